// The steps either side of the decode matvec: RMS normalisation of the bf16
// activation rows before it (norm / add_norm, shaders/elementwise.metal:6-58)
// and greedy token selection over the f32 logits after the lm_head
// (argmax_f32, shaders/argmax.metal:1-47).
//
// The row statistic is computed by one routine, block_inv_rms (norm.h),
// shared with the streaming matvec's fused-norm staging, so a fused and an
// unfused path see the same inverse RMS, bit for bit.
#include "norm.h"

namespace oco {

// ---- RMS norm ------------------------------------------------------------------

template <bool ADD>
__global__ __launch_bounds__(256) void norm_kernel(uint16_t *x, const uint16_t *y, const float *w, uint16_t *out,
                                                   uint32_t n, float epsilon, uint32_t full_layer) {
    __shared__ float partial[4];
    uint16_t *xr = x + (uint64_t)blockIdx.x * n;
    uint16_t *orow = out + (uint64_t)blockIdx.x * n;
    if constexpr (ADD) {  // the residual stream takes bf16(x + y) first (elementwise.metal:41-43)
        const uint16_t *yr = y + (uint64_t)blockIdx.x * n;
        for (uint32_t i = threadIdx.x; i < n; i += 256)
            xr[i] = f32_to_bf16_bits(bf16_bits_to_f32(xr[i]) + bf16_bits_to_f32(yr[i]));
        __syncthreads();  // each thread re-reads only its own elements, but keep the order explicit
    }
    const float inv = block_inv_rms(xr, n, epsilon, partial);
    // eight values per thread through 16-byte accesses when every row is aligned
    uint32_t i0 = 0;
    if ((((uintptr_t)xr | (uintptr_t)orow | (uintptr_t)w) & 15u) == 0) {
        for (uint32_t c = threadIdx.x; 8 * c + 8 <= n; c += 256) {
            const uint4 u = *reinterpret_cast<const uint4 *>(xr + 8 * c);
            const float4 w0 = *reinterpret_cast<const float4 *>(w + 8 * c), w1 = *reinterpret_cast<const float4 *>(w + 8 * c + 4);
            const uint32_t h[4] = {u.x, u.y, u.z, u.w};
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                o[j] = (uint32_t)norm_value_bits(__uint_as_float(h[j] << 16), inv, wv[2 * j], full_layer) |
                       ((uint32_t)norm_value_bits(__uint_as_float(h[j] & 0xffff0000u), inv, wv[2 * j + 1], full_layer) << 16);
            *reinterpret_cast<uint4 *>(orow + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
        }
        i0 = n / 8 * 8;
    }
    for (uint32_t i = i0 + threadIdx.x; i < n; i += 256) orow[i] = norm_value_bits(bf16_bits_to_f32(xr[i]), inv, w[i], full_layer);
}

// ---- argmax ----------------------------------------------------------------------

// Order key of a logit (argmax.metal:11-17): finite values as integers after
// folding the sign, -0 as +0; packed with the complement of the index so
// that the 64-bit maximum is the largest value at the lowest index.  Key 0 is
// below every finite logit (no element yet).
__device__ __forceinline__ uint64_t argmax_pack(float f, uint32_t i, uint32_t &bad) {
    uint32_t bits = __float_as_uint(f);
    if ((bits & 0x7f800000u) == 0x7f800000u) {
        bad = 1;
        return 0;
    }
    bits = (bits & 0x7fffffffu) == 0 ? 0u : bits;
    const uint32_t v = bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
    return ((uint64_t)v << 32) | (uint32_t)~i;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Workgroup-wide (max pack, OR bad) into thread 0.
__device__ __forceinline__ void argmax_block(uint64_t &best, uint32_t &bad, uint64_t *sb, uint32_t *sf) {
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, o), hi = (uint32_t)__shfl_xor((int)(best >> 32), o);
        best = max_u64(best, ((uint64_t)hi << 32) | lo);
        bad |= (uint32_t)__shfl_xor((int)bad, o);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sb[wave] = best;
        sf[wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int v = 1; v < (int)(blockDim.x >> 6); v++) {
            best = max_u64(best, sb[v]);
            bad |= sf[v];
        }
    }
}

// Pass 1: each workgroup's (pack, bad) over a grid-strided range; with one
// workgroup the answer goes straight to `out`.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *x, uint32_t n, uint64_t *part_best,
                                                             uint32_t *part_bad, uint32_t *out) {
    __shared__ uint64_t sb[4];
    __shared__ uint32_t sf[4];
    uint64_t best = 0;
    uint32_t bad = 0;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
        best = max_u64(best, argmax_pack(x[i], i, bad));
    argmax_block(best, bad, sb, sf);
    if (threadIdx.x == 0) {
        if (gridDim.x == 1) {
            out[0] = bad ? 0xffffffffu : ~(uint32_t)best;
        } else {
            part_best[blockIdx.x] = best;
            part_bad[blockIdx.x] = bad;
        }
    }
}

// Pass 2: one workgroup over the partials.
__global__ __launch_bounds__(256) void argmax_final_kernel(const uint64_t *part_best, const uint32_t *part_bad,
                                                           uint32_t parts, uint32_t *out) {
    __shared__ uint64_t sb[4];
    __shared__ uint32_t sf[4];
    uint64_t best = 0;
    uint32_t bad = 0;
    for (uint32_t i = threadIdx.x; i < parts; i += 256) {
        best = max_u64(best, part_best[i]);
        bad |= part_bad[i];
    }
    argmax_block(best, bad, sb, sf);
    if (threadIdx.x == 0) out[0] = bad ? 0xffffffffu : ~(uint32_t)best;
}

}  // namespace oco

using namespace oco;

extern "C" int oco_norm(const void *x, const float *w, void *y, uint32_t rows, uint32_t n, float epsilon,
                        int full_layer, oco_stream stream) {
    if (rows == 0 || n == 0) return OCO_OK;
    if (!x || !w || !y) return fail(OCO_ERR_INVALID, "oco_norm: null pointer");
    if (rows > 0x7fffffffu) return fail(OCO_ERR_INVALID, "oco_norm: %u rows", rows);
    hipLaunchKernelGGL(norm_kernel<false>, dim3(rows), dim3(256), 0, (hipStream_t)stream,
                       const_cast<uint16_t *>((const uint16_t *)x), (const uint16_t *)nullptr, w, (uint16_t *)y, n,
                       epsilon, (uint32_t)(full_layer != 0));
    return launch_check("oco_norm");
}

extern "C" int oco_add_norm(void *x, const void *y, const float *w, void *out, uint32_t rows, uint32_t n,
                            float epsilon, int full_layer, oco_stream stream) {
    if (rows == 0 || n == 0) return OCO_OK;
    if (!x || !y || !w || !out) return fail(OCO_ERR_INVALID, "oco_add_norm: null pointer");
    if (rows > 0x7fffffffu) return fail(OCO_ERR_INVALID, "oco_add_norm: %u rows", rows);
    hipLaunchKernelGGL(norm_kernel<true>, dim3(rows), dim3(256), 0, (hipStream_t)stream, (uint16_t *)x,
                       (const uint16_t *)y, w, (uint16_t *)out, n, epsilon, (uint32_t)(full_layer != 0));
    return launch_check("oco_add_norm");
}

// Partials: up to 256 workgroups, each over >= 8 elements per thread.
static uint32_t argmax_parts(uint32_t n) {
    const uint32_t by_work = (n + 256 * 8 - 1) / (256 * 8);
    return by_work < 1 ? 1 : by_work > 256 ? 256 : by_work;
}

extern "C" uint64_t oco_argmax_workspace(uint32_t n) {
    const uint32_t parts = argmax_parts(n);
    return parts == 1 ? 0 : (uint64_t)parts * 12;
}

extern "C" int oco_argmax_f32_ws(const float *logits, uint32_t n, uint32_t *out, void *workspace,
                                 uint64_t workspace_bytes, oco_stream stream) {
    if (!out) return fail(OCO_ERR_INVALID, "oco_argmax_f32: null output");
    if (n && !logits) return fail(OCO_ERR_INVALID, "oco_argmax_f32: null logits");
    const uint32_t parts = argmax_parts(n);
    if (parts > 1 && (!workspace || workspace_bytes < (uint64_t)parts * 12))
        return fail(OCO_ERR_INVALID, "oco_argmax_f32_ws: workspace of %llu bytes, need %llu",
                    (unsigned long long)workspace_bytes, (unsigned long long)parts * 12);
    uint64_t *best = (uint64_t *)workspace;
    uint32_t *bad = parts > 1 ? (uint32_t *)(best + parts) : nullptr;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(256), 0, (hipStream_t)stream, logits, n, best, bad,
                       out);
    OCO_TRY(launch_check("oco_argmax_f32"));
    if (parts > 1) {
        hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, best, bad, parts, out);
        OCO_TRY(launch_check("oco_argmax_f32 (final)"));
    }
    return OCO_OK;
}

extern "C" int oco_argmax_f32(const float *logits, uint32_t n, uint32_t *out, oco_stream stream) {
    const uint64_t need = oco_argmax_workspace(n);
    if (!need) return oco_argmax_f32_ws(logits, n, out, nullptr, 0, stream);
    void *ws = nullptr;
    OCO_TRY(hip_check(hipMallocAsync(&ws, need, (hipStream_t)stream), "oco_argmax_f32: hipMallocAsync"));
    const int rc = oco_argmax_f32_ws(logits, n, out, ws, need, stream);
    const int rc2 = hip_check(hipFreeAsync(ws, (hipStream_t)stream), "oco_argmax_f32: hipFreeAsync");
    return rc != OCO_OK ? rc : rc2;
}
