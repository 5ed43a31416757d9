// Prefill matmul on CDNA4 MFMA: Y[m, n] = X[m, k] W[n, k]^T (+ bias) with
// GGUF-block weights dequantized into LDS.  Replaces DenseMatrix::apply's
// tiled plans (src/weights/compute/matrix.rs:130-379: `matmul`,
// `matmul_q4*`, `matmul_tensor_*`, shaders/matrix/batch.metal:24-79,
// tensor.metal:9-102).
//
// Operands: MXFP4 weights (E2M1 x 2^e) and bf16 activations are exact in
// bf16, so MXFP4 runs v_mfma_f32_16x16x32_bf16 with exact products.  The
// other formats decode to f16 -- the reference's half(w) operand
// (tile.metal:16-80) -- and the activations convert to f16, on
// v_mfma_f32_16x16x32_f16.  Accumulation is fp32.
//
// Tile: a 256-thread workgroup computes 64 activation rows x 64 weight rows;
// each wavefront owns a 32 x 32 quadrant as 2 x 2 MFMA blocks.  K advances
// 32 at a time (one Q8_0/MXFP4 block, an eighth of a K-quant super-block).
#include "formats.h"

namespace oco {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MatmulArgs {
    const uint8_t *w;
    const void *x;
    void *y;
    const float *bias;
    uint32_t m, n, k;
    uint64_t row_bytes;
    uint32_t x_f16, y_bf16;
};

// 16-bit operand bits of a float: bf16 (round to nearest even) or f16.
template <bool BF>
__device__ __forceinline__ uint16_t operand_bits(float v) {
    if constexpr (BF) {
        return f32_to_bf16_bits(v);
    } else {
        _Float16 h = (_Float16)v;
        uint16_t b;
        __builtin_memcpy(&b, &h, 2);
        return b;
    }
}

template <int FMT>
struct BlockShape {
    static constexpr uint32_t BE = FMT == OCO_F32 || FMT == OCO_F16 || FMT == OCO_BF16 ? 1
                                   : (FMT == OCO_Q4_K || FMT == OCO_Q5_K || FMT == OCO_Q6_K) ? 256 : 32;
    static constexpr uint32_t BB = FMT == OCO_F32 ? 4 : (FMT == OCO_F16 || FMT == OCO_BF16) ? 2
                                   : FMT == OCO_Q4_0 ? 18 : FMT == OCO_Q4_1 ? 20 : FMT == OCO_Q8_0 ? 34
                                   : FMT == OCO_Q4_K ? 144 : FMT == OCO_Q5_K ? 176 : FMT == OCO_Q6_K ? 210 : 17;
};

template <int FMT, bool BF>
__global__ __launch_bounds__(256) void matmul_kernel(MatmulArgs a) {
    constexpr int BM = 64, BN = 64, BK = 32, LD = BK + 8;  // LDS row stride in 16-bit words (80 bytes)
    __shared__ __attribute__((aligned(16))) uint16_t xs[BM * LD];
    __shared__ __attribute__((aligned(16))) uint16_t ws[BN * LD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int tm = (wave >> 1) * 32, tn = (wave & 1) * 32;
    const int srow = tid >> 2, schunk = (tid & 3) * 8;  // staging: 64 rows x 4 chunks of 8

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t xrow = m0 + srow, wrow = n0 + srow;
    const uint8_t *wr = a.w + (uint64_t)min(wrow, a.n - 1) * a.row_bytes;
    for (uint32_t k0 = 0; k0 < a.k; k0 += BK) {
        // Activations: 8 consecutive values of one row per thread.
        uint16_t xv[8];
        if (xrow < a.m) {
            uint4 raw = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.x) +
                                                         (uint64_t)xrow * a.k + k0 + schunk);
            const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint16_t lo = (uint16_t)(w4[i] & 0xffffu), hi = (uint16_t)(w4[i] >> 16);
                if (!BF && !a.x_f16) {  // bf16 -> f16
                    lo = operand_bits<false>(bf16_bits_to_f32(lo));
                    hi = operand_bits<false>(bf16_bits_to_f32(hi));
                }
                xv[2 * i] = lo;
                xv[2 * i + 1] = hi;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) xv[i] = 0;
        }
        // Weights: decode 8 coefficients of one row.
        uint16_t wv[8];
        {
            constexpr uint32_t BE = BlockShape<FMT>::BE, BB = BlockShape<FMT>::BB;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t col = k0 + schunk + i;
                wv[i] = operand_bits<BF>(decode_scalar(FMT, wr + (uint64_t)(col / BE) * BB, col % BE));
            }
        }
        __syncthreads();  // previous step's fragments are consumed
        *reinterpret_cast<uint4 *>(&xs[srow * LD + schunk]) =
            make_uint4(xv[0] | (uint32_t)xv[1] << 16, xv[2] | (uint32_t)xv[3] << 16, xv[4] | (uint32_t)xv[5] << 16,
                       xv[6] | (uint32_t)xv[7] << 16);
        *reinterpret_cast<uint4 *>(&ws[srow * LD + schunk]) =
            make_uint4(wv[0] | (uint32_t)wv[1] << 16, wv[2] | (uint32_t)wv[3] << 16, wv[4] | (uint32_t)wv[5] << 16,
                       wv[6] | (uint32_t)wv[7] << 16);
        __syncthreads();
        // Fragments: lane l holds row/column l % 16, k = 8 (l / 16) .. + 8.
        const int fr = lane & 15, fk = (lane >> 4) * 8;
        uint4 af[2], bfm[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            af[i] = *reinterpret_cast<const uint4 *>(&xs[(tm + i * 16 + fr) * LD + fk]);
            bfm[i] = *reinterpret_cast<const uint4 *>(&ws[(tn + i * 16 + fr) * LD + fk]);
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if constexpr (BF) {
                    bf16x8 av, bv;
                    __builtin_memcpy(&av, &af[i], 16);
                    __builtin_memcpy(&bv, &bfm[j], 16);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[i][j], 0, 0, 0);
                } else {
                    f16x8 av, bv;
                    __builtin_memcpy(&av, &af[i], 16);
                    __builtin_memcpy(&bv, &bfm[j], 16);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[i][j], 0, 0, 0);
                }
            }
    }
    // C fragment: lane l holds column l % 16, rows 4 (l / 16) .. + 4.
    const int cc = lane & 15, cr = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t col = n0 + tn + j * 16 + cc;
            if (col >= a.n) continue;
            const float b = a.bias ? round_bf16(a.bias[col]) : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t row = m0 + tm + i * 16 + cr + v;
                if (row >= a.m) continue;
                const float r = acc[i][j][v] + b;
                const uint64_t o = (uint64_t)row * a.n + col;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(r);
                else
                    reinterpret_cast<float *>(a.y)[o] = r;
            }
        }
}

typedef void (*MatmulFn)(MatmulArgs);

static MatmulFn matmul_pick(uint32_t fmt) {
    switch (fmt) {
    case OCO_MXFP4: return matmul_kernel<OCO_MXFP4, true>;
    case OCO_BF16: return matmul_kernel<OCO_BF16, true>;
    case OCO_Q8_0: return matmul_kernel<OCO_Q8_0, false>;
    case OCO_Q4_K: return matmul_kernel<OCO_Q4_K, false>;
    case OCO_Q5_K: return matmul_kernel<OCO_Q5_K, false>;
    case OCO_Q6_K: return matmul_kernel<OCO_Q6_K, false>;
    case OCO_Q4_0: return matmul_kernel<OCO_Q4_0, false>;
    case OCO_Q4_1: return matmul_kernel<OCO_Q4_1, false>;
    case OCO_F16: return matmul_kernel<OCO_F16, false>;
    case OCO_F32: return matmul_kernel<OCO_F32, false>;
    }
    return nullptr;
}

}  // namespace oco

using namespace oco;

extern "C" int oco_matmul(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                          oco_dtype y_dtype, const float *bias, const oco_matrix *p, oco_stream stream) {
    if (!p || !w || !x || !y) return fail(OCO_ERR_INVALID, "oco_matmul: null argument");
    uint32_t e, bb;
    OCO_TRY(oco_block_layout(format, &e, &bb));
    if (p->k == 0 || p->k % 32 || p->k % e)
        return fail(OCO_ERR_INVALID, "oco_matmul: k=%u must be a multiple of 32 and of the block", p->k);
    if (p->m == 0 || p->n == 0) return OCO_OK;
    if (p->experts > 1) return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: routed rows go through oco_experts_apply");
    if (p->has_bias && !bias) return fail(OCO_ERR_INVALID, "oco_matmul: has_bias without bias");
    if (x_dtype != OCO_DT_BF16 && x_dtype != OCO_DT_F16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: activations must be bf16 or f16");
    if (x_dtype == OCO_DT_F16 && (format == OCO_MXFP4 || format == OCO_BF16))
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: MXFP4/BF16 weights take bf16 activations");
    if (y_dtype != OCO_DT_F32 && y_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: output must be f32 or bf16");
    MatmulFn fn = matmul_pick(format);
    if (!fn) return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: format %u", format);
    MatmulArgs a;
    a.w = (const uint8_t *)w;
    a.x = x;
    a.y = y;
    a.bias = p->has_bias ? bias : nullptr;
    a.m = p->m;
    a.n = p->n;
    a.k = p->k;
    a.row_bytes = oco_row_bytes(format, p->k);
    a.x_f16 = x_dtype == OCO_DT_F16;
    a.y_bf16 = y_dtype == OCO_DT_BF16;
    dim3 grid((p->n + 63) / 64, (p->m + 63) / 64);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    return launch_check("oco_matmul");
}
