// Decode matvec: GGUF dequantization fused into y = W x for batch-1 decode
// and for routed (per-expert) rows.  Replaces oco's vector kernels
// (shaders/matrix/vector.metal:66-394, q8-dot.metal:39-86,
// mxfp4-dot.metal:9-45, projections.metal:140-182) and the kernel choice of
// Builder::vector_kernel (src/weights/pipelines.rs:227-265).
//
// Geometry.  A 256-thread workgroup is four wavefronts.  A wavefront owns R
// output rows; KS wavefronts may split one row group's K range (partials
// meet in LDS), so a workgroup covers (4/KS)*R rows.  Inside a wavefront, P
// lanes share a GGUF block and each lane decodes one piece, so a step reads
// 64/P consecutive blocks of each of the R rows as one contiguous span.  The
// lane's activation values are loaded once per step and reused by all R
// rows.  The K loop is unrolled so several independent weight loads per lane
// are in flight, which is what a weight stream at HBM speed needs.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "stream.h"
#include "norm.h"

namespace oco {

struct MatvecArgs {
    const uint8_t *w;
    const void *x;
    void *y;
    const float *bias;
    const uint32_t *ids;
    oco_matrix p;
    uint64_t row_bytes;
    int y_bf16;
    int relu_sqr;  // relu² of x on load
};

template <int FMT, typename XT, int R, int KS>
__global__ __launch_bounds__(256) void matvec_kernel(MatvecArgs a) {
    using F = Piece<FMT>;
    constexpr int WAVES = 4, GROUPS = WAVES / KS;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int group = wave / KS, split = wave % KS;
    const oco_matrix &p = a.p;
    const uint32_t row0 = (blockIdx.x * GROUPS + group) * R;
    if (row0 >= p.n) {  // whole wavefront past the end (only when KS == 1: no barrier below)
        if (KS == 1) return;
    }
    const uint32_t route = blockIdx.y;
    const uint32_t expert = p.experts > 1 ? a.ids[route] : 0;
    const uint32_t input = (p.experts > 1 && !p.route_major) ? route / p.routes : route;
    const XT *xr = reinterpret_cast<const XT *>(a.x) + (uint64_t)input * p.k;

    // One buffer resource over this wavefront's R rows; rows past n read as
    // zero (out of the resource's range) and are never stored.
    const uint32_t live = row0 < p.n ? min((uint32_t)R, p.n - row0) : 0u;
    const WSrc src(a.w + ((uint64_t)expert * p.n + row0) * a.row_bytes, (uint64_t)live * a.row_bytes);
    const uint32_t rb = (uint32_t)a.row_bytes;

    const uint32_t blocks = p.k / F::BLOCK;
    constexpr int BPS = 64 / F::P;  // blocks per wavefront step
    const int piece = lane % F::P;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

#pragma unroll 2
    for (uint32_t b = (uint32_t)split * BPS + lane / F::P; b < blocks; b += BPS * KS) {
        typename F::X xv;
        F::load_x(xr, b, piece, xv, a.relu_sqr != 0);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += F::dot(src, r * rb + b * F::BYTES, piece, xv);
    }

#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);

    if (KS > 1) {
        __shared__ float partial[WAVES][R];
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) partial[wave][r] = acc[r];
        }
        __syncthreads();
        if (split != 0) return;
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < KS; j++) s += partial[group * KS + j][r];
            acc[r] = s;
        }
    }

    if (lane < R) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < R; r++)
            if (lane == r) v = acc[r];
        uint32_t row = row0 + lane;
        if (row < p.n) {
            if (p.has_bias)
                v += round_bf16(a.bias[(uint64_t)expert * p.n + row] + (p.has_bias == 2 ? 1.0f : 0.0f));
            uint64_t o = (uint64_t)route * p.n + row;
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(v);
            else
                reinterpret_cast<float *>(a.y)[o] = v;
        }
    }
}

}  // namespace oco

#include "stream_kernel.h"

namespace oco {

static bool streamable(uint32_t fmt) {
    return fmt == OCO_Q8_0 || fmt == OCO_MXFP4 || fmt == OCO_Q4_K || fmt == OCO_Q6_K || fmt == OCO_Q4_0 ||
           fmt == OCO_Q4_1 || fmt == OCO_Q5_K;
}

struct StreamPlan {
    int r, ks, wg_per_cu;
};

// Geometry for the streaming kernel: R rows per half-wavefront, KS
// wavefronts per K range, workgroups per CU (the analogue of
// Builder::vector_kernel's table, pipelines.rs:227-265).
static StreamPlan stream_plan(uint32_t fmt, uint32_t k, uint32_t n, uint32_t m, bool fused_norm) {
    int32_t ov[4];
    if (plan_override(OCO_KNOB_STREAM_PLAN, ov) == 3 && ov[0] > 0) return {ov[0], ov[1], ov[2]};
    uint64_t row_bytes = oco_row_bytes(fmt, k);
    int ks = row_bytes > 6144 ? 4 : row_bytes > 3072 ? 2 : 1;
    // Q8_0 decodes at one conversion and one FMA per weight, so one
    // wavefront per row set holds up while its pieces fit a lane (k <= 4096;
    // measured, 4096 x 4096: 7.28 -> 6.55 us against a K split of 2).  The
    // K-quants lose without the split (lm_head 111 -> 148 us, Q4_K
    // 12288 x 4096 10.9 -> 14.5 us).
    if (fmt == OCO_Q8_0 && k / 32 <= 128) ks = 1;
    (void)m;
    // Workgroups per CU, measured: three pay off on long streams (the 510 MB
    // Q6_K lm_head 3.6 -> 4.2 TB/s) and for MXFP4 and Q4_K at every measured
    // size (the headline 5760 x 2880 5.30 -> 5.17 us, its 720 row groups one
    // per workgroup; Q4_K 12288 x 4096 10.86 -> 10.66 us); mid-size Q5_K and
    // Q6_K lose with three (12288 x 4096 13.6 -> 16.0 us, 4096 x 12288
    // 14.3 -> 15.7 us), and Q8_0 4096 x 4096 is level.  A fused norm, which
    // every workgroup repeats while staging, keeps two (Qwen3-8B's norm +
    // ffn_up + ffn_gate: 24.60 -> 24.17 us against three).
    const bool long_stream = (uint64_t)n * row_bytes > (128ull << 20);
    const int wg = long_stream || (!fused_norm && (fmt == OCO_MXFP4 || fmt == OCO_Q4_K)) ? 3 : 2;
    return {1, ks, wg};
}

typedef void (*MatvecFn)(MatvecArgs);

template <int FMT, typename XT>
static MatvecFn pick(int r, int ks) {
    if (r == 4 && ks == 1) return matvec_kernel<FMT, XT, 4, 1>;
    if (r == 2 && ks == 1) return matvec_kernel<FMT, XT, 2, 1>;
    if (r == 4 && ks == 4) return matvec_kernel<FMT, XT, 4, 4>;
    if (r == 2 && ks == 4) return matvec_kernel<FMT, XT, 2, 4>;
    if (r == 1 && ks == 4) return matvec_kernel<FMT, XT, 1, 4>;
    if (r == 2 && ks == 2) return matvec_kernel<FMT, XT, 2, 2>;
    return matvec_kernel<FMT, XT, 1, 1>;
}

template <typename XT>
static MatvecFn pick_format(uint32_t fmt, int r, int ks) {
    switch (fmt) {
    case OCO_Q8_0: return pick<OCO_Q8_0, XT>(r, ks);
    case OCO_MXFP4: return pick<OCO_MXFP4, XT>(r, ks);
    case OCO_Q4_K: return pick<OCO_Q4_K, XT>(r, ks);
    case OCO_Q5_K: return pick<OCO_Q5_K, XT>(r, ks);
    case OCO_Q6_K: return pick<OCO_Q6_K, XT>(r, ks);
    case OCO_Q4_0: return pick<OCO_Q4_0, XT>(r, ks);
    case OCO_Q4_1: return pick<OCO_Q4_1, XT>(r, ks);
    case OCO_F32: return pick<OCO_F32, XT>(r, ks);
    case OCO_F16: return pick<OCO_F16, XT>(r, ks);
    case OCO_BF16: return pick<OCO_BF16, XT>(r, ks);
    }
    return nullptr;
}

// Geometry table: the analogue of Builder::vector_kernel's per-format
// choice (pipelines.rs:227-265), keyed on the number of wavefront-row
// groups the matrix yields so small matrices still put many independent
// loads in flight on every CU.
struct MatvecPlan {
    int r, ks;
};

MatvecPlan matvec_plan(uint32_t fmt, uint32_t k, uint32_t n, uint32_t m) {
    int32_t ov[4];
    if (plan_override(OCO_KNOB_MATVEC_PLAN, ov) == 2 && ov[0] > 0) return {ov[0], ov[1]};
    uint32_t e, bb;
    oco_block_layout(fmt, &e, &bb);
    uint64_t rows = (uint64_t)n * m;
    uint64_t blocks = k / e;
    // Lanes per block and thus blocks per wavefront step.
    int P = (fmt == OCO_Q8_0) ? 4 : (fmt == OCO_Q4_K || fmt == OCO_Q5_K || fmt == OCO_Q6_K) ? 8
            : (fmt == OCO_MXFP4 || fmt == OCO_Q4_0 || fmt == OCO_Q4_1) ? 2 : 1;
    uint64_t steps = (blocks + 64 / P - 1) / (64 / P);
    // Enough wavefronts for ~16 per CU on 256 CUs before splitting K.
    if (rows >= 16384 * 4) return {4, 1};
    if (rows >= 16384 * 2) return {2, 1};
    if (steps >= 4) return rows >= 8192 ? MatvecPlan{2, 4} : MatvecPlan{1, 4};
    return {2, 1};
}

}  // namespace oco

using namespace oco;

struct NormSpec {
    const float *w;
    float epsilon;
    int full_layer;
};

// Several matrices of one format and shape over the same input rows, in one
// grid (oco_matvec_group).
struct GroupSpec {
    uint32_t count;
    const void *const *w;
    void *const *y;
    const float *const *bias;
};

namespace oco {
// The grouped kernels, instantiated in matvec_group.hip.
StreamFn stream_pick_group(bool x_bf16, uint32_t fmt, int xs, int npl, bool direct, int &lpr);
}

// oco_matvec, optionally with the RMS norm of each bf16 input row fused
// into the streaming kernel's staging (norm != nullptr, x bf16).  Formats
// without a streaming kernel normalise into a stream-ordered temporary first.
static int matvec_impl(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                       oco_dtype y_dtype, const float *bias, const uint32_t *ids, const oco_matrix *p,
                       const NormSpec *norm, oco_stream stream, const GroupSpec *grp = nullptr,
                       bool relu_sqr = false) {
    if (!p || !w || !x || !y) return fail(OCO_ERR_INVALID, "oco_matvec: null argument");
    if (relu_sqr && (norm || grp)) return fail(OCO_ERR_INVALID, "oco_matvec: relu_sqr takes neither a norm nor a group");
    uint32_t e, bb;
    OCO_TRY(oco_block_layout(format, &e, &bb));
    uint32_t align = e;
    if (format == OCO_F32) align = 4;
    if (format == OCO_F16 || format == OCO_BF16) align = 8;
    if (p->k == 0 || p->k % align)
        return fail(OCO_ERR_INVALID, "oco_matvec: k=%u is not a multiple of %u", p->k, align);
    if (p->n == 0 || p->m == 0) return OCO_OK;
    if (p->m > 65535) return fail(OCO_ERR_INVALID, "oco_matvec: m=%u exceeds 65535 routes", p->m);
    if (p->experts > 1 && !ids) return fail(OCO_ERR_INVALID, "oco_matvec: routed matrix needs ids");
    if (p->has_bias && !bias) return fail(OCO_ERR_INVALID, "oco_matvec: has_bias without bias");
    if (p->experts > 1 && !p->route_major && p->routes == 0)
        return fail(OCO_ERR_INVALID, "oco_matvec: routes must be > 0");
    if (x_dtype != OCO_DT_F32 && x_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: activations must be f32 or bf16");
    if (y_dtype != OCO_DT_F32 && y_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: output must be f32 or bf16");
    const int routed_f32 = p->experts > 1 && !p->route_major;
    int32_t plain[4];
    // The streaming kernel reads x in 16-byte (f32) or 8-byte (bf16) vectors.
    const bool x_vec = ((uintptr_t)x & (x_dtype == OCO_DT_F32 ? 15u : 7u)) == 0;
    if (streamable(format) && x_vec && !(plan_override(OCO_KNOB_MATVEC_PLAIN, plain) && plain[0])) {
        static int cus = 0;
        if (!cus) {
            int dev = 0;
            hipGetDevice(&dev);
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
            if (cus <= 0) cus = 256;
        }
        uint32_t be, bbytes;
        oco_block_layout(format, &be, &bbytes);
        const uint32_t P = (format == OCO_Q4_K || format == OCO_Q5_K || format == OCO_Q6_K) ? 8 : 1;
        const uint32_t nblocks = p->k / be;
        const uint32_t nmat = grp ? grp->count : 1u;
        StreamPlan sp = stream_plan(format, p->k, p->n * nmat, p->m, norm != nullptr && !grp);
        if (sp.ks != 1 && sp.ks != 2 && sp.ks != 4) sp.ks = 1;
        uint32_t slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
        int npl = (int)((slice_blocks * P + 31) / 32);
        while (npl > 4 && sp.ks < 4) {  // widen the K split until a lane's pieces fit
            sp.ks *= 2;
            slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
            npl = (int)((slice_blocks * P + 31) / 32);
        }
        // Q4_K / Q5_K blocks are whole 16-byte chunks: on a 16-byte aligned
        // base every lane loads its own pieces (OCO_KNOB_STREAM_DIRECT 0 turns
        // this off).
        int32_t dov[4];
        bool aligned = ((uintptr_t)w & 15u) == 0;
        for (uint32_t i = 0; grp && i < grp->count; i++) aligned = aligned && ((uintptr_t)grp->w[i] & 15u) == 0;
        const bool direct = (format == OCO_Q4_K || format == OCO_Q5_K) && aligned &&
                            !(plan_override(OCO_KNOB_STREAM_DIRECT, dov) && dov[0] == 0);
        // Direct loads hold three register sets of pieces: past two pieces per
        // lane that costs occupancy, so split K further (measured: Q4_K and
        // Q5_K 12288 x 4096, 14.7 -> 11.1 us).
        int32_t sov[4];
        while (direct && npl > 2 && sp.ks < 4 && plan_override(OCO_KNOB_STREAM_PLAN, sov) != 3) {
            sp.ks *= 2;
            slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
            npl = (int)((slice_blocks * P + 31) / 32);
        }
        // Where the activations come from: a fused norm stages them through
        // LDS; otherwise rows past 8192 values read them straight into
        // registers, since staged x would take LDS that occupancy needs
        // (measured, Q6_K 4096 x 12288: 15.2 -> 14.5 us), while shorter rows
        // stage (MXFP4 5760 x 2880: 5.25 us staged, 7.7 us from registers).
        // OCO_KNOB_STREAM_DIRECT's second value, when given, picks: 0 staged,
        // 1 registers.
        int xs = norm ? (norm->full_layer ? XS_NORM_FULL : XS_NORM) : p->k > 8192 ? XS_REG : XS_STAGED;
        if (!norm && plan_override(OCO_KNOB_STREAM_DIRECT, dov) >= 2) xs = dov[1] ? XS_REG : XS_STAGED;
        int lpr = 0;
        StreamFn fn = npl > 4  ? nullptr
                    : grp      ? stream_pick_group(x_dtype == OCO_DT_BF16, format, xs, npl, direct, lpr)
                    : x_dtype == OCO_DT_F32 ? stream_pick_format<float, false>(format, xs, npl, direct, lpr)
                                            : stream_pick_format<bf16_t, false>(format, xs, npl, direct, lpr);
        if (fn) {
            StreamArgs a;
            a.w = (const uint8_t *)w;
            a.x = x;
            a.y = y;
            a.bias = bias;
            a.ids = ids;
            a.p = *p;
            a.row_bytes = oco_row_bytes(format, p->k);
            a.y_bf16 = (y_dtype == OCO_DT_BF16) && !routed_f32;
            a.ks = sp.ks;
            a.slice_blocks = slice_blocks;
            a.norm_mode = norm ? (norm->full_layer ? 2u : 1u) : 0u;
            a.norm_eps = norm ? norm->epsilon : 0.f;
            a.norm_w = norm ? norm->w : nullptr;
            const uint32_t rows_per_group = (4 / sp.ks) * 2;
            a.ngroups = (p->n + rows_per_group - 1) / rows_per_group;
            a.nmat = nmat;
            for (uint32_t i = 0; i < OCO_MATVEC_GROUP_MAX; i++) {
                a.wm[i] = grp && i < nmat ? (const uint8_t *)grp->w[i] : nullptr;
                a.ym[i] = grp && i < nmat ? grp->y[i] : nullptr;
                a.bm[i] = grp && i < nmat && grp->bias ? grp->bias[i] : nullptr;
            }
            const uint32_t nsum = (format == OCO_Q8_0 || format == OCO_Q4_0 || format == OCO_Q4_1) ? 1
                                  : (format == OCO_Q4_K || format == OCO_Q5_K)                    ? 2
                                  : format == OCO_Q6_K                                            ? 4
                                                                                                  : 0;
            const size_t tile = direct ? 0 : (size_t)2 * lpr * 1024;
            const size_t xbytes = xs != XS_REG ? (size_t)p->k * 4 + (size_t)nsum * (p->k / 32) * 4 : 0;
            const size_t lds = xbytes + 4 * tile + 32 * sizeof(float);
            if (lds > 160 * 1024)
                return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: k=%u needs %zu bytes of LDS", p->k, lds);
            if (lds > 64 * 1024)
                OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn,
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                                  "hipFuncSetAttribute"));
            const uint32_t grid = std::min<uint32_t>(a.ngroups * nmat, (uint32_t)(cus * sp.wg_per_cu));
            if (a.p.routes > 0x7fffffffu) return fail(OCO_ERR_INVALID, "oco_matvec: routes=%u", a.p.routes);
            const uint32_t mode = (sp.ks == 4 ? 2u : sp.ks == 2 ? 1u : 0u) | (relu_sqr ? 4u : 0u);
            hipLaunchKernelGGL(fn, dim3(grid, p->m), dim3(256), lds, (hipStream_t)stream, a.w, a.x,
                               (uint32_t)a.row_bytes, a.p.n, a.p.k, mode, a.slice_blocks, a.ngroups, a.p.experts,
                               a.p.routes | (a.p.route_major ? 0x80000000u : 0u), a);
            return launch_check("oco_matvec");
        }
    }
    if (grp) {  // no streaming kernel: one call per matrix
        for (uint32_t i = 0; i < grp->count; i++)
            OCO_TRY(matvec_impl(format, grp->w[i], x, x_dtype, grp->y[i], y_dtype, grp->bias ? grp->bias[i] : nullptr,
                                ids, p, norm, stream));
        return OCO_OK;
    }
    if (norm) {  // no streaming kernel: normalise the input rows, then the plain matvec
        const uint32_t in_rows =
            (p->experts > 1 && !p->route_major) ? (p->m + p->routes - 1) / p->routes : p->m;
        void *tmp = nullptr;
        const size_t bytes = (size_t)in_rows * p->k * 2;
        OCO_TRY(hip_check(hipMallocAsync(&tmp, bytes, (hipStream_t)stream), "oco_matvec_norm: hipMallocAsync"));
        int rc = oco_norm(x, norm->w, tmp, in_rows, p->k, norm->epsilon, norm->full_layer, stream);
        if (rc == OCO_OK) rc = matvec_impl(format, w, tmp, OCO_DT_BF16, y, y_dtype, bias, ids, p, nullptr, stream);
        const int rc2 = hip_check(hipFreeAsync(tmp, (hipStream_t)stream), "oco_matvec_norm: hipFreeAsync");
        return rc != OCO_OK ? rc : rc2;
    }
    MatvecPlan plan = matvec_plan(format, p->k, p->n, p->m);
    MatvecFn fn = x_dtype == OCO_DT_F32 ? pick_format<float>(format, plan.r, plan.ks)
                                        : pick_format<bf16_t>(format, plan.r, plan.ks);
    if (!fn) return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: format %u", format);
    MatvecArgs a;
    a.w = (const uint8_t *)w;
    a.x = x;
    a.y = y;
    a.bias = bias;
    a.ids = ids;
    a.p = *p;
    a.row_bytes = oco_row_bytes(format, p->k);
    // Routed, non-route-major outputs are always f32 (vector.metal:142-146).
    a.y_bf16 = (y_dtype == OCO_DT_BF16) && !(p->experts > 1 && !p->route_major);
    a.relu_sqr = relu_sqr;
    uint32_t rows_per_group = (4 / plan.ks) * plan.r;
    dim3 grid((p->n + rows_per_group - 1) / rows_per_group, p->m);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    return launch_check("oco_matvec");
}


extern "C" int oco_matvec(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                          oco_dtype y_dtype, const float *bias, const uint32_t *ids,
                          const oco_matrix *p, oco_stream stream) {
    return matvec_impl(format, w, x, x_dtype, y, y_dtype, bias, ids, p, nullptr, stream);
}

extern "C" int oco_matvec_relu_sqr(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                                   oco_dtype y_dtype, const float *bias, const uint32_t *ids, const oco_matrix *p,
                                   oco_stream stream) {
    return matvec_impl(format, w, x, x_dtype, y, y_dtype, bias, ids, p, nullptr, stream, nullptr, true);
}

extern "C" int oco_matvec_norm(uint32_t format, const void *w, const void *x, const float *norm_w, float epsilon,
                               int full_layer, void *y, oco_dtype y_dtype, const float *bias,
                               const uint32_t *ids, const oco_matrix *p, oco_stream stream) {
    if (!norm_w) return fail(OCO_ERR_INVALID, "oco_matvec_norm: null norm weights");
    const NormSpec n{norm_w, epsilon, full_layer};
    return matvec_impl(format, w, x, OCO_DT_BF16, y, y_dtype, bias, ids, p, &n, stream);
}

extern "C" int oco_matvec_group(uint32_t format, uint32_t count, const void *const *w, const void *x,
                                oco_dtype x_dtype, const float *norm_w, float epsilon, int full_layer,
                                void *const *y, oco_dtype y_dtype, const float *const *bias, const oco_matrix *p,
                                oco_stream stream) {
    if (!w || !y || !p) return fail(OCO_ERR_INVALID, "oco_matvec_group: null argument");
    if (count == 0 || count > OCO_MATVEC_GROUP_MAX)
        return fail(OCO_ERR_INVALID, "oco_matvec_group: count=%u is not 1..%u", count, OCO_MATVEC_GROUP_MAX);
    if (p->experts > 1) return fail(OCO_ERR_UNSUPPORTED, "oco_matvec_group: routed matrices go through oco_matvec");
    for (uint32_t i = 0; i < count; i++) {
        if (!w[i] || !y[i]) return fail(OCO_ERR_INVALID, "oco_matvec_group: null matrix or output %u", i);
        if (p->has_bias && (!bias || !bias[i])) return fail(OCO_ERR_INVALID, "oco_matvec_group: has_bias without bias %u", i);
    }
    if (norm_w && x_dtype != OCO_DT_BF16) return fail(OCO_ERR_UNSUPPORTED, "oco_matvec_group: the fused norm takes bf16 rows");
    const NormSpec n{norm_w, epsilon, full_layer};
    const GroupSpec g{count, w, y, bias};
    return matvec_impl(format, w[0], x, x_dtype, y[0], y_dtype, bias ? bias[0] : nullptr, nullptr, p,
                       norm_w ? &n : nullptr, stream, &g);
}
