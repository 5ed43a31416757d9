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
#include "formats.h"

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
};

template <int FMT, typename XT, int R, int KS>
__global__ __launch_bounds__(256) void matvec_kernel(MatvecArgs a) {
    using F = Piece<FMT>;
    constexpr int WAVES = 4, GROUPS = WAVES / KS;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int group = wave / KS, split = wave % KS;
    const oco_matrix &p = a.p;
    const uint32_t row0 = (blockIdx.x * GROUPS + group) * R;
    const uint32_t route = blockIdx.y;
    const uint32_t expert = p.experts > 1 ? a.ids[route] : 0;
    const uint32_t input = (p.experts > 1 && !p.route_major) ? route / p.routes : route;
    const XT *xr = reinterpret_cast<const XT *>(a.x) + (uint64_t)input * p.k;

    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t row = min(row0 + r, p.n - 1);  // tail rows re-read the last row, never stored
        rows[r] = a.w + ((uint64_t)expert * p.n + row) * a.row_bytes;
    }

    const uint32_t blocks = p.k / F::BLOCK;
    constexpr int BPS = 64 / F::P;  // blocks per wavefront step
    const int piece = lane % F::P;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

#pragma unroll 2
    for (uint32_t b = (uint32_t)split * BPS + lane / F::P; b < blocks; b += BPS * KS) {
        typename F::X xv;
        F::load_x(xr, b, piece, xv);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += F::dot(rows[r] + (uint64_t)b * F::BYTES, piece, xv);
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

extern "C" int oco_matvec(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                          oco_dtype y_dtype, const float *bias, const uint32_t *ids,
                          const oco_matrix *p, oco_stream stream) {
    if (!p || !w || !x || !y) return fail(OCO_ERR_INVALID, "oco_matvec: null argument");
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
    uint32_t rows_per_group = (4 / plan.ks) * plan.r;
    dim3 grid((p->n + rows_per_group - 1) / rows_per_group, p->m);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    return launch_check("oco_matvec");
}
