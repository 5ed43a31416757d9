// Routed expert path for decode: gate/up projections of the selected experts
// with the activation fused, the down projection, and the weighted combine.
// Replaces oco's Bindings::experts (src/weights/compute/feed_forward.rs:
// 107-275) with its kernels expert_expand (projections.metal:78-137),
// matvec_mxfp4 (:140-182) and moe_sum (routing.metal:157-168).
//
// Each workgroup takes one tile of the route plan -- one expert and up to T
// of the routes that chose it -- and streams that expert's rows once through
// the LDS tile path of the decode matvec (stream.h), applying every row to
// all of the tile's routes.  An expert picked by several tokens is therefore
// read from HBM once per call, not once per route; experts nobody picked are
// never touched.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "matmul.h"
#include "route.h"
#include "stream.h"

#include <atomic>
#include <mutex>

namespace oco {

// The first 56 bytes arrive in SGPRs (KPre): what the tile choice and the
// first weight loads depend on comes first.
struct MoeArgs {
    const uint8_t *w[2];     // gated: {gate, up}; otherwise {down, unused}
    const float *logits;     // single token: select the experts in-kernel
    const uint32_t *ids;     // [routes] expert per route (no plan, no logits)
    const uint32_t *plan;    // route plan (tile = (expert, first row)) or null (tile = route)
    uint32_t k, n, experts, topk;
    const void *x;           // activations
    uint32_t x_bf16;         // activation element type
    uint32_t input_div;      // route -> activation row: route / input_div
    const float *bias[2];    // per-matrix f32 biases [experts * n] or null
    float *out0, *out1;      // gated: activation, up (may be null); otherwise y
    uint32_t *ids_out;       // with logits: selected ids / probabilities
    float *probs_out;
    uint32_t routes;
    uint64_t row_bytes;
    uint32_t ngroups;
    uint32_t act, up_one;
};

__device__ __forceinline__ float activation(uint32_t act, float g, float u) {
    if ((__float_as_uint(g) & 0x7f800000u) == 0x7f800000u || (__float_as_uint(u) & 0x7f800000u) == 0x7f800000u)
        return __uint_as_float(0x7fc00000u);
    if (act == OCO_ACT_SWIGLU_CLIPPED) {  // projections.metal:4-13
        g = fminf(g, 7.0f);
        u = fminf(fmaxf(u, -6.0f), 8.0f);
        float e = expf(-fabsf(g) * 1.702f);
        float sig = (g < 0 ? e : 1.0f) / (1.0f + e);
        return sig * g * u;
    }
    float e = expf(-fabsf(g));  // silu(g) * u (elementwise.metal:70-88, in f32)
    float sig = (g < 0 ? e : 1.0f) / (1.0f + e);
    return sig * g * u;
}

constexpr uint32_t PLAN_TILE = 16;  // routes per route-plan tile (its minimum, see oco_route_plan)

template <int FMT, bool GATED, int T, int NPL>
__global__ __launch_bounds__(256) void moe_kernel(KPRE_PARAMS, MoeArgs a) {
    KPRE_APPLY(a);
    using Tl = Tile<FMT>;
    a.row_bytes = (uint64_t)(a.k / Tl::BLOCK) * Tl::BYTES;
    constexpr int NM = GATED ? 2 : 1;             // matrices streamed together
    constexpr int LPR = (NPL * 32 * Tl::BYTES / Tl::P + 32 + 1023) / 1024;
    constexpr int TROWS = 2 * NM;                 // tile rows per wavefront (R = 1 per half)
    constexpr int TILE = TROWS * LPR * 1024;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t K = a.k, PT = K / Tl::BLOCK * Tl::P;
    float4 *xs4 = reinterpret_cast<float4 *>(smem);                       // [T][8][PT]
    float *xsum = reinterpret_cast<float *>(smem + (size_t)T * K * 4);   // [T][NSUM][PT]
    uint8_t *tiles = smem + (size_t)T * K * 4 + (size_t)T * Tl::NSUM * PT * 4;
    __shared__ uint32_t sel_ids[8], tile_routes[T], tile_meta[2];
    __shared__ float sel_probs[8];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, c = lane & 31;

    // Which expert and which routes this workgroup serves.
    if (threadIdx.x < 64) {
        if (a.logits) {
            select_topk<1>(a.logits, a.experts, a.topk, sel_ids, sel_probs);
            if (lane == 0) {
                const uint32_t y = blockIdx.y;
                tile_meta[0] = sel_ids[y];
                tile_meta[1] = 1;
                tile_routes[0] = y;
                if (blockIdx.x == 0 && blockIdx.y == 0 && a.ids_out)
                    for (uint32_t r = 0; r < a.topk; r++) {
                        a.ids_out[r] = sel_ids[r];
                        a.probs_out[r] = sel_probs[r];
                    }
            }
        } else if (a.plan) {
            if (lane == 0) {
                // Plan tiles hold up to PLAN_TILE routes; each is served as
                // PLAN_TILE / T sub-tiles of T routes.
                const uint32_t y = blockIdx.y / (PLAN_TILE / T), sub = blockIdx.y % (PLAN_TILE / T);
                const uint32_t ntiles = a.plan[1];
                uint32_t count = 0, expert = 0;
                if (y < ntiles) {
                    expert = a.plan[6 + 2 * y];
                    const uint32_t first = a.plan[7 + 2 * y] + sub * T;
                    const uint64_t grouped = 6 + 2 * ((uint64_t)(a.routes + 15) / 16 + a.experts);
                    const uint64_t base = grouped + (uint64_t)expert * (a.routes + 1);
                    const uint32_t total = a.plan[base];
                    count = first < total ? min((uint32_t)T, total - first) : 0u;
                    for (uint32_t j = 0; j < count; j++) tile_routes[j] = a.plan[base + 1 + first + j];
                }
                tile_meta[0] = expert;
                tile_meta[1] = count;
            }
        } else if (lane == 0) {
            tile_meta[0] = a.ids[blockIdx.y];
            tile_meta[1] = 1;
            tile_routes[0] = blockIdx.y;
        }
    }
    __syncthreads();
    const uint32_t expert = tile_meta[0], count = tile_meta[1];
    if (count == 0) return;  // uniform across the workgroup

    // This expert's rows of each matrix: offsets from the 16-byte boundary
    // at or below their start.
    uint32_t shift[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) shift[m] = (uint32_t)((uintptr_t)(a.w[m] + (uint64_t)expert * a.n * a.row_bytes) & 15);
    const uint32_t row_span = (uint32_t)a.row_bytes, pieces = PT;
    u32x4 regs[TROWS * LPR];
    // Tile row i: matrix i / 2, row (group rows) wave*2 + i % 2.
    auto row_offset = [&](uint32_t g, int i) -> uint32_t {
        const uint32_t row = g * 8 + wave * 2 + (i & 1);
        return (uint32_t)(shift[i >> 1] + (uint64_t)row * a.row_bytes);
    };
    // One buffer resource per tile row, from the 16-byte boundary at or
    // below the row to its end rounded up to a whole chunk: the loads need no
    // per-lane test (a branch around them would make the compiler wait for
    // every load before the join), since chunks past the range read as zero
    // without touching memory.  Rows past n get an empty range.
    const uint8_t *mb[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) mb[m] = a.w[m] + (uint64_t)expert * a.n * a.row_bytes;
    auto issue = [&](uint32_t g) {
#pragma unroll
        for (int i = 0; i < TROWS; i++) {
            const uint32_t off = row_offset(g, i), start = off & ~15u;
            const uint32_t row = g * 8 + wave * 2 + (i & 1);
            const uint32_t need = row < a.n ? (off & 15u) + row_span : 0u;
            const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(((uintptr_t)mb[i >> 1] & ~(uintptr_t)15) + start), 0, (need + 15u) & ~15u, 0x00020000);
#pragma unroll
            for (int u = 0; u < LPR; u++)
                regs[i * LPR + u] = __builtin_amdgcn_raw_buffer_load_b128(rr, 16 * (u * 64 + lane), 0, 2);
        }
    };
    // One-route tiles request four float4 of x per thread (the first 1024)
    // before the weights: loads return in issue order, so x is in registers
    // while the weights are still in flight, as in the decode matvec.  (Plan
    // tiles, whose accumulators already take the registers, do not.)
    float xpre[4][4];
    if constexpr (T == 1) {
        const uint32_t in = tile_routes[0] / a.input_div;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t f = threadIdx.x + 256u * u;
            if (f < K / 4) {
                if (!a.x_bf16) {
                    const uint4 t = ld_u128((gbytes)a.x + ((uint64_t)in * (K / 4) + f) * 16);
                    xpre[u][0] = __uint_as_float(t.x); xpre[u][1] = __uint_as_float(t.y);
                    xpre[u][2] = __uint_as_float(t.z); xpre[u][3] = __uint_as_float(t.w);
                } else {
                    const uint2 t = ld_u64((gbytes)a.x + ((uint64_t)in * (K / 4) + f) * 8);
                    xpre[u][0] = __uint_as_float(t.x << 16); xpre[u][1] = __uint_as_float(t.x & 0xffff0000u);
                    xpre[u][2] = __uint_as_float(t.y << 16); xpre[u][3] = __uint_as_float(t.y & 0xffff0000u);
                }
            }
        }
    }
    uint32_t g = blockIdx.x;
    if (g < a.ngroups) issue(g);

    // Stage each route's activation row (piece-major) and its piece sums.
    for (uint32_t j = 0; j < count; j++) {
        const uint32_t in = tile_routes[j] / a.input_div;
        uint32_t f0 = threadIdx.x;
        if constexpr (T == 1) {  // one route: its first 1024 float4 are in xpre
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t f = threadIdx.x + 256u * u;
                if (f < K / 4) {
                    uint32_t pp, tt;
                    Tl::map(f, pp, tt);
                    xs4[tt * PT + pp] = make_float4(xpre[u][0], xpre[u][1], xpre[u][2], xpre[u][3]);
                }
            }
            f0 = threadIdx.x + 1024;
        }
        for (uint32_t f = f0; f < K / 4; f += 256) {
            float v[4];
            if (!a.x_bf16) {
                const uint4 t = ld_u128((gbytes)a.x + ((uint64_t)in * (K / 4) + f) * 16);
                v[0] = __uint_as_float(t.x); v[1] = __uint_as_float(t.y);
                v[2] = __uint_as_float(t.z); v[3] = __uint_as_float(t.w);
            } else {
                const uint2 t = ld_u64((gbytes)a.x + ((uint64_t)in * (K / 4) + f) * 8);
                v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
                v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
            }
            uint32_t pp, tt;
            Tl::map(f, pp, tt);
            xs4[(j * 8 + tt) * PT + pp] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    if constexpr (Tl::NSUM > 0) {
        __syncthreads();
        for (uint32_t q = threadIdx.x; q < count * PT; q += 256) {
            const uint32_t j = q / PT, pp = q % PT;
            float xv[32], sv[Tl::NSUM > 0 ? Tl::NSUM : 1];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                float4 v = xs4[(j * 8 + t) * PT + pp];
                xv[4 * t] = v.x; xv[4 * t + 1] = v.y; xv[4 * t + 2] = v.z; xv[4 * t + 3] = v.w;
            }
            Tl::sums(xv, sv);
#pragma unroll
            for (int s = 0; s < Tl::NSUM; s++) xsum[(j * Tl::NSUM + s) * PT + pp] = sv[s];
        }
    }
    __syncthreads();

    uint8_t *tile = tiles + (size_t)wave * TILE;
    for (; g < a.ngroups; g += gridDim.x) {
#pragma unroll
        for (int i = 0; i < TROWS * LPR; i++) reinterpret_cast<u32x4 *>(tile)[i * 64 + lane] = regs[i];
        uint32_t rbase[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const int i = 2 * m + half;
            rbase[m] = i * LPR * 1024 + (row_offset(g, i) & 15u);
        }
        if (g + gridDim.x < a.ngroups) issue(g + gridDim.x);

        float acc[NM][T];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int j = 0; j < T; j++) acc[m][j] = 0.f;
#pragma unroll
        for (int s = 0; s < NPL; s++) {
            const uint32_t pl = c + 32 * s;
            if (pl < pieces) {
                const uint32_t blk = pl / Tl::P, cc = pl % Tl::P;
                typename Tl::Raw raw[NM];
#pragma unroll
                for (int m = 0; m < NM; m++) raw[m] = Tl::load(tile + rbase[m] + blk * Tl::BYTES, cc);
#pragma unroll
                for (int j = 0; j < T; j++) {
                    if ((uint32_t)j < count) {
                        float xv[32], sv[Tl::NSUM > 0 ? Tl::NSUM : 1];
#pragma unroll
                        for (int t = 0; t < 8; t++) {
                            float4 v = xs4[(j * 8 + t) * PT + pl];
                            xv[4 * t] = v.x; xv[4 * t + 1] = v.y; xv[4 * t + 2] = v.z; xv[4 * t + 3] = v.w;
                        }
#pragma unroll
                        for (int q = 0; q < Tl::NSUM; q++) sv[q] = xsum[(j * Tl::NSUM + q) * PT + pl];
#pragma unroll
                        for (int m = 0; m < NM; m++) acc[m][j] += tile_dot<FMT>(raw[m], xv, sv, cc);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int j = 0; j < T; j++) acc[m][j] = half_sum(acc[m][j]);

        const uint32_t row = g * 8 + wave * 2 + half;
        if (c < count && row < a.n) {
            float v0 = acc[0][0], v1 = NM > 1 ? acc[NM - 1][0] : 0.f;
#pragma unroll
            for (int j = 1; j < T; j++)
                if (c == (uint32_t)j) {
                    v0 = acc[0][j];
                    v1 = acc[NM - 1][j];
                }
            const uint32_t route = tile_routes[c];
            const uint64_t bi = (uint64_t)expert * a.n + row, o = (uint64_t)route * a.n + row;
            if (a.bias[0]) v0 += round_bf16(a.bias[0][bi]);
            if (GATED) {
                if (a.bias[1]) v1 += round_bf16(a.bias[1][bi] + (a.up_one ? 1.0f : 0.0f));
                else if (a.up_one) v1 += 1.0f;
                a.out0[o] = activation(a.act, v0, v1);
                if (a.out1) a.out1[o] = v1;
            } else {
                a.out0[o] = v0;
            }
        }
    }
}

typedef void (*MoeFn)(u32x4, u32x4, u32x4, u32x2, MoeArgs);
constexpr int MOE_T = 4;  // routes per tile (plan tiles); one-route tiles without a plan use T = 1

template <int FMT, bool GATED, int T>
static MoeFn moe_pick(int npl) {
    switch (npl) {
    case 1: return moe_kernel<FMT, GATED, T, 1>;
    case 2: return moe_kernel<FMT, GATED, T, 2>;
    case 3: return moe_kernel<FMT, GATED, T, 3>;
    case 4: return moe_kernel<FMT, GATED, T, 4>;
    }
    return nullptr;
}

template <int T>
static MoeFn moe_pick_t(uint32_t fmt, bool gated, int npl) {
    switch (fmt) {
    case OCO_MXFP4: return gated ? moe_pick<OCO_MXFP4, true, T>(npl) : moe_pick<OCO_MXFP4, false, T>(npl);
    case OCO_Q4_K: return gated ? moe_pick<OCO_Q4_K, true, T>(npl) : moe_pick<OCO_Q4_K, false, T>(npl);
    case OCO_Q6_K: return gated ? moe_pick<OCO_Q6_K, true, T>(npl) : moe_pick<OCO_Q6_K, false, T>(npl);
    case OCO_Q8_0: return gated ? moe_pick<OCO_Q8_0, true, T>(npl) : moe_pick<OCO_Q8_0, false, T>(npl);
    }
    return nullptr;
}

static MoeFn moe_pick_format(uint32_t fmt, bool gated, int npl, int t) {
    return t == 1 ? moe_pick_t<1>(fmt, gated, npl) : moe_pick_t<MOE_T>(fmt, gated, npl);
}

static int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        hipGetDevice(&dev);
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (cus <= 0) cus = 256;
    }
    return cus;
}

// Launch one grouped projection over `tiles` tiles.
static int moe_launch(uint32_t fmt, bool gated, MoeArgs a, uint32_t tiles, uint32_t parallel_tiles,
                      hipStream_t stream) {
    uint32_t be, bb;
    OCO_TRY(oco_block_layout(fmt, &be, &bb));
    if (a.k % be || a.k % 32) return fail(OCO_ERR_INVALID, "experts: k=%u is not block aligned", a.k);
    const uint32_t P = (fmt == OCO_Q4_K || fmt == OCO_Q6_K) ? 8 : 1;
    const uint32_t pieces = a.k / be * P;
    const int npl = (int)((pieces + 31) / 32);
    // Without a plan every tile is one route: a one-route kernel, whose
    // staged activations take a quarter of the LDS.
    const int t = a.plan ? MOE_T : 1;
    MoeFn fn = npl <= 4 ? moe_pick_format(fmt, gated, npl, t) : nullptr;
    if (!fn)
        return fail(OCO_ERR_UNSUPPORTED, "experts: format %u with k=%u has no routed kernel (rows over %u bytes)",
                    fmt, a.k, 4 * 32 * bb / P);
    a.row_bytes = oco_row_bytes(fmt, a.k);
    a.ngroups = (a.n + 7) / 8;
    const uint32_t nsum = fmt == OCO_Q8_0 ? 1 : fmt == OCO_Q4_K ? 2 : fmt == OCO_Q6_K ? 4 : 0;
    const int lpr = (npl * 32 * (int)bb / (int)P + 32 + 1023) / 1024;
    const size_t lds = (size_t)t * a.k * 4 + (size_t)t * nsum * (a.k / 32) * 4 +
                       4 * (size_t)(2 * (gated ? 2 : 1) * lpr * 1024);
    if (lds > 150 * 1024) return fail(OCO_ERR_UNSUPPORTED, "experts: k=%u needs %zu bytes of LDS", a.k, lds);
    if (lds > 64 * 1024)
        OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                          "hipFuncSetAttribute"));
    int32_t ov[4];
    // Three workgroups per CU for MXFP4 banks (gpt-oss B = 1: 33.6 -> 32.4
    // us against two), two for the others.
    const uint32_t per_cu = plan_override(OCO_KNOB_MOE_WG, ov) && ov[0] > 0 ? (uint32_t)ov[0] : fmt == OCO_MXFP4 ? 3u : 2u;
    const uint32_t target = per_cu * device_cus();
    uint32_t gx = std::max<uint32_t>(1, target / std::max<uint32_t>(1, parallel_tiles));
    gx = std::min(gx, a.ngroups);
    hipLaunchKernelGGL(fn, dim3(gx, tiles), dim3(256), lds, stream, KPRE_ARGS(a), a);
    return launch_check("experts projection");
}

// hidden is the reduction length of gate/up and must be whole blocks; ffn is
// the reduction length of down, so only callers that run down (need_down)
// require it in whole blocks (expand alone takes any ffn).
static int check_bank(const oco_experts *w, bool need_down) {
    if (!w) return fail(OCO_ERR_INVALID, "experts: null descriptor");
    if (!w->gate || !w->up || !w->down) return fail(OCO_ERR_INVALID, "experts: null weights");
    if (w->experts == 0 || w->experts > 256 || w->k == 0 || w->k > 8 || w->k > w->experts)
        return fail(OCO_ERR_INVALID, "experts: need 0 < k <= 8, k <= experts <= 256");
    if (w->activation > OCO_ACT_SWIGLU) return fail(OCO_ERR_INVALID, "experts: unknown activation");
    if (w->hidden == 0 || w->ffn == 0) return fail(OCO_ERR_INVALID, "experts: empty geometry");
    uint32_t be, bb;
    OCO_TRY(oco_block_layout(w->format, &be, &bb));
    if (w->hidden % be) return fail(OCO_ERR_INVALID, "experts: hidden=%u must be whole blocks of %u", w->hidden, be);
    if (need_down && w->ffn % be)
        return fail(OCO_ERR_INVALID, "experts: ffn=%u must be whole blocks of %u", w->ffn, be);
    return OCO_OK;
}

static uint64_t align256(uint64_t v) { return (v + 255) & ~255ull; }

// Prefill: from this many tokens on, the routed layer runs as grouped MFMA
// GEMMs over the route plan's expert tiles.
constexpr uint32_t MOE_MFMA_TOKENS = 32;
// MXFP4 banks take the block-scaled MFMA path from this many tokens on.
constexpr uint32_t MOE_MX_TOKENS = 4;  // measured (gpt-oss): B=4 on these tiles beats the routed kernel, B=1 does not

// Gate/up activations to f16 rows for the Q4_K down tiles: each row scaled
// by the power of two (row_gain) that brings its max |activation| into
// [2^14, 2^15), which is exact, then rounded to f16; the down epilogue
// multiplies the gain back out, also exactly.  Four elements per thread
// (cols % 4 == 0).
__global__ __launch_bounds__(256) void act_f16_kernel(const float *x, const uint32_t *rowmax, uint16_t *y,
                                                      uint32_t cols8, uint32_t n8) {
    // Eight values per thread (cols % 8 == 0: one row each), 32-byte loads,
    // one 16-byte store.
    const uint32_t i8 = blockIdx.x * 256 + threadIdx.x;
    if (i8 >= n8) return;
    const float g = row_gain(gp(rowmax)[i8 / cols8]);
    const auto src = gp(reinterpret_cast<const u32x4 *>(x) + 2 * (uint64_t)i8);
    const u32x4 v0 = src[0], v1 = src[1];
    const uint32_t vb[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float e[8];
#pragma unroll
    for (int j = 0; j < 8; j++) e[j] = __uint_as_float(vb[j]) * g;
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const _Float16 h = (_Float16)e[j];
        uint16_t u;
        __builtin_memcpy(&u, &h, 2);
        b[j] = u;
    }
    gp(reinterpret_cast<u32x4 *>(y))[i8] = u32x4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
}

}  // namespace oco

using namespace oco;

extern "C" {

uint64_t oco_experts_workspace(const oco_experts *w, uint32_t tokens) {
    if (!w) return 0;
    const uint64_t routes = (uint64_t)tokens * w->k;
    // plan, f32 activations, f16 copy of f32 inputs and activation row maxima
    // (prefill), route outputs, f16 activations (Q4_K prefill); MXFP4 banks
    // also the E2M3 splits of the inputs and of the activations
    uint64_t bytes = align256(oco_route_plan_words((uint32_t)routes, w->experts) * 4) + align256(routes * w->ffn * 4) +
                     align256((uint64_t)tokens * w->hidden * 2) + align256(routes * 4) + align256(routes * w->hidden * 4);
    if (w->format == OCO_Q4_K) bytes += align256(routes * w->ffn * 2);
    if (w->format == OCO_MXFP4)  // ... and the plan's tile descriptors (tiles of up to 32 rows)
        bytes += align256(mx_rows_bytes(tokens, w->hidden)) + align256(mx_rows_bytes((uint32_t)routes, w->ffn)) +
                 align256(plan_desc_words((uint32_t)routes, w->experts, 32) * 4);
    // router logits of oco_experts_forward, last
    return bytes + align256((uint64_t)tokens * w->experts * 4);
}

}  // extern "C"

// The layer after the router logits.  With `logits`, the experts are
// selected on the device (ids/probs are written): at one token inside the
// routed gate/up kernel (expert_expand's selection), else inside the route
// plan's launch.
// The MXFP4 tiles at a small decode batch: every gate/up workgroup builds
// the route plan itself (route.h), the input rows are split beside the
// router logits, or by a launch of their own without a router.
static bool mx_small_path(const oco_experts *w, uint32_t tokens) {
    int32_t ov[4];
    const uint32_t mx_tokens = plan_override(OCO_KNOB_MOE_MX_TOKENS, ov) ? (uint32_t)ov[0] : MOE_MX_TOKENS;
    return w->format == OCO_MXFP4 && w->hidden % 32 == 0 && w->ffn % 32 == 0 && tokens >= mx_tokens &&
           small_plan_fits(tokens, tokens * w->k, w->experts);
}

// The input rows' split records in the workspace (MXFP4 banks).
static uint8_t *mx_xrec(const oco_experts *w, uint8_t *ws, uint32_t tokens) {
    const uint32_t routes = tokens * w->k;
    return ws + align256(oco_route_plan_words(routes, w->experts) * 4) + align256((uint64_t)routes * w->ffn * 4) +
           align256((uint64_t)tokens * w->hidden * 2) + align256((uint64_t)routes * 4) +
           align256((uint64_t)routes * w->hidden * 4);
}

static int experts_apply(const oco_experts *w, const void *x, oco_dtype x_dtype, uint32_t *ids, float *probs,
                         const float *logits, uint32_t tokens, uint16_t *out, float *routed, void *workspace,
                         uint64_t workspace_bytes, hipStream_t s, const char *who, bool split_done = false) {
    OCO_TRY(check_bank(w, true));
    if (!tokens) return OCO_OK;
    if (!x || !ids || !probs || !out || !workspace) return fail(OCO_ERR_INVALID, "%s: null pointer", who);
    if (x_dtype != OCO_DT_F32 && x_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "%s: activations must be f32 or bf16", who);
    if (workspace_bytes < oco_experts_workspace(w, tokens))
        return fail(OCO_ERR_INVALID, "%s: workspace of %llu bytes, need %llu", who,
                    (unsigned long long)workspace_bytes, (unsigned long long)oco_experts_workspace(w, tokens));
    oco_stream stream = (oco_stream)s;
    // Selection inside the gate/up kernel covers one token over <= 64 experts;
    // otherwise it runs in the route plan's workgroup, before the plan.
    const bool small = mx_small_path(w, tokens);
    const bool fused_select = logits && tokens == 1 && w->experts <= 64 && !small;
    PlanSide sel = {};
    if (logits && !fused_select) {
        sel.logits = logits;
        sel.tokens = tokens;
        sel.topk = w->k;
        sel.ids_out = ids;
        sel.probs_out = probs;
    }
    const uint32_t routes = tokens * w->k;
    uint8_t *ws = (uint8_t *)workspace;
    uint32_t *plan = (uint32_t *)ws;
    float *act = (float *)(ws + align256(oco_route_plan_words(routes, w->experts) * 4));
    uint16_t *x16 = (uint16_t *)((uint8_t *)act + align256((uint64_t)routes * w->ffn * 4));
    uint32_t *rowmax = (uint32_t *)((uint8_t *)x16 + align256((uint64_t)tokens * w->hidden * 2));
    uint8_t *own_down = (uint8_t *)rowmax + align256((uint64_t)routes * 4);
    float *down = routed ? routed : (float *)own_down;
    uint8_t *xrec = mx_xrec(w, ws, tokens);  // MXFP4 only (just past the route outputs)
    uint8_t *arec = xrec + align256(mx_rows_bytes(tokens, w->hidden));
    uint16_t *act16 = (uint16_t *)xrec;  // Q4_K only (in place of the MXFP4 splits)

    int32_t ov[4];
    const uint32_t mx_tokens = plan_override(OCO_KNOB_MOE_MX_TOKENS, ov) ? (uint32_t)ov[0] : MOE_MX_TOKENS;
    // The MFMA tiles and the E2M3 row split read whole 32-element k groups
    // and n tiles; other geometries take the routed matvec path below.
    const bool tiled = w->hidden % 32 == 0 && w->ffn % 32 == 0;
    if (tiled && w->format == OCO_MXFP4 && tokens >= mx_tokens) {
        // MXFP4 banks: block-scaled FP6 x FP4 MFMA on the GGUF bytes (no
        // weight decode); activations split per row into four E2M3 terms.
        // Decode batches take 16-row tiles (half the staged activations).
        const uint32_t tile_rows = tokens <= 16 ? 16 : 32;
        // The input rows' split runs beside the router or the plan; the
        // activations are split by the gate/up tiles themselves.
        uint32_t *desc = (uint32_t *)(arec + align256(mx_rows_bytes(routes, w->ffn)));
        MatmulArgs g = {};
        if (small) {
            if (!split_done)
                OCO_TRY(router_logits_launch(x, x_dtype, nullptr, nullptr, tokens, w->hidden, w->experts, nullptr, xrec,
                                             s));
            g.small = 1;
            g.logits = logits;
            g.ids = ids;
            g.ids_out = ids;
            g.probs_out = probs;
            g.desc_out = desc;
            g.plan_out = plan;
        } else {
            PlanSide side = sel;
            side.desc = desc;
            side.x = x;
            side.x_bf16 = x_dtype == OCO_DT_BF16 ? 1u : 0u;
            side.rec = xrec;
            side.rows = tokens;
            side.k = w->hidden;
            OCO_TRY(route_plan_launch(ids, routes, w->experts, tile_rows, 0, 0, plan, &side, s));
        }
        g.desc = desc;
        g.w = (const uint8_t *)w->gate;
        g.w2 = (const uint8_t *)w->up;
        g.bias = w->gate_bias;
        g.bias2 = w->up_bias;
        g.yrec = arec;  // split records [routes][ffn], expert-sorted rows
        g.m = routes;
        g.n = w->ffn;
        g.k = w->hidden;
        g.row_bytes = (uint32_t)oco_row_bytes(w->format, w->hidden);
        g.expert_bytes = (uint64_t)g.row_bytes * w->ffn;
        g.plan = plan;
        g.routes = routes;
        g.experts = w->experts;
        g.topk = w->k;
        g.act = w->activation;
        g.up_one = w->up_bias_one;
        OCO_TRY(mx_experts_launch(MM_GATE_UP, g, xrec, tile_rows, s));
        MatmulArgs d = g;
        d.small = 0;
        d.yrec = nullptr;
        d.w = (const uint8_t *)w->down;
        d.w2 = nullptr;
        d.bias = w->down_bias;
        d.bias2 = nullptr;
        d.y = down;
        d.y_bf16 = routed ? 0 : 1;
        d.n = w->hidden;
        d.k = w->ffn;
        d.row_bytes = (uint32_t)oco_row_bytes(w->format, w->ffn);
        d.expert_bytes = (uint64_t)d.row_bytes * w->hidden;
        OCO_TRY(mx_experts_launch(MM_DOWN, d, arec, tile_rows, s));
        return oco_moe_sum(down, routed ? OCO_DT_F32 : OCO_DT_BF16, probs, out, w->hidden, tokens, w->k, stream);
    }

    const uint32_t mfma_tokens = plan_override(OCO_KNOB_MOE_MFMA_TOKENS, ov) ? (uint32_t)ov[0] : MOE_MFMA_TOKENS;
    if (tiled && tokens >= mfma_tokens) {
        // Prefill: grouped MFMA GEMMs (expert_up_tensor / moe_activate /
        // expert_down_tensor, projections.metal:192-376, routing.metal:44-64).
        // Rows per tile: most experts in one tile (mean routes per expert,
        // plus room for the spread).  An OCO_KNOB_MOE_Q4_ROWS override of 0
        // sends Q4_K to the f16 LDS tiles of the other formats.
        const int q4_rows = plan_override(OCO_KNOB_MOE_Q4_ROWS, ov) ? ov[0] : -1;
        const bool q4 = w->format == OCO_Q4_K && q4_rows != 0;
        const uint32_t mean = routes / w->experts;
        const uint32_t bm = q4 ? (q4_rows > 0 ? (uint32_t)q4_rows : mean <= 20 ? 32 : mean <= 36 ? 48 : 64)
                               : (mean <= 40 ? 32 : 64);
        // The tiles take f16 rows (the reference's half(x)); the conversion
        // and the clearing of the row maxima run beside the plan.
        PlanSide side = sel;
        side.x = x;
        side.x_bf16 = x_dtype == OCO_DT_BF16 ? 1u : 0u;
        side.y = x16;
        side.n = (uint64_t)tokens * w->hidden;
        side.zero = rowmax;
        side.nzero = routes;
        OCO_TRY(route_plan_launch(ids, routes, w->experts, bm, 0, 0, plan, &side, s));
        const void *xin = x16;
        MatmulArgs g = {};
        g.w = (const uint8_t *)w->gate;
        g.w2 = (const uint8_t *)w->up;
        g.bias = w->gate_bias;
        g.bias2 = w->up_bias;
        g.x = xin;
        g.x_f16 = 1;
        g.y = act;  // f32 [routes][ffn], expert-sorted rows
        g.rowmax = rowmax;
        g.m = routes;
        g.n = w->ffn;
        g.k = w->hidden;
        g.row_bytes = (uint32_t)oco_row_bytes(w->format, w->hidden);
        g.expert_bytes = (uint64_t)g.row_bytes * w->ffn;
        g.plan = plan;
        g.routes = routes;
        g.experts = w->experts;
        g.topk = w->k;
        g.act = w->activation;
        g.up_one = w->up_bias_one;
        OCO_TRY(q4 ? moe_q4k_launch(MM_GATE_UP, g, bm, s) : grouped_matmul_launch(MM_GATE_UP, w->format, g, bm, s));
        MatmulArgs d = g;
        d.w = (const uint8_t *)w->down;
        d.w2 = nullptr;
        d.bias = w->down_bias;
        d.bias2 = nullptr;
        d.x = act;
        d.x_f16 = 1;
        if (q4) {
            const uint64_t n8 = (uint64_t)routes * w->ffn / 8;  // ffn % 256 == 0 (Q4_K rows)
            if (n8 > 0xffffffffull - 255)
                return fail(OCO_ERR_INVALID, "experts: %llu activations", (unsigned long long)n8 * 8);
            hipLaunchKernelGGL(act_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, act, rowmax,
                               act16, w->ffn / 8, (uint32_t)n8);
            OCO_TRY(launch_check("experts f16 activations"));
            d.x = act16;
        }
        // Route outputs: f32 when the caller asks for them, else bf16 as the
        // reference stores them (moe_sum rounds f32 routes to bf16 anyway).
        d.y = down;
        d.y_bf16 = routed ? 0 : 1;
        d.n = w->hidden;
        d.k = w->ffn;
        d.row_bytes = (uint32_t)oco_row_bytes(w->format, w->ffn);
        d.expert_bytes = (uint64_t)d.row_bytes * w->hidden;
        OCO_TRY(q4 ? moe_q4k_launch(MM_DOWN, d, bm, s) : grouped_matmul_launch(MM_DOWN, w->format, d, bm, s));
        return oco_moe_sum(down, routed ? OCO_DT_F32 : OCO_DT_BF16, probs, out, w->hidden, tokens, w->k, stream);
    }

    uint32_t tiles = routes, parallel = routes;
    const uint32_t *use_plan = nullptr;
    if (fused_select) {
        // expert_expand (projections.metal:78-137): every gate/up workgroup
        // selects the token's experts from the logits; workgroup (0, 0)
        // records ids and probabilities for the down pass and the combine.
        MoeArgs a = {};
        a.w[0] = (const uint8_t *)w->gate;
        a.w[1] = (const uint8_t *)w->up;
        a.bias[0] = w->gate_bias;
        a.bias[1] = w->up_bias;
        a.x = x;
        a.x_bf16 = x_dtype == OCO_DT_BF16;
        a.input_div = w->k;
        a.out0 = act;
        a.logits = logits;
        a.ids_out = ids;
        a.probs_out = probs;
        a.k = w->hidden;
        a.n = w->ffn;
        a.experts = w->experts;
        a.topk = w->k;
        a.routes = routes;
        a.act = w->activation;
        a.up_one = w->up_bias_one;
        OCO_TRY(moe_launch(w->format, true, a, routes, routes, s));
        MoeArgs d = {};
        d.w[0] = (const uint8_t *)w->down;
        d.bias[0] = w->down_bias;
        d.x = act;
        d.input_div = 1;
        d.out0 = down;
        d.ids = ids;
        d.k = w->ffn;
        d.n = w->hidden;
        d.experts = w->experts;
        d.topk = w->k;
        d.routes = routes;
        d.act = w->activation;
        d.up_one = w->up_bias_one;
        OCO_TRY(moe_launch(w->format, false, d, routes, routes, s));
        return oco_moe_sum(down, OCO_DT_F32, probs, out, w->hidden, tokens, w->k, stream);
    }
    if (tokens > 1) {
        OCO_TRY(route_plan_launch(ids, routes, w->experts, PLAN_TILE, 0, 0, plan, &sel, s));
        use_plan = plan;
        tiles = ((routes + PLAN_TILE - 1) / PLAN_TILE + w->experts) * (PLAN_TILE / MOE_T);
        parallel = std::min(routes, w->experts);
    }
    MoeArgs a = {};
    a.w[0] = (const uint8_t *)w->gate;
    a.w[1] = (const uint8_t *)w->up;
    a.bias[0] = w->gate_bias;
    a.bias[1] = w->up_bias;
    a.x = x;
    a.x_bf16 = x_dtype == OCO_DT_BF16;
    a.input_div = w->k;
    a.out0 = act;
    a.out1 = nullptr;
    a.ids = ids;
    a.plan = use_plan;
    a.k = w->hidden;
    a.n = w->ffn;
    a.experts = w->experts;
    a.topk = w->k;
    a.routes = routes;
    a.act = w->activation;
    a.up_one = w->up_bias_one;
    OCO_TRY(moe_launch(w->format, true, a, tiles, parallel, s));

    MoeArgs d = a;
    d.w[0] = (const uint8_t *)w->down;
    d.w[1] = nullptr;
    d.bias[0] = w->down_bias;
    d.bias[1] = nullptr;
    d.x = act;
    d.x_bf16 = 0;
    d.input_div = 1;
    d.out0 = down;
    d.k = w->ffn;
    d.n = w->hidden;
    OCO_TRY(moe_launch(w->format, false, d, tiles, parallel, s));
    return oco_moe_sum(down, OCO_DT_F32, probs, out, w->hidden, tokens, w->k, stream);
}

extern "C" {

int oco_experts_apply(const oco_experts *w, const void *x, oco_dtype x_dtype, const uint32_t *ids,
                      const float *probs, uint32_t tokens, uint16_t *out, float *routed, void *workspace,
                      uint64_t workspace_bytes, oco_stream stream) {
    return experts_apply(w, x, x_dtype, const_cast<uint32_t *>(ids), const_cast<float *>(probs), nullptr, tokens,
                         out, routed, workspace, workspace_bytes, (hipStream_t)stream, "oco_experts_apply");
}

int oco_experts_forward(const oco_experts *w, const float *router_w, const float *router_bias, const void *x,
                        oco_dtype x_dtype, uint32_t tokens, uint16_t *out, uint32_t *ids, float *probs,
                        float *routed, void *workspace, uint64_t workspace_bytes, oco_stream stream) {
    OCO_TRY(check_bank(w, true));
    if (!tokens) return OCO_OK;
    if (!router_w || !x || !workspace) return fail(OCO_ERR_INVALID, "oco_experts_forward: null pointer");
    if (workspace_bytes < oco_experts_workspace(w, tokens))
        return fail(OCO_ERR_INVALID, "oco_experts_forward: workspace of %llu bytes, need %llu",
                    (unsigned long long)workspace_bytes, (unsigned long long)oco_experts_workspace(w, tokens));
    hipStream_t s = (hipStream_t)stream;
    float *logits = (float *)((uint8_t *)workspace + oco_experts_workspace(w, tokens) -
                              align256((uint64_t)tokens * w->experts * 4));
    // the MXFP4 decode tiles' input split rides in the router's launch
    const bool split = mx_small_path(w, tokens) && (x_dtype == OCO_DT_F32 || x_dtype == OCO_DT_BF16);
    OCO_TRY(router_logits_launch(x, x_dtype, router_w, router_bias, tokens, w->hidden, w->experts, logits,
                                 split ? mx_xrec(w, (uint8_t *)workspace, tokens) : nullptr, s));
    return experts_apply(w, x, x_dtype, ids, probs, logits, tokens, out, routed, workspace, workspace_bytes, s,
                         "oco_experts_forward", split);
}

}  // extern "C"

// ---- the layer without allocation -------------------------------------------
// A file-scope device array stands in for the caller's workspace.  In host
// code `scratch` names a host-side stand-in, never its device memory: its
// address on each device comes from hipGetSymbolAddress, once per device,
// and only that address is handed to kernels.
static __device__ __align__(256) uint8_t scratch[OCO_EXPERTS_SCRATCH_BYTES];
constexpr int SCRATCH_DEVICES = 64;
static std::atomic<void *> g_scratch[SCRATCH_DEVICES];
static std::mutex g_scratch_lock;

namespace oco {
int experts_scratch_init(int device) {
    if (device < 0 || device >= SCRATCH_DEVICES)
        return fail(OCO_ERR_UNSUPPORTED, "experts scratch: device %d beyond %d", device, SCRATCH_DEVICES);
    std::lock_guard<std::mutex> hold(g_scratch_lock);
    if (g_scratch[device].load(std::memory_order_acquire)) return OCO_OK;
    void *p = nullptr;
    OCO_TRY(hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    if (!p) return fail(OCO_ERR_HIP, "hipGetSymbolAddress(scratch): null address");
    g_scratch[device].store(p, std::memory_order_release);
    return OCO_OK;
}
}  // namespace oco

extern "C" {

int oco_experts_forward_static(const oco_experts *w, const float *router_w, const float *router_bias, const void *x,
                               oco_dtype x_dtype, uint32_t tokens, uint16_t *out, uint32_t *ids, float *probs,
                               float *routed, oco_stream stream) {
    OCO_TRY(check_bank(w, true));
    if (!tokens) return OCO_OK;
    const uint64_t need = oco_experts_workspace(w, tokens);
    if (need > OCO_EXPERTS_SCRATCH_BYTES)
        return fail(OCO_ERR_INVALID,
                    "oco_experts_forward_static: %u tokens need %llu bytes of scratch, over its %llu (use "
                    "oco_experts_forward with a workspace)",
                    tokens, (unsigned long long)need, (unsigned long long)OCO_EXPERTS_SCRATCH_BYTES);
    int dev = 0;
    OCO_TRY(hip_check(hipGetDevice(&dev), "hipGetDevice"));
    if (dev < 0 || dev >= SCRATCH_DEVICES || !g_scratch[dev].load(std::memory_order_acquire))
        OCO_TRY(experts_scratch_init(dev));
    return oco_experts_forward(w, router_w, router_bias, x, x_dtype, tokens, out, ids, probs, routed,
                               g_scratch[dev].load(std::memory_order_acquire), need, stream);
}

int oco_expert_expand(const oco_experts *w, const void *x, oco_dtype x_dtype, const float *logits, uint32_t *ids,
                      float *probs, float *up_out, float *act_out, oco_stream stream) {
    OCO_TRY(check_bank(w, false));
    if (!x || !logits || !ids || !probs || !act_out) return fail(OCO_ERR_INVALID, "oco_expert_expand: null pointer");
    if (w->experts > 64) return fail(OCO_ERR_UNSUPPORTED, "oco_expert_expand: fused selection covers <= 64 experts");
    if (x_dtype != OCO_DT_F32 && x_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_expert_expand: activations must be f32 or bf16");
    MoeArgs a = {};
    a.w[0] = (const uint8_t *)w->gate;
    a.w[1] = (const uint8_t *)w->up;
    a.bias[0] = w->gate_bias;
    a.bias[1] = w->up_bias;
    a.x = x;
    a.x_bf16 = x_dtype == OCO_DT_BF16;
    a.input_div = w->k;
    a.out0 = act_out;
    a.out1 = up_out;
    a.logits = logits;
    a.ids_out = ids;
    a.probs_out = probs;
    a.k = w->hidden;
    a.n = w->ffn;
    a.experts = w->experts;
    a.topk = w->k;
    a.routes = w->k;
    a.act = w->activation;
    a.up_one = w->up_bias_one;
    return moe_launch(w->format, true, a, w->k, w->k, (hipStream_t)stream);
}

}  // extern "C"
