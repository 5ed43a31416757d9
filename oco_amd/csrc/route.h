// Top-k expert selection shared by the routing and expert kernels.
#pragma once
#include "common.h"

namespace oco {

// A job run beside the route plan, in the same launch (workgroups 1..):
// activation rows to f16 (the reference's half(x)) from bf16 or f32, four
// elements per thread, and `nzero` words of `zero` cleared; or, with `rec`
// set, the rows' split records (mxsplit.h: three E2M3 terms) in place of the
// f16 copy.
//
// Also optional, in the plan's own workgroup: the expert selection itself
// (`logits` set: top-`topk` of each of `tokens` rows of `experts` logits, as
// oco_route_select, into ids_out / probs_out, which then are the plan's ids),
// and per-tile descriptors (`desc` set), so that a tile's consumer finds all
// it needs in one contiguous read: PLAN_DESC_HEAD words {expert, rows (0 for
// an unused tile slot), first sorted row, first list row} then the tile's
// `tile_rows` route ids in list order, for every one of the plan's
// ceil(routes / 16) + experts tile slots.
struct PlanSide {
    const void *x;
    uint32_t x_bf16;
    uint16_t *y;
    uint64_t n;
    uint32_t *zero;
    uint32_t nzero;
    uint8_t *rec;       // split records of rows x k (k % 32 == 0), or null
    uint32_t rows, k;
    const float *logits;
    uint32_t tokens, topk;
    uint32_t *ids_out;
    float *probs_out;
    uint32_t *desc;
};
constexpr uint32_t PLAN_DESC_HEAD = 4;
__host__ __device__ inline uint64_t plan_desc_words(uint32_t routes, uint32_t experts, uint32_t tile_rows) {
    return ((uint64_t)(routes + 15) / 16 + experts) * (PLAN_DESC_HEAD + tile_rows);
}

// Router logits [tokens, experts] (routing.metal:96-146) into `logits` (or
// none: null), and with `rec` set, in the same launch, the rows' split
// records (mxsplit.h: three E2M3 terms).
int router_logits_launch(const void *x, oco_dtype x_dtype, const float *w, const float *bias, uint32_t tokens,
                         uint32_t hidden, uint32_t experts, float *logits, uint8_t *rec, hipStream_t stream);
// oco_route_plan with an optional side job (null: none).
int route_plan_launch(const uint32_t *ids, uint32_t routes, uint32_t experts, uint32_t tile_rows, uint32_t up_tiles,
                      uint32_t down_tiles, uint32_t *plan, const PlanSide *side, hipStream_t stream);

// Wave-wide max / min over 64 lanes with DPP and permlane swaps (all lanes
// receive the result).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_u32<0x124>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_u32<0x128>(__float_as_uint(v))));
    auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
    auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_u32<0xB1>(v));
    v = min(v, dpp_u32<0x4E>(v));
    v = min(v, dpp_u32<0x124>(v));
    v = min(v, dpp_u32<0x128>(v));
    auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = min((uint32_t)s16[0], (uint32_t)s16[1]);
    auto s32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return min((uint32_t)s32[0], (uint32_t)s32[1]);
}

__device__ __forceinline__ bool finite_bits(float v) {
    return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u;
}

// Top-k of one token's logits by one wavefront (routing.metal:71-94,
// generalised to k-of-E, E <= 256): repeatedly take the maximum, ties to the
// lowest expert index; non-finite logits rank as -inf and turn every
// probability NaN; chosen logits are rounded to bf16 and the probabilities
// are bf16 of the softmax over the chosen k.  Lane 0 receives ids/probs.
template <int PER>  // logits per lane: experts <= 64 * PER
__device__ void select_topk(const float *logits, uint32_t experts, uint32_t k, uint32_t *ids,
                            float *probs) {
    const uint32_t lane = threadIdx.x & 63;
    float v[PER];
    bool avail[PER];
    bool invalid = false;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        uint32_t e = lane + 64 * j;
        float l = e < experts ? logits[e] : -INFINITY;
        bool fin = finite_bits(l);
        if (e < experts && !fin) invalid = true;
        v[j] = fin ? l : -INFINITY;
        avail[j] = e < experts;
    }
    invalid = __ballot(invalid) != 0;  // any lane saw a non-finite logit
    float chosen[8];
    uint32_t sel[8];
    for (uint32_t r = 0; r < k; r++) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (avail[j]) m = fmaxf(m, v[j]);
        m = wave_max(m);
        uint32_t cand = 0xffffffffu;
#pragma unroll
        for (int j = PER - 1; j >= 0; j--)
            if (avail[j] && v[j] == m) cand = lane + 64 * j;
        cand = wave_min_u32(cand);
        sel[r] = cand;
        chosen[r] = round_bf16(m);
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (lane + 64 * j == cand) avail[j] = false;
    }
    if (lane != 0) return;
    for (uint32_t r = 0; r < k; r++)
        if (!finite_bits(chosen[r])) invalid = true;
    if (invalid) {
        for (uint32_t r = 0; r < k; r++) {
            ids[r] = sel[r] < experts ? sel[r] : 0;
            probs[r] = __uint_as_float(0x7fc00000u);
        }
        return;
    }
    float sum = 0.f;
    for (uint32_t r = 0; r < k; r++) sum += expf(chosen[r] - chosen[0]);
    for (uint32_t r = 0; r < k; r++) {
        ids[r] = sel[r];
        probs[r] = round_bf16(expf(chosen[r] - chosen[0]) / sum);
    }
}

// ---- the route plan inside a consumer's workgroup (small decode batches) ----
// For up to 64 routes, 64 experts and 16 tokens every workgroup of the
// gate/up launch builds the plan itself instead of waiting on a plan launch.
//
// Selection ranks every (token, expert) logit against its token's row at
// once by 64-bit keys (the logit's order-preserving bits, then the inverted
// expert index): rank = #{j : key_j > key_e}, so the k of rank < k are
// exactly what select_topk's repeated maximum takes, in the same order
// (non-finite logits rank as -inf, -0 as +0, ties to the lowest expert); the
// probabilities are select_topk's expressions in its order.
//
// The plan itself is ballots within each wavefront (lane r = route r): with
// B_b the mask of routes whose expert has bit b set, a lane's masks of the
// routes with its expert (`eq`) and with a lower expert (`lt`) follow bit by
// bit, and counts and offsets are their population counts: rank in the list
// = popc(eq below the lane), first sorted row = popc(lt), tile = popc(lt &
// heads) + rank / TR, heads being the routes with rank % TR == 0.
constexpr uint32_t SMALL_PLAN_ROUTES = 64, SMALL_PLAN_EXPERTS = 64, SMALL_PLAN_KEYS = 512;
__host__ __device__ inline uint32_t small_plan_stride(uint32_t experts) { return experts <= 32 ? 32u : 64u; }
__host__ __device__ inline bool small_plan_fits(uint32_t tokens, uint32_t routes, uint32_t experts) {
    return routes <= SMALL_PLAN_ROUTES && experts <= SMALL_PLAN_EXPERTS &&
           tokens * small_plan_stride(experts) <= SMALL_PLAN_KEYS;
}
// LDS words: keys (two words each), then route ids, chosen logits,
// probabilities, per-token non-finite flags, a tile's route ids
constexpr uint32_t SMALL_PLAN_WORDS = 2 * SMALL_PLAN_KEYS + 4 * 64 + 64;
__device__ __forceinline__ uint32_t *sh_ids(uint32_t *sh) { return sh + 2 * SMALL_PLAN_KEYS; }
__device__ __forceinline__ float *sh_chosen(uint32_t *sh) {
    return reinterpret_cast<float *>(sh + 2 * SMALL_PLAN_KEYS + 64);
}
__device__ __forceinline__ float *sh_probs(uint32_t *sh) {
    return reinterpret_cast<float *>(sh + 2 * SMALL_PLAN_KEYS + 128);
}
__device__ __forceinline__ uint32_t *sh_nonfinite(uint32_t *sh) { return sh + 2 * SMALL_PLAN_KEYS + 192; }
__device__ __forceinline__ uint32_t *sh_tile(uint32_t *sh) { return sh + 2 * SMALL_PLAN_KEYS + 256; }

__device__ __forceinline__ uint64_t small_key(float v, uint32_t e) {
    const uint32_t b = __float_as_uint(v), o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (0xffffffffu - e);
}
// #{j < S : key_j > key}, all S keys read before the first compare (keys
// past the experts are 0: below every real key)
template <int S>
__device__ __forceinline__ uint32_t small_rank(const uint64_t *row, uint64_t key) {
    uint64_t u[S];
#pragma unroll
    for (int q = 0; q < S / 2; q++) {
        const u32x4 f = reinterpret_cast<const u32x4 *>(row)[q];
        u[2 * q] = ((uint64_t)f.y << 32) | f.x;
        u[2 * q + 1] = ((uint64_t)f.w << 32) | f.z;
    }
    uint32_t rank = 0;
#pragma unroll
    for (int j = 0; j < S; j++) rank += u[j] > key ? 1u : 0u;
    return rank;
}

// Per-lane view of the plan, the same in every wavefront: lane r as route r.
struct SmallPlan {
    uint32_t e;      // expert (>= experts: none)
    uint32_t rk;     // rank in the expert's list (route order)
    uint64_t eq;     // routes of the same expert
    uint64_t lt;     // routes of lower experts
    uint64_t heads;  // routes that open a tile (uniform)
};

// Selection (logits set) or the given ids, then the plan, for tiles of TR
// rows; every thread of the workgroup (NTH threads) calls it; the
// probabilities only `with_probs`.  `sh` holds SMALL_PLAN_WORDS words of LDS.
template <int NTH, int TR>
__device__ __forceinline__ SmallPlan small_plan(const float *logits, const uint32_t *ids, uint32_t tokens, uint32_t experts,
                                uint32_t k, uint32_t *sh, bool with_probs) {
    uint32_t *sid = sh_ids(sh), *nf = sh_nonfinite(sh);
    float *sch = sh_chosen(sh), *sprob = sh_probs(sh);
    const uint32_t routes = tokens * k, tid = threadIdx.x, l = tid & 63;
    if (logits) {
        static_assert(SMALL_PLAN_KEYS % NTH == 0, "whole key slots per thread");
        constexpr int PER = SMALL_PLAN_KEYS / NTH;
        uint64_t *keys = reinterpret_cast<uint64_t *>(sh);
        const uint32_t S = small_plan_stride(experts);
        float v[PER];
        bool raw_fin[PER];
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint32_t i = tid + NTH * j, t = i / S, e = i % S;
            const float x = t < tokens && e < experts ? logits[t * experts + e] : 0.f;
            raw_fin[j] = finite_bits(x);
            v[j] = raw_fin[j] ? (x == 0.f ? 0.f : x) : -INFINITY;
        }
        if (tid < 64) nf[tid] = 0;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint32_t i = tid + NTH * j, t = i / S, e = i % S;
            keys[i] = t < tokens && e < experts ? small_key(v[j], e) : 0ull;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint32_t i = tid + NTH * j, t = i / S, e = i % S;
            if (t >= tokens || e >= experts) continue;
            if (!raw_fin[j]) nf[t] = 1;
            const uint64_t key = keys[i];
            const uint32_t rank = S == 32 ? small_rank<32>(keys + t * 32, key) : small_rank<64>(keys + t * 64, key);
            if (rank < k) {
                sid[t * k + rank] = e;
                sch[t * k + rank] = round_bf16(v[j]);
            }
        }
        if (with_probs) {
            __syncthreads();
            for (uint32_t r = tid; r < routes; r += NTH) {
                const uint32_t t = r / k, r0 = t * k;
                bool invalid = nf[t] != 0;
                for (uint32_t j = 0; j < k; j++) invalid |= !finite_bits(sch[r0 + j]);
                float p = __uint_as_float(0x7fc00000u);
                if (!invalid) {
                    float sum = 0.f;
                    for (uint32_t j = 0; j < k; j++) sum += expf(sch[r0 + j] - sch[r0]);
                    p = round_bf16(expf(sch[r] - sch[r0]) / sum);
                }
                sprob[r] = p;
            }
        }
    } else {
        for (uint32_t r = tid; r < routes; r += NTH) sid[r] = ids[r];
    }
    __syncthreads();
    SmallPlan sp;
    sp.e = l < routes ? sid[l] : 0xffffffffu;
    const bool valid = sp.e < experts;
    const uint64_t vmask = __ballot(valid);
    uint64_t eq = vmask, lt = 0;
    const uint32_t id_bits = experts > 1 ? 32u - (uint32_t)__builtin_clz(experts - 1) : 0u;
    for (int bit = (int)id_bits - 1; bit >= 0; bit--) {  // uniform
        const uint64_t b = __ballot(valid && ((sp.e >> bit) & 1u));
        if ((sp.e >> bit) & 1u) {
            lt |= eq & ~b;
            eq &= b;
        } else {
            eq &= ~b;
        }
    }
    sp.eq = valid ? eq : 0ull;
    sp.lt = valid ? lt : 0ull;
    sp.rk = (uint32_t)__popcll(sp.eq & ((1ull << l) - 1ull));
    sp.heads = __ballot(valid && sp.rk % TR == 0);
    return sp;
}

__device__ __forceinline__ uint32_t small_tiles(const SmallPlan &sp) { return (uint32_t)__popcll(sp.heads); }

// Tile y (< small_tiles) of the plan: its expert, rows, first sorted row and
// list row; the tile's route ids go to sh_tile(sh) (read after a barrier).
struct SmallTile {
    uint32_t expert, rows, sorted0, first;
};
template <int TR>
__device__ __forceinline__ SmallTile small_tile(const SmallPlan &sp, uint32_t y, uint32_t *sh) {
    const uint32_t l = threadIdx.x & 63;
    const bool head = (sp.heads >> l) & 1ull;
    const uint32_t tile = (uint32_t)__popcll(sp.lt & sp.heads) + sp.rk / TR;  // a route's tile
    const uint64_t own = __ballot(head && tile == y);
    const int h = (int)__builtin_ctzll(own);  // the tile's first route (uniform)
    SmallTile t;
    t.expert = (uint32_t)__builtin_amdgcn_readlane((int)sp.e, h);
    t.first = (uint32_t)__builtin_amdgcn_readlane((int)sp.rk, h);
    const uint32_t cnt = (uint32_t)__builtin_amdgcn_readlane((int)__popcll(sp.eq), h);
    t.rows = min((uint32_t)TR, cnt - t.first);
    t.sorted0 = (uint32_t)__builtin_amdgcn_readlane((int)__popcll(sp.lt), h) + t.first;
    if (threadIdx.x < 64 && sp.e == t.expert && tile == y) sh_tile(sh)[sp.rk - t.first] = l;
    return t;
}

// The plan as the down launch reads it: tile descriptors (PLAN_DESC_HEAD
// words {expert, rows, first sorted row, first list row}, then the tile's
// route ids) for the tiles in use, plan word 1 = tiles in use; and the
// selection (ids/probs) when it was made here.  Threads 0-63 of one
// workgroup.
template <int TR>
__device__ __forceinline__ void small_plan_store(const SmallPlan &sp, uint32_t routes, uint32_t *desc, uint32_t *plan, uint32_t *sh,
                                 uint32_t *ids_out, float *probs_out) {
    if (threadIdx.x >= 64) return;
    const uint32_t l = threadIdx.x, DW = PLAN_DESC_HEAD + TR;
    if (ids_out && l < routes) {
        ids_out[l] = sh_ids(sh)[l];
        probs_out[l] = sh_probs(sh)[l];
    }
    if (sp.eq) {  // a valid route
        const uint32_t tile = (uint32_t)__popcll(sp.lt & sp.heads) + sp.rk / TR, cnt = (uint32_t)__popcll(sp.eq);
        uint32_t *d = desc + (uint64_t)tile * DW;
        d[PLAN_DESC_HEAD + sp.rk % TR] = l;
        if (sp.rk % TR == 0) {
            const uint32_t first = sp.rk;
            d[0] = sp.e;
            d[1] = min((uint32_t)TR, cnt - first);
            d[2] = (uint32_t)__popcll(sp.lt) + first;
            d[3] = first;
        }
    }
    if (l == 0) plan[1] = small_tiles(sp);
}

}  // namespace oco
