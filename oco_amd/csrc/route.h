// Top-k expert selection shared by the routing and expert kernels.
#pragma once
#include "common.h"

namespace oco {

// A job run beside the route plan, in the same launch (workgroups 1..):
// activation rows to f16 (the reference's half(x)) from bf16 or f32, four
// elements per thread, and `nzero` words of `zero` cleared; or, with `rec`
// set, the rows' E4M3 split records (mxsplit.h: bf16 rows in two terms, f32
// rows in three) in place of the f16 copy.
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

// oco_route_plan with an optional side job (null: none).
// Router logits [tokens, experts] (routing.metal:96-146) into `logits`.
int router_logits_launch(const void *x, oco_dtype x_dtype, const float *w, const float *bias, uint32_t tokens,
                         uint32_t hidden, uint32_t experts, float *logits, hipStream_t stream);
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

}  // namespace oco
