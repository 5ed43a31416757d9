// Routing for the expert path: top-k selection, router logits, per-expert
// route plans and the weighted combine.  Replaces oco's
// shaders/experts/routing.metal (select_expert_values :71-94, router
// :96-128, router_logits :131-146, route_plan_64 :4-39, moe_sum :157-168) and
// nemotron.metal's route_plan_n (:238-273).
#include <algorithm>

#include "mxsplit.h"
#include "route.h"

namespace oco {

template <int PER>
__global__ __launch_bounds__(64) void route_select_kernel(const float *logits, uint32_t tokens,
                                                          uint32_t experts, uint32_t k, uint32_t *ids,
                                                          float *probs) {
    const uint32_t t = blockIdx.x;
    if (t >= tokens) return;
    select_topk<PER>(logits + (uint64_t)t * experts, experts, k, ids + (uint64_t)t * k,
                     probs + (uint64_t)t * k);
}

// Router logits = sum_k bf16(x) bf16(W[e]) + bf16(bias[e]) (routing.metal:96-146):
// one wavefront per (token, expert), fp32 FMA accumulation.
template <typename XT>
__global__ __launch_bounds__(256) void router_logits_kernel(const XT *x, const float *w, const float *bias,
                                                            uint32_t tokens, uint32_t hidden,
                                                            uint32_t experts, float *logits) {
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wave >= tokens * experts) return;
    const uint32_t t = wave / experts, e = wave % experts;
    float acc = 0.f;
    for (uint32_t i = lane; i < hidden; i += 64) {
        float xv = XLoad<XT>::one(x + (uint64_t)t * hidden, i);
        if constexpr (sizeof(XT) == 4) xv = round_bf16(xv);
        acc = fmaf(xv, round_bf16(w[(uint64_t)e * hidden + i]), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) logits[(uint64_t)t * experts + e] = acc + (bias ? round_bf16(bias[e]) : 0.f);
}

// The same logits with the reduction spread over a workgroup: workgroup
// g * experts + e takes expert e and tokens 4g .. 4g + 3, each thread four columns per
// 1024-column chunk (16-byte weight loads, all of a thread's loads issued
// before its first FMA), partial sums over DPP and then LDS.  Needs hidden %
// 4 == 0 and 16-byte (f32) or 8-byte (bf16) aligned rows.  Workgroups past
// the logits' (`rec` set) split the rows into records of four E2M3 terms
// (mxsplit.h), one split item (row, K step, block) per thread.
constexpr int ROUTER_TOKENS = 4;
template <typename XT>
__global__ __launch_bounds__(256) void router_logits_wide_kernel(const XT *x, const float *w, const float *bias,
                                                                 uint32_t tokens, uint32_t hidden,
                                                                 uint32_t experts, float *logits, uint8_t *rec) {
    constexpr int TT = ROUTER_TOKENS, U = 4;  // tokens per workgroup, chunks in flight per thread
    __shared__ float part[4][TT];
    const uint32_t groups = (tokens + TT - 1) / TT;
    if (blockIdx.x >= experts * groups) {  // the split job
        const uint64_t item = (uint64_t)(blockIdx.x - experts * groups) * 256 + threadIdx.x;
        if (item < (uint64_t)tokens * ((hidden + 63) / 64) * 2) {
            if constexpr (sizeof(XT) == 4)
                mx6_split_item<float>(reinterpret_cast<const float *>(x), rec, hidden, item);
            else
                mx6_split_item<uint16_t>(reinterpret_cast<const uint16_t *>(x), rec, hidden, item);
        }
        return;
    }
    const uint32_t e = blockIdx.x % experts, t0 = blockIdx.x / experts * TT, wave = threadIdx.x >> 6;
    const uint32_t nt = min((uint32_t)TT, tokens - t0), quads = hidden / 4;
    const float4 *wr = reinterpret_cast<const float4 *>(w + (uint64_t)e * hidden);
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.f;
    for (uint32_t f0 = threadIdx.x; f0 < quads; f0 += 256 * U) {
        float4 wv[U];
        float xv[TT][U][4];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t f = f0 + 256 * u;
            wv[u] = f < quads ? wr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const uint32_t tt = t0 + min((uint32_t)t, nt - 1);
                if (f < quads) {
                    if constexpr (sizeof(XT) == 4) {
                        const float4 v = reinterpret_cast<const float4 *>(x + (uint64_t)tt * hidden)[f];
                        xv[t][u][0] = v.x; xv[t][u][1] = v.y; xv[t][u][2] = v.z; xv[t][u][3] = v.w;
                    } else {
                        const uint2 v = reinterpret_cast<const uint2 *>(x + (uint64_t)tt * hidden)[f];
                        xv[t][u][0] = __uint_as_float(v.x << 16); xv[t][u][1] = __uint_as_float(v.x & 0xffff0000u);
                        xv[t][u][2] = __uint_as_float(v.y << 16); xv[t][u][3] = __uint_as_float(v.y & 0xffff0000u);
                    }
                } else {
                    xv[t][u][0] = xv[t][u][1] = xv[t][u][2] = xv[t][u][3] = 0.f;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float wq[4] = {round_bf16(wv[u].x), round_bf16(wv[u].y), round_bf16(wv[u].z), round_bf16(wv[u].w)};
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[t] = fmaf(sizeof(XT) == 4 ? round_bf16(xv[t][u][j]) : xv[t][u][j], wq[j], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TT; t++) {
        const float v = wave_sum(acc[t]);
        if ((threadIdx.x & 63) == 0) part[wave][t] = v;
    }
    __syncthreads();
    if (threadIdx.x < nt) {
        const uint32_t t = threadIdx.x;
        const float v = (part[0][t] + part[1][t]) + (part[2][t] + part[3][t]);
        logits[(uint64_t)(t0 + t) * experts + e] = v + (bias ? round_bf16(bias[e]) : 0.f);
    }
}

// Route plan (routing.metal:4-39, nemotron.metal:238-273) by one workgroup:
// per-expert route lists in route order, expert-sorted first rows, each
// route's sorted row, (expert, first list row) tiles of `tile_rows`, and the
// two dispatch grids at words 0-5.  Routes are taken 1024 at a time; a
// route's place in its expert's list is the expert's running count plus the
// number of earlier routes of the chunk with the same expert, so lists keep
// route order: up to 256 experts from ballot-matched peers inside each
// wavefront and per-wavefront histograms in LDS, beyond that by broadcast
// LDS reads of the whole chunk.  Ids >= experts are left out.
constexpr uint32_t PLAN_THREADS = 1024;
constexpr uint32_t PLAN_HIST_EXPERTS = 256;  // per-wavefront histograms in LDS up to this many experts
constexpr uint32_t PLAN_ONEPASS_CHUNKS = 8;   // the one-pass plan: up to this many chunks of 1024 routes
constexpr uint32_t PLAN_ONEPASS_WORDS = 12288;  // and per-(chunk, wavefront, expert) counts up to this many words (48 KB)

__host__ __device__ inline bool plan_one_pass(uint32_t routes, uint32_t experts) {
    const uint32_t nchunks = (routes + 1023) / 1024;
    return experts <= PLAN_HIST_EXPERTS && nchunks <= PLAN_ONEPASS_CHUNKS && nchunks * 16 * experts <= PLAN_ONEPASS_WORDS;
}

__global__ __launch_bounds__(PLAN_THREADS) void route_plan_kernel(const uint32_t *ids, uint32_t routes,
                                                                  uint32_t experts, uint32_t tile_rows,
                                                                  uint32_t up_tiles, uint32_t down_tiles,
                                                                  uint32_t *plan, PlanSide side) {
    if (blockIdx.x > 0) {  // the side job: four elements (or one split item) and one cleared word per thread
        const uint64_t t = (uint64_t)(blockIdx.x - 1) * PLAN_THREADS + threadIdx.x;
        if (t < side.nzero) side.zero[t] = 0;
        if (side.rec) {  // one split item (row, K step, block) per thread
            const uint64_t item = t;
            if (item < (uint64_t)side.rows * ((side.k + 63) / 64) * 2) {
                if (side.x_bf16)
                    mx6_split_item<uint16_t>(reinterpret_cast<const uint16_t *>(side.x), side.rec, side.k, item);
                else
                    mx6_split_item<float>(reinterpret_cast<const float *>(side.x), side.rec, side.k, item);
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint64_t i = 4 * t + j;
            if (i >= side.n) break;
            const float v = side.x_bf16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(side.x)[i] << 16)
                                        : reinterpret_cast<const float *>(side.x)[i];
            const _Float16 h = (_Float16)v;
            __builtin_memcpy(&side.y[i], &h, 2);
        }
        return;
    }
    // The expert selection first, a token per wavefront; the plan then reads
    // the selected ids back (written and read by this workgroup only).
    if (side.logits) {
        const uint32_t wave0 = threadIdx.x >> 6;
        for (uint32_t t = wave0; t < side.tokens; t += PLAN_THREADS / 64) {
            const float *lt = side.logits + (uint64_t)t * experts;
            uint32_t *it = side.ids_out + (uint64_t)t * side.topk;
            float *pt = side.probs_out + (uint64_t)t * side.topk;
            if (experts <= 64)
                select_topk<1>(lt, experts, side.topk, it, pt);
            else if (experts <= 128)
                select_topk<2>(lt, experts, side.topk, it, pt);
            else
                select_topk<4>(lt, experts, side.topk, it, pt);
        }
        __threadfence_block();
        __syncthreads();
        ids = side.ids_out;
    }
    // LDS: chunk ids [1024]; run, tile base, offset [experts]; per-wavefront
    // histograms [16][experts] (experts <= PLAN_HIST_EXPERTS)
    extern __shared__ __attribute__((aligned(16))) uint32_t sh[];
    uint32_t *chunk = sh, *run = sh + PLAN_THREADS, *tbase = run + experts, *offs = tbase + experts;
    uint32_t *hist = offs + experts;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint64_t grouped = 6 + 2 * ((uint64_t)(routes + 15) / 16 + experts);
    const uint64_t sorted = grouped + (uint64_t)experts * (routes + 1);

    // One pass (experts <= PLAN_HIST_EXPERTS, up to PLAN_ONEPASS_CHUNKS chunks
    // of 1024 routes whose per-wavefront histograms fit the LDS): every
    // route's rank among its wavefront's peers by ballots, the counts per
    // (chunk, wavefront, expert) in LDS, one exclusive scan per expert over
    // those slots (which also gives the counts), then every placement at
    // once -- a handful of barriers instead of four per chunk.
    const uint32_t nchunks = (routes + PLAN_THREADS - 1) / PLAN_THREADS;
    const bool one_pass = plan_one_pass(routes, experts);
    uint32_t ev[PLAN_ONEPASS_CHUNKS], rk[PLAN_ONEPASS_CHUNKS];
    if (one_pass) {
        // counts of (chunk, wavefront) slot q of expert e at hist[e * HS + q]:
        // an odd row stride keeps the scan's reads (threads of several
        // experts, each over a run of slots) on distinct banks
        const uint32_t slots = nchunks * 16, HS = slots + 1;
        for (uint32_t t = tid; t < HS * experts; t += PLAN_THREADS) hist[t] = 0;
        const uint32_t id_bits = experts > 1 ? 32u - (uint32_t)__builtin_clz(experts - 1) : 0u;
#pragma unroll
        for (uint32_t c = 0; c < PLAN_ONEPASS_CHUNKS; c++) {
            ev[c] = 0xffffffffu;
            rk[c] = 0;
            if (c < nchunks) {
                const uint32_t i = c * PLAN_THREADS + tid;
                ev[c] = i < routes ? ids[i] : 0xffffffffu;
            }
        }
        __syncthreads();  // hist cleared
#pragma unroll
        for (uint32_t c = 0; c < PLAN_ONEPASS_CHUNKS; c++) {
            if (c >= nchunks) break;  // uniform
            const uint32_t e = ev[c];
            uint64_t peers = __ballot(e < experts);
            if (e >= experts) peers = ~peers;
            for (uint32_t bit = 0; bit < id_bits; bit++) {
                const uint64_t b = __ballot((e >> bit) & 1u);
                peers &= ((e >> bit) & 1u) ? b : ~b;
            }
            rk[c] = (uint32_t)__popcll(peers & ((1ull << lane) - 1ull));
            if (e < experts && (peers >> lane) == 1ull) hist[e * HS + c * 16 + wave] = rk[c] + 1;
        }
        __syncthreads();
        // exclusive scan per expert over the slots (chunk, wavefront) in
        // route order: G consecutive threads per expert, each over a run of
        // slots, joined by a shuffle scan within the group
        uint32_t G = 1;
        while (G * 2 * experts <= PLAN_THREADS && G < 64) G *= 2;
        const uint32_t e = tid / G, j = tid % G, per = (slots + G - 1) / G;
        uint32_t local = 0;
        if (e < experts)
            for (uint32_t q = j * per; q < min(slots, j * per + per); q++) local += hist[e * HS + q];
        uint32_t incl = local;
        for (uint32_t o = 1; o < G; o <<= 1) {
            const uint32_t v = (uint32_t)__shfl_up((int)incl, o, (int)G);
            if (j >= o) incl += v;
        }
        if (e < experts) {
            uint32_t run_e = incl - local;
            for (uint32_t q = j * per; q < min(slots, j * per + per); q++) {
                const uint32_t v = hist[e * HS + q];
                hist[e * HS + q] = run_e;
                run_e += v;
            }
            if (j == G - 1) run[e] = incl;
        }
        __syncthreads();
    }
    // 1. counts per expert (four ids in flight per thread)
    for (uint32_t e = tid; e < experts && !one_pass; e += PLAN_THREADS) run[e] = 0;
    __syncthreads();
    for (uint32_t base = tid; base < routes && !one_pass; base += 4 * PLAN_THREADS) {
        uint32_t ev[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t i = base + u * PLAN_THREADS;
            ev[u] = i < routes ? ids[i] : 0xffffffffu;
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (ev[u] < experts) atomicAdd(&run[ev[u]], 1u);
    }
    __syncthreads();
    // 2. offsets and tile bases: a block-wide exclusive scan over experts
    // (thread t owns experts [t P, t P + P)), then counts, offsets, tiles
    const uint32_t P = (experts + PLAN_THREADS - 1) / PLAN_THREADS, e0 = tid * P;
    uint32_t my_c = 0, my_t = 0;
    for (uint32_t e = e0; e < min(e0 + P, experts); e++) {
        my_c += run[e];
        my_t += (run[e] + tile_rows - 1) / tile_rows;
    }
    uint32_t inc_c = my_c, inc_t = my_t;  // inclusive scans within the wavefront
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t c2 = (uint32_t)__shfl_up((int)inc_c, o), t2 = (uint32_t)__shfl_up((int)inc_t, o);
        if ((int)lane >= o) {
            inc_c += c2;
            inc_t += t2;
        }
    }
    uint32_t *wsum = chunk;  // [16] counts, [16] tiles (chunk is free until step 3)
    if (lane == 63) {
        wsum[wave] = inc_c;
        wsum[16 + wave] = inc_t;
    }
    __syncthreads();
    uint32_t off_c = inc_c - my_c, off_t = inc_t - my_t;
    for (uint32_t w = 0; w < wave; w++) {
        off_c += wsum[w];
        off_t += wsum[16 + w];
    }
    for (uint32_t e = e0; e < min(e0 + P, experts); e++) {
        const uint32_t count = run[e];
        plan[grouped + (uint64_t)e * (routes + 1)] = count;
        plan[sorted + e] = off_c;
        offs[e] = off_c;
        tbase[e] = off_t;
        off_c += count;
        off_t += (count + tile_rows - 1) / tile_rows;
    }
    if (tid == PLAN_THREADS - 1) {  // the last thread ends with the totals
        plan[0] = up_tiles;
        plan[1] = off_t;
        plan[2] = 1;
        plan[3] = down_tiles;
        plan[4] = off_t;
        plan[5] = 1;
    }
    __syncthreads();
    const uint32_t DW = PLAN_DESC_HEAD + tile_rows;  // descriptor words per tile
    for (uint32_t e = tid; e < experts; e += PLAN_THREADS) {
        uint32_t t = tbase[e];
        for (uint32_t b = 0; b < run[e]; b += tile_rows, t++) {
            plan[6 + 2 * (uint64_t)t] = e;
            plan[6 + 2 * (uint64_t)t + 1] = b;
            if (side.desc) {
                uint32_t *d = side.desc + (uint64_t)t * DW;
                d[0] = e;
                d[1] = min(tile_rows, run[e] - b);
                d[2] = offs[e] + b;
                d[3] = b;
            }
        }
    }
    if (side.desc) {  // unused tile slots: no rows
        const uint32_t slots = (routes + 15) / 16 + experts;
        uint32_t total = 0;  // tiles in use: the per-wavefront tile sums of step 2
        for (uint32_t w = 0; w < 16; w++) total += wsum[16 + w];
        for (uint32_t t = total + tid; t < slots; t += PLAN_THREADS) side.desc[(uint64_t)t * DW + 1] = 0;
    }
    if (one_pass) {
        __syncthreads();  // offs[] is complete
        // Every route's place goes to an expert-sorted array in LDS first,
        // (expert << 16) | route, and the lists and descriptors are written
        // from it in sorted order: consecutive threads then store consecutive
        // words, where storing from each route's own thread scatters every
        // wavefront instruction over 64 lines through this one CU's address
        // unit.
        uint32_t *srt = hist + max(16 * experts, (nchunks * 16 + 1) * experts);
#pragma unroll
        for (uint32_t c = 0; c < PLAN_ONEPASS_CHUNKS; c++) {
            if (c >= nchunks) break;  // uniform
            const uint32_t e = ev[c], i = c * PLAN_THREADS + tid;
            if (e < experts) {
                const uint32_t pos = hist[e * (nchunks * 16 + 1) + c * 16 + wave] + rk[c];
                srt[offs[e] + pos] = (e << 16) | i;
                plan[sorted + experts + i] = offs[e] + pos;
            }
        }
        uint32_t placed = 0;  // routes with a valid expert: the per-wavefront count sums of step 2
        for (uint32_t w = 0; w < 16; w++) placed += wsum[w];
        __syncthreads();
        for (uint32_t j = tid; j < placed; j += PLAN_THREADS) {
            const uint32_t v = srt[j], e = v >> 16, i = v & 0xffffu, pos = j - offs[e];
            plan[grouped + (uint64_t)e * (routes + 1) + 1 + pos] = i;
            if (side.desc)
                side.desc[(uint64_t)(tbase[e] + pos / tile_rows) * DW + PLAN_DESC_HEAD + pos % tile_rows] = i;
        }
        return;
    }
    __syncthreads();
    for (uint32_t e = tid; e < experts; e += PLAN_THREADS) run[e] = 0;  // reused as the running count of step 3
    __syncthreads();
    // 3. stable placement, 1024 routes at a time: a route's place in its
    // expert's list is the running count plus its rank among the chunk's
    // earlier routes of the same expert
    const uint32_t id_bits = experts > 1 ? 32u - (uint32_t)__builtin_clz(experts - 1) : 0u;
    uint32_t e_next = tid < routes ? ids[tid] : 0xffffffffu;
    for (uint32_t base = 0; base < routes; base += PLAN_THREADS) {
        const uint32_t i = base + tid, e = e_next;
        e_next = i + PLAN_THREADS < routes ? ids[i + PLAN_THREADS] : 0xffffffffu;  // next chunk, in flight
        uint32_t rank = 0;
        if (experts <= PLAN_HIST_EXPERTS) {
            // Lanes of the wavefront holding the same expert: one ballot per
            // bit of the id (and one for validity) narrows each lane's peer
            // mask; the rank is the count of earlier peers, and the last peer
            // carries the wavefront's count.
            uint64_t peers = __ballot(e < experts);
            if (e >= experts) peers = ~peers;
            for (uint32_t bit = 0; bit < id_bits; bit++) {
                const uint64_t b = __ballot((e >> bit) & 1u);
                peers &= ((e >> bit) & 1u) ? b : ~b;
            }
            rank = (uint32_t)__popcll(peers & ((1ull << lane) - 1ull));
            const bool last = (peers >> lane) == 1ull;
            for (uint32_t t = tid; t < 16 * experts; t += PLAN_THREADS) hist[t] = 0;
            __syncthreads();
            if (e < experts && last) hist[wave * experts + e] = rank + 1;
            __syncthreads();
            if (e < experts)
                for (uint32_t w = 0; w < wave; w++) rank += hist[w * experts + e];
        } else {
            chunk[tid] = e;
            __syncthreads();
            if (e < experts) {
                const uint4 *c4 = reinterpret_cast<const uint4 *>(chunk);
                uint32_t j = 0;
                for (; j + 4 <= tid; j += 4) {
                    const uint4 v = c4[j / 4];
                    rank += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
                }
                for (; j < tid; j++) rank += chunk[j] == e;
            }
        }
        const uint32_t pos = e < experts ? run[e] + rank : 0;
        __syncthreads();  // every read of run[], chunk[] and hist[] is done
        if (e < experts) {
            plan[grouped + (uint64_t)e * (routes + 1) + 1 + pos] = i;
            plan[sorted + experts + i] = offs[e] + pos;
            if (side.desc)
                side.desc[(uint64_t)(tbase[e] + pos / tile_rows) * DW + PLAN_DESC_HEAD + pos % tile_rows] = i;
            atomicAdd(&run[e], 1u);
        }
        __syncthreads();
    }
}

// out[t, d] = bf16(out + bf16(sum_r route[t*k + r, d] * p[t, r])), the sum in
// route order in fp32 (routing.metal:157-168).  The reference stores route
// outputs as bf16, so f32 route values are rounded to bf16 first.
template <typename RT>
__global__ __launch_bounds__(256) void moe_sum_kernel(const RT *routes, const float *probs, uint16_t *out,
                                                      uint32_t hidden, uint32_t tokens, uint32_t k) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)hidden * tokens) return;
    const uint64_t t = i / hidden, d = i % hidden;
    // all k (<= 8) route values requested before the first FMA
    float v[8], p[8];
#pragma unroll
    for (uint32_t r = 0; r < 8; r++) {
        if (r >= k) break;
        if constexpr (sizeof(RT) == 4)
            v[r] = round_bf16(routes[(t * k + r) * hidden + d]);
        else
            v[r] = bf16_bits_to_f32(routes[(t * k + r) * hidden + d].bits);
        p[r] = probs[t * k + r];
    }
    float s = 0.f;
#pragma unroll
    for (uint32_t r = 0; r < 8; r++) {
        if (r >= k) break;
        s = fmaf(v[r], p[r], s);
    }
    out[i] = f32_to_bf16_bits(bf16_bits_to_f32(out[i]) + round_bf16(s));
}

// The same for bf16 routes and hidden % 8 == 0, eight outputs per thread
// with 16-byte loads; the per-element arithmetic and order are unchanged.
__global__ __launch_bounds__(256) void moe_sum8_kernel(const uint16_t *routes, const float *probs, uint16_t *out,
                                                       uint32_t hidden, uint32_t tokens, uint32_t k) {
    const uint64_t i8 = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i8 * 8 >= (uint64_t)hidden * tokens) return;
    const uint64_t i = i8 * 8, t = i / hidden, d = i % hidden;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // all k (<= 8) routes' words requested before the first FMA
    uint4 rv[8];
    float pv[8];
#pragma unroll
    for (uint32_t r = 0; r < 8; r++) {
        if (r >= k) break;
        rv[r] = *reinterpret_cast<const uint4 *>(routes + (t * k + r) * hidden + d);
        pv[r] = probs[t * k + r];
    }
#pragma unroll
    for (uint32_t r = 0; r < 8; r++) {
        if (r >= k) break;
        const uint32_t w[4] = {rv[r].x, rv[r].y, rv[r].z, rv[r].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            s[2 * j] = fmaf(__uint_as_float(w[j] << 16), pv[r], s[2 * j]);
            s[2 * j + 1] = fmaf(__uint_as_float(w[j] & 0xffff0000u), pv[r], s[2 * j + 1]);
        }
    }
    uint4 o = *reinterpret_cast<const uint4 *>(out + i);
    uint32_t ow[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t lo = f32_to_bf16_bits(bf16_bits_to_f32(ow[j] & 0xffffu) + round_bf16(s[2 * j]));
        const uint32_t hi = f32_to_bf16_bits(bf16_bits_to_f32(ow[j] >> 16) + round_bf16(s[2 * j + 1]));
        ow[j] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4 *>(out + i) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

}  // namespace oco

using namespace oco;

namespace oco {

int route_plan_launch(const uint32_t *ids, uint32_t routes, uint32_t experts, uint32_t tile_rows, uint32_t up_tiles,
                      uint32_t down_tiles, uint32_t *plan, const PlanSide *side, hipStream_t stream) {
    if (!ids || !plan) return fail(OCO_ERR_INVALID, "oco_route_plan: null pointer");
    if (experts == 0 || experts > 4096 || tile_rows < 16)
        return fail(OCO_ERR_INVALID,
                    "oco_route_plan: need 0 < experts <= 4096 and tile_rows >= 16 (the plan holds ceil(routes/16) + "
                    "experts tiles)");
    PlanSide sj = side ? *side : PlanSide{};
    if (sj.rec && sj.k % 32) return fail(OCO_ERR_INVALID, "oco_route_plan: split rows need k %% 32 == 0 (k=%u)", sj.k);
    const uint64_t side_items = sj.rec ? (uint64_t)sj.rows * ((sj.k + 63) / 64) * 2 : (sj.n + 3) / 4;  // threads
    const uint64_t side_blocks =
        std::max<uint64_t>((side_items + PLAN_THREADS - 1) / PLAN_THREADS, (sj.nzero + PLAN_THREADS - 1) / PLAN_THREADS);
    if (side_blocks >= 0x7fffffffu) return fail(OCO_ERR_INVALID, "oco_route_plan: side job of %llu elements", (unsigned long long)sj.n);
    // LDS words: chunk ids, run / tile base / offset per expert, then the
    // histograms and (one pass) the expert-sorted routes.
    const size_t lds = (size_t)(PLAN_THREADS + 3 * experts +
                                (plan_one_pass(routes, experts)
                                     ? std::max(16 * experts, ((routes + 1023) / 1024 * 16 + 1) * experts) + routes
                                 : experts <= PLAN_HIST_EXPERTS ? 16 * experts
                                                                : 0)) * 4;
    if (lds > 64 * 1024)
        OCO_TRY(hip_check(hipFuncSetAttribute((const void *)route_plan_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                          "hipFuncSetAttribute"));
    hipLaunchKernelGGL(route_plan_kernel, dim3(1 + (unsigned)side_blocks), dim3(PLAN_THREADS), lds, stream, ids, routes,
                       experts, tile_rows, up_tiles, down_tiles, plan, sj);
    return launch_check("oco_route_plan");
}

}  // namespace oco

extern "C" {

int oco_route_select(const float *logits, uint32_t tokens, uint32_t experts, uint32_t k, uint32_t *ids,
                     float *probs, oco_stream stream) {
    if (!tokens) return OCO_OK;
    if (!logits || !ids || !probs) return fail(OCO_ERR_INVALID, "oco_route_select: null pointer");
    if (experts == 0 || experts > 256 || k == 0 || k > 8 || k > experts)
        return fail(OCO_ERR_INVALID, "oco_route_select: need 0 < k <= 8, k <= experts <= 256");
    hipStream_t s = (hipStream_t)stream;
    if (experts <= 64)
        hipLaunchKernelGGL(route_select_kernel<1>, dim3(tokens), dim3(64), 0, s, logits, tokens, experts, k, ids, probs);
    else if (experts <= 128)
        hipLaunchKernelGGL(route_select_kernel<2>, dim3(tokens), dim3(64), 0, s, logits, tokens, experts, k, ids, probs);
    else
        hipLaunchKernelGGL(route_select_kernel<4>, dim3(tokens), dim3(64), 0, s, logits, tokens, experts, k, ids, probs);
    return launch_check("oco_route_select");
}

int oco_router(const void *x, oco_dtype x_dtype, const float *w, const float *bias, uint32_t tokens,
               uint32_t hidden, uint32_t experts, uint32_t k, float *logits, uint32_t *ids, float *probs,
               oco_stream stream) {
    if (!tokens) return OCO_OK;
    if (!x || !w || !ids || !probs) return fail(OCO_ERR_INVALID, "oco_router: null pointer");
    if (experts == 0 || experts > 256 || k == 0 || k > 8 || k > experts)
        return fail(OCO_ERR_INVALID, "oco_router: need 0 < k <= 8, k <= experts <= 256");
    hipStream_t s = (hipStream_t)stream;
    float *l = logits;
    if (!l) {
        // Caller did not ask for the logits: keep them in a per-call allocation.
        OCO_TRY(hip_check(hipMallocAsync((void **)&l, (size_t)tokens * experts * 4, s), "hipMallocAsync"));
    }
    int rc = router_logits_launch(x, x_dtype, w, bias, tokens, hidden, experts, l, nullptr, s);
    if (rc == OCO_OK) rc = oco_route_select(l, tokens, experts, k, ids, probs, stream);
    if (!logits) (void)hipFreeAsync(l, s);
    return rc;
}

}  // extern "C"

namespace oco {
int router_logits_launch(const void *x, oco_dtype x_dtype, const float *w, const float *bias, uint32_t tokens,
                         uint32_t hidden, uint32_t experts, float *logits, uint8_t *rec, hipStream_t s) {
    const uint32_t waves = tokens * experts;
    const uint32_t xal = x_dtype == OCO_DT_F32 ? 16 : 8;
    const uint64_t split_blocks = rec ? ((uint64_t)tokens * ((hidden + 63) / 64) * 2 + 255) / 256 : 0;
    const uint64_t router_blocks = (uint64_t)experts * ((tokens + ROUTER_TOKENS - 1) / ROUTER_TOKENS);
    if (rec && hidden % 32) return fail(OCO_ERR_INVALID, "router: split rows need hidden %% 32 == 0 (hidden=%u)", hidden);
    const bool wide = hidden % 4 == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & (xal - 1)) == 0 &&
                      (x_dtype == OCO_DT_F32 || x_dtype == OCO_DT_BF16);
    if (wide || (rec && !logits)) {
        if (router_blocks + split_blocks >= 0x7fffffffull)
            return fail(OCO_ERR_INVALID, "router: %u tokens x %u experts over one grid", tokens, experts);
        // a split alone (no logits): no router workgroups
        const uint32_t ex = logits ? experts : 0;
        const dim3 grid((unsigned)((logits ? router_blocks : 0) + split_blocks));
        if (grid.x == 0) return OCO_OK;
        if (x_dtype == OCO_DT_F32)
            hipLaunchKernelGGL(router_logits_wide_kernel<float>, grid, dim3(256), 0, s, (const float *)x, w, bias,
                               tokens, hidden, ex, logits, rec);
        else if (x_dtype == OCO_DT_BF16)
            hipLaunchKernelGGL(router_logits_wide_kernel<bf16_t>, grid, dim3(256), 0, s, (const bf16_t *)x, w, bias,
                               tokens, hidden, ex, logits, rec);
        else
            return fail(OCO_ERR_UNSUPPORTED, "router: activations must be f32 or bf16");
        return launch_check("router logits");
    }
    if (x_dtype == OCO_DT_F32)
        hipLaunchKernelGGL(router_logits_kernel<float>, dim3((waves + 3) / 4), dim3(256), 0, s,
                           (const float *)x, w, bias, tokens, hidden, experts, logits);
    else if (x_dtype == OCO_DT_BF16)
        hipLaunchKernelGGL(router_logits_kernel<bf16_t>, dim3((waves + 3) / 4), dim3(256), 0, s,
                           (const bf16_t *)x, w, bias, tokens, hidden, experts, logits);
    else
        return fail(OCO_ERR_UNSUPPORTED, "router: activations must be f32 or bf16");
    OCO_TRY(launch_check("router logits"));
    // the split apart when the rows did not suit the wide kernel
    return rec ? router_logits_launch(x, x_dtype, w, bias, tokens, hidden, experts, nullptr, rec, s) : OCO_OK;
}
}  // namespace oco

extern "C" {

uint64_t oco_route_plan_words(uint32_t routes, uint32_t experts) {
    return 6 + 2 * ((uint64_t)(routes + 15) / 16 + experts) + (uint64_t)experts * (routes + 1) + experts +
           routes;
}


int oco_route_plan(const uint32_t *ids, uint32_t routes, uint32_t experts, uint32_t tile_rows,
                   uint32_t up_tiles, uint32_t down_tiles, uint32_t *plan, oco_stream stream) {
    return route_plan_launch(ids, routes, experts, tile_rows, up_tiles, down_tiles, plan, nullptr,
                             (hipStream_t)stream);
}


int oco_moe_sum(const void *routes, oco_dtype routes_dtype, const float *probs, uint16_t *out,
                uint32_t hidden, uint32_t tokens, uint32_t k, oco_stream stream) {
    uint64_t n = (uint64_t)hidden * tokens;
    if (!n) return OCO_OK;
    if (!routes || !probs || !out) return fail(OCO_ERR_INVALID, "oco_moe_sum: null pointer");
    if (k > 8) return fail(OCO_ERR_INVALID, "oco_moe_sum: k=%u routes per token, at most 8", k);
    hipStream_t s = (hipStream_t)stream;
    unsigned grid = (unsigned)((n + 255) / 256);
    if (routes_dtype == OCO_DT_F32)
        hipLaunchKernelGGL(moe_sum_kernel<float>, dim3(grid), dim3(256), 0, s, (const float *)routes, probs,
                           out, hidden, tokens, k);
    else if (routes_dtype == OCO_DT_BF16 && hidden % 8 == 0 && ((uintptr_t)routes & 15) == 0 && ((uintptr_t)out & 15) == 0)
        hipLaunchKernelGGL(moe_sum8_kernel, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, s,
                           (const uint16_t *)routes, probs, out, hidden, tokens, k);
    else if (routes_dtype == OCO_DT_BF16)
        hipLaunchKernelGGL(moe_sum_kernel<bf16_t>, dim3(grid), dim3(256), 0, s, (const bf16_t *)routes, probs,
                           out, hidden, tokens, k);
    else
        return fail(OCO_ERR_UNSUPPORTED, "oco_moe_sum: routes must be f32 or bf16");
    return launch_check("oco_moe_sum");
}

}  // extern "C"
