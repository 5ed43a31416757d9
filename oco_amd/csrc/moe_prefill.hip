// Routed-expert prefill for Q4_K banks with the weights decoded in registers:
// the grouped expert GEMMs of expert_up_tensor / moe_activate /
// expert_down_tensor (projections.metal:192-376, routing.metal:44-64) at
// the few dozen routes per expert of MoE prefill, where each weight is used
// by only that many rows and staging decoded weights through LDS costs more
// than the multiply.
//
// v_mfma_f32_16x16x32_f16: lane l supplies row / column l % 16 and the
// eight K values 8 (l / 16) .. + 8.  K order is free as long as both
// operands agree, so each lane group q = l / 16 takes Q4_K sub-block pair q
// of a super-block (32 qs bytes: 64 weights, low nibbles then high nibbles)
// and MFMA chunk c (0..7) of the super-block pairs
//     k = 64 q + 8 c + e,   e = 0..7
// -- for the weights, byte 32 q + 8 (c % 4) + e, nibble c / 4; for the
// activations, a contiguous 16-byte run of the staged row.  A lane decodes
// exactly the weights it multiplies (half(d sc q - dmin mn), as the
// reference's half tiles: tile.metal:35-52); weights pass through LDS as raw
// bytes only, never decoded.
//
// Work: a unit is (route-plan tile of 16 MI rows, column chunk of NW x 16
// gate/up columns or NW x 32 down columns).  The grid is persistent: each
// workgroup takes a contiguous range of units (tile-major) and runs one flat
// pipeline of (unit, super-block) steps across them, so the prefetch does
// not restart per unit.  Each step:
//   - activations of the step two ahead go straight from global memory into
//     a three-stage LDS ring (global_load_lds_dwordx4, no registers), rows
//     swizzled so that the MFMA A reads are conflict-free;
//   - weights of the step two ahead load into a three-set register ring as
//     whole-line chunks (each row's 144-byte super-block is nine consecutive
//     16-byte chunks), and at the step pass through a per-wavefront LDS
//     region to the lanes that decode them;
//   - the wavefront decodes and multiplies its two 16-row fragments
//     (gate/up: the 16 gate rows and the same 16 up rows, so the activation
//     is fused in-lane; down: two groups of 16 rows).
// Both GEMMs read f16 rows: the caller's inputs (gathered per route) for
// gate/up, and for down the gate/up activations already scaled per row by a
// power of two into f16 range (act_f16_kernel).
#include "matmul.h"
#include "formats.h"

#include <algorithm>

namespace oco {

typedef _Float16 q4f16x8 __attribute__((ext_vector_type(8)));
typedef float q4f32x4 __attribute__((ext_vector_type(4)));

struct Q4Raw {  // one lane's bytes of one super-block: header and its 32 qs bytes
    uint4 hdr, q0, q1;
};
// A wavefront's weights of one step as loaded: its 32 rows' super-blocks
// (144 bytes each), 288 16-byte chunks, chunk lane + 64 i in c[i].
struct Q4Set {
    uint4 c[5];
};

// Scales of sub-block pair q: a = d sc, m = dmin mn for the low (0) and high
// (1) nibbles (get_scale_min_k4, weights.metal:67-77).
struct Q4Scales {
    float a0, m0, a1, m1;
};
__device__ __forceinline__ Q4Scales q4_scales(const uint4 &hdr, int q) {
    // scales[12] = hdr.y (bytes 0..3), hdr.z (4..7), hdr.w (8..11); sub-block
    // j < 4: sc = scales[j] & 63, mn = scales[j+4] & 63; j >= 4: sc =
    // (scales[j+4] & 15) | (scales[j-4] >> 6) << 4, mn = (scales[j+4] >> 4) |
    // (scales[j] >> 6) << 4.  Pair q holds j = 2q, 2q + 1; with b = 2 (q & 1)
    // both forms read bytes b, b + 1 of hdr.y and hdr.z, and the second also
    // bytes b, b + 1 of hdr.w, so two byte permutes gather the lane's
    // [sc0, sc1, mn0, mn1].
    const uint32_t b = 2u * (uint32_t)(q & 1);
    const uint32_t sel = b | ((b + 1) << 8) | ((b + 4) << 16) | ((b + 5) << 24);
    const uint32_t yz = __builtin_amdgcn_perm(hdr.z, hdr.y, sel);                                 // y_b, y_b1, z_b, z_b1
    const uint32_t ww = __builtin_amdgcn_perm(hdr.w, hdr.w, (sel & 0x0000ffffu) | ((sel & 0xffffu) << 16));  // w_b, w_b1, w_b, w_b1
    const uint32_t lo6 = yz & 0x3f3f3f3fu;
    const uint32_t hi6 = (ww & 0x00000f0fu) | ((ww >> 4) & 0x0f0f0000u) | ((yz >> 2) & 0x30303030u);
    const uint32_t v = q < 2 ? lo6 : hi6;
    const float d = half_bits_to_f32(hdr.x & 0xffffu), dmin = half_bits_to_f32(hdr.x >> 16);
    return {d * (float)(v & 0xffu), dmin * (float)((v >> 16) & 0xffu), d * (float)((v >> 8) & 0xffu),
            dmin * (float)(v >> 24)};
}

// Eight f16 weights of chunk c from the lane's qs bytes (q0 = bytes 0..15,
// q1 = 16..31 of its pair).
template <int C>
__device__ __forceinline__ q4f16x8 q4_chunk(const Q4Raw &r, const Q4Scales &s) {
    const uint4 &src = (C % 4) < 2 ? r.q0 : r.q1;
    const uint32_t w0 = (C % 2) == 0 ? src.x : src.z, w1 = (C % 2) == 0 ? src.y : src.w;
    const float a = C < 4 ? s.a0 : s.a1, m = C < 4 ? s.m0 : s.m1;
    const int sh = C < 4 ? 0 : 4;
    uint32_t o[4];
    q4_four((w0 >> sh) & 0x0f0f0f0fu, a, m, o[0], o[1]);
    q4_four((w1 >> sh) & 0x0f0f0f0fu, a, m, o[2], o[3]);
    q4f16x8 v;
    __builtin_memcpy(&v, o, 16);
    return v;
}

// A workgroup's range holds at most Q4_UNITS units over at most Q4_TILES
// tiles (the launch sizes the grid for that); their route rows and biases
// are read once, into LDS, before the pipeline starts.
constexpr int Q4_TILES = 4, Q4_UNITS = 8;

template <int B, int E, typename F>
__device__ __forceinline__ void q4_static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        q4_static_for<B + 1, E>(f);
    }
}

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void q4_vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Max over the 16 lanes of a DPP row (lanes 16 r .. 16 r + 15).
__device__ __forceinline__ uint32_t q4_row_max(uint32_t m) {
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xf, 0xf, false));   // quad xor 1
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xf, 0xf, false));   // quad xor 2
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xf, 0xf, false));  // half-row mirror
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x140, 0xf, 0xf, false));  // row mirror
    return m;
}

// LDS reads outside the ring, as inline asm: the compiler cannot tell the
// arrays they read from the ring's stages, so a read it sees waits for every
// global->LDS load in flight.  The caller's s_waitcnt lgkmcnt(0) (inline asm
// too) takes the results as operands, so no use moves above it.
__device__ __forceinline__ uint32_t q4_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ __forceinline__ uint32_t q4_lds_b32(const void *p) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(q4_lds_addr(p)));
    return v;
}
typedef uint32_t q4u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ q4u32x4 q4_lds_b128(const void *p) {
    q4u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(q4_lds_addr(p)));
    return v;
}

// A use of v the compiler cannot see through (it must have landed here).
__device__ __forceinline__ void q4_touch(const uint4 &v) {
    q4u32x4 t;
    __builtin_memcpy(&t, &v, 16);
    asm volatile("" ::"v"(t));
}

// 16 bytes per lane from global memory straight into LDS: lane l writes
// lds + 16 l (global_load_lds_dwordx4; lds must be uniform).
__device__ __forceinline__ void q4_load_lds16(gbytes src, void *lds) {
    __builtin_amdgcn_global_load_lds((const GLOBAL void *)src, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}


template <int G, int MI, int NW>
__global__ __launch_bounds__(64 * NW) void moe_q4k_kernel(KPRE_PARAMS, MatmulArgs a, uint32_t chunks) {
    KPRE_APPLY(a);
    constexpr int ROWS = 16 * MI;
    constexpr int XL = ROWS / (2 * NW);  // activation loads per lane per step (16 bytes each)
    constexpr int STAGE = ROWS * 512;    // one super-block of f16 rows
    constexpr int COLS = G == MM_GATE_UP ? 16 : 32;
    constexpr int LOADS = XL + 5;        // vector loads per lane per step
    static_assert(ROWS % (2 * NW) == 0, "whole 16-byte runs per lane");
    static_assert(Q4_TILES * ROWS <= 64 * NW, "one thread per (tile, row) in the prologue");
    // Three separate arrays, so the compiler can tell an LDS load of one stage
    // from the asynchronous global->LDS loads into another (one array would
    // make it wait for every outstanding load before each LDS read).
    __shared__ __attribute__((aligned(16))) uint8_t xs0[STAGE], xs1[STAGE], xs2[STAGE];
    __shared__ __attribute__((aligned(16))) uint32_t t_route[Q4_TILES][ROWS];
    __shared__ __attribute__((aligned(16))) float t_inv[G == MM_DOWN ? Q4_TILES : 1][ROWS];
    __shared__ __attribute__((aligned(16))) uint32_t t_info[Q4_TILES][4];  // expert, rows, first sorted row
    __shared__ float u_bias[Q4_UNITS][2 * 16 * NW];  // gate/up: gate then up biases; down: biases
    // Each wavefront's weights of the step it computes, [row][144 bytes]
    // (320 chunk slots: the loads past the 288 land in the tail).
    __shared__ __attribute__((aligned(16))) uint8_t wst[NW * 5120];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c16 = lane & 15, q = lane >> 4;
    const uint32_t grid = gridDim.x, lg = xcd_order(blockIdx.x, grid);
    const auto plan = gp(a.plan);
    const uint32_t U = plan[1] * chunks;
    const uint32_t lo = (uint32_t)((uint64_t)lg * U / grid), hi = (uint32_t)((uint64_t)(lg + 1) * U / grid);
    if (lo >= hi) return;  // uniform
    const uint32_t y0 = lo / chunks, ny = (hi - 1) / chunks - y0 + 1;  // <= Q4_TILES (launch)
    const uint32_t nu = hi - lo;                                        // <= Q4_UNITS (launch)

    // Tile prologue: per (tile, row) the route, the inverse row gain (down),
    // and the tile's expert / row count / first expert-sorted row.
    const uint64_t grouped = 6 + 2 * ((uint64_t)(a.routes + 15) / 16 + a.experts);
    const uint64_t sorted = grouped + (uint64_t)a.experts * (a.routes + 1);
    {
        const uint32_t ti = tid / ROWS, r = tid % ROWS;
        if (ti < ny) {
            const uint32_t y = y0 + ti;
            const uint32_t expert = plan[6 + 2 * y], first = plan[7 + 2 * y];
            const uint64_t list = grouped + (uint64_t)expert * (a.routes + 1);
            const uint32_t rows = min((uint32_t)ROWS, plan[list] - first);
            const uint32_t sorted0 = plan[sorted + expert] + first;
            const uint32_t rr = min(r, rows - 1);  // padding rows repeat the last row (discarded)
            t_route[ti][r] = plan[list + 1 + first + rr];
            if constexpr (G == MM_DOWN) t_inv[ti][r] = 1.0f / row_gain(gp(a.rowmax)[sorted0 + rr]);
            if (r == 0) {
                t_info[ti][0] = expert;
                t_info[ti][1] = rows;
                t_info[ti][2] = sorted0;
            }
        }
    }
    // Biases of each unit's columns (as bf16, the reference's bias tensors;
    // the up bias folds in the clipped SwiGLU's + 1).
    for (uint32_t e = tid; e < nu * 2 * 16 * NW; e += 64 * NW) {
        const uint32_t j = e / (2 * 16 * NW), c = e % (2 * 16 * NW), u = lo + j, y = u / chunks, ch = u - y * chunks;
        const uint32_t expert = plan[6 + 2 * y];
        float b = 0.f;
        if constexpr (G == MM_GATE_UP) {
            const bool up = c >= 16 * NW;
            const uint32_t col = ch * (NW * COLS) + c % (16 * NW);
            const float *bias = up ? a.bias2 : a.bias;
            const float one = up && a.up_one ? 1.0f : 0.0f;
            b = col < a.n && bias ? round_bf16(gp(bias)[(uint64_t)expert * a.n + col] + one) : one;
        } else {
            const uint32_t col = ch * (NW * COLS) + c;
            b = col < a.n && a.bias ? round_bf16(gp(a.bias)[(uint64_t)expert * a.n + col]) : 0.f;
        }
        u_bias[j][c] = b;
    }
    __syncthreads();

    const uint32_t nsb = a.k / 256, T = nu * nsb;
    const uint64_t xrow = (uint64_t)a.k * 2;
    const gbytes x8 = gp(reinterpret_cast<const uint8_t *>(a.x));

    // Prefetch cursor: unit pu, super-block psb; per-lane source offsets.
    uint32_t pu = lo, psb = 0;
    uint32_t xoff[XL];
    gbytes cptr[5];
    auto set_unit = [&](uint32_t u) __attribute__((always_inline)) {
        const uint32_t y = u / chunks, ch = u - y * chunks, ti = y - y0;
        const uint32_t expert = __builtin_amdgcn_readfirstlane(t_info[ti][0]);
        const uint32_t rows = __builtin_amdgcn_readfirstlane(t_info[ti][1]);
        const uint32_t sorted0 = __builtin_amdgcn_readfirstlane(t_info[ti][2]);
#pragma unroll
        for (int i = 0; i < XL; i++) {
            const uint32_t r = 2 * (wave + NW * i) + (lane >> 5), j = (lane & 31) ^ (r & 15);
            const uint32_t src = G == MM_GATE_UP ? t_route[ti][r] / a.topk : sorted0 + min(r, rows - 1);
            xoff[i] = (uint32_t)(src * xrow) + 16 * j;
        }
        // Weight chunk j = lane + 64 i: row j / 9 of the wavefront's 32
        // (fragment f = row / 16), 16-byte piece j % 9 of its super-block.
        const uint64_t eoff = (uint64_t)expert * a.expert_bytes;
        const gbytes bank0 = gp(a.w) + eoff, bank1 = gp(G == MM_GATE_UP ? a.w2 : a.w) + eoff;
#pragma unroll
        for (int i = 0; i < 5; i++) {
            const uint32_t j = min(lane + 64u * i, 287u), r = j / 9, p = j - 9 * r, f = r >> 4;
            const uint32_t col = ch * (NW * COLS) + wave * COLS + (G == MM_GATE_UP ? 0 : 16 * f) + (r & 15);
            const uint64_t off = (uint64_t)min(col, a.n - 1) * a.row_bytes + 16 * p;
            cptr[i] = (G == MM_GATE_UP && f ? bank1 : bank0) + off;
        }
    };
    // Refill of stage nst / register set wn for the cursor's step, as
    // LOADS items: 0..4 the weight chunks (whole lines per instruction:
    // each row's super-block is nine consecutive chunks), 5.. the activation
    // rows.  The items are spread over the eight MFMA chunks of a step:
    // issued all at once, every wavefront's loads queued behind each other's
    // at the address units.
    auto load_item = [&](auto kk, int nst, Q4Set *wn) __attribute__((always_inline)) {
        constexpr int K = decltype(kk)::value;
        if constexpr (K < 5) {
            wn->c[K] = ld_u128(cptr[K] + psb * 144);
        } else {
            constexpr int i = K - 5;
            uint8_t *stage = nst == 0 ? xs0 : nst == 1 ? xs1 : xs2;
            q4_load_lds16(x8 + xoff[i] + psb * 512, stage + (wave + NW * i) * 1024);
        }
    };
    auto advance = [&]() __attribute__((always_inline)) {
        if (++psb == nsb) {  // uniform
            psb = 0;
            if (++pu < hi) set_unit(pu);
        }
    };
    q4f32x4 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = q4f32x4{0.f, 0.f, 0.f, 0.f};

    // 16-row fragments of the computing unit's tile that hold routes: the
    // MFMAs of the others are skipped (their rows are never stored).
    auto tile_live = [&](uint32_t u) __attribute__((always_inline)) {
        const uint32_t rows = __builtin_amdgcn_readfirstlane(t_info[u / chunks - y0][1]);
        return (min(rows, (uint32_t)ROWS) + 15) / 16;
    };
    uint32_t live = tile_live(lo);

    // One step: eight MFMA chunks of 32 k, each issuing its share of the
    // refill for step t + 2.
    auto compute = [&](int st, const Q4Set *wc, int nst, Q4Set *wn) __attribute__((always_inline)) {
        // The step's chunks through the wavefront's LDS region to the lanes
        // that decode them: lane (c16, q) takes fragment f's row 16 f + c16,
        // its header and its pair q of qs halves.
        uint8_t *ws = wst + wave * 5120;
#pragma unroll
        for (int i = 0; i < 5; i++) *reinterpret_cast<uint4 *>(ws + 16 * (lane + 64 * i)) = wc->c[i];
        // (Reads as inline asm, with their own wait: the compiler cannot tell
        // this region from the ring's stages and would wait for every
        // global->LDS load in flight.)
        asm volatile("" ::: "memory");  // the writes stay above the reads
        q4u32x4 v[6];
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const uint8_t *blk = ws + (16 * f + c16) * 144;
            v[3 * f] = q4_lds_b128(blk);
            v[3 * f + 1] = q4_lds_b128(blk + 16 + 32 * q);
            v[3 * f + 2] = q4_lds_b128(blk + 32 + 32 * q);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]));
        Q4Raw r[2];
#pragma unroll
        for (int f = 0; f < 2; f++) {
            __builtin_memcpy(&r[f].hdr, &v[3 * f], 16);
            __builtin_memcpy(&r[f].q0, &v[3 * f + 1], 16);
            __builtin_memcpy(&r[f].q1, &v[3 * f + 2], 16);
        }
        const uint8_t *xb = (st == 0 ? xs0 : st == 1 ? xs1 : xs2) + c16 * 512;
        const Q4Scales s0 = q4_scales(r[0].hdr, q), s1 = q4_scales(r[1].hdr, q);
        auto chunk = [&](auto cc) __attribute__((always_inline)) {
            constexpr int C = decltype(cc)::value;
            q4_static_for<C * LOADS / 8, (C + 1) * LOADS / 8>([&](auto kk) { load_item(kk, nst, wn); });
            q4f16x8 av[MI];
#pragma unroll
            for (int i = 0; i < MI; i++)
                __builtin_memcpy(&av[i], xb + i * 16 * 512 + 16 * ((8 * q + C) ^ c16), 16);
            const q4f16x8 b0 = q4_chunk<C>(r[0], s0), b1 = q4_chunk<C>(r[1], s1);
#pragma unroll
            for (int i = 0; i < MI; i++) {
                if (i > 0 && (uint32_t)i >= live) continue;  // uniform: a fragment past the tile's routes
                acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], b0, acc[i][0], 0, 0, 0);
                acc[i][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], b1, acc[i][1], 0, 0, 0);
            }
        };
        q4_static_for<0, 8>(chunk);
        advance();
    };

    // Gate/up: per lane, max |activation| bits of its rows over the tile's
    // units so far.
    uint32_t rmax[G == MM_GATE_UP ? MI : 1][4] = {};

    // C fragment: lane l holds column l % 16, rows 4 (l / 16) .. + 4.
    auto epilogue = [&](uint32_t u) __attribute__((always_inline)) {
        const uint32_t y = u / chunks, ch = u - y * chunks, ti = y - y0;
        const float *ub = u_bias[u - lo];
        const int cr = q * 4;
        q4u32x4 info = q4_lds_b128(t_info[ti]);
        if constexpr (G == MM_GATE_UP) {
            uint32_t bgb = q4_lds_b32(ub + wave * 16 + c16), bub = q4_lds_b32(ub + 16 * NW + wave * 16 + c16);
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(info), "+v"(bgb), "+v"(bub));
            const uint32_t rows = info.y, sorted0 = info.z;
            const float bg = __uint_as_float(bgb), bu = __uint_as_float(bub);
            const uint32_t col = ch * (NW * COLS) + wave * COLS + c16;
            const bool cok = col < a.n;
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const uint32_t r = i * 16 + cr + v;
                    const float act = expert_activation(a.act, acc[i][0][v] + bg, acc[i][1][v] + bu);
                    if (cok && r < rows) gp(reinterpret_cast<float *>(a.y))[(uint64_t)(sorted0 + r) * a.n + col] = act;
                    if (cok) rmax[i][v] = max(rmax[i][v], __float_as_uint(act) & 0x7fffffffu);
                }
            // Row maxima go out once per (workgroup, tile): after the tile's
            // last unit in this range.
            if (u + 1 == hi || (u + 1) / chunks != y) {
#pragma unroll
                for (int i = 0; i < MI; i++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const uint32_t r = i * 16 + cr + v, m = q4_row_max(rmax[i][v]);
                        if (c16 == 0 && r < rows) atomicMax(&a.rowmax[sorted0 + r], m);
                        rmax[i][v] = 0;
                    }
            }
        } else {
            // this lane's rows 16 i + 4 q .. + 3: routes and inverse gains
            uint32_t bb[2];
            q4u32x4 rt[MI], ig[MI];
#pragma unroll
            for (int f = 0; f < 2; f++) bb[f] = q4_lds_b32(ub + wave * COLS + 16 * f + c16);
#pragma unroll
            for (int i = 0; i < MI; i++) {
                rt[i] = q4_lds_b128(&t_route[ti][i * 16 + cr]);
                ig[i] = q4_lds_b128(&t_inv[ti][i * 16 + cr]);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(info), "+v"(bb[0]), "+v"(bb[1]));
#pragma unroll
            for (int i = 0; i < MI; i++) asm volatile("" : "+v"(rt[i]), "+v"(ig[i]));
            const uint32_t rows = info.y;
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const uint32_t col = ch * (NW * COLS) + wave * COLS + 16 * f + c16;
                if (col >= a.n) continue;
                const float b = __uint_as_float(bb[f]);
#pragma unroll
                for (int i = 0; i < MI; i++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const uint32_t r = i * 16 + cr + v;
                        if (r >= rows) continue;
                        // the inverse gain is a power of two: exact, as the division
                        const float val = acc[i][f][v] * __uint_as_float(ig[i][v]) + b;
                        const uint64_t o = (uint64_t)rt[i][v] * a.n + col;
                        if (a.y_bf16)
                            gp(reinterpret_cast<uint16_t *>(a.y))[o] = f32_to_bf16_bits(val);
                        else
                            gp(reinterpret_cast<float *>(a.y))[o] = val;
                    }
            }
        }
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = q4f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // Step t computes stage t % 3 with register set t % 3 and refills stage
    // and set (t + 2) % 3, consumed at step t - 1; past the last step the
    // refills repeat the last unit's first super-block, never consumed.
    Q4Set w0, w1, w2;
    set_unit(lo);
    // Steps 0 and 1's loads.
    q4_static_for<0, LOADS>([&](auto kk) { load_item(kk, 0, &w0); });
    advance();
    q4_static_for<0, LOADS>([&](auto kk) { load_item(kk, 1, &w1); });
    advance();
    uint32_t cu = lo, csb = 0;
    bool pend = false;  // unit cu - 1's results are in acc, not yet stored
    // Start of step t (compute register set wc): its loads landed in every
    // wavefront, a finished unit's stores go out, and wc is marked in use
    // (the compiler's own wait for it then sits here, where it has landed).
    auto start = [&](int t, const Q4Set *wc) __attribute__((always_inline)) {
        q4_vm_wait<LOADS>();                      // step t's loads (step t + 1's may be in flight)
        asm volatile("s_barrier" ::: "memory");  // every wavefront's LDS loads landed; stage (t + 2) % 3 is free
#pragma unroll
        for (int i = 0; i < 5; i++) q4_touch(wc->c[i]);
        // A finished unit's stores go out before this step's loads, so that
        // reusing their registers later waits only as far as those loads.
        if (pend) {
            epilogue(cu - 1);
            pend = false;
        }
    };
    auto body = [&](int st, int t, const Q4Set *wc, Q4Set *wn) __attribute__((always_inline)) {
        compute(st, wc, (st + 2) % 3, wn);  // issues step t + 2's loads on the way
        if (++csb == nsb) {
            csb = 0;
            cu++;
            pend = true;
            if (cu < hi) live = tile_live(cu);
        }
    };
    // The loop starts with step t's compute (its start is the previous
    // iteration's last act, or the prologue's), so that its entry and its
    // back edge hold the same loads in flight.
    start(0, &w0);
    for (int t = 0;; t += 3) {
        body(0, t, &w0, &w2);
        if (t + 1 >= (int)T) break;
        start(t + 1, &w1);
        body(1, t + 1, &w1, &w0);
        if (t + 2 >= (int)T) break;
        start(t + 2, &w2);
        body(2, t + 2, &w2, &w1);
        if (t + 3 >= (int)T) break;
        start(t + 3, &w0);
    }
    epilogue(cu - 1);  // the last unit ends on the last step
    q4_vm_wait<0>();  // no LDS load may land after the workgroup exits
}

// Eight wavefronts (two per SIMD; the registers allow no more); rows per
// tile bm = 16 MI routes (32, 48 or 64).
constexpr int Q4_NW = 8;

template <int G, int MI>
static int q4_launch(const MatmulArgs &a, uint32_t bm, hipStream_t stream) {
    static int per_cu = 0, cus = 0;
    if (!per_cu) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, moe_q4k_kernel<G, MI, Q4_NW>, 64 * Q4_NW, 0) != hipSuccess || per_cu <= 0)
            per_cu = 1;
        if (cus <= 0) cus = 256;
    }
    const uint32_t cols = (G == MM_GATE_UP ? 16 : 32) * Q4_NW;
    const uint32_t chunks = (a.n + cols - 1) / cols;
    const uint64_t max_units = (uint64_t)((a.routes + bm - 1) / bm + a.experts) * chunks;
    // Enough workgroups that no range holds more than Q4_UNITS units or
    // spans more than Q4_TILES tiles.
    const uint64_t span = std::min<uint64_t>(Q4_UNITS, (uint64_t)(Q4_TILES - 1) * chunks + 1);
    uint64_t grid = std::min<uint64_t>(max_units, (uint64_t)per_cu * cus);
    grid = std::max<uint64_t>(grid, (max_units + span - 1) / span);
    if (grid > 0x7fffffffu) return fail(OCO_ERR_INVALID, "experts: Q4_K grid of %llu units", (unsigned long long)max_units);
    hipLaunchKernelGGL((moe_q4k_kernel<G, MI, Q4_NW>), dim3((unsigned)grid), dim3(64 * Q4_NW), 0, stream, KPRE_ARGS(a), a, chunks);
    return OCO_OK;
}


int moe_q4k_launch(int mode, const MatmulArgs &a, uint32_t bm, hipStream_t stream) {
    if (a.k % 256) return fail(OCO_ERR_INVALID, "experts: Q4_K rows need k %% 256 == 0 (k=%u)", a.k);
    if (bm != 32 && bm != 48 && bm != 64) return fail(OCO_ERR_INVALID, "experts: Q4_K tile of %u rows", bm);
    // Activation rows are addressed with 32-bit byte offsets.
    const uint64_t xrows = mode == MM_GATE_UP ? (uint64_t)a.routes / std::max(a.topk, 1u) : (uint64_t)a.routes;
    if (xrows * a.k * 2 >= 0xffffffffull)
        return fail(OCO_ERR_INVALID, "experts: Q4_K activations of %llu bytes exceed 4 GiB",
                    (unsigned long long)(xrows * a.k * 2));
    int rc = OCO_OK;
    if (mode == MM_GATE_UP) {
        if (bm == 32) rc = q4_launch<MM_GATE_UP, 2>(a, bm, stream);
        if (bm == 48) rc = q4_launch<MM_GATE_UP, 3>(a, bm, stream);
        if (bm == 64) rc = q4_launch<MM_GATE_UP, 4>(a, bm, stream);
    } else {
        if (bm == 32) rc = q4_launch<MM_DOWN, 2>(a, bm, stream);
        if (bm == 48) rc = q4_launch<MM_DOWN, 3>(a, bm, stream);
        if (bm == 64) rc = q4_launch<MM_DOWN, 4>(a, bm, stream);
    }
    OCO_TRY(rc);
    return launch_check("experts Q4_K grouped matmul");
}

}  // namespace oco
