// MXFP4 prefill on CDNA4's block-scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4).
// Same operation as the MXFP4 case of oco_matmul -- Y = X W^T (+ bias) for
// DenseMatrix::apply's MXFP4 plans (src/weights/compute/matrix.rs:130-379,
// shaders/matrix/batch.metal:24-79) -- without decoding a single weight:
//
//  * W (GGUF MXFP4: per 32 values one E8M0 byte, then 16 bytes of E2M1 nibbles,
//    value j in the low nibble of byte j and value j+16 in the high nibble) is
//    the B operand as stored.  Its E8M0 byte is the B block scale.
//  * X (bf16) is split once per call into two E4M3 terms with their own E8M0
//    scale per 32-block: x = s1 q1 + s2 q2.  s1 is the smallest power of two
//    with max|x| / s1 <= 448; the residual x - s1 q1 is exact in fp32 and its
//    rounding to E4M3 under s2 leaves at most 2^-8 of the residual's block
//    maximum.  The split stores the terms in the MFMA's register order with
//    the k order of each block permuted to match W's nibble order, so every
//    operand load is one contiguous 16-byte access.
//
// Operand layout of the 32x32x64 scaled MFMA (measured on gfx950), row
// (column, for B) r = l % 32, block b = 0, 1 of the K=64 step:
//  * B, E2M1: lane r + 32b holds block b as 16 bytes, element e in nibble
//    e & 1 of byte e / 2 -- exactly a GGUF MXFP4 block's payload;
//  * A, E4M3: block b's elements 0..15 are bytes 16b .. 16b + 15 of lane r,
//    elements 16..31 the same bytes of lane r + 32;
//  * block b's scale is in lane r + 32b (A and B), byte chosen by op_sel.
// The accumulator holds column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "stream.h"

namespace oco {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// One record per (32-row tile, K step of 64): [term 2][block 2][lane 64][16 B]
// of E4M3 codes, then [lane 64] u32 of E8M0 scales (byte t = term t).
constexpr uint32_t MX_DATA = 2 * 2 * 64 * 16, MX_REC = MX_DATA + 64 * 4;

struct MxSplitArgs {
    const uint16_t *x;
    uint8_t *frag;
    uint32_t m, k, ksteps, records;
};

// Smallest E with amax <= 448 * 2^E, as the E8M0 byte E + 127 (0 for a zero
// block, 255 -- NaN -- for a non-finite one).
__device__ __forceinline__ int mx_scale_exp(float amax) {
    if (!(amax <= 3.402823466e38f)) return 128;
    if (amax == 0.f) return -127;
    const uint32_t b = __float_as_uint(amax);
    int e;
    uint32_t mant;
    if (b >> 23) {
        e = (int)(b >> 23) - 127;
        mant = b & 0x7fffffu;
    } else {  // subnormal amax: normalise
        const int lz = __builtin_clz(b) - 8;
        e = -126 - lz;
        mant = (b << lz) & 0x7fffffu;
    }
    const int E = mant <= 0x600000u ? e - 8 : e - 7;  // m <= 1.75 <=> m * 256 <= 448
    return E < -127 ? -127 : E;
}

// One workgroup per record: four lanes per (row, block), each holding 8 of
// the block's 32 values (q = lane % 4: values 8q .. 8q + 7).  The block's
// maximum meets over the quad through DPP; in the record, chunk p of a
// (term, block) interleaves groups p and p + 2 (byte 2i: value 8p + i,
// byte 2i + 1: value 8p + 16 + i), so partner lanes q and q ^ 2 swap their
// codes and each stores 8 of the chunk's 16 bytes.
__global__ __launch_bounds__(256) void mx_split_kernel(KPRE_PARAMS, MxSplitArgs a) {
    KPRE_APPLY(a);
    const uint32_t rec = blockIdx.x;
    const uint32_t tile = rec / a.ksteps, s = rec % a.ksteps;
    const int tid = threadIdx.x, q = tid & 3, pair = tid >> 2, r = pair & 31, blk = pair >> 5;
    const uint32_t row = tile * 32 + r, k0 = s * 64 + 32 * blk;
    float v[8];
    if (row < a.m && k0 < a.k) {
        const uint4 u = *reinterpret_cast<const uint4 *>(a.x + (uint64_t)row * a.k + k0 + 8 * q);
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = __uint_as_float(w4[j] << 16);
            v[2 * j + 1] = __uint_as_float(w4[j] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.f;
    }
    uint8_t *out = a.frag + (uint64_t)rec * MX_REC;
    uint32_t scales = 0;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        // |x| bit patterns order like the values, with Inf above every
        // finite value and NaN above Inf: the integer maximum carries both.
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) m = max(m, __float_as_uint(v[i]) & 0x7fffffffu);
        m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xf, 0xf, false));  // quad xor 1
        m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xf, 0xf, false));  // quad xor 2
        const int E = mx_scale_exp(__uint_as_float(m));
        scales |= (uint32_t)(E + 127) << (8 * t);
        const float inv = E == 128 ? 0.f : __builtin_ldexpf(1.f, -E), sc = E == 128 ? 0.f : __builtin_ldexpf(1.f, E);
        uint32_t c[2];  // codes of values 8q .. 8q + 3 and 8q + 4 .. 8q + 7
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int pk = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h] * inv, v[4 * h + 1] * inv, 0, false);
            pk = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h + 2] * inv, v[4 * h + 3] * inv, pk, true);
            c[h] = (uint32_t)pk;
            v[4 * h] -= __builtin_amdgcn_cvt_f32_fp8(pk, 0) * sc;
            v[4 * h + 1] -= __builtin_amdgcn_cvt_f32_fp8(pk, 1) * sc;
            v[4 * h + 2] -= __builtin_amdgcn_cvt_f32_fp8(pk, 2) * sc;
            v[4 * h + 3] -= __builtin_amdgcn_cvt_f32_fp8(pk, 3) * sc;
        }
        const uint32_t o0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)c[0], 0x4E, 0xf, 0xf, false);
        const uint32_t o1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)c[1], 0x4E, 0xf, 0xf, false);
        // Lane q < 2 (group p = q) stores bytes 0..7 of chunk p: its values
        // 0..3 with the partner's; lane q >= 2 (group p + 2) bytes 8..15: the
        // partner's values 4..7 with its own.
        const uint32_t ev = q < 2 ? c[0] : o1, od = q < 2 ? o0 : c[1];
        const uint32_t lo = __builtin_amdgcn_perm(od, ev, 0x05010400u), hi = __builtin_amdgcn_perm(od, ev, 0x07030602u);
        const int p = q & 1;
        *reinterpret_cast<uint2 *>(out + ((t * 2 + blk) * 64 + r + 32 * p) * 16 + (q >= 2 ? 8 : 0)) = make_uint2(lo, hi);
    }
    if (q == 0) *reinterpret_cast<uint32_t *>(out + MX_DATA + (r + 32 * blk) * 4) = scales;
}

// The first 56 bytes arrive in SGPRs (KPre).
struct MxArgs {
    const uint8_t *w;
    const uint8_t *frag;
    uint32_t m, n, k, ksteps, tiles;
    uint32_t row_bytes;
    uint32_t wspan;  // weight bytes from the dword-aligned base, rounded up to 4 (< 4 GiB)
    uint32_t y_bf16;
    void *y;
    const float *bias;
};

template <int I>
struct Int {
    static constexpr int value = I;
};
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(Int<I>{});
        static_for<N, I + 1>(f);
    }
}

typedef void (*MxFn)(u32x4, u32x4, u32x4, u32x2, MxArgs);

// A buffer resource the compiler keeps in SGPRs: every field goes through
// readfirstlane (the values are uniform; without this a resource built next
// to divergent code may land in VGPRs and every load becomes a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void *p, uint32_t bytes) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(uintptr_t)(((uint64_t)hi << 32) | lo), 0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// ---------------------------------------------------------------------------
// Prefill tile: workgroup = four wavefronts, WM along the activation rows
// and 4 / WM along the weight rows (output columns); each wavefront owns one
// 32-row activation tile and CTW 32-column weight tiles, so a K step is
// 2 CTW independent MFMAs (the two activation terms of every column tile).
//
// Sizing (measured on MI355X): an L2-resident operand stream reaches about
// 33 bytes/clock per CU, and a 32x32x64 MFMA takes 64 clocks.  A workgroup
// tile of BM rows x BN columns loads 2 BM x 64 bytes of activations and
// 34 BN / 32 bytes of weights per K step.  At 128 x 96 (WM = 4) that is
// 53 bytes per 384 MFMA clocks: the L2 stream, not the MFMA, sets the pace.
// At 64 x 192 (WM = 2) the two wavefronts of a row tile read the same
// activation records (the second from the CU's L1), and L2 traffic falls to
// 39 bytes per 384 clocks for the same number of workgroups.
//
//  * A: each wavefront's split records go straight into a register ring RA
//    K steps deep, through a buffer resource whose step offset is scalar.
//  * B: GGUF rows staged a double step (4 blocks, 68 bytes) at a time: each
//    thread moves whole blocks (the 20-byte dword-aligned span holding 17
//    bytes), realigned into LDS as [block][row] 16-byte payloads and scale
//    words whose byte (step parity) the MFMA's op_sel picks.  A register
//    ring RB double steps deep feeds three LDS stages; one barrier per
//    double step.
template <int WM, int CTW, int RB>
struct MxPlan {
    static constexpr int WN = 4 / WM, BM = 32 * WM, BN = 32 * CTW * WN, BLOCKS = 4 * BN, BU = (BLOCKS + 255) / 256;
    static constexpr int PAY = 4 * BN * 16, SCL = 2 * BN * 4, STAGE = PAY + SCL + 16;  // + landing pad of unused slots
    static constexpr int NST = 3, LDS = NST * STAGE, RA = 6;
    static_assert(WM * WN == 4, "four wavefronts");
    static_assert(RB % 3 == 0 && RB >= 3, "the B ring is a whole number of LDS stage rounds");
};

template <int WM, int CTW, int RB>
__global__ __launch_bounds__(256) void mx_matmul_kernel(KPRE_PARAMS, MxArgs a) {
    KPRE_APPLY(a);
    using P = MxPlan<WM, CTW, RB>;
    constexpr int BN = P::BN, BU = P::BU, STAGE = P::STAGE, RA = P::RA, CT = CTW;
    constexpr int PER = RB;  // double steps per unrolled round: RB, 3 stages and RA / 2 all divide it
    static_assert(PER % 3 == 0 && (2 * PER) % RA == 0, "ring periods");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // The wavefront index is uniform: readfirstlane keeps the A resource in SGPRs.
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
              part = lane >> 5;
    const int wm = wave % WM, wn = wave / WM;
    // Logical (column tile, row group), column-major per XCD: the row groups
    // of one weight column tile share its GGUF bytes in one L2.
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
    const uint32_t bx = lin / gridDim.y, by = lin % gridDim.y;
    const uint32_t tile = by * WM + wm, col0 = bx * BN;
    const uint32_t nblk = a.k / 32, nsteps = a.ksteps;

    // A: this wavefront's records; steps past the end read as zero.
    const __amdgpu_buffer_rsrc_t ra_rs =
        uniform_rsrc(a.frag + (uint64_t)min(tile, a.tiles - 1) * a.ksteps * MX_REC, a.ksteps * MX_REC);
    // B: the tensor from its dword-aligned base; bytes past the end read as zero.
    const uint32_t wsh = (uint32_t)((uintptr_t)a.w & 3u);
    const __amdgpu_buffer_rsrc_t rb_rs = uniform_rsrc(a.w - wsh, a.wspan);
    const uint32_t rbytes = (uint32_t)a.row_bytes;
    // Staging: thread slot g = tid + 256 u moves block g % 4 of row g / 4 of
    // each double step, realigned into the payload and scale arrays.
    uint32_t boff[BU], bsh[BU], bpay[BU], bscl[BU];
#pragma unroll
    for (int u = 0; u < BU; u++) {
        const uint32_t g = tid + 256 * u, row = min(g / 4, (uint32_t)BN - 1), blk = g % 4;
        const uint32_t at = wsh + min(col0 + row, a.n - 1) * rbytes + 17 * blk;
        const bool live = g < (uint32_t)P::BLOCKS;
        boff[u] = at & ~3u;
        bsh[u] = at & 3u;
        bpay[u] = live ? (blk * BN + row) * 16 : P::PAY + P::SCL;  // unused slots: the landing pad
        bscl[u] = live ? P::PAY + ((blk & 1) * BN + row) * 4 + (blk >> 1) : P::PAY + P::SCL;
    }
    const uint32_t wcol = wn * CT * 32;  // this wavefront's first column within the tile

    i32x8 av[RA][2];
    uint32_t as[RA];
    u32x4 bv[RB][BU];
    uint32_t bx4[RB][BU];
    auto load_a = [&](auto slot, uint32_t s) {
        constexpr int U = decltype(slot)::value;
        const uint32_t so = s * MX_REC;
#pragma unroll
        for (int t = 0; t < 2; t++) {
#if defined(OCO_ABL) && OCO_ABL == 6
            const u32x4 lo = u32x4{so, (uint32_t)t, 3u, 4u}, hi = u32x4{(uint32_t)lane, so, 1u, 2u};
#else
            const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(ra_rs, lane * 16 + 2 * t * 1024, so, 0);
            const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(ra_rs, lane * 16 + (2 * t + 1) * 1024, so, 0);
#endif
            av[U][t] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
        as[U] = __builtin_amdgcn_raw_buffer_load_b32(ra_rs, MX_DATA + lane * 4, so, 0);
    };
    auto load_b = [&](auto slot, uint32_t j) {
        constexpr int U = decltype(slot)::value;
#pragma unroll
        for (int u = 0; u < BU; u++) {
#if defined(OCO_ABL) && OCO_ABL == 7
            bv[U][u] = u32x4{boff[u], j, 5u, 6u};
            bx4[U][u] = boff[u] ^ j;
#else
            bv[U][u] = __builtin_amdgcn_raw_buffer_load_b128(rb_rs, boff[u], j * 68, 0);
            bx4[U][u] = __builtin_amdgcn_raw_buffer_load_b32(rb_rs, boff[u] + 16, j * 68, 0);
#endif
        }
    };
    auto store_b = [&](auto slot, auto stage) {
        constexpr int U = decltype(slot)::value, S = decltype(stage)::value;
#pragma unroll
        for (int u = 0; u < BU; u++) {
            const u32x4 v = bv[U][u];
            const uint32_t w4 = bx4[U][u], sh = bsh[u];
            // Span bytes: scale at sh, payload at sh + 1 .. sh + 16.
            // alignbyte shifts by 0..3 bytes: a shift of 4 is the next dword.
            const uint32_t sh1 = sh + 1;
            const uint32_t d0 = sh1 == 4 ? v.y : __builtin_amdgcn_alignbyte(v.y, v.x, sh1);
            const uint32_t d1 = sh1 == 4 ? v.z : __builtin_amdgcn_alignbyte(v.z, v.y, sh1);
            const uint32_t d2 = sh1 == 4 ? v.w : __builtin_amdgcn_alignbyte(v.w, v.z, sh1);
            const uint32_t d3 = sh1 == 4 ? w4 : __builtin_amdgcn_alignbyte(w4, v.w, sh1);
            *reinterpret_cast<u32x4 *>(lds + S * STAGE + bpay[u]) = u32x4{d0, d1, d2, d3};
            lds[S * STAGE + bscl[u]] = (uint8_t)(v.x >> (8 * sh));
        }
    };

    // One accumulator per column tile; a step issues term 0 over all tiles,
    // then term 1, so consecutive MFMAs never share an accumulator.
    f32x16 acc[CT];
#pragma unroll
    for (int j = 0; j < CT; j++) acc[j] = f32x16{};

    // B fragments: payload per step (double-buffered by parity), scales per
    // double step (byte = step parity, chosen by op_sel).
    i32x8 bf[2][CT];
    uint32_t sw[CT];
    auto frag_read = [&](auto stage, auto par) {
        constexpr int S = decltype(stage)::value, PA = decltype(par)::value;
        const uint8_t *base = lds + S * STAGE;
#pragma unroll
        for (int j = 0; j < CT; j++) {
            const u32x4 q = *reinterpret_cast<const u32x4 *>(base + ((2 * PA + part) * BN + wcol + j * 32 + c) * 16);
            bf[PA][j] = i32x8{(int)q.x, (int)q.y, (int)q.z, (int)q.w, 0, 0, 0, 0};
            if (PA == 0)
                sw[j] = *reinterpret_cast<const uint32_t *>(base + P::PAY + (part * BN + wcol + j * 32 + c) * 4);
        }
    };
    // Local K step s = 2 j + PA (A slot U): read step s + 1's payload (and,
    // at the end of a double step, the next double step's scales) from LDS
    // stage NS, then multiply step s.
    auto step = [&](auto par, auto aslot, auto nstage, uint32_t s) {
        constexpr int PA = decltype(par)::value, U = decltype(aslot)::value;
        if (s < nsteps) {
            uint32_t scl[CT];
#pragma unroll
            for (int j = 0; j < CT; j++) scl[j] = sw[j];
            frag_read(nstage, Int<1 - PA>{});
            // A block past K (odd block count, last step): its scale byte may be
            // E8M0 255 (NaN); the activations there are zero, so scale 1 keeps it out.
            const bool dead = part && (nblk & 1) && s == a.ksteps - 1;
#pragma unroll
            for (int j = 0; j < CT; j++) scl[j] = dead ? 0x7f7f7f7fu : scl[j];
#if defined(OCO_ABL) && OCO_ABL == 5
#pragma unroll
            for (int j = 0; j < CT; j++) acc[j][0] += __int_as_float(av[U][0][0] ^ av[U][1][7] ^ bf[PA][j][0] ^ bf[PA][j][3] ^ (int)scl[j] ^ (int)as[U]);
            return;
#endif
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < CT; j++) {
                    if (t == 0)
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[U][0], bf[PA][j], acc[j], 0, 4, 0,
                                                                                  (int)as[U], PA, (int)scl[j]);
                    else
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[U][1], bf[PA][j], acc[j], 0, 4, 1,
                                                                                  (int)as[U], PA, (int)scl[j]);
                }
        }
    };

    // Double step j (ring position Q = j mod PER): stage j % 3 holds B of j
    // (steps 2j, 2j + 1) and stage (j + 1) % 3 B of j + 1 (read for step
    // 2j + 2 before this round's barrier); B of j + 2 goes to stage
    // (j + 2) % 3, last read before the previous barrier.
    auto body = [&](auto q, uint32_t j) {
        constexpr int Q = decltype(q)::value;
        store_b(Int<(Q + 2) % RB>{}, Int<(Q + 2) % 3>{});
        load_b(Int<(Q + 2) % RB>{}, j + 2 + RB);
        step(Int<0>{}, Int<(2 * Q) % RA>{}, Int<Q % 3>{}, 2 * j);
        load_a(Int<(2 * Q) % RA>{}, 2 * j + RA);
        step(Int<1>{}, Int<(2 * Q + 1) % RA>{}, Int<(Q + 1) % 3>{}, 2 * j + 1);
        load_a(Int<(2 * Q + 1) % RA>{}, 2 * j + 1 + RA);
        __syncthreads();
    };

    // Prologue, in the order the first steps need the data.
    load_b(Int<0>{}, 0);
    load_b(Int<1>{}, 1);
    static_for<RA>([&](auto u) { load_a(u, u.value); });
    static_for<RB - 2>([&](auto u) { load_b(Int<u.value + 2>{}, u.value + 2); });
    store_b(Int<0>{}, Int<0>{});
    store_b(Int<1>{}, Int<1>{});
    load_b(Int<0>{}, RB);
    load_b(Int<1>{}, RB + 1);
    __syncthreads();
    frag_read(Int<0>{}, Int<0>{});
    const uint32_t nd = (nsteps + 1) / 2;
    for (uint32_t j = 0; j < nd; j += PER)
        static_for<PER>([&](auto q) { body(q, j + q.value); });

    if (tile >= a.tiles) return;
#pragma unroll
    for (int j = 0; j < CT; j++) {
        const uint32_t col = col0 + wcol + j * 32 + c;
        if (col >= a.n) continue;
        const float bias = a.bias ? round_bf16(a.bias[col]) : 0.f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const uint32_t row = tile * 32 + 8 * (v / 4) + 4 * part + (v % 4);
            if (row >= a.m) continue;
            const float r = acc[j][v] + bias;
            const uint64_t o = (uint64_t)row * a.n + col;
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(r);
            else
                reinterpret_cast<float *>(a.y)[o] = r;
        }
    }
}

// Tile plan of one call: wavefronts along the activation rows (WM) and
// column tiles per wavefront (CTW).
struct MxTilePlan {
    int wm, ctw;
    uint32_t col_tiles, groups;
};
static MxTilePlan mx_plan(uint32_t m, uint32_t n) {
    int wm = 4, ctw = 3;  // 128 x 96: measured fastest at 512 x 5760 x 2880
    int32_t ov[4];
    if (plan_override(OCO_KNOB_MX_TILE, ov) == 2) {
        const int w2 = ov[0], c2 = ov[1];
        if ((w2 == 2 || w2 == 4) && (c2 == 3 || c2 == 6)) {
            wm = w2;
            ctw = c2;
        }
    }
    MxTilePlan p;
    p.wm = wm;
    p.ctw = ctw;
    const uint32_t bn = 32 * ctw * (4 / wm), bm = 32 * wm;
    p.col_tiles = (n + bn - 1) / bn;
    p.groups = (m + bm - 1) / bm;
    return p;
}

uint64_t mx_workspace_bytes(uint32_t m, uint32_t n, uint32_t k) {
    (void)n;
    return (uint64_t)((m + 31) / 32) * ((k + 63) / 64) * MX_REC;
}

template <int WM, int CTW>
static MxFn mx_kernel_fn(size_t &lds) {
    lds = (size_t)MxPlan<WM, CTW, 3>::LDS;
    return mx_matmul_kernel<WM, CTW, 3>;
}

int mx_matmul_launch(const void *w, const void *x, void *y, bool y_bf16, const float *bias, uint32_t m, uint32_t n,
                     uint32_t k, void *workspace, hipStream_t stream) {
    const uint32_t ksteps = (k + 63) / 64, tiles = (m + 31) / 32;
    const MxTilePlan plan = mx_plan(m, n);
    MxSplitArgs sa;
    sa.x = (const uint16_t *)x;
    sa.frag = (uint8_t *)workspace;
    sa.m = m;
    sa.k = k;
    sa.ksteps = ksteps;
    sa.records = tiles * ksteps;
    hipLaunchKernelGGL(mx_split_kernel, dim3(sa.records), dim3(256), 0, stream, KPRE_ARGS(sa), sa);
    OCO_TRY(launch_check("oco_matmul (mx split)"));
    size_t lds = 0;
    MxFn fn = plan.wm == 2 ? (plan.ctw == 3 ? mx_kernel_fn<2, 3>(lds) : mx_kernel_fn<2, 6>(lds))
                           : (plan.ctw == 3 ? mx_kernel_fn<4, 3>(lds) : mx_kernel_fn<4, 6>(lds));
    if (lds > 64 * 1024)
        OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                          "hipFuncSetAttribute"));
    MxArgs a;
    a.w = (const uint8_t *)w;
    a.frag = (const uint8_t *)workspace;
    a.y = y;
    a.bias = bias;
    a.m = m;
    a.n = n;
    a.k = k;
    a.ksteps = ksteps;
    a.tiles = tiles;
    a.row_bytes = (k / 32) * 17;
    a.y_bf16 = y_bf16;
    const uint64_t wspan = ((uint64_t)n * a.row_bytes + ((uintptr_t)w & 3u) + 3) & ~3ull;
    if (wspan > 0xffffff00ull)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: MXFP4 weight of %llu bytes (4 GiB limit)",
                    (unsigned long long)wspan);
    a.wspan = (uint32_t)wspan;
    hipLaunchKernelGGL(fn, dim3(plan.col_tiles, plan.groups), dim3(256), lds, stream, KPRE_ARGS(a), a);
    return launch_check("oco_matmul (mx)");
}

}  // namespace oco
