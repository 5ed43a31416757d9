// MXFP4 prefill on CDNA4's block-scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4).
// Same operation as the MXFP4 case of oco_matmul -- Y = X W^T (+ bias) for
// DenseMatrix::apply's MXFP4 plans (src/weights/compute/matrix.rs:130-379,
// shaders/matrix/batch.metal:24-79) -- without decoding a single weight:
//
//  * W (GGUF MXFP4: per 32 values one E8M0 byte, then 16 bytes of E2M1 nibbles,
//    value j in the low nibble of byte j and value j+16 in the high nibble) is
//    the B operand as stored.  Its E8M0 byte is the B block scale.
//  * X (bf16) is split once per call into two E2M3 (FP6) terms with their own
//    E8M0 scale per 32-block: x = s1 q1 + s2 q2.  s1 is the smallest power
//    of two with max|x| / s1 <= 7.5; the residual x - s1 q1 is exact in fp32
//    and its rounding to E2M3 under s2 leaves at most 1/225 of the block
//    maximum per value (relative L2 ~3.4e-4 on the product for N(0,1)
//    activations, ~4.4e-4 for values spanning 2^+-30 in a block).  FP6 x
//    FP4 issues in 40 clocks against 64 for FP8 x FP4 (measured), and the
//    terms are 24 bytes per 32 values against 32.  The split stores the
//    terms in the MFMA's register order, so every operand load is
//    contiguous.
//
// Operand layout of the 32x32x64 scaled MFMA (measured on gfx950), row
// (column, for B) r = l % 32, block b = 0, 1 of the K=64 step:
//  * B, E2M1: lane r + 32b holds block b as 16 bytes, element e in nibble
//    e & 1 of byte e / 2 -- exactly a GGUF MXFP4 block's payload;
//  * A, E2M3: lane r + 32b holds block b as 24 bytes, element e in bits
//    6e .. 6e + 5; element e of both operands is block column e / 2 for even
//    e and 16 + e / 2 for odd e (the GGUF nibble order);
//  * block b's scale is in lane r + 32b (A and B), byte chosen by op_sel.
// The accumulator holds column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "mxsplit.h"
#include "stream.h"

namespace oco {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// One record per (32-row tile, K step of 64): [term 2][lane 64][16 B] then
// [term 2][lane 64][8 B] of E2M3 codes (lane l's 24-byte fragment is its
// 16-byte part and its 8-byte part), then [lane 64] u32 of E8M0 scales
// (byte t = term t).  Lane l = row l % 32, block l / 32 of the step.
constexpr uint32_t MX_LO = 2 * 64 * 16, MX_DATA = 2 * 64 * 24, MX_REC = MX_DATA + 64 * 4;

typedef mx_f32x32 f32x32;
typedef mx_i32x6 i32x6;

struct MxSplitArgs {
    const uint16_t *x;
    uint8_t *frag;
    uint32_t m, k, ksteps, records;
};

// One wavefront (workgroup) per record, so the records spread over every CU;
// lane l = (row l % 32, block l / 32), each lane
// splitting its whole block in registers: x = s1 q1 + s2 q2 with E2M3 codes
// q and E8M0 scales s (s1 the smallest power of two with max|x| / s1 <= 7.5,
// s2 likewise for the residual x - s1 q1, which is exact in fp32).  The
// codes go in MFMA k order: k = 2i is the block's column i, k = 2i + 1 its
// column 16 + i -- the nibble order of the GGUF MXFP4 payload the B operand
// holds as stored.  The second term leaves at most 1/225 of the block
// maximum per value: a few 1e-4 relative L2 on the product (N(0,1) rows).
__global__ __launch_bounds__(64) void mx_split_kernel(KPRE_PARAMS, MxSplitArgs a) {
    KPRE_APPLY(a);
    const uint32_t rec = blockIdx.x;
    const uint32_t lane = threadIdx.x, tile = rec / a.ksteps, s = rec % a.ksteps;
    const uint32_t row = tile * 32 + (lane & 31), k0 = s * 64 + 32 * (lane >> 5);
    uint32_t w[16];
    if (row < a.m && k0 < a.k) {
        const auto src = gp(reinterpret_cast<const u32x4 *>(a.x + (uint64_t)row * a.k + k0));
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const u32x4 u = src[q];
            w[4 * q] = u.x; w[4 * q + 1] = u.y; w[4 * q + 2] = u.z; w[4 * q + 3] = u.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = 0;
    }
    float v[32];  // column order
#pragma unroll
    for (int i = 0; i < 16; i++) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
    auto out = gp(a.frag + (uint64_t)rec * MX_REC);
    uint32_t scales = 0;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        // |x| bit patterns order like the values, with Inf above every finite
        // value and NaN above Inf: the integer maximum carries both.
        // (a tree, so the 32-value maximum is five dependent steps, not 16)
        uint32_t mt[16];
#pragma unroll
        for (int i = 0; i < 16; i++) mt[i] = max(__float_as_uint(v[i]) & 0x7fffffffu, __float_as_uint(v[16 + i]) & 0x7fffffffu);
#pragma unroll
        for (int w = 8; w > 0; w >>= 1)
#pragma unroll
            for (int i = 0; i < w; i++) mt[i] = max(mt[i], mt[i + w]);
        const int E = mx6_scale_exp(mt[0]);
        scales |= (uint32_t)(E + 127) << (8 * t);
        const float inv = E == 128 ? 0.f : __builtin_ldexpf(1.f, -E), sc = E == 128 ? 0.f : __builtin_ldexpf(1.f, E);
        f32x16 lo, hi;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            lo[i] = v[i] * inv;
            hi[i] = v[16 + i] * inv;
        }
        const i32x6 c = fp6_pack(lo, hi);
        *reinterpret_cast<__attribute__((address_space(1))) u32x4 *>(out + (t * 64 + lane) * 16) =
            u32x4{(uint32_t)c[0], (uint32_t)c[1], (uint32_t)c[2], (uint32_t)c[3]};
        *reinterpret_cast<__attribute__((address_space(1))) u32x2 *>(out + MX_LO + (t * 64 + lane) * 8) = u32x2{(uint32_t)c[4], (uint32_t)c[5]};
        if (t == 0) {
            const f32x32 d = fp6_unpack(c);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                v[i] -= d[2 * i] * sc;
                v[16 + i] -= d[2 * i + 1] * sc;
            }
        }
    }
    *reinterpret_cast<__attribute__((address_space(1))) uint32_t *>(out + MX_DATA + lane * 4) = scales;
}

// The first 56 bytes arrive in SGPRs (KPre).
struct MxArgs {
    const uint8_t *w;
    const uint8_t *frag;
    uint32_t m, n, k, ksteps, tiles;
    uint32_t row_bytes;
    uint32_t wspan;  // weight bytes from the 16-byte aligned base, rounded up to 16 (< 4 GiB)
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

// ---------------------------------------------------------------------------
// Prefill tile: workgroup = four wavefronts, WM along the activation rows
// and 4 / WM along the weight rows (output columns); each wavefront owns one
// 32-row activation tile and CTW 32-column weight tiles, so a K step is
// 2 CTW independent MFMAs (the two activation terms of every column tile).
//
//  * A: each wavefront's split records go straight into a register ring RA
//    K steps deep, through a buffer resource whose step offset is scalar.
//  * B: GGUF rows staged eight K steps (16 blocks, 272 bytes) at a time.
//    272 is a multiple of 16, so a row's stage span starts at the same
//    misalignment every time: it is fetched as the 18 aligned 16-byte
//    chunks that cover it, 18 consecutive lanes per row -- nearly the
//    contiguous pattern L2 serves best (measured from L2: contiguous 1 KB
//    wavefront loads ~55 bytes/clock per CU; four lanes per 68-byte row
//    segment ~19).  The chunks land in a raw LDS buffer as they are; one
//    pass per stage, shared by the workgroup, realigns every 17-byte block
//    into an aligned [block][row] payload array and a [row][block] array
//    of scale bytes.  A step then reads one aligned 16-byte fragment per
//    column tile, and the stage's eight scales per row come in one 8-byte
//    read (op_sel picks the step's byte).  Realigning per wavefront at
//    fragment-read time instead put five dependent LDS reads and four
//    v_alignbyte per fragment on every wavefront's critical path
//    (measured: that loop alone, without loads or MFMAs, took 15 us).
//
//    Per stage o (one barrier): realign raw stage o + 1; write stage
//    o + 2's chunks (in registers since stage o - 1) to the other raw
//    buffer; request stage o + 3's chunks; run the eight steps of stage o.
template <int WM, int CTW>
struct MxPlan {
    static constexpr int WN = 4 / WM, BM = 32 * WM, BN = 32 * CTW * WN;
    static constexpr int OCT = 8;     // K steps per B stage
    static constexpr int CH = 18;     // 16-byte chunks per row and stage
    static constexpr int RSTR = 296;  // raw LDS bytes per row (18 chunks + pad)
    static constexpr int NTH = 512;                          // threads: two wavefronts per (row tile, columns)
    static constexpr int BU = (BN * CH + NTH - 1) / NTH;      // chunk slots per thread
    static constexpr int RU = (BN * 2 * OCT + NTH - 1) / NTH; // realigned blocks per thread
    static constexpr int PROW = BN + 1;                     // payload slots per block row
    static constexpr int RAW = BN * RSTR, PAY = 2 * OCT * PROW * 16, SCL = BN * 2 * OCT;
    static constexpr int ALN = PAY + SCL;
    static constexpr int LDS = 2 * RAW + 2 * ALN;
    static constexpr int RA = 2;  // A ring: this wavefront's next two own steps (four K steps ahead)
    static_assert((OCT / 2) % RA == 0, "ring slots repeat every stage");
    static constexpr int RED = 4 * CTW * 16 * 64 * 4, OROW = BN + 4, OUT = BM * OROW * 4;
    static_assert(RED + OUT <= LDS, "the K-half sums and the output tile fit the stage buffers");
};

template <int WM, int CTW>
__global__ __launch_bounds__(512) void mx_matmul_kernel(KPRE_PARAMS, MxArgs a) {
    KPRE_APPLY(a);
    using P = MxPlan<WM, CTW>;
    constexpr int BN = P::BN, BU = P::BU, RU = P::RU, RA = P::RA, CT = CTW, OCT = P::OCT;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t *const raw = lds, *const aln = lds + 2 * P::RAW;
    // The wavefront index is uniform: readfirstlane keeps the A resource in SGPRs.
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
              part = lane >> 5;
    // Wavefronts w and w + 4 share a row tile and its column tiles: kw = 0
    // takes the even steps of every stage, kw = 1 the odd ones.
    const int kw = wave >> 2, w4 = wave & 3, wm = w4 % WM, wn = w4 / WM;
    // Logical (column tile, row group), column-major per XCD: the row groups
    // of one weight column tile share its GGUF bytes in one L2.
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
    const uint32_t bx = lin / gridDim.y, by = lin % gridDim.y;
    const uint32_t tile = by * WM + wm, col0 = bx * BN;
    const uint32_t nblk = a.k / 32, nsteps = a.ksteps;

    // A: this wavefront's records; steps past the end read as zero.
    const __amdgpu_buffer_rsrc_t ra_rs =
        uniform_rsrc(a.frag + (uint64_t)min(tile, a.tiles - 1) * a.ksteps * MX_REC, a.ksteps * MX_REC);
    // B: the tensor from its 16-byte aligned base; bytes past the end read as zero.
    const uint32_t wsh = (uint32_t)((uintptr_t)a.w & 15u);
    const __amdgpu_buffer_rsrc_t rb_rs = uniform_rsrc(a.w - wsh, a.wspan);
    const uint32_t rbytes = (uint32_t)a.row_bytes;
    // Chunk slot q = tid + 512 u: chunk q % 18 of tile row q / 18 (rows past
    // n repeat row n - 1 and are never stored).
    uint32_t boff[BU], bdst[BU];
#pragma unroll
    for (int u = 0; u < BU; u++) {
        const uint32_t q = tid + P::NTH * u, row = min(q / P::CH, (uint32_t)BN - 1), ch = q % P::CH;
        const bool live = q < (uint32_t)(BN * P::CH);
        boff[u] = live ? ((wsh + min(col0 + row, a.n - 1) * rbytes) & ~15u) + 16 * ch : 0u;
        bdst[u] = live ? row * P::RSTR + 16 * ch : ~0u;  // ~0: no slot (the last round's spare threads)
    }
    // Realign slot r = tid + 512 u: block r / BN of tile row r % BN; its
    // scale byte sits at rsrc in the raw buffer, its payload right after.
    uint32_t rsrc[RU], rpay[RU], rscl[RU];
#pragma unroll
    for (int u = 0; u < RU; u++) {
        const uint32_t r = tid + P::NTH * u, row = r % BN, blk = r / BN;
        const bool live = r < (uint32_t)(BN * 2 * OCT);
        rsrc[u] = row * P::RSTR + ((wsh + min(col0 + row, a.n - 1) * rbytes) & 15u) + 17 * blk;
        rpay[u] = live ? (blk * P::PROW + row) * 16 : ~0u;
        rscl[u] = P::PAY + row * 2 * OCT + (blk & 1) * OCT + (blk >> 1);
    }
    const uint32_t wcol = wn * CT * 32;  // this wavefront's first column within the tile

    i32x8 av[RA][2];
    uint32_t as[RA];
    u32x4 bv[BU];
    auto load_a = [&](auto slot, uint32_t s) {
        constexpr int U = decltype(slot)::value;
        const uint32_t so = s * MX_REC;
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(ra_rs, (t * 64 + lane) * 16, so, 0);
            const u32x2 hi = __builtin_amdgcn_raw_buffer_load_b64(ra_rs, MX_LO + (t * 64 + lane) * 8, so, 0);
            av[U][t] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, 0, 0};
        }
        as[U] = __builtin_amdgcn_raw_buffer_load_b32(ra_rs, MX_DATA + lane * 4, so, 0);
    };
    // B chunks of stage o (steps 8 o .. 8 o + 7).
    const uint32_t nst = (nsteps + OCT - 1) / OCT;
    auto load_b = [&](uint32_t o) {
#pragma unroll
        for (int u = 0; u < BU; u++) bv[u] = __builtin_amdgcn_raw_buffer_load_b128(rb_rs, boff[u], o * 272, 0);
    };
    auto store_b = [&](auto buf) {
        constexpr int S = decltype(buf)::value;
#pragma unroll
        for (int u = 0; u < BU; u++) {
            if ((BN * P::CH) % P::NTH == 0 || u + 1 < BU || bdst[u] != ~0u) {
                *reinterpret_cast<u32x2 *>(raw + S * P::RAW + bdst[u]) = u32x2{bv[u].x, bv[u].y};
                *reinterpret_cast<u32x2 *>(raw + S * P::RAW + bdst[u] + 8) = u32x2{bv[u].z, bv[u].w};
            }
        }
    };
    // Raw buffer S to aligned buffer S.
    auto realign = [&](auto buf) {
        constexpr int S = decltype(buf)::value;
#pragma unroll
        for (int u = 0; u < RU; u++) {
            if ((BN * 2 * OCT) % P::NTH == 0 || u + 1 < RU || rpay[u] != ~0u) {
                const uint32_t o = S * P::RAW + rsrc[u], p = o + 1, sh = p & 3u;
                const uint32_t *w = reinterpret_cast<const uint32_t *>(raw + (p & ~3u));
                const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
                *reinterpret_cast<u32x4 *>(aln + S * P::ALN + rpay[u]) =
                    u32x4{__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
                          __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(w4, w3, sh)};
                aln[S * P::ALN + rscl[u]] = raw[o];
            }
        }
    };

    // One accumulator per column tile; a step issues term 0 over all tiles,
    // then term 1, so consecutive MFMAs never share an accumulator.
    f32x16 acc[CT];
#pragma unroll
    for (int j = 0; j < CT; j++) acc[j] = f32x16{};

    // The stage's scale bytes of this lane's rows: 8 steps, byte L of word L / 4.
    u32x2 sw[CT];
    // Fragments of step L of aligned buffer S, read one own step (two steps)
    // ahead of their MFMAs, into set (L / 2) & 1.
    i32x8 bf[2][CT];
    auto frag = [&](auto buf, auto local) {
        constexpr int S = decltype(buf)::value, L = decltype(local)::value;
#pragma unroll
        for (int t = 0; t < CT; t++) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(aln + S * P::ALN +
                                                             ((2 * L + part) * P::PROW + wcol + t * 32 + c) * 16);
            bf[(L / 2) & 1][t] = i32x8{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
        }
    };
    // Step s = 8 o + L of stage o (aligned buffer S), A ring slot (L / 2) % RA.
    auto step = [&](auto buf, auto local, uint32_t s) {
        constexpr int S = decltype(buf)::value, L = decltype(local)::value;
        if constexpr (L + 2 < OCT) frag(buf, Int<L + 2>{});
        if (s < nsteps) {
            // A block past K (odd block count, last step): its weight scale
            // byte may be E8M0 255 (NaN); the activations there are zero, so
            // scale 1 keeps it out.
            const bool dead = part && (nblk & 1) && s == nsteps - 1;
            uint32_t scl[CT];
#pragma unroll
            for (int t = 0; t < CT; t++) scl[t] = dead ? 0x7f7f7f7fu : (L < 4 ? sw[t].x : sw[t].y);
            constexpr int U = (L / 2) % RA, B = L & 3, F = (L / 2) & 1;
#pragma unroll
            for (int t = 0; t < CT; t++)
                acc[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[U][0], bf[F][t], acc[t], 2, 4, 0,
                                                                          (int)as[U], B, (int)scl[t]);
#pragma unroll
            for (int t = 0; t < CT; t++)
                acc[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[U][1], bf[F][t], acc[t], 2, 4, 1,
                                                                          (int)as[U], B, (int)scl[t]);
        }
        (void)S;
    };
    // Stage o: realign raw stage o + 1; write stage o + 2's chunks to the
    // other raw buffer; request stage o + 3's; then this wavefront's four
    // steps of stage o (parity kw), each followed by the A request of the
    // same step one stage ahead.
    auto body = [&](auto par, uint32_t o) {
        constexpr int S = decltype(par)::value;
        realign(Int<1 - S>{});
        if (o + 2 < nst) store_b(Int<S>{});
        // (no requests past the last stage: they would be HBM reads that
        // the kernel's tail waits behind)
        if (o + 3 < nst) load_b(o + 3);
#pragma unroll
        for (int t = 0; t < CT; t++)
            sw[t] = *reinterpret_cast<const u32x2 *>(aln + S * P::ALN + P::PAY + (wcol + t * 32 + c) * 2 * OCT + part * OCT);
        if (kw == 0) {
            frag(Int<S>{}, Int<0>{});
            static_for<OCT / 2>([&](auto i) {
                step(Int<S>{}, Int<2 * i.value>{}, o * OCT + 2 * i.value);
                load_a(Int<i.value % RA>{}, o * OCT + 2 * (i.value + RA));
            });
        } else {
            frag(Int<S>{}, Int<1>{});
            static_for<OCT / 2>([&](auto i) {
                step(Int<S>{}, Int<2 * i.value + 1>{}, o * OCT + 2 * i.value + 1);
                load_a(Int<i.value % RA>{}, o * OCT + 2 * (i.value + RA) + 1);
            });
        }
        __syncthreads();
    };

    // Prologue: stage 0 realigned, stage 1 raw in LDS, stage 2 in registers.
    load_b(0);
    static_for<RA>([&](auto u) { load_a(u, 2 * u.value + kw); });
    store_b(Int<0>{});
    if (nst > 1) load_b(1);
    __syncthreads();
    realign(Int<0>{});
    if (nst > 1) store_b(Int<1>{});
    if (nst > 2) load_b(2);
    __syncthreads();
    for (uint32_t o = 0; o < nst; o += 2) {
        body(Int<0>{}, o);
        if (o + 1 < nst) body(Int<1>{}, o + 1);
    }

    // The odd-step wavefronts hand their sums to the even-step ones, which
    // put the tile in LDS (f32, [row][column]; the stage buffers are free
    // after the loop's last barrier); then all threads store it as rows of
    // 4-column chunks -- contiguous 8- or 16-byte stores instead of one
    // 2-byte store per accumulator.
    float *red = reinterpret_cast<float *>(lds);
    float *ot = reinterpret_cast<float *>(lds + P::RED);
    constexpr int OROW = P::OROW;  // floats per LDS row (pad: rows 4 banks apart)
    if (kw == 1) {
#pragma unroll
        for (int j = 0; j < CT; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) red[((w4 * CT + j) * 16 + v) * 64 + lane] = acc[j][v];
    }
    __syncthreads();
    if (kw == 0) {
#pragma unroll
        for (int j = 0; j < CT; j++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                ot[(wm * 32 + 8 * (v / 4) + 4 * part + (v % 4)) * OROW + wcol + j * 32 + c] =
                    acc[j][v] + red[((w4 * CT + j) * 16 + v) * 64 + lane];
    }
    __syncthreads();
    const uint32_t rows = min((uint32_t)P::BM, a.m - min(a.m, by * P::BM));
    if (a.y_bf16 && col0 + BN <= a.n && (a.n & 7) == 0 && ((uintptr_t)a.y & 15) == 0) {
        // bf16 rows of whole 8-column chunks: one 16-byte store each
        constexpr int CPR8 = BN / 8;
        for (uint32_t q = tid; q < rows * CPR8; q += P::NTH) {
            const uint32_t r = q / CPR8, cc = (q % CPR8) * 8, col = col0 + cc;
            const float4 f0 = *reinterpret_cast<const float4 *>(ot + r * OROW + cc);
            const float4 f1 = *reinterpret_cast<const float4 *>(ot + r * OROW + cc + 4);
            float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
            if (a.bias) {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] += round_bf16(gp(a.bias)[col + e]);
            }
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[e] = (uint32_t)f32_to_bf16_bits(v[2 * e]) | ((uint32_t)f32_to_bf16_bits(v[2 * e + 1]) << 16);
            const uint64_t o = (uint64_t)(by * P::BM + r) * a.n + col;
            *reinterpret_cast<__attribute__((address_space(1))) u32x4 *>(gp(reinterpret_cast<uint16_t *>(a.y) + o)) =
                u32x4{w[0], w[1], w[2], w[3]};
        }
        return;
    }
    constexpr int CPR = BN / 4;  // chunks per row
    for (uint32_t q = tid; q < rows * CPR; q += P::NTH) {
        const uint32_t r = q / CPR, cc = (q % CPR) * 4, col = col0 + cc;
        if (col >= a.n) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = ot[r * OROW + cc + e];
        if (a.bias) {
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] += col + e < a.n ? round_bf16(gp(a.bias)[col + e]) : 0.f;
        }
        const uint64_t o = (uint64_t)(by * P::BM + r) * a.n + col;
        const bool whole = col + 4 <= a.n;
        if (a.y_bf16) {
            auto y = gp(reinterpret_cast<uint16_t *>(a.y) + o);
            if (whole && (o & 3) == 0) {
                *reinterpret_cast<__attribute__((address_space(1))) u32x2 *>(y) =
                    u32x2{(uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16),
                          (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16)};
            } else {
                for (uint32_t e = 0; e < 4 && col + e < a.n; e++) y[e] = f32_to_bf16_bits(v[e]);
            }
        } else {
            auto y = gp(reinterpret_cast<float *>(a.y) + o);
            if (whole && (o & 3) == 0) {
                *reinterpret_cast<__attribute__((address_space(1))) u32x4 *>(y) =
                    u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
            } else {
                for (uint32_t e = 0; e < 4 && col + e < a.n; e++) y[e] = v[e];
            }
        }
    }
}

// Tile plan of one call: wavefronts along the activation rows (WM) and
// column tiles per wavefront (CTW); 128 x 96 is the one that fits LDS with
// both buffer pairs (192 columns would need 219 KB).
struct MxTilePlan {
    int wm, ctw;
    uint32_t col_tiles, groups;
};
static MxTilePlan mx_plan(uint32_t m, uint32_t n) {
    const int wm = 4, ctw = 3;  // 128 x 96: 240 workgroups at 512 x 5760
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
    lds = (size_t)MxPlan<WM, CTW>::LDS;
    return mx_matmul_kernel<WM, CTW>;
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
    hipLaunchKernelGGL(mx_split_kernel, dim3(sa.records), dim3(64), 0, stream, KPRE_ARGS(sa), sa);
    OCO_TRY(launch_check("oco_matmul (mx split)"));
    size_t lds = 0;
    MxFn fn = mx_kernel_fn<4, 3>(lds);
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
    // Bytes from the 16-byte aligned base through the last row, rounded up
    // to a whole chunk (stage spans past the end read as zero).
    const uint64_t wspan = ((uint64_t)n * a.row_bytes + ((uintptr_t)w & 15u) + 15) & ~15ull;
    if (wspan > 0xffffff00ull)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: MXFP4 weight of %llu bytes (4 GiB limit)",
                    (unsigned long long)wspan);
    a.wspan = (uint32_t)wspan;
    hipLaunchKernelGGL(fn, dim3(plan.col_tiles, plan.groups), dim3(MxPlan<4, 3>::NTH), lds, stream, KPRE_ARGS(a), a);
    return launch_check("oco_matmul (mx)");
}

}  // namespace oco
