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
#include "norm.h"
#include "stream.h"

namespace oco {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Split activations, lane l = (row l % 32, block l / 32) of a 32-row tile
// and K step of 64:
//  * codes: one record per (tile, step), [chunk 3][lane 64][16 B]: lane l's
//    48 bytes are term 0's 24 bytes of E2M3 codes, then term 1's, so three
//    aligned 16-byte loads give both MFMA operands in six consecutive
//    dwords each;
//  * scales: one record per (tile, stage of 8 steps), [lane 64][16 B]:
//    byte 2 L + t is step L's term-t E8M0 scale (dword L / 2, selected by
//    the MFMA's op_sel).
// Steps are counted to whole stages; the split writes the padding steps as
// zero codes under scale byte 0 (2^-127), which add nothing.
constexpr uint32_t MX_STAGE = 8, MX_REC = 3 * 64 * 16, MX_SREC = 64 * 16;

typedef mx_f32x32 f32x32;
typedef mx_i32x6 i32x6;

struct MxSplitArgs {
    const uint16_t *x;
    uint8_t *frag, *scl;
    uint32_t m, k, kpad, records;
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
// One block's split: v holds its 32 values in column order (consumed);
// lane `lane`'s three chunks of record `out` receive the codes, and the
// return value the two E8M0 scale bytes (term 0 low).
__device__ __forceinline__ uint32_t mx_split_block(float *v, __attribute__((address_space(1))) uint8_t *out,
                                                   uint32_t lane) {
    uint32_t scales = 0;
    i32x6 c0;
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
        auto chunk = [&](int q, u32x4 v) {
            *reinterpret_cast<__attribute__((address_space(1))) u32x4 *>(out + (q * 64 + lane) * 16) = v;
        };
        if (t == 0) {
            chunk(0, u32x4{(uint32_t)c[0], (uint32_t)c[1], (uint32_t)c[2], (uint32_t)c[3]});
            c0 = c;
        } else {
            chunk(1, u32x4{(uint32_t)c0[4], (uint32_t)c0[5], (uint32_t)c[0], (uint32_t)c[1]});
            chunk(2, u32x4{(uint32_t)c[2], (uint32_t)c[3], (uint32_t)c[4], (uint32_t)c[5]});
        }
        if (t == 0) {
            const f32x32 d = fp6_unpack(c);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                v[i] -= d[2 * i] * sc;
                v[16 + i] -= d[2 * i + 1] * sc;
            }
        }
    }
    return scales;
}

// Record and scale-word addresses of (32-row tile, K step, lane).
__device__ __forceinline__ __attribute__((address_space(1))) uint8_t *mx_rec(uint8_t *frag, uint32_t tile, uint32_t s,
                                                                             uint32_t kpad) {
    return gp(frag + ((uint64_t)tile * kpad + s) * MX_REC);
}
__device__ __forceinline__ __attribute__((address_space(1))) uint16_t *mx_scale_slot(uint8_t *scl, uint32_t tile,
                                                                                      uint32_t s, uint32_t kpad,
                                                                                      uint32_t lane) {
    return reinterpret_cast<__attribute__((address_space(1))) uint16_t *>(
        gp(scl + ((uint64_t)tile * (kpad / MX_STAGE) + s / MX_STAGE) * MX_SREC + lane * 16 + 2 * (s % MX_STAGE)));
}

__global__ __launch_bounds__(64) void mx_split_kernel(KPRE_PARAMS, MxSplitArgs a) {
    KPRE_APPLY(a);
    const uint32_t rec = blockIdx.x;
    const uint32_t lane = threadIdx.x, tile = rec / a.kpad, s = rec % a.kpad;
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
    *mx_scale_slot(a.scl, tile, s, a.kpad, lane) = (uint16_t)mx_split_block(v, mx_rec(a.frag, tile, s, a.kpad), lane);
}

// The RMS norm (elementwise.metal:6-28, oco_norm's rounding) with the split
// of its output rows: one 256-thread workgroup per row of the 32-row tiles
// (rows past m write zero records); each thread splits whole blocks of the
// normalised bf16 row, so the records are bit for bit the split of
// oco_norm's output.  `y`, when set, receives that bf16 row too.
struct MxNormSplitArgs {
    uint16_t *x;
    const uint16_t *res;  // add form: the rows added into x first
    const float *w;
    uint16_t *y;
    uint8_t *frag, *scl;
    uint32_t m, k, kpad, full_layer;
    float epsilon;
};

template <bool ADD>
__global__ __launch_bounds__(256) void mx_norm_split_kernel(MxNormSplitArgs a) {
    __shared__ float partial[4];
    extern __shared__ __attribute__((aligned(16))) uint16_t nrow[];  // the normalised row, bf16 [k]
    const uint32_t row = blockIdx.x, tile = row / 32, r = row % 32;
    const bool live = row < a.m;  // uniform
    uint16_t *xr = a.x + (uint64_t)row * a.k;
    if (live) {
        if constexpr (ADD) {  // the residual stream takes bf16(x + y) first, as oco_add_norm
            const uint16_t *yr = a.res + (uint64_t)row * a.k;
            for (uint32_t i = threadIdx.x; i < a.k; i += 256)
                xr[i] = f32_to_bf16_bits(bf16_bits_to_f32(xr[i]) + bf16_bits_to_f32(yr[i]));
            __syncthreads();
        }
        const float inv = block_inv_rms(xr, a.k, a.epsilon, partial);
        // eight consecutive values per thread, coalesced, into LDS (and y)
        uint16_t *yr = a.y ? a.y + (uint64_t)row * a.k : nullptr;
        const bool vec = (((uintptr_t)xr | (uintptr_t)a.w | (uintptr_t)yr) & 15u) == 0;
        for (uint32_t c = threadIdx.x; 8 * c < a.k; c += 256) {
            float xv[8], wv[8];
            if (vec) {
                const uint4 u = *reinterpret_cast<const uint4 *>(xr + 8 * c);
                const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    xv[2 * j] = __uint_as_float(h[j] << 16);
                    xv[2 * j + 1] = __uint_as_float(h[j] & 0xffff0000u);
                }
                const float4 w0 = *reinterpret_cast<const float4 *>(a.w + 8 * c);
                const float4 w1 = *reinterpret_cast<const float4 *>(a.w + 8 * c + 4);
                wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
                wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    xv[j] = bf16_bits_to_f32(xr[8 * c + j]);
                    wv[j] = a.w[8 * c + j];
                }
            }
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                o[j] = (uint32_t)norm_value_bits(xv[2 * j], inv, wv[2 * j], a.full_layer) |
                       ((uint32_t)norm_value_bits(xv[2 * j + 1], inv, wv[2 * j + 1], a.full_layer) << 16);
            *reinterpret_cast<uint4 *>(nrow + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
            if (yr) {
                if (vec) {
                    *reinterpret_cast<uint4 *>(yr + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        yr[8 * c + 2 * j] = (uint16_t)o[j];
                        yr[8 * c + 2 * j + 1] = (uint16_t)(o[j] >> 16);
                    }
                }
            }
        }
        __syncthreads();
    }
    // one whole block per thread (padding steps and rows past m: zeros)
    for (uint32_t b = threadIdx.x; b < 2 * a.kpad; b += 256) {
        const uint32_t s = b / 2, lane = r + 32 * (b & 1), k0 = 32 * b;
        float v[32];  // column order
        if (live && k0 < a.k) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint4 u = *reinterpret_cast<const uint4 *>(nrow + k0 + 8 * q);
                const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    v[8 * q + 2 * j] = __uint_as_float(h[j] << 16);
                    v[8 * q + 2 * j + 1] = __uint_as_float(h[j] & 0xffff0000u);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = 0.f;
        }
        *mx_scale_slot(a.scl, tile, s, a.kpad, lane) = (uint16_t)mx_split_block(v, mx_rec(a.frag, tile, s, a.kpad), lane);
    }
}

// The first 56 bytes arrive in SGPRs (KPre).
struct MxArgs {
    const uint8_t *w;
    const uint8_t *frag;
    uint32_t m, n, k, ksteps, tiles;
    uint32_t kpad;
    const uint8_t *scl;
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
// Prefill tile: 32 RT activation rows x 32 CT weight rows (output columns)
// per workgroup of eight wavefronts in two roles, one of each per SIMD:
//
//  * Wavefronts 0 .. RT - 1 (one per 32-row activation tile) only issue
//    MFMAs.  A K step is 2 CT independent MFMAs (the two activation terms of
//    every column tile).  Their split records go straight into a register
//    ring RA K steps deep, through a buffer resource whose step offset is
//    scalar; their B fragments come from LDS, one aligned 16-byte read per
//    column tile, read one step ahead.
//  * Wavefronts RT .. 7 only stage the weights.  GGUF rows are staged eight
//    K steps (16 blocks, 272 bytes) at a time.  272 is a multiple of 16, so
//    a row's stage span starts at the same misalignment every time: it is
//    fetched as the 18 aligned 16-byte chunks that cover it, 18 consecutive
//    lanes per row (nearly the contiguous pattern L2 serves best), and
//    written to a raw LDS buffer as it comes.  One pass per stage realigns
//    every 17-byte block into an aligned [block][row] payload array and a
//    [row][block] array of scale bytes (unaligned 16-byte LDS reads are
//    correct on gfx950 but run at an eighth of the aligned rate; five dword
//    reads and four v_alignbyte per block cost the staging wavefronts, not
//    the MFMA issue).
//
// Per stage o (one barrier): the staging wavefronts realign raw stage
// o + 1, write stage o + 2's chunks (in their registers since stage o - 1)
// to the other raw buffer and request stage o + 3's; meanwhile the MFMA
// wavefronts run the eight steps of stage o from the aligned buffer written
// during stage o - 1.
template <int CT>
struct MxPlan {
    static constexpr int RT = 4, BM = 32 * RT, BN = 32 * CT;
    static constexpr int OCT = 8;     // K steps per B stage
    static constexpr int CH = 18;     // 16-byte chunks per row and stage
    static constexpr int RSTR = 296;  // raw LDS bytes per row (18 chunks + pad)
    static constexpr int NTH = 512, NL = NTH - 64 * RT;     // threads; staging threads
    static constexpr int BU = (BN * CH + NL - 1) / NL;       // chunk slots per staging thread
    static constexpr int RU = (BN * 2 * OCT + NL - 1) / NL;  // realigned blocks per staging thread
    static constexpr int PROW = BN + 1;                      // payload slots per block row
    static constexpr int RAW = BN * RSTR, PAY = 2 * OCT * PROW * 16, SCL = BN * 2 * OCT;
    static constexpr int ALN = PAY + SCL;
    static constexpr int LDS = 2 * RAW + 2 * ALN;
    static constexpr int RA = OCT;  // A ring: one stage of K steps ahead
    static_assert(OCT == (int)MX_STAGE, "A scale records cover one B stage");
    static constexpr int OROW = BN + 4, OUT = BM * OROW * 4;
    static_assert(OUT <= LDS, "the output tile fits the stage buffers");
};

template <int CT>
__global__ __launch_bounds__(512) void mx_matmul_kernel(KPRE_PARAMS, MxArgs a) {
    KPRE_APPLY(a);
    using P = MxPlan<CT>;
    constexpr int BN = P::BN, BU = P::BU, RU = P::RU, RA = P::RA, OCT = P::OCT, RT = P::RT;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t *const raw = lds, *const aln = lds + 2 * P::RAW;
    // The wavefront index is uniform: readfirstlane keeps the role and the
    // A resource in SGPRs.
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
              part = lane >> 5;
    const bool mfma_wave = wave < RT;
    // Logical (column tile, row group), column-major per XCD: the row groups
    // of one weight column tile share its GGUF bytes in one L2.
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
    const uint32_t bx = lin / gridDim.y, by = lin % gridDim.y;
    const uint32_t col0 = bx * BN;
    const uint32_t nblk = a.k / 32, nsteps = a.ksteps;
    const uint32_t nst = (nsteps + OCT - 1) / OCT;

    // ---- staging wavefronts: B chunk slots and realignment slots ----
    // B: the tensor from its 16-byte aligned base; bytes past the end read as zero.
    const uint32_t wsh = (uint32_t)((uintptr_t)a.w & 15u);
    const __amdgpu_buffer_rsrc_t rb_rs = uniform_rsrc(a.w - wsh, a.wspan);
    const uint32_t rbytes = (uint32_t)a.row_bytes, st = (uint32_t)(tid - 64 * RT);
    // Chunk slot q = st + NL u: chunk q % 18 of tile row q / 18 (rows past
    // n repeat row n - 1 and are never stored).
    uint32_t boff[BU], bdst[BU];
    // Realign slot r = st + NL u: block r / BN of tile row r % BN; its scale
    // byte sits at rsrc in the raw buffer, its payload right after.
    uint32_t rsrc[RU], rpay[RU], rscl[RU];
    u32x4 bv[BU];
    if (!mfma_wave) {
#pragma unroll
        for (int u = 0; u < BU; u++) {
            const uint32_t q = st + P::NL * u, row = min(q / P::CH, (uint32_t)BN - 1), ch = q % P::CH;
            const bool live = q < (uint32_t)(BN * P::CH);
            boff[u] = live ? ((wsh + min(col0 + row, a.n - 1) * rbytes) & ~15u) + 16 * ch : 0u;
            bdst[u] = live ? row * P::RSTR + 16 * ch : ~0u;  // ~0: no slot (the last round's spare threads)
        }
#pragma unroll
        for (int u = 0; u < RU; u++) {
            const uint32_t r = st + P::NL * u, row = r % BN, blk = r / BN;
            const bool live = r < (uint32_t)(BN * 2 * OCT);
            rsrc[u] = row * P::RSTR + ((wsh + min(col0 + row, a.n - 1) * rbytes) & 15u) + 17 * blk;
            rpay[u] = live ? (blk * P::PROW + row) * 16 : ~0u;
            rscl[u] = P::PAY + row * 2 * OCT + (blk & 1) * OCT + (blk >> 1);
        }
    }
    // B chunks of stage o (steps 8 o .. 8 o + 7).
    auto load_b = [&](uint32_t o) {
#pragma unroll
        for (int u = 0; u < BU; u++) bv[u] = __builtin_amdgcn_raw_buffer_load_b128(rb_rs, boff[u], o * 272, 0);
    };
    auto store_b = [&](auto buf) {
        constexpr int S = decltype(buf)::value;
#pragma unroll
        for (int u = 0; u < BU; u++) {
            if ((BN * P::CH) % P::NL == 0 || u + 1 < BU || bdst[u] != ~0u) {
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
            if ((BN * 2 * OCT) % P::NL == 0 || u + 1 < RU || rpay[u] != ~0u) {
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

    // ---- MFMA wavefronts ----
    const uint32_t tile = by * RT + (mfma_wave ? wave : 0);
    // A: this wavefront's records; steps past the end read as zero.
    const uint32_t atile = min(tile, a.tiles - 1);
    const __amdgpu_buffer_rsrc_t ra_rs = uniform_rsrc(a.frag + (uint64_t)atile * a.kpad * MX_REC, a.kpad * MX_REC);
    const __amdgpu_buffer_rsrc_t rs_rs =
        uniform_rsrc(a.scl + (uint64_t)atile * (a.kpad / OCT) * MX_SREC, (a.kpad / OCT) * MX_SREC);
    u32x4 av[RA][3];
    auto load_a = [&](auto slot, uint32_t s) {
        constexpr int U = decltype(slot)::value;
#pragma unroll
        for (int q = 0; q < 3; q++) av[U][q] = __builtin_amdgcn_raw_buffer_load_b128(ra_rs, (q * 64 + lane) * 16, s * MX_REC, 0);
    };
    // The A scales of a stage, one word per pair of steps.
    u32x4 asv[2];
    auto load_as = [&](auto buf, uint32_t o) {
        constexpr int S = decltype(buf)::value;
        asv[S] = __builtin_amdgcn_raw_buffer_load_b128(rs_rs, lane * 16, o * MX_SREC, 0);
    };
    // One accumulator per column tile; a step issues term 0 over all tiles,
    // then term 1, so consecutive MFMAs never share an accumulator.
    f32x16 acc[CT];
#pragma unroll
    for (int j = 0; j < CT; j++) acc[j] = f32x16{};
    // The stage's scale bytes of this lane's rows: 8 steps, byte L of word L / 4.
    u32x2 sw[CT];
    // Fragments of step L of aligned buffer S, read one step ahead of their
    // MFMAs, into set L & 1.
    i32x8 bf[2][CT];
    auto frag = [&](auto buf, auto local) {
        constexpr int S = decltype(buf)::value, L = decltype(local)::value;
#pragma unroll
        for (int t = 0; t < CT; t++) {
            const u32x4 v =
                *reinterpret_cast<const u32x4 *>(aln + S * P::ALN + ((2 * L + part) * P::PROW + t * 32 + c) * 16);
            bf[L & 1][t] = i32x8{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
        }
    };
    // Step s = 8 o + L of stage o (aligned buffer S), A ring slot L.  The
    // step runs whether or not s < nsteps: branches around the loads or the
    // MFMAs would make the compiler wait for every outstanding load at each
    // step.  Past the last step the A records read as zero (codes 0, scale
    // byte 0) and the weight scales are forced to 1, so the stage span's
    // bytes of the next row (which may hold the NaN scale byte) add zero.
    auto step = [&](auto buf, auto local, uint32_t s) {
        constexpr int S = decltype(buf)::value, L = decltype(local)::value;
        if constexpr (L + 1 < OCT) frag(buf, Int<L + 1>{});
        // A block past K (odd block count, last step): its weight scale byte
        // may be E8M0 255 (NaN); the activations there are zero, so scale 1
        // keeps it out.
        const bool dead = (s >= nsteps) | ((part != 0) & ((nblk & 1) != 0) & (s + 1 == nsteps));
        uint32_t scl[CT];
#pragma unroll
        for (int t = 0; t < CT; t++) scl[t] = dead ? 0x7f7f7f7fu : (L < 4 ? sw[t].x : sw[t].y);
        constexpr int B = L & 3, F = L & 1, AW = L / 2, AB = 2 * (L & 1);
        const uint32_t asw = asv[S][AW];
        const u32x4 c0 = av[L][0], c1 = av[L][1], c2 = av[L][2];
        const i32x8 a0 = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, 0, 0};
        const i32x8 a1 = {(int)c1.z, (int)c1.w, (int)c2.x, (int)c2.y, (int)c2.z, (int)c2.w, 0, 0};
#pragma unroll
        for (int t = 0; t < CT; t++)
            acc[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a0, bf[F][t], acc[t], 2, 4, AB, (int)asw, B,
                                                                      (int)scl[t]);
#pragma unroll
        for (int t = 0; t < CT; t++)
            acc[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a1, bf[F][t], acc[t], 2, 4, AB + 1, (int)asw, B,
                                                                      (int)scl[t]);
    };
    // The two roles run separate loops with the same barriers, so that
    // neither role's registers are live in the other's.
    if (mfma_wave) {
        // The A ring fills in two halves: at the start every workgroup's
        // requests meet in HBM and L2 at once, and the first B stage (needed
        // before any MFMA) should not queue behind A steps that are needed
        // later.
        load_as(Int<0>{}, 0);
        static_for<RA / 2>([&](auto u) { load_a(u, u.value); });
        __syncthreads();
        static_for<RA / 2>([&](auto u) { load_a(Int<RA / 2 + u.value>{}, RA / 2 + u.value); });
        __syncthreads();
        auto body = [&](auto par, uint32_t o) {
            constexpr int S = decltype(par)::value;
#pragma unroll
            for (int t = 0; t < CT; t++)
                sw[t] = *reinterpret_cast<const u32x2 *>(aln + S * P::ALN + P::PAY + (t * 32 + c) * 2 * OCT + part * OCT);
            frag(Int<S>{}, Int<0>{});
            load_as(Int<1 - S>{}, o + 1);  // past the records: zeros, no memory access
            static_for<OCT>([&](auto i) {
                step(Int<S>{}, i, o * OCT + i.value);
                load_a(i, o * OCT + i.value + RA);  // past the records: zeros, no memory access
                // Keep each step's fragment reads and loads in place: hoisted
                // reads of later steps only occupy registers.
                __builtin_amdgcn_sched_barrier(0);
            });
            __syncthreads();
        };
        // Stages run in pairs (static buffer indices); an odd count gets one
        // stage of dead steps.
        for (uint32_t o = 0; o < nst; o += 2) {
            body(Int<0>{}, o);
            body(Int<1>{}, o + 1);
        }
    } else {
        // Prologue: stage 0 realigned, stage 1 raw in LDS, stage 2 in registers.
        load_b(0);
        store_b(Int<0>{});
        if (nst > 1) load_b(1);
        __syncthreads();
        realign(Int<0>{});
        if (nst > 1) store_b(Int<1>{});
        if (nst > 2) load_b(2);
        __syncthreads();
        auto body = [&](auto par, uint32_t o) {
            constexpr int S = decltype(par)::value;
            if (o + 1 < nst) realign(Int<1 - S>{});
            if (o + 2 < nst) store_b(Int<S>{});
            // (no requests past the last stage: they would be HBM reads that
            // the kernel's tail waits behind)
            if (o + 3 < nst) load_b(o + 3);
            __syncthreads();
        };
        for (uint32_t o = 0; o < nst; o += 2) {
            body(Int<0>{}, o);
            body(Int<1>{}, o + 1);
        }
    }

    // The MFMA wavefronts put the tile in LDS (f32, [row][column]; the stage
    // buffers are free after the loop's last barrier); then all threads
    // store it as rows of 8- or 4-column chunks -- contiguous 16- or 8-byte
    // stores instead of one 2-byte store per accumulator.
    float *ot = reinterpret_cast<float *>(lds);
    constexpr int OROW = P::OROW;  // floats per LDS row (pad: rows 4 banks apart)
    if (mfma_wave) {
#pragma unroll
        for (int j = 0; j < CT; j++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                ot[(wave * 32 + 8 * (v / 4) + 4 * part + (v % 4)) * OROW + j * 32 + c] = acc[j][v];
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

// Tile plan of one call: 128 x 96 (three column tiles per MFMA wavefront)
// is the one that fits LDS with both buffer pairs (192 columns would need
// 219 KB).
struct MxTilePlan {
    uint32_t col_tiles, groups;
};
static MxTilePlan mx_plan(uint32_t m, uint32_t n) {
    MxTilePlan p;  // 128 x 96: 240 workgroups at 512 x 5760
    const uint32_t bn = MxPlan<3>::BN, bm = MxPlan<3>::BM;
    p.col_tiles = (n + bn - 1) / bn;
    p.groups = (m + bm - 1) / bm;
    return p;
}

uint64_t mx_workspace_bytes(uint32_t m, uint32_t n, uint32_t k) {
    (void)n;
    const uint64_t tiles = (m + 31) / 32, stages = ((k + 63) / 64 + MX_STAGE - 1) / MX_STAGE;
    return tiles * stages * (MX_STAGE * MX_REC + MX_SREC);
}

template <int CT>
static MxFn mx_kernel_fn(size_t &lds) {
    lds = (size_t)MxPlan<CT>::LDS;
    return mx_matmul_kernel<CT>;
}

// The workspace: the code records of every (tile, step), then the scale
// words of every (tile, stage).
struct MxSplitLayout {
    uint32_t ksteps, tiles, kpad;
    uint8_t *frag, *scl;
};
static MxSplitLayout mx_layout(uint32_t m, uint32_t k, void *workspace) {
    MxSplitLayout l;
    l.ksteps = (k + 63) / 64;
    l.tiles = (m + 31) / 32;
    l.kpad = (l.ksteps + MX_STAGE - 1) / MX_STAGE * MX_STAGE;
    l.frag = (uint8_t *)workspace;
    l.scl = l.frag + (uint64_t)l.tiles * l.kpad * MX_REC;
    return l;
}

int mx_norm_split_launch(void *x, const void *res, const float *w, void *y, uint32_t m, uint32_t k, float epsilon,
                         bool full_layer, void *workspace, hipStream_t stream) {
    const MxSplitLayout l = mx_layout(m, k, workspace);
    MxNormSplitArgs a;
    a.x = (uint16_t *)x;
    a.res = (const uint16_t *)res;
    a.w = w;
    a.y = (uint16_t *)y;
    a.frag = l.frag;
    a.scl = l.scl;
    a.m = m;
    a.k = k;
    a.kpad = l.kpad;
    a.full_layer = full_layer ? 1u : 0u;
    a.epsilon = epsilon;
    const size_t lds = (size_t)k * 2;
    auto fn = res ? mx_norm_split_kernel<true> : mx_norm_split_kernel<false>;
    if (lds > 64 * 1024)
        OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                          "hipFuncSetAttribute"));
    hipLaunchKernelGGL(fn, dim3(l.tiles * 32), dim3(256), lds, stream, a);
    return launch_check("oco_norm_mx_split");
}

int mx_matmul_launch(const void *w, const void *x, void *y, bool y_bf16, const float *bias, uint32_t m, uint32_t n,
                     uint32_t k, void *workspace, hipStream_t stream, bool presplit) {
    const MxSplitLayout l = mx_layout(m, k, workspace);
    const uint32_t ksteps = l.ksteps, tiles = l.tiles, kpad = l.kpad;
    uint8_t *const frag = l.frag, *const scl = l.scl;
    const MxTilePlan plan = mx_plan(m, n);
    if (!presplit) {
        MxSplitArgs sa;
        sa.x = (const uint16_t *)x;
        sa.frag = frag;
        sa.scl = scl;
        sa.m = m;
        sa.k = k;
        sa.kpad = kpad;
        sa.records = tiles * kpad;
        hipLaunchKernelGGL(mx_split_kernel, dim3(sa.records), dim3(64), 0, stream, KPRE_ARGS(sa), sa);
        OCO_TRY(launch_check("oco_matmul (mx split)"));
    }
    size_t lds = 0;
    MxFn fn = mx_kernel_fn<3>(lds);
    if (lds > 64 * 1024)
        OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                          "hipFuncSetAttribute"));
    MxArgs a;
    a.w = (const uint8_t *)w;
    a.frag = frag;
    a.scl = scl;
    a.kpad = kpad;
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
    hipLaunchKernelGGL(fn, dim3(plan.col_tiles, plan.groups), dim3(MxPlan<3>::NTH), lds, stream, KPRE_ARGS(a), a);
    return launch_check("oco_matmul (mx)");
}

}  // namespace oco
