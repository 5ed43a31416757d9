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

__global__ __launch_bounds__(256) void mx_split_kernel(MxSplitArgs a) {
    const uint32_t rec = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (rec >= a.records) return;
    const uint32_t tile = rec / a.ksteps, s = rec % a.ksteps;
    const int l = threadIdx.x & 63, r = l & 31, blk = l >> 5;
    const uint32_t row = tile * 32 + r, k0 = s * 64 + 32 * blk;
    float v[32];
    if (row < a.m && k0 < a.k) {
        const uint4 *src = reinterpret_cast<const uint4 *>(a.x + (uint64_t)row * a.k + k0);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 u = src[q];
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[8 * q + 2 * j] = __uint_as_float(w4[j] << 16);
                v[8 * q + 2 * j + 1] = __uint_as_float(w4[j] & 0xffff0000u);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = 0.f;
    }
    uint8_t *out = a.frag + (uint64_t)rec * MX_REC;
    uint32_t scales = 0;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        float amax = 0.f;
        bool nan = false;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            amax = fmaxf(amax, fabsf(v[i]));
            nan |= v[i] != v[i];
        }
        if (nan) amax = __uint_as_float(0x7fc00000u);
        const int E = mx_scale_exp(amax);
        scales |= (uint32_t)(E + 127) << (8 * t);
        const float inv = E == 128 ? 0.f : __builtin_ldexpf(1.f, -E), sc = E == 128 ? 0.f : __builtin_ldexpf(1.f, E);
        uint32_t codes[8];  // 32 E4M3 codes, block value order
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            int p = __builtin_amdgcn_cvt_pk_fp8_f32(v[i] * inv, v[i + 1] * inv, 0, false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(v[i + 2] * inv, v[i + 3] * inv, p, true);
            codes[i / 4] = (uint32_t)p;
        }
#pragma unroll
        for (int q = 0; q < 8; q++) {
            v[4 * q] -= __builtin_amdgcn_cvt_f32_fp8((int)codes[q], 0) * sc;
            v[4 * q + 1] -= __builtin_amdgcn_cvt_f32_fp8((int)codes[q], 1) * sc;
            v[4 * q + 2] -= __builtin_amdgcn_cvt_f32_fp8((int)codes[q], 2) * sc;
            v[4 * q + 3] -= __builtin_amdgcn_cvt_f32_fp8((int)codes[q], 3) * sc;
        }
        // Lane r + 32p, byte e of this block: the value W keeps in nibble e & 1 of
        // payload byte 8p + e / 2, i.e. value 8p + e / 2 + 16 (e & 1).
#pragma unroll
        for (int p = 0; p < 2; p++) {
            uint32_t o[4];
#pragma unroll
            for (int d = 0; d < 4; d++) {
                uint32_t word = 0;
#pragma unroll
                for (int bb = 0; bb < 4; bb++) {
                    const int e = 4 * d + bb, idx = 8 * p + e / 2 + 16 * (e & 1);
                    word |= ((codes[idx / 4] >> (8 * (idx & 3))) & 0xffu) << (8 * bb);
                }
                o[d] = word;
            }
            *reinterpret_cast<uint4 *>(out + ((t * 2 + blk) * 64 + r + 32 * p) * 16) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    *reinterpret_cast<uint32_t *>(out + MX_DATA + (r + 32 * blk) * 4) = scales;
}

struct MxArgs {
    const uint8_t *w;
    const uint8_t *frag;
    void *y;
    const float *bias;
    uint32_t m, n, k, ksteps, tiles;
    uint64_t row_bytes;
    uint32_t y_bf16;
};

// Workgroup tile: 4 x NW wavefronts; wavefront (wm, wn) owns MI activation
// row tiles of 32 and CW = CT / NW weight row tiles of 32 (workgroup tile
// BM = 128 MI rows x BN = 32 CT columns).
//  * A (the split activations) goes straight from the split records
//    (16-byte lanes, coalesced) into registers, D steps ahead.
//  * B (the GGUF bytes) is shared by the workgroup and staged through LDS:
//    per K step of 64, each weight row's two blocks (34 bytes) are fetched
//    as the dword-aligned span that holds them, ten consecutive lanes per
//    row, so each byte crosses the address units once.  Three LDS buffers:
//    at step t the MFMAs of t run on operands already in registers while
//    the B fragments of t + 1 are read from LDS and B of t + 2 is written.
// One barrier per step; the MFMA pipe never waits for LDS.
constexpr int MX_BSLOT = 44;  // LDS bytes per weight row per step: 34 + alignment, 11 dwords (odd: no bank conflicts)

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

template <int MI, int CT, int NW, int D>
struct MxPlan {
    static constexpr int THREADS = 256 * NW, CW = CT / NW;  // CW column tiles per wavefront
    static constexpr int BM = 128 * MI, BN = 32 * CT;
    static constexpr int BD = BN * 10, BU = (BD + THREADS - 1) / THREADS;  // B dwords per step, per thread
    static constexpr int STAGE = BN * MX_BSLOT, LDS = 3 * STAGE;
    static_assert(CT % NW == 0, "column tiles split evenly");
    static_assert(D % 2 == 0 && D >= 2, "even ring depth");
};

template <int MI, int CT, int NW, int D>
struct MxRing {
    using P = MxPlan<MI, CT, NW, D>;
    const uint8_t *arec[MI];  // this lane's records, step 0
    const uint8_t *brow[P::BU];
    uint32_t bdst[P::BU], bd[P::BU];
    i32x8 ra[D][MI][2];  // A of step t in slot t % D: [tile][term], already in MFMA operand form
    uint32_t rs[D][MI];
    uint32_t rb[D][P::BU];  // B of step t (awaiting its LDS store) in slot t % D

    __device__ __forceinline__ void init(const MxArgs &a, int tid, int lane, uint32_t tile0, uint32_t col0) {
#pragma unroll
        for (int i = 0; i < MI; i++)
            arec[i] = a.frag + (uint64_t)min(tile0 + i, a.tiles - 1) * a.ksteps * MX_REC + lane * 16;
#pragma unroll
        for (int u = 0; u < P::BU; u++) {
            const int f = min(tid + P::THREADS * u, P::BD - 1), col = f / 10;  // surplus lanes repeat the last dword
            bd[u] = f % 10;
            brow[u] = a.w + (uint64_t)min(col0 + col, a.n - 1) * a.row_bytes;
            bdst[u] = col * MX_BSLOT + bd[u] * 4;
        }
    }
    // Loads are unconditional (a step past the end re-reads the last one):
    // a branch around a load makes the compiler wait for all loads at the join.
    template <int SLOT>
    __device__ __forceinline__ void load_a(const MxArgs &a, int lane, uint32_t s) {
        s = min(s, a.ksteps - 1);
#pragma unroll
        for (int i = 0; i < MI; i++) {
            const uint8_t *rec = arec[i] + (uint64_t)s * MX_REC;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint4 lo = *reinterpret_cast<const uint4 *>(rec + (2 * t) * 1024);
                const uint4 hi = *reinterpret_cast<const uint4 *>(rec + (2 * t + 1) * 1024);
                ra[SLOT][i][t] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
            rs[SLOT][i] = *reinterpret_cast<const uint32_t *>(rec - lane * 16 + MX_DATA + lane * 4);
        }
    }
    template <int SLOT>
    __device__ __forceinline__ void load_b(const MxArgs &a, uint32_t s) {
        s = min(s, a.ksteps - 1);
        const uint32_t len = 2 * s + 1 < a.k / 32 ? 34 : 17;
#pragma unroll
        for (int u = 0; u < P::BU; u++) {
            const uint8_t *p = brow[u] + (uint64_t)s * 34;
            const uint32_t lo = (uint32_t)(uintptr_t)p & 3u, last = (lo + len - 1) / 4;
            // only dwords holding bytes of this step's blocks
            rb[SLOT][u] = *reinterpret_cast<const uint32_t *>(p - lo + 4 * min(bd[u], last));
        }
    }
    template <int SLOT>
    __device__ __forceinline__ void store_b(uint8_t *base) const {
#pragma unroll
        for (int u = 0; u < P::BU; u++) *reinterpret_cast<uint32_t *>(base + bdst[u]) = rb[SLOT][u];
    }
};

template <int MI, int CT, int NW, int D>
__global__ __launch_bounds__(256 * NW) void mx_matmul_kernel(MxArgs a) {
    using P = MxPlan<MI, CT, NW, D>;
    constexpr int CW = P::CW;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // [3][STAGE]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 31, part = lane >> 5;
    const int wm = wave & 3, wn = wave >> 2;
    // Logical (column tile, row tile), column-major per XCD: the row tiles of
    // one weight column tile share its GGUF bytes in one L2, and each XCD's
    // share of the split activations stays resident.
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
    const uint32_t bx = lin / gridDim.y, by = lin % gridDim.y;
    const uint32_t tile0 = by * (4 * MI) + wm * MI, col0 = bx * P::BN;
    const uint32_t nblk = a.k / 32;

    MxRing<MI, CT, NW, D> ring;
    ring.init(a, tid, lane, tile0, col0);
    uint32_t wlow[CW];  // weight row address mod 4 (fixes the span alignment)
#pragma unroll
    for (int j = 0; j < CW; j++)
        wlow[j] = (uint32_t)(uintptr_t)(a.w + (uint64_t)min(col0 + (wn * CW + j) * 32 + c, a.n - 1) * a.row_bytes) & 3u;

    f32x16 acc[MI][CW];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < CW; j++) acc[i][j] = f32x16{};

    i32x8 bf[2][CW];  // B fragments of steps of parity 0 / 1
    int sb[2][CW];
    auto frags = [&](auto par, uint32_t t) {  // B fragments of step t from LDS buffer t % 3
        constexpr int PA = decltype(par)::value;
        const uint8_t *base = lds + (t % 3) * P::STAGE;
        const bool live = 2 * t + part < nblk;
#pragma unroll
        for (int j = 0; j < CW; j++) {
            const uint8_t *row = base + ((wn * CW + j) * 32 + c) * MX_BSLOT;
            const uint32_t off = ((wlow[j] + 34 * t) & 3u) + 17 * part;  // scale byte of block 2t + part
            uint32_t q[4];
            lds_bytes<16>(row + off + 1, q);
            bf[PA][j] = live ? i32x8{(int)q[0], (int)q[1], (int)q[2], (int)q[3], 0, 0, 0, 0} : i32x8{};
            sb[PA][j] = live ? row[off] : 127;
        }
    };
    auto mma = [&](auto slot, auto par) {
        constexpr int SL = decltype(slot)::value, PA = decltype(par)::value;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < MI; i++) {
                const i32x8 &av = ring.ra[SL][i][t];
#pragma unroll
                for (int j = 0; j < CW; j++) {
                    if (t == 0)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bf[PA][j], acc[i][j], 0, 4, 0,
                                                                                     (int)ring.rs[SL][i], 0, sb[PA][j]);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bf[PA][j], acc[i][j], 0, 4, 1,
                                                                                     (int)ring.rs[SL][i], 0, sb[PA][j]);
                }
            }
    };
    // One step t (u = t mod D): read B fragments of t + 1, multiply t, load
    // A of t + D, store B of t + 2 to LDS and load B of t + 2 + D.
    auto body = [&](auto u, uint32_t t) {
        constexpr int U = decltype(u)::value, B2 = (U + 2) % D;
        frags(Int<(U + 1) & 1>{}, t + 1);  // harmless past the end
        mma(u, Int<U & 1>{});
        ring.template load_a<U>(a, lane, t + D);
        ring.template store_b<B2>(lds + ((t + 2) % 3) * P::STAGE);
        ring.template load_b<B2>(a, t + 2 + D);
        __syncthreads();
    };

    static_for<D>([&](auto u) {
        ring.template load_a<u.value>(a, lane, u.value);
        ring.template load_b<u.value>(a, u.value);
    });
    ring.template store_b<0>(lds);
    ring.template store_b<1>(lds + P::STAGE);
    ring.template load_b<0>(a, D);
    ring.template load_b<1>(a, D + 1);
    __syncthreads();
    frags(Int<0>{}, 0);
    uint32_t s = 0;
    for (; s + D <= a.ksteps; s += D)  // whole rounds: no branch between a load and its use
        static_for<D>([&](auto u) { body(u, s + u.value); });
    static_for<D>([&](auto u) {
        if (s + u.value < a.ksteps) body(u, s + u.value);
    });

#pragma unroll
    for (int j = 0; j < CW; j++) {
        const uint32_t col = col0 + (wn * CW + j) * 32 + c;
        if (col >= a.n) continue;
        const float bias = a.bias ? round_bf16(a.bias[col]) : 0.f;
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t row = (tile0 + i) * 32 + 8 * (v / 4) + 4 * part + (v % 4);
                if (row >= a.m) continue;
                const float r = acc[i][j][v] + bias;
                const uint64_t o = (uint64_t)row * a.n + col;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(r);
                else
                    reinterpret_cast<float *>(a.y)[o] = r;
            }
    }
}

uint64_t mx_workspace_bytes(uint32_t m, uint32_t k) {
    return (uint64_t)((m + 31) / 32) * ((k + 63) / 64) * MX_REC;
}

typedef void (*MxFn)(MxArgs);

template <int MI, int CT, int NW, int D>
static MxFn mx_kernel(int &rows, int &cols, int &threads, size_t &lds) {
    using P = MxPlan<MI, CT, NW, D>;
    rows = P::BM;
    cols = P::BN;
    threads = P::THREADS;
    lds = (size_t)P::LDS;
    return mx_matmul_kernel<MI, CT, NW, D>;
}

// Tile shapes: workgroup rows x columns = 128 MI x 32 CT.  Measured on
// MI355X: 128 x 64 with four wavefronts while 128 x 128 tiles would not
// cover the 256 CUs (gpt-oss 5760 x 2880 at 512 tokens), else 128 x 192
// with eight.
static MxFn mx_pick(uint32_t m, uint32_t n, int &rows, int &cols, int &threads, size_t &lds) {
    int choice = -1;
    if (const char *env = getenv("OCO_MX_TILE")) choice = atoi(env);  // tuning runs only
    if (choice < 0) {
        const uint64_t big = (uint64_t)((m + 127) / 128) * ((n + 127) / 128);
        choice = big < 256 ? 2 : 5;
    }
    switch (choice) {
    case 1: return mx_kernel<1, 4, 1, 2>(rows, cols, threads, lds);  // 128 x 128, 4 waves
    case 2: return mx_kernel<1, 2, 1, 2>(rows, cols, threads, lds);  // 128 x 64, 4 waves
    case 3: return mx_kernel<1, 4, 2, 2>(rows, cols, threads, lds);  // 128 x 128, 8 waves
    case 4: return mx_kernel<2, 2, 1, 2>(rows, cols, threads, lds);  // 256 x 64, 4 waves
    case 5: return mx_kernel<1, 6, 2, 2>(rows, cols, threads, lds);  // 128 x 192, 8 waves
    default: return mx_kernel<1, 2, 2, 2>(rows, cols, threads, lds);  // 128 x 64, 8 waves
    }
}

int mx_matmul_launch(const void *w, const void *x, void *y, bool y_bf16, const float *bias, uint32_t m, uint32_t n,
                     uint32_t k, void *workspace, hipStream_t stream) {
    const uint32_t ksteps = (k + 63) / 64, tiles = (m + 31) / 32;
    MxSplitArgs sa;
    sa.x = (const uint16_t *)x;
    sa.frag = (uint8_t *)workspace;
    sa.m = m;
    sa.k = k;
    sa.ksteps = ksteps;
    sa.records = tiles * ksteps;
    hipLaunchKernelGGL(mx_split_kernel, dim3((sa.records + 3) / 4), dim3(256), 0, stream, sa);
    OCO_TRY(launch_check("oco_matmul (mx split)"));
    int rows, cols, threads;
    size_t lds;
    MxFn fn = mx_pick(m, n, rows, cols, threads, lds);
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
    a.row_bytes = (uint64_t)(k / 32) * 17;
    a.y_bf16 = y_bf16;
    hipLaunchKernelGGL(fn, dim3((n + cols - 1) / cols, (m + rows - 1) / rows), dim3(threads), lds, stream, a);
    return launch_check("oco_matmul (mx)");
}

}  // namespace oco
