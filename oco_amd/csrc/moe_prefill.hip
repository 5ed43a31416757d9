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
// reference's half tiles: tile.metal:35-52); no weight goes through LDS.
//
// Workgroup: NW wavefronts, each owning 16 weight columns (gate/up: the 16
// gate rows and the same 16 up rows, so the activation is fused in-lane;
// down: two groups of 16 rows), over one route-plan tile of 16 MI routes.
// Activations are staged per super-block into LDS (double-buffered, f16);
// weights are loaded a super-block ahead.
#include "matmul.h"
#include "formats.h"

namespace oco {

typedef _Float16 q4f16x8 __attribute__((ext_vector_type(8)));
typedef float q4f32x4 __attribute__((ext_vector_type(4)));

struct Q4Raw {  // one lane's bytes of one super-block: header and its 32 qs bytes
    uint4 hdr, q0, q1;
};


__device__ __forceinline__ float q4_row_gain(uint32_t bits) {
    if (bits == 0 || bits >= 0x7f800000u) return 1.0f;
    const int e = (int)(bits >> 23) - 127;
    return __builtin_ldexpf(1.0f, max(-100, min(100, 14 - e)));
}

__device__ __forceinline__ uint32_t f16_pair(float lo, float hi) {
    const _Float16 a = (_Float16)lo, b = (_Float16)hi;
    uint16_t x, y;
    __builtin_memcpy(&x, &a, 2);
    __builtin_memcpy(&y, &b, 2);
    return (uint32_t)x | ((uint32_t)y << 16);
}

// Scales of sub-block pair q: a = d sc, m = dmin mn for the low (0) and high
// (1) nibbles (get_scale_min_k4, weights.metal:67-77).
struct Q4Scales {
    float a0, m0, a1, m1;
};
__device__ __forceinline__ Q4Scales q4_scales(const uint4 &hdr, int q) {
    // scales[12] = hdr.y (bytes 0..3), hdr.z (4..7), hdr.w (8..11); sub-block
    // j < 4: sc = scales[j] & 63, mn = scales[j+4] & 63; j >= 4: sc =
    // (scales[j+4] & 15) | (scales[j-4] >> 6) << 4, mn = (scales[j+4] >> 4) |
    // (scales[j] >> 6) << 4.  Pair q holds j = 2q, 2q + 1: bit offsets per
    // lane, one select between the two forms.
    uint32_t sc[2], mn[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t t = 8 * ((2 * q + h) & 3);
        const uint32_t sc_lo = __builtin_amdgcn_ubfe(hdr.y, t, 6), mn_lo = __builtin_amdgcn_ubfe(hdr.z, t, 6);
        const uint32_t sc_hi = __builtin_amdgcn_ubfe(hdr.w, t, 4) | (__builtin_amdgcn_ubfe(hdr.y, t + 6, 2) << 4);
        const uint32_t mn_hi = __builtin_amdgcn_ubfe(hdr.w, t + 4, 4) | (__builtin_amdgcn_ubfe(hdr.z, t + 6, 2) << 4);
        sc[h] = q < 2 ? sc_lo : sc_hi;
        mn[h] = q < 2 ? mn_lo : mn_hi;
    }
    const float d = half_bits_to_f32(hdr.x & 0xffffu), dmin = half_bits_to_f32(hdr.x >> 16);
    return {d * (float)sc[0], dmin * (float)mn[0], d * (float)sc[1], dmin * (float)mn[1]};
}

// Four weights from the nibbles of one dword, rounded to f16 as a * q - m:
// byte i -> v_cvt_f32_ubyte<i>, then v_fma_mix{lo,hi}_f16 writes each
// result into its half of the packed pair (a * q is exact, so this is the
// reference's scale * value - minimum rounded to half).
__device__ __forceinline__ void q4_four(uint32_t n, float a, float m, uint32_t &p01, uint32_t &p23) {
    float f0, f1, f2, f3;
    asm volatile("v_cvt_f32_ubyte0 %0, %1" : "=v"(f0) : "v"(n));
    asm volatile("v_cvt_f32_ubyte1 %0, %1" : "=v"(f1) : "v"(n));
    asm volatile("v_cvt_f32_ubyte2 %0, %1" : "=v"(f2) : "v"(n));
    asm volatile("v_cvt_f32_ubyte3 %0, %1" : "=v"(f3) : "v"(n));
    const float nm = -m;
    uint32_t lo, hi;  // mixlo's high half is don't-care: mixhi overwrites it
    asm volatile("v_fma_mixlo_f16 %0, %1, %2, %3" : "=v"(lo) : "v"(a), "v"(f0), "v"(nm));
    asm volatile("v_fma_mixhi_f16 %0, %1, %2, %3" : "+v"(lo) : "v"(a), "v"(f1), "v"(nm));
    asm volatile("v_fma_mixlo_f16 %0, %1, %2, %3" : "=v"(hi) : "v"(a), "v"(f2), "v"(nm));
    asm volatile("v_fma_mixhi_f16 %0, %1, %2, %3" : "+v"(hi) : "v"(a), "v"(f3), "v"(nm));
    p01 = lo;
    p23 = hi;
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

template <int G, int MI, int NW>
__global__ __launch_bounds__(64 * NW) void moe_q4k_kernel(MatmulArgs a) {
    constexpr int THREADS = 64 * NW, ROWS = 16 * MI;
    constexpr int LD = 256 + 8;                                    // f16 per staged row (+16 bytes: no bank conflicts)
    constexpr int XV = ROWS * 256 / THREADS;                       // activations per thread per super-block
    static_assert(ROWS * 256 % (8 * THREADS) == 0, "whole 16-byte runs per thread");
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][ROWS * LD];
    __shared__ uint32_t tile_route[ROWS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c16 = lane & 15, q = lane >> 4;
    // Logical (column group, tile), tile-major per XCD: the column groups of
    // one tile share its activation rows in one L2.
    const uint32_t used = gridDim.x * min(a.plan[1], gridDim.y);  // the plan's real tiles
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, used);
    if (lin >= used) return;  // uniform: a surplus workgroup
    const uint32_t bx = lin % gridDim.x, y = lin / gridDim.x;
    const uint32_t expert = a.plan[6 + 2 * y], first = a.plan[7 + 2 * y];
    const uint64_t grouped = 6 + 2 * ((uint64_t)(a.routes + 15) / 16 + a.experts);
    const uint64_t list = grouped + (uint64_t)expert * (a.routes + 1);
    const uint64_t sorted = grouped + (uint64_t)a.experts * (a.routes + 1);
    const uint32_t rows = min((uint32_t)ROWS, a.plan[list] - first);
    const uint32_t sorted0 = a.plan[sorted + expert] + first;
    for (uint32_t r = tid; r < rows; r += THREADS) tile_route[r] = a.plan[list + 1 + first + r];
    __syncthreads();

    // This wavefront's two 16-row weight fragments.
    const uint32_t col0 = (bx * NW + wave) * (G == MM_GATE_UP ? 16 : 32);
    const uint8_t *wrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t col = G == MM_GATE_UP ? col0 + c16 : col0 + 16 * j + c16;
        const uint8_t *base = (G == MM_GATE_UP && j == 1 ? a.w2 : a.w) + expert * a.expert_bytes;
        wrow[j] = base + (uint64_t)min(col, a.n - 1) * a.row_bytes;
    }
    const uint32_t nsb = a.k / 256;

    // Activation staging: run f = tid + THREADS i (i < RUNS) is row f / 32,
    // 16-byte run f % 32 (consecutive lanes, consecutive runs: coalesced
    // loads, conflict-free LDS stores).
    constexpr int RUNS = XV / 8;
    uint32_t xsrc[RUNS], xrun[RUNS], xrow_[RUNS];
    bool xlive[RUNS];
    float gain[G == MM_DOWN ? RUNS : 1];
#pragma unroll
    for (int i = 0; i < RUNS; i++) {
        const uint32_t f = tid + THREADS * i, r = f / 32;
        xrow_[i] = r;
        xrun[i] = f % 32;
        xlive[i] = r < rows;
        xsrc[i] = !xlive[i] ? 0u : G == MM_GATE_UP ? tile_route[r] / a.topk : sorted0 + r;
        if constexpr (G == MM_DOWN) gain[i] = xlive[i] ? q4_row_gain(a.rowmax[xsrc[i]]) : 1.0f;
    }
    uint4 xv[RUNS * (G == MM_DOWN ? 2 : 1)];
    auto xload = [&](uint32_t sb) {
        sb = min(sb, nsb - 1);
#pragma unroll
        for (int i = 0; i < RUNS; i++) {
            const uint64_t off = (uint64_t)xsrc[i] * a.k + (uint64_t)sb * 256 + 8 * xrun[i];
            if constexpr (G == MM_DOWN) {
                const uint4 *src = reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(a.x) + off);
                xv[2 * i] = xlive[i] ? src[0] : make_uint4(0, 0, 0, 0);
                xv[2 * i + 1] = xlive[i] ? src[1] : make_uint4(0, 0, 0, 0);
            } else {
                xv[i] = xlive[i] ? *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.x) + off)
                                 : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto xstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < RUNS; i++) {
            uint16_t *dst = &xs[buf][xrow_[i] * LD + 8 * xrun[i]];
            uint4 o;
            if constexpr (G == MM_DOWN) {
                const uint4 u0 = xv[2 * i], u1 = xv[2 * i + 1];
                const float g = gain[i];
                o = make_uint4(f16_pair(__uint_as_float(u0.x) * g, __uint_as_float(u0.y) * g),
                               f16_pair(__uint_as_float(u0.z) * g, __uint_as_float(u0.w) * g),
                               f16_pair(__uint_as_float(u1.x) * g, __uint_as_float(u1.y) * g),
                               f16_pair(__uint_as_float(u1.z) * g, __uint_as_float(u1.w) * g));
            } else {  // gate/up: the caller hands f16 rows
                o = xv[i];
            }
            *reinterpret_cast<uint4 *>(dst) = o;
        }
    };
    Q4Raw wr[2][2];  // [register stage][fragment]
    auto wload = [&](Q4Raw *r, uint32_t sb) {
        sb = min(sb, nsb - 1);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint8_t *blk = wrow[j] + (uint64_t)sb * 144;
            r[j].hdr = ld_u128(blk);
            r[j].q0 = ld_u128(blk + 16 + 32 * q);
            r[j].q1 = ld_u128(blk + 32 + 32 * q);
        }
    };

    q4f32x4 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = q4f32x4{0.f, 0.f, 0.f, 0.f};

    auto step = [&](const Q4Raw *r, int buf) {
        const Q4Scales s0 = q4_scales(r[0].hdr, q), s1 = q4_scales(r[1].hdr, q);
        const uint16_t *xb = xs[buf];
        auto chunk = [&](auto cc) {
            constexpr int C = decltype(cc)::value;
            const q4f16x8 b0 = q4_chunk<C>(r[0], s0), b1 = q4_chunk<C>(r[1], s1);
#pragma unroll
            for (int i = 0; i < MI; i++) {
                q4f16x8 av;
                __builtin_memcpy(&av, &xb[(i * 16 + c16) * LD + 64 * q + 8 * C], 16);
                acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b0, acc[i][0], 0, 0, 0);
                acc[i][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b1, acc[i][1], 0, 0, 0);
            }
        };
        chunk(std::integral_constant<int, 0>{});
        chunk(std::integral_constant<int, 1>{});
        chunk(std::integral_constant<int, 2>{});
        chunk(std::integral_constant<int, 3>{});
        chunk(std::integral_constant<int, 4>{});
        chunk(std::integral_constant<int, 5>{});
        chunk(std::integral_constant<int, 6>{});
        chunk(std::integral_constant<int, 7>{});
    };

    // Super-block sb: activations in LDS buffer sb % 2, weights in register
    // stage sb % 2; sb + 1's activations are in registers, sb + 2's loading.
    xload(0);
    wload(wr[0], 0);
    xstore(0);
    xload(1);
    wload(wr[1], 1);
    __syncthreads();
    uint32_t sb = 0;
    for (; sb + 2 <= nsb; sb += 2) {  // whole pairs: register stages by name
        step(wr[0], 0);
        xstore(1);
        xload(sb + 2);
        wload(wr[0], sb + 2);
        __syncthreads();
        step(wr[1], 1);
        xstore(0);
        xload(sb + 3);
        wload(wr[1], sb + 3);
        __syncthreads();
    }
    if (sb < nsb) step(wr[0], 0);

    // C fragment: lane l holds column l % 16, rows 4 (l / 16) .. + 4.
    const int cr = q * 4;
    if constexpr (G == MM_GATE_UP) {
        const uint32_t col = col0 + c16;
        const bool cok = col < a.n;
        const uint64_t bi = (uint64_t)expert * a.n + (cok ? col : 0);
        const float bg = a.bias && cok ? round_bf16(a.bias[bi]) : 0.f;
        const float bu = a.bias2 && cok ? round_bf16(a.bias2[bi] + (a.up_one ? 1.0f : 0.0f)) : (a.up_one ? 1.0f : 0.0f);
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t r = i * 16 + cr + v;
                const float act = expert_activation(a.act, acc[i][0][v] + bg, acc[i][1][v] + bu);
                if (cok && r < rows) reinterpret_cast<float *>(a.y)[(uint64_t)(sorted0 + r) * a.n + col] = act;
                uint32_t m = cok ? __float_as_uint(act) & 0x7fffffffu : 0u;
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o));
                if (c16 == 0 && r < rows) atomicMax(&a.rowmax[sorted0 + r], m);
            }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t col = col0 + 16 * j + c16;
            if (col >= a.n) continue;
            const float b = a.bias ? round_bf16(a.bias[(uint64_t)expert * a.n + col]) : 0.f;
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const uint32_t r = i * 16 + cr + v;
                    if (r >= rows) continue;
                    const float val = acc[i][j][v] / q4_row_gain(a.rowmax[sorted0 + r]) + b;
                    const uint64_t o = (uint64_t)tile_route[r] * a.n + col;
                    if (a.y_bf16)
                        reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(val);
                    else
                        reinterpret_cast<float *>(a.y)[o] = val;
                }
        }
    }
}

// Eight wavefronts (two per SIMD); rows per tile bm = 16 MI routes (32, 48 or 64).
constexpr int Q4_NW = 8;

template <int MI>
static void q4_launch(int mode, const MatmulArgs &a, dim3 grid, hipStream_t stream) {
    if (mode == MM_GATE_UP)
        hipLaunchKernelGGL((moe_q4k_kernel<MM_GATE_UP, MI, Q4_NW>), grid, dim3(64 * Q4_NW), 0, stream, a);
    else
        hipLaunchKernelGGL((moe_q4k_kernel<MM_DOWN, MI, Q4_NW>), grid, dim3(64 * Q4_NW), 0, stream, a);
}

int moe_q4k_launch(int mode, const MatmulArgs &a, uint32_t bm, hipStream_t stream) {
    if (a.k % 256) return fail(OCO_ERR_INVALID, "experts: Q4_K rows need k %% 256 == 0 (k=%u)", a.k);
    if (bm != 32 && bm != 48 && bm != 64) return fail(OCO_ERR_INVALID, "experts: Q4_K tile of %u rows", bm);
    const uint32_t cols = (mode == MM_GATE_UP ? 16 : 32) * Q4_NW;
    const dim3 grid((a.n + cols - 1) / cols, (a.routes + bm - 1) / bm + a.experts);
    if (bm == 32) q4_launch<2>(mode, a, grid, stream);
    if (bm == 48) q4_launch<3>(mode, a, grid, stream);
    if (bm == 64) q4_launch<4>(mode, a, grid, stream);
    return launch_check("experts Q4_K grouped matmul");
}

}  // namespace oco
