// Prefill matmul on CDNA4 MFMA: Y[m, n] = X[m, k] W[n, k]^T (+ bias) with
// GGUF-block weights dequantized into LDS.  Replaces DenseMatrix::apply's
// tiled plans (src/weights/compute/matrix.rs:130-379: `matmul`,
// `matmul_q4*`, `matmul_tensor_*`, shaders/matrix/batch.metal:24-79,
// tensor.metal:9-102).
//
// Operands: MXFP4 weights (E2M1 x 2^e) and bf16 activations are exact in
// bf16, so MXFP4 runs v_mfma_f32_16x16x32_bf16 with exact products.  The
// other formats decode to f16 -- the reference's half(w) operand
// (tile.metal:16-80) -- and the activations convert to f16, on
// v_mfma_f32_16x16x32_f16.  Accumulation is fp32.
//
// Tile: a 256-thread workgroup computes 128 activation rows x 64 weight rows
// with K steps of 128 (see matmul_kernel).
#include <hipblaslt/hipblaslt.h>
#include <stdlib.h>

#include <map>
#include <mutex>
#include <tuple>

#include "formats.h"
#include "matmul.h"

namespace oco {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));


// 16-bit operand bits of a float: bf16 (round to nearest even) or f16.
template <bool BF>
__device__ __forceinline__ uint16_t operand_bits(float v) {
    if constexpr (BF) {
        return f32_to_bf16_bits(v);
    } else {
        _Float16 h = (_Float16)v;
        uint16_t b;
        __builtin_memcpy(&b, &h, 2);
        return b;
    }
}

template <int FMT>
struct BlockShape {
    static constexpr uint32_t BE = FMT == OCO_F32 || FMT == OCO_F16 || FMT == OCO_BF16 ? 1
                                   : (FMT == OCO_Q4_K || FMT == OCO_Q5_K || FMT == OCO_Q6_K) ? 256 : 32;
    static constexpr uint32_t BB = FMT == OCO_F32 ? 4 : (FMT == OCO_F16 || FMT == OCO_BF16) ? 2
                                   : FMT == OCO_Q4_0 ? 18 : FMT == OCO_Q4_1 ? 20 : FMT == OCO_Q8_0 ? 34
                                   : FMT == OCO_Q4_K ? 144 : FMT == OCO_Q5_K ? 176 : FMT == OCO_Q6_K ? 210 : 17;
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }



// One thread's share of a weight tile step: a 32-coefficient piece of one
// row, decoded to MFMA operand bits as four runs of eight consecutive
// columns.  `col0[r]` receives each run's first column within the 128-wide
// K step; out[4r .. 4r+3] its eight 16-bit operands.  Loading (global reads
// of the piece's bytes) and decoding are separate so the loads of later
// steps can be in flight while the current step is decoded.
//   32-blocks (Q8_0, MXFP4, Q4_0, Q4_1, BF16, F16, F32): piece c = block c of
//     the step, runs at 32c + 8r.
//   K-quants: the step is half a super-block; piece c is the lane
//     decomposition of the streaming decoder (piece c + 4 * half).
template <int FMT, bool BF>
struct PrefillPiece {
    static constexpr uint32_t BE = BlockShape<FMT>::BE, BB = BlockShape<FMT>::BB;
    struct Raw {
        uint32_t w[FMT == OCO_Q4_K || FMT == OCO_Q6_K ? 8 : FMT == OCO_MXFP4 ? 5 : 1];
        gbytes row;
    };
    __device__ __forceinline__ static Raw load(gbytes row, uint32_t k0, int c) {
        Raw r;
        r.row = row;
        if constexpr (FMT == OCO_MXFP4 && BF) {
            const gbytes b = row + (uint64_t)(k0 / 32 + c) * BB;
            const uint4 q = ld_u128(b + 1);
            r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
            r.w[4] = ld_u8(b);
        } else if constexpr (FMT == OCO_Q4_K) {
            const uint32_t cc = (k0 % 256) / 128 * 4 + c;
            const gbytes b = row + (uint64_t)(k0 / 256) * BB;
            const uint4 hdr = ld_u128(b), qs = ld_u128(b + 16 + 16 * cc);
            r.w[0] = hdr.x; r.w[1] = hdr.y; r.w[2] = hdr.z; r.w[3] = hdr.w;
            r.w[4] = qs.x; r.w[5] = qs.y; r.w[6] = qs.z; r.w[7] = qs.w;
        } else if constexpr (FMT == OCO_Q6_K) {
            const uint32_t hb = (k0 % 256) / 128, l0 = 8 * c;
            const gbytes b = row + (uint64_t)(k0 / 256) * BB;
            const uint2 ql0 = ld_u64(b + hb * 64 + l0), ql1 = ld_u64(b + hb * 64 + 32 + l0),
                        qh = ld_u64(b + 128 + hb * 32 + l0);
            r.w[0] = ql0.x; r.w[1] = ql0.y; r.w[2] = ql1.x; r.w[3] = ql1.y; r.w[4] = qh.x; r.w[5] = qh.y;
            // four quarter scales (bytes 0, 2, 4, 6 of this 8-byte window) and d
            const uint2 scw = ld_u64(b + 192 + hb * 8 + (l0 >> 4));
            r.w[6] = (scw.x & 0xffu) | ((scw.x >> 8) & 0xff00u) | ((scw.y << 16) & 0xff0000u) | ((scw.y << 8) & 0xff000000u);
            r.w[7] = ld_u16(b + 208);
        }
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw &r, uint32_t k0, int c, uint32_t *out, uint32_t *col0) {
        if constexpr (FMT == OCO_MXFP4 && BF) {
            const float scale = e8m0_scale(r.w[4]);
            uint32_t pk[16];  // byte i -> (column i, column 16 + i)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
                bf16x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(r.w[j], scale, 0);
                bf16x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(r.w[j], scale, 1);
                bf16x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(r.w[j], scale, 2);
                bf16x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(r.w[j], scale, 3);
                __builtin_memcpy(&pk[4 * j], &v0, 4);
                __builtin_memcpy(&pk[4 * j + 1], &v1, 4);
                __builtin_memcpy(&pk[4 * j + 2], &v2, 4);
                __builtin_memcpy(&pk[4 * j + 3], &v3, 4);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                out[i] = __builtin_amdgcn_perm(pk[2 * i + 1], pk[2 * i], 0x05040100u);      // columns 2i, 2i+1
                out[8 + i] = __builtin_amdgcn_perm(pk[2 * i + 1], pk[2 * i], 0x07060302u);  // columns 16+2i, 17+2i
            }
#pragma unroll
            for (int q = 0; q < 4; q++) col0[q] = 32 * c + 8 * q;
        } else if constexpr (FMT == OCO_Q4_K) {
            const uint32_t cc = (k0 % 256) / 128 * 4 + c, g = cc >> 1, odd = cc & 1;
            uint8_t sb[12];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sb[i] = (uint8_t)byte_of(r.w[1], i);
                sb[4 + i] = (uint8_t)byte_of(r.w[2], i);
                sb[8 + i] = (uint8_t)byte_of(r.w[3], i);
            }
            uint32_t sc0, mn0, sc1, mn1;
            kquant_scale_min(sb, 2 * g, sc0, mn0);
            kquant_scale_min(sb, 2 * g + 1, sc1, mn1);
            const float d = half_bits_to_f32(r.w[0] & 0xffffu), dmin = half_bits_to_f32(r.w[0] >> 16);
            const float a0 = d * (float)sc0, m0 = dmin * (float)mn0, a1 = d * (float)sc1, m1 = dmin * (float)mn1;
            // half(a q - m): a q is exact in f32 (a = d sc has at most 17
            // significant bits, q 4), so the fused multiply-add rounds the
            // same value the reference's multiply and subtract do
            static_assert(!BF, "K-quants take f16 operands");
#pragma unroll
            for (int j = 0; j < 4; j++) {
                q4_four(r.w[4 + j] & 0x0f0f0f0fu, a0, m0, out[2 * j], out[2 * j + 1]);
                q4_four((r.w[4 + j] >> 4) & 0x0f0f0f0fu, a1, m1, out[8 + 2 * j], out[8 + 2 * j + 1]);
            }
            const uint32_t base = 64 * g + 16 * odd - (k0 % 256) / 128 * 128;
            col0[0] = base;
            col0[1] = base + 8;
            col0[2] = base + 32;
            col0[3] = base + 40;
        } else if constexpr (FMT == OCO_Q6_K) {
            const uint32_t l0 = 8 * c;
            const float d = half_bits_to_f32(r.w[7]);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t lw0 = (q & 1) ? r.w[2] : r.w[0], lw1 = (q & 1) ? r.w[3] : r.w[1];
                const int shift = (q >> 1) * 4;
                const float sc = d * (float)(int8_t)byte_of(r.w[6], q);
                uint16_t v[8];
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const uint32_t lw = half ? lw1 : lw0, hw = half ? r.w[5] : r.w[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int code =
                            (int)(((lw >> (8 * i + shift)) & 15u) | (((hw >> (8 * i + 2 * q)) & 3u) << 4)) - 32;
                        v[4 * half + i] = operand_bits<BF>(__fmul_rn(sc, (float)code));
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; i++) out[4 * q + i] = pack2(v[2 * i], v[2 * i + 1]);
                col0[q] = 32 * q + l0;
            }
        } else {
            // Generic: decode each coefficient of the 32 columns 32c .. 32c+31.
            const uint32_t kbase = k0 + 32 * c;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t col = kbase + 2 * i;
                uint16_t v0 = operand_bits<BF>(decode_scalar(FMT, (const uint8_t *)r.row + (uint64_t)(col / BE) * BB, col % BE));
                uint16_t v1 =
                    operand_bits<BF>(decode_scalar(FMT, (const uint8_t *)r.row + (uint64_t)((col + 1) / BE) * BB, (col + 1) % BE));
                out[i] = pack2(v0, v1);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) col0[q] = 32 * c + 8 * q;
        }
    }
};

// Tile BM activation rows x BN weight rows, K step 128.  Four wavefronts in
// a 2 x 2 grid, each (BM/2) x (BN/2) as blocks of v_mfma_f32_16x16x32.
// Two LDS buffers: while the MFMAs of step s read buffer s % 2, the same
// wavefronts decode step s+1 (loaded into registers a step earlier) into the
// other buffer, and the loads for step s+2 are in flight; one barrier per
// step.  Weight piece p = tid + 256 u goes to row p % BN, piece p / BN, so a
// wavefront's 64 lanes write 64 different rows (conflict-free LDS stores).
template <int FMT, bool BF, int BM, int BN, int G>
struct Stage {
    static constexpr int XPT = BM * 16 / 256, WPT = BN * 4 / 256;
    uint4 x[G == MM_DOWN ? 2 * XPT : XPT];  // down mode: eight f32 activations per chunk
    typename PrefillPiece<FMT, BF>::Raw w[WPT];
};

//
// Grouped modes (MM_GATE_UP, MM_DOWN) serve routed experts at prefill
// (expert_up_tensor / expert_down_tensor, projections.metal:192-376): tile y
// is the route plan's tile (expert e, first list row b), its rows the routes
// list[e][b ..] (gate/up: their tokens' activation rows; down: the
// expert-sorted activation rows).  In gate/up mode the BN weight rows are
// BN/2 gate and the same BN/2 up rows, placed so each wavefront holds a gate
// column and its up column in the same lane: the activation is fused.
template <int FMT, bool BF, int BM, int BN, int G = MM_DENSE>
__global__ __launch_bounds__(256) void matmul_kernel(KPRE_PARAMS, MatmulArgs a) {
    KPRE_APPLY(a);
    using PP = PrefillPiece<FMT, BF>;
    using ST = Stage<FMT, BF, BM, BN, G>;
    constexpr int BK = 128, LD = BK + 8;  // LDS row stride: 136 halves (272 bytes, conflict-free fragments)
    constexpr int MI = BM / 32, NJ = BN / 32, XPT = ST::XPT, WPT = ST::WPT;
    constexpr int XS = BM * LD, WS = BN * LD;
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];  // [2][XS] then [2][WS]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // Logical (column tile bx, row tile / plan tile by) in XCD order: dense
    // tiles column-major (the row tiles of a weight column tile share one
    // L2), grouped tiles tile-major (the column tiles of a route tile share
    // its activation rows).
    const uint32_t used = G == MM_DENSE ? gridDim.x * gridDim.y : gridDim.x * min(a.plan[1], gridDim.y);
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, used);
    if (lin >= used) return;  // uniform: a surplus workgroup (grouped grids are sized for the tile bound)
    const uint32_t bx = G == MM_DENSE ? lin / gridDim.y : lin % gridDim.x;
    const uint32_t by = G == MM_DENSE ? lin % gridDim.y : lin / gridDim.x;
    uint32_t m0 = by * BM;
    const uint32_t n0 = bx * (G == MM_GATE_UP ? BN / 2 : BN);
    const int tm = (wave >> 1) * (BM / 2), tn = (wave & 1) * (BN / 2);

    // Grouped tile: expert, rows, and each row's route (gate/up and down) or
    // expert-sorted row.
    __shared__ uint32_t tile_route[G == MM_DENSE ? 1 : BM];
    uint32_t expert = 0, rows = a.m, sorted0 = 0;
    if constexpr (G != MM_DENSE) {
        const uint32_t y = by;
        if (y >= a.plan[1]) return;  // uniform: past the plan's tile count
        expert = a.plan[6 + 2 * y];
        const uint32_t first = a.plan[7 + 2 * y];
        const uint64_t grouped = 6 + 2 * ((uint64_t)(a.routes + 15) / 16 + a.experts);
        const uint64_t list = grouped + (uint64_t)expert * (a.routes + 1);
        const uint64_t sorted = grouped + (uint64_t)a.experts * (a.routes + 1);
        rows = min((uint32_t)BM, a.plan[list] - first);
        sorted0 = a.plan[sorted + expert] + first;
        for (uint32_t r = tid; r < rows; r += 256) tile_route[r] = a.plan[list + 1 + first + r];
        __syncthreads();
        m0 = 0;
    }

    f32x4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const GLOBAL uint16_t *xg = gp(reinterpret_cast<const uint16_t *>(a.x));
    gbytes wr[WPT];
    int wrow[WPT], wpc[WPT];
#pragma unroll
    for (int u = 0; u < WPT; u++) {
        const int p = tid + 256 * u;
        wrow[u] = p % BN;
        wpc[u] = p / BN;
        if constexpr (G == MM_GATE_UP) {
            // LDS row q: column half h = q / (BN/2); its first BN/4 rows gate, the next BN/4 up
            const int q = wrow[u], h = q / (BN / 2), rr = q % (BN / 2);
            const uint32_t col = n0 + h * (BN / 4) + rr % (BN / 4);
            const gbytes base = gp(rr < BN / 4 ? a.w : a.w2) + expert * a.expert_bytes;
            wr[u] = base + (uint64_t)min(col, a.n - 1) * a.row_bytes;
        } else {
            wr[u] = gp(a.w) + expert * a.expert_bytes + (uint64_t)min(n0 + wrow[u], a.n - 1) * a.row_bytes;
        }
    }
    // Activation row of each X chunk this thread stages (fixed over K).  In
    // down mode the rows are f32 activations, scaled by a power of two
    // (row_gain) into f16 range; the epilogue divides it back out exactly.
    const GLOBAL uint16_t *xrow[XPT];
    bool xlive[XPT];
    float xgain[G == MM_DOWN ? XPT : 1];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int r = (tid + 256 * i) >> 4;
        uint32_t src = m0 + r;
        if constexpr (G == MM_GATE_UP) src = r < (int)rows ? tile_route[r] / a.topk : 0;
        if constexpr (G == MM_DOWN) src = sorted0 + r;
        xlive[i] = (uint32_t)r < rows && (G != MM_DENSE || m0 + r < a.m);
        const uint32_t row = xlive[i] ? src : 0;
        if constexpr (G == MM_DOWN) {
            xrow[i] = reinterpret_cast<const GLOBAL uint16_t *>(gp(reinterpret_cast<const float *>(a.x)) + (uint64_t)row * a.k);
            xgain[i] = row_gain(a.rowmax[row]);
        } else {
            xrow[i] = xg + (uint64_t)row * a.k;
        }
    }

    // Loads are unconditional (addresses clamped into the operands; what lies
    // past k is zeroed when the step is stored), so the compiler can count
    // them: with a branch around them it waits for every load in flight
    // before each step.
    auto load = [&](ST &st, uint32_t k0) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int chunk = tid + 256 * i;
            const uint32_t kc = min(k0 + (chunk & 15) * 8, a.k - 8);
            if constexpr (G == MM_DOWN) {
                const gbytes src = reinterpret_cast<gbytes>(reinterpret_cast<const GLOBAL float *>(xrow[i]) + kc);
                st.x[2 * i] = ld_u128(src);
                st.x[2 * i + 1] = ld_u128(src + 16);
            } else {
                st.x[i] = ld_u128(reinterpret_cast<gbytes>(xrow[i] + kc));
            }
        }
#pragma unroll
        for (int u = 0; u < WPT; u++) {  // 32-block formats: the last step may cover a partial 128
            const bool ok = k0 + 32 * wpc[u] < a.k;
            st.w[u] = PP::load(wr[u], ok ? k0 : 0, ok ? wpc[u] : 0);
        }
    };
    auto store = [&](const ST &st, uint32_t k0, int buf) {
        uint16_t *xs = lds + buf * XS;
        uint16_t *ws = lds + 2 * XS + buf * WS;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int chunk = tid + 256 * i, r = chunk >> 4, cc = (chunk & 15) * 8;
            const bool ok = xlive[i] && k0 + cc < a.k;
            uint4 v;
            if constexpr (G == MM_DOWN) {
                float f[8];
                __builtin_memcpy(f, &st.x[2 * i], 16);
                __builtin_memcpy(f + 4, &st.x[2 * i + 1], 16);
                const float g = xgain[i];
                v = make_uint4(pack2(operand_bits<false>(f[0] * g), operand_bits<false>(f[1] * g)),
                               pack2(operand_bits<false>(f[2] * g), operand_bits<false>(f[3] * g)),
                               pack2(operand_bits<false>(f[4] * g), operand_bits<false>(f[5] * g)),
                               pack2(operand_bits<false>(f[6] * g), operand_bits<false>(f[7] * g)));
            } else {
                v = st.x[i];
            }
            if (!ok) v = make_uint4(0, 0, 0, 0);
            if (G != MM_DOWN && !BF && !a.x_f16) {  // bf16 activations -> f16 operands
                uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; j++)
                    w4[j] = pack2(operand_bits<false>(bf16_bits_to_f32(w4[j] & 0xffffu)),
                                  operand_bits<false>(bf16_bits_to_f32(w4[j] >> 16)));
                v = make_uint4(w4[0], w4[1], w4[2], w4[3]);
            }
            *reinterpret_cast<uint4 *>(&xs[r * LD + cc]) = v;
        }
#pragma unroll
        for (int u = 0; u < WPT; u++) {
            uint32_t out[16], col0[4];
            if (k0 + 32 * wpc[u] < a.k) {
                PP::decode(st.w[u], k0, wpc[u], out, col0);
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) out[i] = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) col0[q] = 32 * wpc[u] + 8 * q;
            }
#pragma unroll
            for (int q = 0; q < 4; q++)
                *reinterpret_cast<uint4 *>(&ws[wrow[u] * LD + col0[q]]) =
                    make_uint4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
        }
    };
    auto mfma_step = [&](int buf) {
        const uint16_t *xs = lds + buf * XS;
        const uint16_t *ws = lds + 2 * XS + buf * WS;
        const int fr = lane & 15, fk = (lane >> 4) * 8;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            uint4 af[MI], bfm[NJ];
#pragma unroll
            for (int i = 0; i < MI; i++) af[i] = *reinterpret_cast<const uint4 *>(&xs[(tm + i * 16 + fr) * LD + kk + fk]);
#pragma unroll
            for (int j = 0; j < NJ; j++) bfm[j] = *reinterpret_cast<const uint4 *>(&ws[(tn + j * 16 + fr) * LD + kk + fk]);
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    if constexpr (BF) {
                        bf16x8 av, bv;
                        __builtin_memcpy(&av, &af[i], 16);
                        __builtin_memcpy(&bv, &bfm[j], 16);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[i][j], 0, 0, 0);
                    } else {
                        f16x8 av, bv;
                        __builtin_memcpy(&av, &af[i], 16);
                        __builtin_memcpy(&bv, &bfm[j], 16);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[i][j], 0, 0, 0);
                    }
                }
        }
    };

    // Prologue: step 0 in LDS buffer 0, step 1 in registers (s1), step 2
    // loading (s0).  Steps run in pairs, every one unconditionally: a step
    // past k stores zeros (its MFMAs add nothing), and loads past the last
    // step re-read it (never stored).
    ST s0, s1;
    const uint32_t steps = (a.k + BK - 1) / BK, last = (steps - 1) * BK;
    load(s0, 0);
    load(s1, min(BK, last));
    store(s0, 0, 0);
    load(s0, min(2 * BK, last));
    __syncthreads();
    for (uint32_t s = 0; s < steps; s += 2) {
        // even step s: compute buffer 0, stage step s+1 (s1) into buffer 1, prefetch s+3 into s1
        mfma_step(0);
        store(s1, (s + 1) * BK, 1);
        load(s1, min((s + 3) * BK, last));
        __syncthreads();
        // odd step s+1: compute buffer 1, stage step s+2 (s0) into buffer 0, prefetch s+4 into s0
        mfma_step(1);
        store(s0, (s + 2) * BK, 0);
        load(s0, min((s + 4) * BK, last));
        __syncthreads();
    }
    // C fragment: lane l holds column l % 16, rows 4 (l / 16) .. + 4.
    const int cc = lane & 15, cr = (lane >> 4) * 4;
    if constexpr (G == MM_GATE_UP) {
        // tiles j < NJ/2: gate columns, j + NJ/2: the same up columns
#pragma unroll
        for (int j = 0; j < NJ / 2; j++) {
            const uint32_t col = n0 + (wave & 1) * (BN / 4) + j * 16 + cc;
            if (col >= a.n) continue;
            const uint64_t bi = (uint64_t)expert * a.n + col;
            const float bg = a.bias ? round_bf16(a.bias[bi]) : 0.f;
            const float bu = a.bias2 ? round_bf16(a.bias2[bi] + (a.up_one ? 1.0f : 0.0f)) : (a.up_one ? 1.0f : 0.0f);
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const uint32_t r = tm + i * 16 + cr + v;
                    const float act = expert_activation(a.act, acc[i][j][v] + bg, acc[i][j + NJ / 2][v] + bu);
                    acc[i][j][v] = act;  // kept for the row maxima
                    if (r < rows) reinterpret_cast<float *>(a.y)[(uint64_t)(sorted0 + r) * a.n + col] = act;
                }
        }
        // Row maxima of |act| over this wavefront's columns (16 lanes share a
        // row), one atomic per row; NaN/Inf rows record 0x7f800000 or more.
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                uint32_t m = 0;
#pragma unroll
                for (int j = 0; j < NJ / 2; j++) {
                    const uint32_t col = n0 + (wave & 1) * (BN / 4) + j * 16 + cc;
                    if (col < a.n) m = max(m, __float_as_uint(acc[i][j][v]) & 0x7fffffffu);
                }
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o));
                const uint32_t r = tm + i * 16 + cr + v;
                if (cc == 0 && r < rows) atomicMax(&a.rowmax[sorted0 + r], m);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t col = n0 + tn + j * 16 + cc;
            if (col >= a.n) continue;
            const float b = a.bias ? round_bf16(a.bias[(uint64_t)expert * a.n + col]) : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t row = m0 + tm + i * 16 + cr + v;
                if (row >= (G == MM_DENSE ? a.m : rows)) continue;
                float r = acc[i][j][v];
                if constexpr (G == MM_DOWN) r /= row_gain(a.rowmax[sorted0 + row]);  // exact: a power of two
                r += b;
                const uint64_t o = (uint64_t)(G == MM_DOWN ? tile_route[row] : row) * a.n + col;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(r);
                else
                    reinterpret_cast<float *>(a.y)[o] = r;
            }
        }
}

typedef void (*MatmulFn)(u32x4, u32x4, u32x4, u32x2, MatmulArgs);

template <int BM, int BN>
static MatmulFn matmul_pick_tile(uint32_t fmt) {
    switch (fmt) {
    case OCO_MXFP4: return matmul_kernel<OCO_MXFP4, true, BM, BN>;
    case OCO_BF16: return matmul_kernel<OCO_BF16, true, BM, BN>;
    case OCO_Q8_0: return matmul_kernel<OCO_Q8_0, false, BM, BN>;
    case OCO_Q4_K: return matmul_kernel<OCO_Q4_K, false, BM, BN>;
    case OCO_Q5_K: return matmul_kernel<OCO_Q5_K, false, BM, BN>;
    case OCO_Q6_K: return matmul_kernel<OCO_Q6_K, false, BM, BN>;
    case OCO_Q4_0: return matmul_kernel<OCO_Q4_0, false, BM, BN>;
    case OCO_Q4_1: return matmul_kernel<OCO_Q4_1, false, BM, BN>;
    case OCO_F16: return matmul_kernel<OCO_F16, false, BM, BN>;
    case OCO_F32: return matmul_kernel<OCO_F32, false, BM, BN>;
    }
    return nullptr;
}

// Tile choice (the prefill half of Builder::dense, pipelines.rs:267-355):
// the largest tile that still gives every CU work.
static MatmulFn matmul_pick(uint32_t fmt, uint32_t m, uint32_t n, int &bm, int &bn) {
    int32_t ov[4];
    int choice = plan_override(OCO_KNOB_MATMUL_TILE, ov) ? ov[0] : -1;
    auto tiles = [&](int tm, int tn) { return (uint64_t)((m + tm - 1) / tm) * ((n + tn - 1) / tn); };
    if (choice < 0) choice = tiles(128, 128) >= 160 ? 3 : 1;  // measured: 128x128 once it fills the chip
    switch (choice) {
    case 3: bm = 128; bn = 128; return matmul_pick_tile<128, 128>(fmt);
    case 2: bm = 128; bn = 64; return matmul_pick_tile<128, 64>(fmt);
    case 1: bm = 64; bn = 64; return matmul_pick_tile<64, 64>(fmt);
    default: bm = 64; bn = 128; return matmul_pick_tile<64, 128>(fmt);
    }
}

// Grouped (routed-expert) prefill GEMMs on f16 operands -- the reference's
// half(w) x half(x) expert tiles (projections.metal:192-376).  Rows per tile
// BM = 32 or 64 (the route plan must use tile_rows = BM), 128 weight rows.
template <int BM, int G>
static MatmulFn grouped_pick(uint32_t fmt) {
    switch (fmt) {
    case OCO_Q4_K: return matmul_kernel<OCO_Q4_K, false, BM, 128, G>;
    case OCO_Q6_K: return matmul_kernel<OCO_Q6_K, false, BM, 128, G>;
    case OCO_Q8_0: return matmul_kernel<OCO_Q8_0, false, BM, 128, G>;
    case OCO_MXFP4: return matmul_kernel<OCO_MXFP4, false, BM, 128, G>;
    }
    return nullptr;
}

int grouped_matmul_launch(int mode, uint32_t fmt, const MatmulArgs &a, uint32_t bm, hipStream_t stream) {
    MatmulFn fn = nullptr;
    if (mode == MM_GATE_UP) fn = bm == 32 ? grouped_pick<32, MM_GATE_UP>(fmt) : grouped_pick<64, MM_GATE_UP>(fmt);
    if (mode == MM_DOWN) fn = bm == 32 ? grouped_pick<32, MM_DOWN>(fmt) : grouped_pick<64, MM_DOWN>(fmt);
    if (!fn) return fail(OCO_ERR_UNSUPPORTED, "experts: format %u has no grouped MFMA kernel", fmt);
    if (a.k % 32) return fail(OCO_ERR_INVALID, "experts: k=%u is not a multiple of 32", a.k);
    constexpr uint32_t BN = 128;
    const uint32_t cols = mode == MM_GATE_UP ? BN / 2 : BN;
    const dim3 grid((a.n + cols - 1) / cols, (a.routes + bm - 1) / bm + a.experts);
    const size_t lds = (size_t)2 * (bm + BN) * (128 + 8) * 2;
    if (lds > 64 * 1024)
        OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                          "hipFuncSetAttribute"));
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, stream, KPRE_ARGS(a), a);
    return launch_check("experts grouped matmul");
}

// ---- Dense prefill as a dequantize pass and a vendor GEMM --------------------
// At prefill sizes the fused tiles above decode every weight once per row
// tile and convert every activation once per column tile, on one wavefront
// per SIMD; the decode alone is about a third of their time.  Here each
// weight is decoded once, into the same f16 operand bits the fused tiles put
// in LDS (PrefillPiece::decode, the reference's half(w)), the bf16
// activations convert once to f16 (as the fused tiles convert them), and the
// product is a plain f16 GEMM with fp32 accumulation on hipBLASLt.  Its
// fp32 result then takes the fused tiles' epilogue: + bf16-rounded bias,
// then f32 or bf16 (weights.metal:24-33).

// Grid: weight blocks first (four (row, 2048-column chunk) tasks each, one
// per wavefront), then activation blocks (eight values per thread).
template <int FMT>
__global__ __launch_bounds__(256) void operand_kernel(const uint8_t *w, uint64_t row_bytes, uint32_t n, uint32_t k,
                                                      uint16_t *wo, const uint16_t *x, uint16_t *xo, uint64_t xchunks,
                                                      uint32_t wblocks) {
    if (blockIdx.x >= wblocks) {
        const uint64_t i = (uint64_t)(blockIdx.x - wblocks) * 256 + threadIdx.x;
        if (i >= xchunks) return;
        const uint4 v = *reinterpret_cast<const uint4 *>(x + 8 * i);
        uint32_t h[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++)
            h[j] = pack2(operand_bits<false>(bf16_bits_to_f32(h[j] & 0xffffu)),
                         operand_bits<false>(bf16_bits_to_f32(h[j] >> 16)));
        *reinterpret_cast<uint4 *>(xo + 8 * i) = make_uint4(h[0], h[1], h[2], h[3]);
        return;
    }
    // Each wavefront: one row's 2048-column chunk.  Lane = piece (step
    // lane / 4, piece lane % 4) decoded into the wavefront's LDS chunk, then
    // the chunk leaves in 16-byte stores at consecutive addresses across the
    // lanes (the pieces' own column runs are interleaved within a step).
    using PP = PrefillPiece<FMT, false>;
    __shared__ __attribute__((aligned(16))) uint16_t chunkbuf[4][2048];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, chunks = (k + 2047) / 2048;
    const uint64_t task = (uint64_t)blockIdx.x * 4 + wave;
    const bool live = task < (uint64_t)n * chunks;  // uniform per wavefront
    const uint32_t row = live ? (uint32_t)(task / chunks) : 0, ch = live ? (uint32_t)(task % chunks) : 0;
    const uint32_t k0 = ch * 2048 + lane / 4 * 128, c = lane % 4;
    uint16_t *lb = chunkbuf[wave];
    if (live && k0 + 32 * c < k) {  // 32-block formats: the last step may be partial
        const typename PP::Raw r = PP::load(gp(w) + (uint64_t)row * row_bytes, k0, c);
        uint32_t out[16], col0[4];
        PP::decode(r, k0, c, out, col0);
#pragma unroll
        for (int q = 0; q < 4; q++)
            *reinterpret_cast<uint4 *>(lb + (k0 - ch * 2048) + col0[q]) =
                make_uint4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
    }
    __syncthreads();
    if (!live) return;
    const uint32_t units = min(2048u, k - ch * 2048) / 8;
    uint16_t *dst = wo + (uint64_t)row * k + ch * 2048;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t u = lane + 64 * i;
        if (u < units) *reinterpret_cast<uint4 *>(dst + 8 * u) = *reinterpret_cast<const uint4 *>(lb + 8 * u);
    }
}

// The scaled Q4_0 / Q4_1 tiles' activations (q4_input_scales and the
// staging of matmul_q4_half: batch.metal:44-68, q4_tile.metal:44-49, 90-93):
// per row a power-of-two gain from the exponent e of its max |x|,
// 2^clamp(141 - e, -120, 120) (1 for a zero row), and the operands
// half(x * gain); `inv` receives 1 / gain for the epilogue.  One
// 256-thread workgroup per row.
__global__ __launch_bounds__(256) void row_gain_f16_kernel(const uint16_t *x, uint16_t *xo, float *inv, uint32_t k) {
    __shared__ float peaks[4];
    const uint16_t *xr = x + (uint64_t)blockIdx.x * k;
    uint16_t *orow = xo + (uint64_t)blockIdx.x * k;
    float peak = 0.f;
    for (uint32_t i = threadIdx.x; i < k; i += 256) peak = fmaxf(peak, fabsf(bf16_bits_to_f32(xr[i])));
    for (int o = 32; o >= 1; o >>= 1) peak = fmaxf(peak, __shfl_xor(peak, o));
    if ((threadIdx.x & 63) == 0) peaks[threadIdx.x >> 6] = peak;
    __syncthreads();
    peak = fmaxf(fmaxf(peaks[0], peaks[1]), fmaxf(peaks[2], peaks[3]));
    const int e = (int)((__float_as_uint(peak) >> 23) & 255u);
    const int shift = peak == 0.f ? 0 : min(max(141 - e, -120), 120);
    const float gain = __uint_as_float((uint32_t)(127 + shift) << 23);
    if (threadIdx.x == 0) inv[blockIdx.x] = __uint_as_float((uint32_t)(127 - shift) << 23);
    for (uint32_t i = threadIdx.x; i < k; i += 256) orow[i] = operand_bits<false>(bf16_bits_to_f32(xr[i]) * gain);
}

// y[m, n] = acc (* 1 / row gain) + bf16(bias), as f32 or bf16: four columns
// per thread.
__global__ __launch_bounds__(256) void gemm_epilogue_kernel(const float *acc, const float *bias, const float *inv_gain,
                                                            void *y, bool y_bf16, uint32_t n, uint64_t quads) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= quads) return;
    const uint32_t col = (uint32_t)(4 * i % n);
    const float g = inv_gain ? inv_gain[4 * i / n] : 1.0f;
    const float4 v = *reinterpret_cast<const float4 *>(acc + 4 * i);
    float r[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) r[j] = r[j] * g + (bias ? round_bf16(bias[col + j]) : 0.f);
    if (y_bf16)
        *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(y) + 4 * i) =
            make_uint2(pack2(f32_to_bf16_bits(r[0]), f32_to_bf16_bits(r[1])),
                       pack2(f32_to_bf16_bits(r[2]), f32_to_bf16_bits(r[3])));
    else
        *reinterpret_cast<float4 *>(reinterpret_cast<float *>(y) + 4 * i) = make_float4(r[0], r[1], r[2], r[3]);
}

// One GEMM shape's hipBLASLt objects, built once per (device, m, n, k): D
// [n rows of m, column-major] = W^T X with W the f16 operands as k x n
// column-major (the weight rows as stored) and X as k x m.
struct BlasPlan {
    hipblasLtHandle_t handle = nullptr;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo;
    uint64_t ws = 0;
    bool ok = false;
};
constexpr uint64_t BLAS_WS_MAX = 32ull << 20;
static std::mutex g_blas_lock;
static std::map<int, hipblasLtHandle_t> g_blas_handles;
static std::map<std::tuple<int, uint32_t, uint32_t, uint32_t>, BlasPlan> g_blas_plans;

// The plan for this shape on the current device; ok == false when hipBLASLt
// offers no algorithm (the fused tiles then run).
static const BlasPlan &blas_plan(uint32_t m, uint32_t n, uint32_t k) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> hold(g_blas_lock);
    const auto key = std::make_tuple(dev, m, n, k);
    auto it = g_blas_plans.find(key);
    if (it != g_blas_plans.end()) return it->second;
    BlasPlan &pl = g_blas_plans[key];
    // hipblasLtCreate ends the process when no device is present: ask first.
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices <= 0) return pl;
    hipblasLtHandle_t &h = g_blas_handles[dev];
    if (!h && hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) {
        h = nullptr;
        return pl;
    }
    pl.handle = h;
    const int32_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescCreate(&pl.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t)) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n)) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&pl.a, HIP_R_16F, k, n, k) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&pl.b, HIP_R_16F, k, m, k) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&pl.d, HIP_R_32F, n, m, n) != HIPBLAS_STATUS_SUCCESS)
        return pl;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return pl;
    const uint64_t wsmax = BLAS_WS_MAX;
    hipblasLtMatmulHeuristicResult_t res;
    int count = 0;
    if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsmax, sizeof(wsmax)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulAlgoGetHeuristic(h, pl.desc, pl.a, pl.b, pl.d, pl.d, pref, 1, &res, &count) ==
            HIPBLAS_STATUS_SUCCESS &&
        count > 0 && res.state == HIPBLAS_STATUS_SUCCESS && res.workspaceSize <= BLAS_WS_MAX) {
        pl.algo = res.algo;
        pl.ws = res.workspaceSize;
        pl.ok = true;
    }
    hipblasLtMatmulPreferenceDestroy(pref);
    return pl;
}

static bool vendor_format(uint32_t format) {
    switch (format) {
    case OCO_Q4_0: case OCO_Q4_1: case OCO_Q8_0: case OCO_Q4_K: case OCO_Q5_K: case OCO_Q6_K: case OCO_F16: case OCO_F32:
        return true;
    }
    return false;
}

// The vendor path from 32 activation rows, where prefill starts (measured
// on the box at 32..256 rows: as fast or faster for Q4_K 12288 x 4096, 2-3x
// for Q8_0 4096 x 4096 and Q6_K 4096 x 12288), unless the
// OCO_KNOB_MATMUL_VENDOR override chooses.
// The reference scales Q4_0 / Q4_1 activation rows by a power-of-two gain
// when the matrix has more than 1024 outputs (pipelines.rs:286-288); only
// the vendor path implements it, so those shapes take it at every tiled m.
// (f16 activations, which the reference does not take, are used as given.)
static bool q4_gain(uint32_t format, uint32_t n, oco_dtype x_dtype) {
    return (format == OCO_Q4_0 || format == OCO_Q4_1) && n > 1024 && x_dtype == OCO_DT_BF16;
}

static bool use_vendor(uint32_t format, uint32_t m, uint32_t n, oco_dtype x_dtype) {
    if (!vendor_format(format)) return false;
    int32_t ov[4];
    if (plan_override(OCO_KNOB_MATMUL_VENDOR, ov)) return ov[0] != 0;
    return m >= 32 || q4_gain(format, n, x_dtype);
}

struct VendorLayout {
    uint64_t w, x, d, gain, blas, total;  // byte offsets in the workspace, and its size
};
static VendorLayout vendor_layout(uint32_t format, oco_dtype x_dtype, uint32_t m, uint32_t n, uint32_t k, uint64_t blas_ws) {
    auto al = [](uint64_t b) { return (b + 255) & ~255ull; };
    VendorLayout v;
    v.w = 0;
    v.x = v.w + (format == OCO_F16 ? 0 : al((uint64_t)n * k * 2));
    v.d = v.x + (x_dtype == OCO_DT_F16 && !q4_gain(format, n, x_dtype) ? 0 : al((uint64_t)m * k * 2));
    v.gain = v.d + al((uint64_t)m * n * 4);
    v.blas = v.gain + (q4_gain(format, n, x_dtype) ? al((uint64_t)m * 4) : 0);
    v.total = v.blas + blas_ws;
    return v;
}

template <int FMT>
static void operand_launch(const void *w, uint64_t row_bytes, uint32_t n, uint32_t k, uint16_t *wo, const void *x,
                           uint16_t *xo, uint64_t xchunks, hipStream_t stream) {
    const uint64_t tasks = (uint64_t)n * ((k + 2047) / 2048);  // (row, 2048-column chunk), four per workgroup
    const uint32_t wblocks = FMT == OCO_F16 ? 0 : (uint32_t)((tasks + 3) / 4);
    const uint32_t xblocks = (uint32_t)((xchunks + 255) / 256);
    hipLaunchKernelGGL(operand_kernel<FMT>, dim3(wblocks + xblocks), dim3(256), 0, stream, (const uint8_t *)w, row_bytes,
                       n, k, wo, (const uint16_t *)x, xo, xchunks, wblocks);
}

static int vendor_matmul(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y, oco_dtype y_dtype,
                         const float *bias, const oco_matrix *p, const BlasPlan &pl, void *workspace,
                         uint64_t workspace_bytes, hipStream_t stream) {
    const uint32_t m = p->m, n = p->n, k = p->k;
    const VendorLayout v = vendor_layout(format, x_dtype, m, n, k, pl.ws);
    if (!workspace || workspace_bytes < v.total)
        return fail(OCO_ERR_INVALID, "oco_matmul_ws: workspace of %llu bytes, need %llu",
                    (unsigned long long)workspace_bytes, (unsigned long long)v.total);
    uint8_t *ws = (uint8_t *)workspace;
    const bool gain = q4_gain(format, n, x_dtype);
    uint16_t *wo = format == OCO_F16 ? nullptr : (uint16_t *)(ws + v.w);
    uint16_t *xo = x_dtype == OCO_DT_F16 && !gain ? nullptr : (uint16_t *)(ws + v.x);
    float *inv = gain ? (float *)(ws + v.gain) : nullptr;
    const uint64_t xchunks = xo && !gain ? (uint64_t)m * k / 8 : 0;
    if (gain) {
        hipLaunchKernelGGL(row_gain_f16_kernel, dim3(m), dim3(256), 0, stream, (const uint16_t *)x, xo, inv, k);
        OCO_TRY(launch_check("oco_matmul: row gains"));
    }
    if (wo || xchunks) {
        const uint64_t rb = oco_row_bytes(format, k);
        switch (format) {
#define CASE(F) case F: operand_launch<F>(w, rb, n, k, wo, x, xo, xchunks, stream); break;
            CASE(OCO_Q4_0) CASE(OCO_Q4_1) CASE(OCO_Q8_0) CASE(OCO_Q4_K) CASE(OCO_Q5_K) CASE(OCO_Q6_K) CASE(OCO_F16)
            CASE(OCO_F32)
#undef CASE
        }
        OCO_TRY(launch_check("oco_matmul: operand pass"));
    }
    // f32 output without bias or gain is the GEMM's own output (when aligned for it)
    const bool direct = y_dtype == OCO_DT_F32 && !(p->has_bias && bias) && !gain && ((uintptr_t)y & 15) == 0;
    float *acc = direct ? (float *)y : (float *)(ws + v.d);
    const float alpha = 1.0f, beta = 0.0f;
    const hipblasStatus_t st = hipblasLtMatmul(pl.handle, pl.desc, &alpha, wo ? (const void *)wo : w, pl.a,
                                               xo ? (const void *)xo : x, pl.b, &beta, acc, pl.d, acc, pl.d, &pl.algo,
                                               pl.ws ? ws + v.blas : nullptr, pl.ws, stream);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail(OCO_ERR_HIP, "oco_matmul: hipblasLtMatmul status %d", (int)st);
    if (!direct) {
        const uint64_t quads = (uint64_t)m * n / 4;
        hipLaunchKernelGGL(gemm_epilogue_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, acc,
                           p->has_bias ? bias : nullptr, inv, y, y_dtype == OCO_DT_BF16, n, quads);
        OCO_TRY(launch_check("oco_matmul: epilogue"));
    }
    return OCO_OK;
}

uint64_t mx_workspace_bytes(uint32_t m, uint32_t n, uint32_t k);
int mx_matmul_launch(const void *w, const void *x, void *y, bool y_bf16, const float *bias, uint32_t m, uint32_t n,
                     uint32_t k, void *workspace, hipStream_t stream, bool presplit = false);
int mx_norm_split_launch(void *x, const void *res, const float *w, void *y, uint32_t m, uint32_t k, float epsilon,
                         bool full_layer, void *workspace, hipStream_t stream);

// MXFP4 goes to the block-scaled FP8 x FP4 MFMA unless the
// OCO_KNOB_MX_PREFILL_OFF override says otherwise (comparisons against the
// f16 decode path).
static bool use_mx(uint32_t format) {
    int32_t ov[4];
    return format == OCO_MXFP4 && !(plan_override(OCO_KNOB_MX_PREFILL_OFF, ov) && ov[0]);
}

static int matmul_check(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, const void *y,
                        oco_dtype y_dtype, const float *bias, const oco_matrix *p) {
    if (!p || !w || !x || !y) return fail(OCO_ERR_INVALID, "oco_matmul: null argument");
    uint32_t e, bb;
    OCO_TRY(oco_block_layout(format, &e, &bb));
    if (p->k == 0 || p->k % 32 || p->k % e)
        return fail(OCO_ERR_INVALID, "oco_matmul: k=%u must be a multiple of 32 and of the block", p->k);
    if (p->experts > 1) return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: routed rows go through oco_experts_apply");
    if (p->has_bias && !bias) return fail(OCO_ERR_INVALID, "oco_matmul: has_bias without bias");
    if (x_dtype != OCO_DT_BF16 && x_dtype != OCO_DT_F16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: activations must be bf16 or f16");
    if (x_dtype == OCO_DT_F16 && (format == OCO_MXFP4 || format == OCO_BF16))
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: MXFP4/BF16 weights take bf16 activations");
    if (y_dtype != OCO_DT_F32 && y_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: output must be f32 or bf16");
    return OCO_OK;
}

static int matmul_decode_launch(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                                oco_dtype y_dtype, const float *bias, const oco_matrix *p, hipStream_t stream) {
    int bm = 128, bn = 64;
    MatmulFn fn = matmul_pick(format, p->m, p->n, bm, bn);
    if (!fn) return fail(OCO_ERR_UNSUPPORTED, "oco_matmul: format %u", format);
    MatmulArgs a;
    a.w = (const uint8_t *)w;
    a.x = x;
    a.y = y;
    a.bias = p->has_bias ? bias : nullptr;
    a.m = p->m;
    a.n = p->n;
    a.k = p->k;
    a.row_bytes = (uint32_t)oco_row_bytes(format, p->k);
    a.x_f16 = x_dtype == OCO_DT_F16;
    a.y_bf16 = y_dtype == OCO_DT_BF16;
    dim3 grid((p->n + bn - 1) / bn, (p->m + bm - 1) / bm);
    const size_t lds = (size_t)2 * (bm + bn) * (128 + 8) * 2;
    if (lds > 64 * 1024)
        OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                          "hipFuncSetAttribute"));
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, stream, KPRE_ARGS(a), a);
    return launch_check("oco_matmul");
}

}  // namespace oco

using namespace oco;

// Builder::dense's vector_rows (pipelines.rs:271-283): a product of at most
// this many rows runs the decode matvec on each row (exact weights, fp32
// accumulation), as DenseMatrix::apply does (compute/matrix.rs:174-200).
// F32 matrices of at most 128 outputs stay on it at every m: the reference
// keeps them in exact fp32 either way (vector, or its tensor tiles' fp32
// staging), which only the matvec does here.
static uint32_t vector_rows(uint32_t format, uint32_t k, uint32_t n) {
    switch (format) {
    case OCO_Q4_0:
    case OCO_Q4_1: return 4;
    case OCO_Q5_K: return k == 6144 && n == 5120 ? 4 : 1;
    case OCO_Q8_0: return k == 2880 && n == 512 ? 128 : (k == 2880 && n == 4096) || (k == 4096 && n == 2880) ? 4 : 1;
    case OCO_F32: return n <= 128 ? 0xffffffffu : 1;
    }
    return 1;
}
static bool as_matvec(uint32_t format, oco_dtype x_dtype, const oco_matrix *p) {
    return x_dtype == OCO_DT_BF16 && p->m <= vector_rows(format, p->k, p->n) && p->m <= 65535;  // the matvec's row limit
}

// The vendor path needs n % 4 == 0 (the epilogue's four columns per thread).
static const BlasPlan *vendor_plan(uint32_t format, oco_dtype x_dtype, const oco_matrix *p) {
    if (!use_vendor(format, p->m, p->n, x_dtype) || p->n % 4 || p->m == 0 || p->n == 0) return nullptr;
    const BlasPlan &pl = blas_plan(p->m, p->n, p->k);
    return pl.ok ? &pl : nullptr;
}

extern "C" uint64_t oco_matmul_workspace(uint32_t format, oco_dtype x_dtype, const oco_matrix *p) {
    if (!p || as_matvec(format, x_dtype, p)) return 0;
    if (use_mx(format)) return mx_workspace_bytes(p->m, p->n, p->k);
    if (const BlasPlan *pl = vendor_plan(format, x_dtype, p)) return vendor_layout(format, x_dtype, p->m, p->n, p->k, pl->ws).total;
    return 0;
}

extern "C" int oco_matmul_ws(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                             oco_dtype y_dtype, const float *bias, const oco_matrix *p, void *workspace,
                             uint64_t workspace_bytes, oco_stream stream) {
    OCO_TRY(matmul_check(format, w, x, x_dtype, y, y_dtype, bias, p));
    if (p->m == 0 || p->n == 0) return OCO_OK;
    if (as_matvec(format, x_dtype, p)) return oco_matvec(format, w, x, x_dtype, y, y_dtype, bias, nullptr, p, stream);
    if (use_mx(format)) {
        const uint64_t need = mx_workspace_bytes(p->m, p->n, p->k);
        if (!workspace || workspace_bytes < need)
            return fail(OCO_ERR_INVALID, "oco_matmul_ws: workspace of %llu bytes, need %llu",
                        (unsigned long long)workspace_bytes, (unsigned long long)need);
        return mx_matmul_launch(w, x, y, y_dtype == OCO_DT_BF16, p->has_bias ? bias : nullptr, p->m, p->n, p->k,
                                workspace, (hipStream_t)stream);
    }
    // Operands the GEMM reads as given (F16 weights, f16 activations) must be
    // 16-byte aligned for it; otherwise the fused tiles run.
    const bool aligned = (format != OCO_F16 || ((uintptr_t)w & 15) == 0) &&
                         (x_dtype != OCO_DT_F16 || ((uintptr_t)x & 15) == 0);
    if (const BlasPlan *pl = aligned ? vendor_plan(format, x_dtype, p) : nullptr)
        return vendor_matmul(format, w, x, x_dtype, y, y_dtype, bias, p, *pl, workspace, workspace_bytes,
                             (hipStream_t)stream);
    return matmul_decode_launch(format, w, x, x_dtype, y, y_dtype, bias, p, (hipStream_t)stream);
}

extern "C" int oco_matmul(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                          oco_dtype y_dtype, const float *bias, const oco_matrix *p, oco_stream stream) {
    OCO_TRY(matmul_check(format, w, x, x_dtype, y, y_dtype, bias, p));
    if (p->m == 0 || p->n == 0) return OCO_OK;
    if (as_matvec(format, x_dtype, p)) return oco_matvec(format, w, x, x_dtype, y, y_dtype, bias, nullptr, p, stream);
    const uint64_t need = oco_matmul_workspace(format, x_dtype, p);
    if (!need) return matmul_decode_launch(format, w, x, x_dtype, y, y_dtype, bias, p, (hipStream_t)stream);
    void *ws = nullptr;
    OCO_TRY(hip_check(hipMallocAsync(&ws, need, (hipStream_t)stream), "oco_matmul: hipMallocAsync"));
    const int rc = oco_matmul_ws(format, w, x, x_dtype, y, y_dtype, bias, p, ws, need, stream);
    const int rf = hip_check(hipFreeAsync(ws, (hipStream_t)stream), "oco_matmul: hipFreeAsync");
    return rc != OCO_OK ? rc : rf;
}

static int norm_split_check(const char *who, uint32_t rows, uint32_t n, uint64_t split_bytes) {
    if (n == 0 || n % 32) return fail(OCO_ERR_INVALID, "%s: n=%u is not whole 32-blocks", who, n);
    if (n > 65536) return fail(OCO_ERR_UNSUPPORTED, "%s: n=%u past 65536 (the row is staged in LDS)", who, n);
    if (rows > 0x7fffffe0u) return fail(OCO_ERR_INVALID, "%s: %u rows", who, rows);
    const uint64_t need = mx_workspace_bytes(rows, 0, n);
    if (split_bytes < need)
        return fail(OCO_ERR_INVALID, "%s: split buffer of %llu bytes, need %llu", who,
                    (unsigned long long)split_bytes, (unsigned long long)need);
    return OCO_OK;
}

extern "C" int oco_norm_mx_split(const void *x, const float *norm_w, void *y, uint32_t rows, uint32_t n,
                                 float epsilon, int full_layer, void *split, uint64_t split_bytes,
                                 oco_stream stream) {
    if (rows == 0) return OCO_OK;
    if (!x || !norm_w || !split) return fail(OCO_ERR_INVALID, "oco_norm_mx_split: null pointer");
    OCO_TRY(norm_split_check("oco_norm_mx_split", rows, n, split_bytes));
    return mx_norm_split_launch(const_cast<void *>(x), nullptr, norm_w, y, rows, n, epsilon, full_layer != 0, split,
                                (hipStream_t)stream);
}

extern "C" int oco_add_norm_mx_split(void *x, const void *y, const float *norm_w, void *out, uint32_t rows,
                                     uint32_t n, float epsilon, int full_layer, void *split, uint64_t split_bytes,
                                     oco_stream stream) {
    if (rows == 0) return OCO_OK;
    if (!x || !y || !norm_w || !split) return fail(OCO_ERR_INVALID, "oco_add_norm_mx_split: null pointer");
    OCO_TRY(norm_split_check("oco_add_norm_mx_split", rows, n, split_bytes));
    return mx_norm_split_launch(x, y, norm_w, out, rows, n, epsilon, full_layer != 0, split, (hipStream_t)stream);
}

extern "C" int oco_matmul_mx_split(const void *w, const void *split, uint64_t split_bytes, void *y, oco_dtype y_dtype,
                                   const float *bias, const oco_matrix *p, oco_stream stream) {
    if (!p || !w || !split || !y) return fail(OCO_ERR_INVALID, "oco_matmul_mx_split: null argument");
    if (p->k == 0 || p->k % 32) return fail(OCO_ERR_INVALID, "oco_matmul_mx_split: k=%u must be a multiple of 32", p->k);
    if (p->experts > 1) return fail(OCO_ERR_UNSUPPORTED, "oco_matmul_mx_split: routed rows go through oco_experts_apply");
    if (p->has_bias && !bias) return fail(OCO_ERR_INVALID, "oco_matmul_mx_split: has_bias without bias");
    if (y_dtype != OCO_DT_F32 && y_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matmul_mx_split: output must be f32 or bf16");
    if (p->m == 0 || p->n == 0) return OCO_OK;
    const uint64_t need = mx_workspace_bytes(p->m, p->n, p->k);
    if (split_bytes < need)
        return fail(OCO_ERR_INVALID, "oco_matmul_mx_split: split buffer of %llu bytes, need %llu",
                    (unsigned long long)split_bytes, (unsigned long long)need);
    return mx_matmul_launch(w, nullptr, y, y_dtype == OCO_DT_BF16, p->has_bias ? bias : nullptr, p->m, p->n, p->k,
                            const_cast<void *>(split), (hipStream_t)stream, true);
}
