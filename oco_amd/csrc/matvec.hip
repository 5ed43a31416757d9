// Decode matvec: GGUF dequantization fused into y = W x for batch-1 decode
// and for routed (per-expert) rows.  Replaces oco's vector kernels
// (shaders/matrix/vector.metal:66-394, q8-dot.metal:39-86,
// mxfp4-dot.metal:9-45, projections.metal:140-182) and the kernel choice of
// Builder::vector_kernel (src/weights/pipelines.rs:227-265).
//
// Geometry.  A 256-thread workgroup is four wavefronts.  A wavefront owns R
// output rows; KS wavefronts may split one row group's K range (partials
// meet in LDS), so a workgroup covers (4/KS)*R rows.  Inside a wavefront, P
// lanes share a GGUF block and each lane decodes one piece, so a step reads
// 64/P consecutive blocks of each of the R rows as one contiguous span.  The
// lane's activation values are loaded once per step and reused by all R
// rows.  The K loop is unrolled so several independent weight loads per lane
// are in flight, which is what a weight stream at HBM speed needs.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "stream.h"
#include "norm.h"

namespace oco {

struct MatvecArgs {
    const uint8_t *w;
    const void *x;
    void *y;
    const float *bias;
    const uint32_t *ids;
    oco_matrix p;
    uint64_t row_bytes;
    int y_bf16;
};

template <int FMT, typename XT, int R, int KS>
__global__ __launch_bounds__(256) void matvec_kernel(MatvecArgs a) {
    using F = Piece<FMT>;
    constexpr int WAVES = 4, GROUPS = WAVES / KS;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int group = wave / KS, split = wave % KS;
    const oco_matrix &p = a.p;
    const uint32_t row0 = (blockIdx.x * GROUPS + group) * R;
    if (row0 >= p.n) {  // whole wavefront past the end (only when KS == 1: no barrier below)
        if (KS == 1) return;
    }
    const uint32_t route = blockIdx.y;
    const uint32_t expert = p.experts > 1 ? a.ids[route] : 0;
    const uint32_t input = (p.experts > 1 && !p.route_major) ? route / p.routes : route;
    const XT *xr = reinterpret_cast<const XT *>(a.x) + (uint64_t)input * p.k;

    // One buffer resource over this wavefront's R rows; rows past n read as
    // zero (out of the resource's range) and are never stored.
    const uint32_t live = row0 < p.n ? min((uint32_t)R, p.n - row0) : 0u;
    const WSrc src(a.w + ((uint64_t)expert * p.n + row0) * a.row_bytes, (uint64_t)live * a.row_bytes);
    const uint32_t rb = (uint32_t)a.row_bytes;

    const uint32_t blocks = p.k / F::BLOCK;
    constexpr int BPS = 64 / F::P;  // blocks per wavefront step
    const int piece = lane % F::P;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

#pragma unroll 2
    for (uint32_t b = (uint32_t)split * BPS + lane / F::P; b < blocks; b += BPS * KS) {
        typename F::X xv;
        F::load_x(xr, b, piece, xv);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += F::dot(src, r * rb + b * F::BYTES, piece, xv);
    }

#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);

    if (KS > 1) {
        __shared__ float partial[WAVES][R];
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) partial[wave][r] = acc[r];
        }
        __syncthreads();
        if (split != 0) return;
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < KS; j++) s += partial[group * KS + j][r];
            acc[r] = s;
        }
    }

    if (lane < R) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < R; r++)
            if (lane == r) v = acc[r];
        uint32_t row = row0 + lane;
        if (row < p.n) {
            if (p.has_bias)
                v += round_bf16(a.bias[(uint64_t)expert * p.n + row] + (p.has_bias == 2 ? 1.0f : 0.0f));
            uint64_t o = (uint64_t)route * p.n + row;
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(v);
            else
                reinterpret_cast<float *>(a.y)[o] = v;
        }
    }
}


// ---------------------------------------------------------------------------
// Streaming matvec (Q8_0, Q4_0, Q4_1, Q4_K, Q5_K, Q6_K, MXFP4).
//
// Persistent workgroups of four wavefronts loop over row groups.  The
// activation vector is staged once per workgroup into LDS in piece-major
// order (see stream.h).  Each wavefront owns a tile of 2R row slices: it
// streams the tile's bytes from HBM with aligned 16-byte buffer loads into
// registers (GGUF blocks are 17, 34, 144 or 210 bytes, so per-lane block
// loads would be unaligned and split), deposits them in its private LDS
// tile, issues the loads of its next tile, and decodes the current tile from
// LDS while those loads are in flight.  Half-wavefront h decodes rows
// h*R .. h*R+R-1 of the tile, lane c taking pieces c, c+32, ...; the
// activation registers of a piece serve all R rows.  KS wavefronts may split
// a row group's K range (partials meet in LDS).
// ---------------------------------------------------------------------------
struct StreamArgs {
    const uint8_t *w;
    const void *x;
    void *y;
    const float *bias;
    const uint32_t *ids;
    oco_matrix p;
    uint64_t row_bytes;
    uint32_t y_bf16;
    uint32_t ks;            // wavefronts sharing a row set (K slices)
    uint32_t slice_blocks;  // blocks per K slice
    uint32_t ngroups;       // row groups per route
    // Fused RMS norm of the (bf16) input row during staging: 0 off, 1 norm,
    // 2 norm with full_layer rounding (elementwise.metal:6-28).
    uint32_t norm_mode;
    float norm_eps;
    const float *norm_w;
};

// Loads per tile row: enough 16-byte chunks for NPL pieces per lane of a
// half-wavefront (32 lanes) plus the row's misalignment.
template <int FMT, int NPL>
struct StreamShape {
    static constexpr int BYTES_MAX = NPL * 32 * Tile<FMT>::BYTES / Tile<FMT>::P + 32;
    static constexpr int LPR = (BYTES_MAX + 1023) / 1024;
};

template <int FMT, typename XT, int R, int NPL>
__global__ __launch_bounds__(256) void stream_kernel(StreamArgs a) {
    using T = Tile<FMT>;
    constexpr int LPR = StreamShape<FMT, NPL>::LPR;
    constexpr int ROWS = 2 * R;                 // tile rows per wavefront
    constexpr int TILE = ROWS * LPR * 1024;     // LDS bytes per wavefront tile
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const oco_matrix &p = a.p;
    const uint32_t PT = p.k / T::BLOCK * T::P;  // pieces per full row
    float4 *xs4 = reinterpret_cast<float4 *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + (size_t)p.k * 4);
    uint8_t *tiles = smem + (size_t)p.k * 4 + (size_t)T::NSUM * PT * 4;
    float *part = reinterpret_cast<float *>(tiles + 4 * TILE);

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, c = lane & 31;
    const uint32_t ks = a.ks, sets = 4 / ks, set = wave / ks, sl = wave % ks;
    const uint32_t route = blockIdx.y;
    const uint32_t expert = p.experts > 1 ? a.ids[route] : 0;
    const uint32_t input = (p.experts > 1 && !p.route_major) ? route / p.routes : route;
    const uint32_t rows_per_group = sets * ROWS;

    // One buffer resource over this expert's rows, based 16-byte aligned.
    // Buffer loads zero any access that straddles num_records, so the range
    // extends to the 16-byte boundary after the last byte: that chunk lies in
    // the same page as the tensor's last byte, and bytes past the end of the
    // last row are never decoded.
    const uint8_t *ebase = a.w + (uint64_t)expert * p.n * a.row_bytes;
    const uintptr_t base_al = (uintptr_t)ebase & ~(uintptr_t)15;
    const uint32_t shift = (uint32_t)((uintptr_t)ebase & 15);
    const uint64_t span = ((uint64_t)p.n * a.row_bytes + shift + 15) & ~15ull;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)base_al, 0, (uint32_t)(span > 0xffffffffull ? 0xffffffffull : span), 0x00020000);

    // This wavefront's K slice.
    const uint32_t nblocks = p.k / T::BLOCK;
    const uint32_t b0 = min(sl * a.slice_blocks, nblocks);
    const uint32_t b1 = min(b0 + a.slice_blocks, nblocks);
    const uint32_t slice_bytes = (b1 - b0) * T::BYTES;
    const uint32_t pieces = (b1 - b0) * T::P;

    u32x4 regs[ROWS * LPR];
    // Byte offset of tile row i of group g from base_al.
    auto row_offset = [&](uint32_t g, int i) -> uint32_t {
        const uint32_t row = g * rows_per_group + set * ROWS + i;
        return (uint32_t)(shift + (uint64_t)row * a.row_bytes + (uint64_t)b0 * T::BYTES);
    };
    auto issue = [&](uint32_t g) {
#pragma unroll
        for (int i = 0; i < ROWS; i++) {
            const uint32_t off = row_offset(g, i), start = off & ~15u, need = (off & 15u) + slice_bytes;
#pragma unroll
            for (int u = 0; u < LPR; u++) {
                const uint32_t j = (uint32_t)(u * 64 + lane);
                regs[i * LPR + u] = 16 * j < need
                                        ? __builtin_amdgcn_raw_buffer_load_b128(rs, start + 16 * j, 0, 2 /* nontemporal */)
                                        : u32x4{0, 0, 0, 0};
            }
        }
    };

    uint32_t g = blockIdx.x;
    if (g < a.ngroups) issue(g);

    // Stage x (f32) in piece-major order, then the per-piece sums.  With a
    // fused norm, x is the bf16 row before normalisation: every workgroup
    // takes its inverse RMS (the same routine and order as oco_norm, so the
    // staged values equal oco_norm's output bit for bit) and normalises
    // while staging.
    {
        const XT *xr = reinterpret_cast<const XT *>(a.x) + (uint64_t)input * p.k;
        float inv = 1.f;
        if (a.norm_mode) inv = block_inv_rms(reinterpret_cast<const uint16_t *>(xr), p.k, a.norm_eps, part);
        // Four loads in flight per thread before any store: x arrives in one
        // memory round trip, not one per loop iteration.
        for (uint32_t f0 = threadIdx.x; f0 < p.k / 4; f0 += 4 * 256) {
            float v[4][4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t f = f0 + 256 * u;
                if (f < p.k / 4) {
                    if constexpr (sizeof(XT) == 4) {
                        const float4 t = reinterpret_cast<const float4 *>(xr)[f];
                        v[u][0] = t.x; v[u][1] = t.y; v[u][2] = t.z; v[u][3] = t.w;
                    } else {
                        const uint2 t = reinterpret_cast<const uint2 *>(xr)[f];
                        v[u][0] = __uint_as_float(t.x << 16); v[u][1] = __uint_as_float(t.x & 0xffff0000u);
                        v[u][2] = __uint_as_float(t.y << 16); v[u][3] = __uint_as_float(t.y & 0xffff0000u);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t f = f0 + 256 * u;
                if (f < p.k / 4) {
                    if (a.norm_mode) {
                        float wn[4];
                        if (((uintptr_t)a.norm_w & 15u) == 0) {
                            const float4 t = reinterpret_cast<const float4 *>(a.norm_w)[f];
                            wn[0] = t.x; wn[1] = t.y; wn[2] = t.z; wn[3] = t.w;
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; e++) wn[e] = a.norm_w[4 * f + e];
                        }
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            v[u][e] = bf16_bits_to_f32(norm_value_bits(v[u][e], inv, wn[e], a.norm_mode == 2));
                    }
                    uint32_t pp, tt;
                    T::map(f, pp, tt);
                    xs4[tt * PT + pp] = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
                }
            }
        }
        if constexpr (T::NSUM > 0) {
            __syncthreads();
            for (uint32_t pp = threadIdx.x; pp < PT; pp += 256) {
                float xv[32], sv[T::NSUM > 0 ? T::NSUM : 1];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    float4 q = xs4[t * PT + pp];
                    xv[4 * t] = q.x; xv[4 * t + 1] = q.y; xv[4 * t + 2] = q.z; xv[4 * t + 3] = q.w;
                }
                T::sums(xv, sv);
#pragma unroll
                for (int j = 0; j < T::NSUM; j++) xsum[j * PT + pp] = sv[j];
            }
        }
        __syncthreads();
    }

    uint8_t *tile = tiles + (size_t)wave * TILE;
    for (; g < a.ngroups; g += gridDim.x) {
#pragma unroll
        for (int i = 0; i < ROWS * LPR; i++) reinterpret_cast<u32x4 *>(tile)[i * 64 + lane] = regs[i];
        uint32_t rbase[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = half * R + r;
            rbase[r] = i * LPR * 1024 + (row_offset(g, i) & 15u);
        }
        const uint32_t gnext = g + gridDim.x;
        if (gnext < a.ngroups) issue(gnext);

        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
        for (int s = 0; s < NPL; s++) {
            const uint32_t pl = c + 32 * s;
            if (pl < pieces) {
                const uint32_t pg = b0 * T::P + pl;  // piece index in the full row
                float xv[32], sv[T::NSUM > 0 ? T::NSUM : 1];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    float4 q = xs4[t * PT + pg];
                    xv[4 * t] = q.x; xv[4 * t + 1] = q.y; xv[4 * t + 2] = q.z; xv[4 * t + 3] = q.w;
                }
#pragma unroll
                for (int j = 0; j < T::NSUM; j++) sv[j] = xsum[j * PT + pg];
                const uint32_t blk = pl / T::P, cc = pl % T::P;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    typename T::Raw raw = T::load(tile + rbase[r] + blk * T::BYTES, cc);
                    acc[r] += tile_dot<FMT>(raw, xv, sv, cc);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = half_sum(acc[r]);

        const uint32_t row0 = g * rows_per_group + set * ROWS + half * R;
        if (ks > 1) {
            if (c == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) part[(wave * 2 + half) * R + r] = acc[r];
            }
            __syncthreads();
            if (sl == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    float v = 0.f;
                    for (uint32_t j = 0; j < ks; j++) v += part[((wave + j) * 2 + half) * R + r];
                    acc[r] = v;
                }
            }
            __syncthreads();
        }
        if (sl == 0 && c < R) {
            float v = acc[0];
#pragma unroll
            for (int r = 1; r < R; r++)
                if (c == (uint32_t)r) v = acc[r];
            const uint32_t row = row0 + c;
            if (row < p.n) {
                if (p.has_bias)
                    v += round_bf16(a.bias[(uint64_t)expert * p.n + row] + (p.has_bias == 2 ? 1.0f : 0.0f));
                const uint64_t o = (uint64_t)route * p.n + row;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(v);
                else
                    reinterpret_cast<float *>(a.y)[o] = v;
            }
        }
    }
}

typedef void (*StreamFn)(StreamArgs);

template <int FMT, typename XT, int R>
static StreamFn stream_pick_npl(int npl) {
    switch (npl) {
    case 1: return stream_kernel<FMT, XT, R, 1>;
    case 2: return stream_kernel<FMT, XT, R, 2>;
    case 3: return stream_kernel<FMT, XT, R, 3>;
    case 4: return stream_kernel<FMT, XT, R, 4>;
    }
    return nullptr;
}

template <int FMT>
static int stream_lpr(int npl) {
    switch (npl) {
    case 1: return StreamShape<FMT, 1>::LPR;
    case 2: return StreamShape<FMT, 2>::LPR;
    case 3: return StreamShape<FMT, 3>::LPR;
    case 4: return StreamShape<FMT, 4>::LPR;
    }
    return 0;
}

template <typename XT>
static StreamFn stream_pick_format(uint32_t fmt, int r, int npl, int &lpr) {
    switch (fmt) {
#define F(FM)                                                                                   \
    case FM:                                                                                    \
        lpr = stream_lpr<FM>(npl);                                                              \
        return r == 1 ? stream_pick_npl<FM, XT, 1>(npl) : stream_pick_npl<FM, XT, 2>(npl);
        F(OCO_Q8_0) F(OCO_MXFP4) F(OCO_Q4_K) F(OCO_Q6_K) F(OCO_Q4_0) F(OCO_Q4_1) F(OCO_Q5_K)
#undef F
    }
    return nullptr;
}

static bool streamable(uint32_t fmt) {
    return fmt == OCO_Q8_0 || fmt == OCO_MXFP4 || fmt == OCO_Q4_K || fmt == OCO_Q6_K || fmt == OCO_Q4_0 ||
           fmt == OCO_Q4_1 || fmt == OCO_Q5_K;
}

struct StreamPlan {
    int r, ks, wg_per_cu;
};

// Geometry for the streaming kernel: R rows per half-wavefront, KS
// wavefronts per K range, workgroups per CU (the analogue of
// Builder::vector_kernel's table, pipelines.rs:227-265).
static StreamPlan stream_plan(uint32_t fmt, uint32_t k, uint32_t n, uint32_t m) {
    int32_t ov[4];
    if (plan_override(OCO_KNOB_STREAM_PLAN, ov) == 3 && ov[0] > 0) return {ov[0], ov[1], ov[2]};
    uint64_t row_bytes = oco_row_bytes(fmt, k);
    int ks = row_bytes > 6144 ? 4 : row_bytes > 3072 ? 2 : 1;
    (void)m;
    // Three workgroups per CU only pay off on long streams (measured: the
    // 510 MB Q6_K lm_head 3.6 -> 4.2 TB/s; 8-41 MB matrices lose with it).
    const int wg = (uint64_t)n * row_bytes > (128ull << 20) ? 3 : 2;
    return {1, ks, wg};
}

typedef void (*MatvecFn)(MatvecArgs);

template <int FMT, typename XT>
static MatvecFn pick(int r, int ks) {
    if (r == 4 && ks == 1) return matvec_kernel<FMT, XT, 4, 1>;
    if (r == 2 && ks == 1) return matvec_kernel<FMT, XT, 2, 1>;
    if (r == 4 && ks == 4) return matvec_kernel<FMT, XT, 4, 4>;
    if (r == 2 && ks == 4) return matvec_kernel<FMT, XT, 2, 4>;
    if (r == 1 && ks == 4) return matvec_kernel<FMT, XT, 1, 4>;
    if (r == 2 && ks == 2) return matvec_kernel<FMT, XT, 2, 2>;
    return matvec_kernel<FMT, XT, 1, 1>;
}

template <typename XT>
static MatvecFn pick_format(uint32_t fmt, int r, int ks) {
    switch (fmt) {
    case OCO_Q8_0: return pick<OCO_Q8_0, XT>(r, ks);
    case OCO_MXFP4: return pick<OCO_MXFP4, XT>(r, ks);
    case OCO_Q4_K: return pick<OCO_Q4_K, XT>(r, ks);
    case OCO_Q5_K: return pick<OCO_Q5_K, XT>(r, ks);
    case OCO_Q6_K: return pick<OCO_Q6_K, XT>(r, ks);
    case OCO_Q4_0: return pick<OCO_Q4_0, XT>(r, ks);
    case OCO_Q4_1: return pick<OCO_Q4_1, XT>(r, ks);
    case OCO_F32: return pick<OCO_F32, XT>(r, ks);
    case OCO_F16: return pick<OCO_F16, XT>(r, ks);
    case OCO_BF16: return pick<OCO_BF16, XT>(r, ks);
    }
    return nullptr;
}

// Geometry table: the analogue of Builder::vector_kernel's per-format
// choice (pipelines.rs:227-265), keyed on the number of wavefront-row
// groups the matrix yields so small matrices still put many independent
// loads in flight on every CU.
struct MatvecPlan {
    int r, ks;
};

MatvecPlan matvec_plan(uint32_t fmt, uint32_t k, uint32_t n, uint32_t m) {
    int32_t ov[4];
    if (plan_override(OCO_KNOB_MATVEC_PLAN, ov) == 2 && ov[0] > 0) return {ov[0], ov[1]};
    uint32_t e, bb;
    oco_block_layout(fmt, &e, &bb);
    uint64_t rows = (uint64_t)n * m;
    uint64_t blocks = k / e;
    // Lanes per block and thus blocks per wavefront step.
    int P = (fmt == OCO_Q8_0) ? 4 : (fmt == OCO_Q4_K || fmt == OCO_Q5_K || fmt == OCO_Q6_K) ? 8
            : (fmt == OCO_MXFP4 || fmt == OCO_Q4_0 || fmt == OCO_Q4_1) ? 2 : 1;
    uint64_t steps = (blocks + 64 / P - 1) / (64 / P);
    // Enough wavefronts for ~16 per CU on 256 CUs before splitting K.
    if (rows >= 16384 * 4) return {4, 1};
    if (rows >= 16384 * 2) return {2, 1};
    if (steps >= 4) return rows >= 8192 ? MatvecPlan{2, 4} : MatvecPlan{1, 4};
    return {2, 1};
}

}  // namespace oco

using namespace oco;

struct NormSpec {
    const float *w;
    float epsilon;
    int full_layer;
};

// oco_matvec, optionally with the RMS norm of each bf16 input row fused
// into the streaming kernel's staging (norm != nullptr, x bf16).  Formats
// without a streaming kernel normalise into a stream-ordered temporary first.
static int matvec_impl(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                       oco_dtype y_dtype, const float *bias, const uint32_t *ids, const oco_matrix *p,
                       const NormSpec *norm, oco_stream stream) {
    if (!p || !w || !x || !y) return fail(OCO_ERR_INVALID, "oco_matvec: null argument");
    uint32_t e, bb;
    OCO_TRY(oco_block_layout(format, &e, &bb));
    uint32_t align = e;
    if (format == OCO_F32) align = 4;
    if (format == OCO_F16 || format == OCO_BF16) align = 8;
    if (p->k == 0 || p->k % align)
        return fail(OCO_ERR_INVALID, "oco_matvec: k=%u is not a multiple of %u", p->k, align);
    if (p->n == 0 || p->m == 0) return OCO_OK;
    if (p->m > 65535) return fail(OCO_ERR_INVALID, "oco_matvec: m=%u exceeds 65535 routes", p->m);
    if (p->experts > 1 && !ids) return fail(OCO_ERR_INVALID, "oco_matvec: routed matrix needs ids");
    if (p->has_bias && !bias) return fail(OCO_ERR_INVALID, "oco_matvec: has_bias without bias");
    if (p->experts > 1 && !p->route_major && p->routes == 0)
        return fail(OCO_ERR_INVALID, "oco_matvec: routes must be > 0");
    if (x_dtype != OCO_DT_F32 && x_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: activations must be f32 or bf16");
    if (y_dtype != OCO_DT_F32 && y_dtype != OCO_DT_BF16)
        return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: output must be f32 or bf16");
    const int routed_f32 = p->experts > 1 && !p->route_major;
    int32_t plain[4];
    if (streamable(format) && !(plan_override(OCO_KNOB_MATVEC_PLAIN, plain) && plain[0])) {
        static int cus = 0;
        if (!cus) {
            int dev = 0;
            hipGetDevice(&dev);
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
            if (cus <= 0) cus = 256;
        }
        uint32_t be, bbytes;
        oco_block_layout(format, &be, &bbytes);
        const uint32_t P = (format == OCO_Q4_K || format == OCO_Q5_K || format == OCO_Q6_K) ? 8 : 1;
        const uint32_t nblocks = p->k / be;
        StreamPlan sp = stream_plan(format, p->k, p->n, p->m);
        if (sp.ks != 1 && sp.ks != 2 && sp.ks != 4) sp.ks = 1;
        if (sp.r != 1 && sp.r != 2) sp.r = 1;
        uint32_t slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
        int npl = (int)((slice_blocks * P + 31) / 32);
        while (npl > 4 && sp.ks < 4) {  // widen the K split until a lane's pieces fit
            sp.ks *= 2;
            slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
            npl = (int)((slice_blocks * P + 31) / 32);
        }
        int lpr = 0;
        StreamFn fn = npl > 4 ? nullptr
                    : x_dtype == OCO_DT_F32 ? stream_pick_format<float>(format, sp.r, npl, lpr)
                                            : stream_pick_format<bf16_t>(format, sp.r, npl, lpr);
        if (fn) {
            StreamArgs a;
            a.w = (const uint8_t *)w;
            a.x = x;
            a.y = y;
            a.bias = bias;
            a.ids = ids;
            a.p = *p;
            a.row_bytes = oco_row_bytes(format, p->k);
            a.y_bf16 = (y_dtype == OCO_DT_BF16) && !routed_f32;
            a.ks = sp.ks;
            a.slice_blocks = slice_blocks;
            a.norm_mode = norm ? (norm->full_layer ? 2u : 1u) : 0u;
            a.norm_eps = norm ? norm->epsilon : 0.f;
            a.norm_w = norm ? norm->w : nullptr;
            const uint32_t rows_per_group = (4 / sp.ks) * 2 * sp.r;
            a.ngroups = (p->n + rows_per_group - 1) / rows_per_group;
            const uint32_t nsum = (format == OCO_Q8_0 || format == OCO_Q4_0 || format == OCO_Q4_1) ? 1
                                  : (format == OCO_Q4_K || format == OCO_Q5_K)                    ? 2
                                  : format == OCO_Q6_K                                            ? 4
                                                                                                  : 0;
            const size_t tile = (size_t)2 * sp.r * lpr * 1024;
            const size_t lds = (size_t)p->k * 4 + (size_t)nsum * (p->k / 32) * 4 + 4 * tile + 32 * sizeof(float);
            if (lds > 160 * 1024)
                return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: k=%u needs %zu bytes of LDS", p->k, lds);
            if (lds > 64 * 1024)
                OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn,
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                                  "hipFuncSetAttribute"));
            const uint32_t grid = std::min<uint32_t>(a.ngroups, (uint32_t)(cus * sp.wg_per_cu));
            hipLaunchKernelGGL(fn, dim3(grid, p->m), dim3(256), lds, (hipStream_t)stream, a);
            return launch_check("oco_matvec");
        }
    }
    if (norm) {  // no streaming kernel: normalise the input rows, then the plain matvec
        const uint32_t in_rows =
            (p->experts > 1 && !p->route_major) ? (p->m + p->routes - 1) / p->routes : p->m;
        void *tmp = nullptr;
        const size_t bytes = (size_t)in_rows * p->k * 2;
        OCO_TRY(hip_check(hipMallocAsync(&tmp, bytes, (hipStream_t)stream), "oco_matvec_norm: hipMallocAsync"));
        int rc = oco_norm(x, norm->w, tmp, in_rows, p->k, norm->epsilon, norm->full_layer, stream);
        if (rc == OCO_OK) rc = matvec_impl(format, w, tmp, OCO_DT_BF16, y, y_dtype, bias, ids, p, nullptr, stream);
        const int rc2 = hip_check(hipFreeAsync(tmp, (hipStream_t)stream), "oco_matvec_norm: hipFreeAsync");
        return rc != OCO_OK ? rc : rc2;
    }
    MatvecPlan plan = matvec_plan(format, p->k, p->n, p->m);
    MatvecFn fn = x_dtype == OCO_DT_F32 ? pick_format<float>(format, plan.r, plan.ks)
                                        : pick_format<bf16_t>(format, plan.r, plan.ks);
    if (!fn) return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: format %u", format);
    MatvecArgs a;
    a.w = (const uint8_t *)w;
    a.x = x;
    a.y = y;
    a.bias = bias;
    a.ids = ids;
    a.p = *p;
    a.row_bytes = oco_row_bytes(format, p->k);
    // Routed, non-route-major outputs are always f32 (vector.metal:142-146).
    a.y_bf16 = (y_dtype == OCO_DT_BF16) && !(p->experts > 1 && !p->route_major);
    uint32_t rows_per_group = (4 / plan.ks) * plan.r;
    dim3 grid((p->n + rows_per_group - 1) / rows_per_group, p->m);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    return launch_check("oco_matvec");
}

extern "C" int oco_matvec(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                          oco_dtype y_dtype, const float *bias, const uint32_t *ids,
                          const oco_matrix *p, oco_stream stream) {
    return matvec_impl(format, w, x, x_dtype, y, y_dtype, bias, ids, p, nullptr, stream);
}

extern "C" int oco_matvec_norm(uint32_t format, const void *w, const void *x, const float *norm_w, float epsilon,
                               int full_layer, void *y, oco_dtype y_dtype, const float *bias,
                               const uint32_t *ids, const oco_matrix *p, oco_stream stream) {
    if (!norm_w) return fail(OCO_ERR_INVALID, "oco_matvec_norm: null norm weights");
    const NormSpec n{norm_w, epsilon, full_layer};
    return matvec_impl(format, w, x, OCO_DT_BF16, y, y_dtype, bias, ids, p, &n, stream);
}
