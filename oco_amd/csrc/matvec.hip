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

// The values the first loads depend on come first, as scalars: the command
// processor preloads leading scalar kernel arguments into SGPRs (built with
// -amdgpu-kernarg-preload-count), so the weight and activation loads issue
// without waiting for a kernarg fetch; the rest of StreamArgs is read behind
// them.
template <int FMT>
struct DirectOk {
    static constexpr bool value = false;
};
template <>
struct DirectOk<OCO_Q4_K> {
    static constexpr bool value = true;
};
template <>
struct DirectOk<OCO_Q5_K> {
    static constexpr bool value = true;
};


// DIRECT (Q4_K / Q5_K on a 16-byte aligned base, whose blocks are then all
// 16-byte aligned): each lane loads its pieces' 16-byte chunks straight into
// registers, with no LDS tile and no realignment.
// Where the streaming kernel's activations come from.
enum { XS_STAGED = 0, XS_NORM = 1, XS_NORM_FULL = 2, XS_REG = 3 };

template <int FMT, typename XT, int NPL, int XS, bool DIRECT>
__global__ __launch_bounds__(256) void stream_kernel(const uint8_t *w_, const void *x_, uint32_t row_bytes_,
                                                     uint32_t n_, uint32_t k_, uint32_t mode_, uint32_t slice_,
                                                     uint32_t ngroups_, uint32_t experts_, uint32_t routes_,
                                                     StreamArgs a) {
    a.w = w_;
    a.x = x_;
    a.row_bytes = row_bytes_;
    a.p.n = n_;
    a.p.k = k_;
    // mode_: bits 0-1 log2 of the K split
    const uint32_t ks_log2 = mode_ & 3u;
    a.ks = 1u << ks_log2;
    a.slice_blocks = slice_;
    a.ngroups = ngroups_;
    // routes_ carries route_major in its top bit
    a.p.experts = experts_;
    a.p.routes = routes_ & 0x7fffffffu;
    a.p.route_major = routes_ >> 31;
    using T = Tile<FMT>;
    constexpr int LPR = StreamShape<FMT, NPL>::LPR;
    constexpr int ROWS = 2;                     // tile rows per wavefront (one per half-wavefront)
    constexpr int TILE = DIRECT ? 0 : ROWS * LPR * 1024;  // LDS bytes per wavefront tile
    constexpr int NS = T::NSUM > 0 ? T::NSUM : 1;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const oco_matrix &p = a.p;
    const uint32_t PT = p.k / T::BLOCK * T::P;  // pieces per full row
    // LDS: [x f32, piece-major][per-piece sums] (staged x only), the
    // wavefronts' tiles, the K-split partials.
    const size_t xbytes = XS != XS_REG ? (size_t)p.k * 4 + (size_t)T::NSUM * PT * 4 : 0;
    float4 *xs4 = reinterpret_cast<float4 *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + (size_t)p.k * 4);
    uint8_t *tiles = smem + xbytes;
    float *part = reinterpret_cast<float *>(tiles + 4 * TILE);

    // The wavefront index is uniform: as a scalar, every row and group offset
    // below is SALU work.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, half = lane >> 5, c = lane & 31;
    const uint32_t ks = a.ks, sets = 4 >> ks_log2, set = wave >> ks_log2, sl = wave & (ks - 1);
    const uint32_t route = blockIdx.y;
    const uint32_t expert = p.experts > 1 ? a.ids[route] : 0;
    const uint32_t input = (p.experts > 1 && !p.route_major) ? route / p.routes : route;
    const uint32_t rows_per_group = sets * ROWS;

    // This expert's rows, from the 16-byte boundary at or below their start.
    const uint8_t *ebase = a.w + (uint64_t)expert * p.n * a.row_bytes;
    const uintptr_t base_al = (uintptr_t)ebase & ~(uintptr_t)15;
    const uint32_t shift = (uint32_t)((uintptr_t)ebase & 15);

    // This wavefront's K slice.
    const uint32_t nblocks = p.k / T::BLOCK;
    const uint32_t b0 = min(sl * a.slice_blocks, nblocks);
    const uint32_t b1 = min(b0 + a.slice_blocks, nblocks);
    const uint32_t slice_bytes = (b1 - b0) * T::BYTES;
    const uint32_t pieces = (b1 - b0) * T::P;

    // Two groups' loads in flight per wavefront: a ring of two register sets.
    u32x4 ra[DIRECT ? 1 : ROWS * LPR], rb[DIRECT ? 1 : ROWS * LPR];
    // DIRECT: a ring of three sets of pieces; a set is refilled right after
    // its group is decoded, so two groups stay in flight with no copies.
    typename T::Raw da[DIRECT ? NPL : 1], db[DIRECT ? NPL : 1], dc[DIRECT ? NPL : 1];
    __amdgpu_buffer_rsrc_t rall;
    if constexpr (DIRECT) {
        // The range ends at a whole dword: a block's dword-aligned span may
        // end up to three bytes past the tensor, and a dword that straddles
        // the range end would read as zero (the same page holds it).
        const uint64_t bytes = ((uint64_t)p.n * a.row_bytes + 3) & ~3ull;
        rall = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(ebase), 0,
                                                 (uint32_t)(bytes > 0xffffffffull ? 0xffffffffull : bytes), 0x00020000);
    }
    // DIRECT: this half-wavefront's row of group g (rows past n read row n - 1
    // and are never stored), pieces past the slice read the last piece.
    auto issue_direct = [&](uint32_t g, typename T::Raw *dst) __attribute__((always_inline)) {
        if constexpr (DIRECT) {
            const uint32_t row = min(g * rows_per_group + set * ROWS + half, p.n - 1);
            const uint32_t roff = row * (uint32_t)a.row_bytes;
#pragma unroll
            for (int s = 0; s < NPL; s++) {
                const uint32_t pl = min(c + 32u * s, pieces - 1), blk = b0 + pl / T::P, cc = pl % T::P;
                dst[s] = T::direct(rall, roff + blk * T::BYTES, cc);
            }
        }
    };
    // Byte offset of tile row i of group g from base_al.
    auto row_offset = [&](uint32_t g, int i) -> uint32_t {
        const uint32_t row = g * rows_per_group + set * ROWS + i;
        return (uint32_t)(shift + (uint64_t)row * a.row_bytes + (uint64_t)b0 * T::BYTES);
    };
    // One buffer resource per tile row, from the 16-byte boundary below the
    // row's slice to the end of the slice rounded up to a whole chunk: the
    // loads need no per-lane range test, since chunks past the range read as
    // zero without touching memory (the range check covers the per-lane
    // offset; the scalar offset stays 0).  The rounded-up chunk ends within
    // the 16 bytes after the slice, in the same page as its last byte.  Rows
    // past n get an empty range.
    auto issue = [&](uint32_t g, u32x4 *regs) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < ROWS; i++) {
            const uint32_t row = g * rows_per_group + set * ROWS + i;
            const uint32_t off = row_offset(g, i), start = off & ~15u;
            const uint32_t need = row < p.n ? (off & 15u) + slice_bytes : 0u;
            const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(base_al + start), 0, (need + 15u) & ~15u, 0x00020000);
#pragma unroll
            for (int u = 0; u < LPR; u++)
                regs[i * LPR + u] = __builtin_amdgcn_raw_buffer_load_b128(rr, 16 * (64 * u + lane), 0, 2 /* nontemporal */);
        }
    };

    // Each lane keeps the activations (and sums) of its pieces -- c + 32 s of
    // this wavefront's K slice, the same for every row group -- in registers.
    float xv[NPL][32], sv[NPL][NS];
    // The first 1024 float4 of x are requested before the weights: they come
    // from L2 and arrive while the weights are still in flight (loads return
    // in issue order).  A fused norm reads x itself first, so it does not.
    const XT *xr = reinterpret_cast<const XT *>(a.x) + (uint64_t)input * p.k;
    float xpre[4][4];
    if constexpr (XS == XS_STAGED) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t f = threadIdx.x + 256 * u;
            if (f < p.k / 4) {
                if constexpr (sizeof(XT) == 4) {
                    const float4 t = reinterpret_cast<const float4 *>(xr)[f];
                    xpre[u][0] = t.x; xpre[u][1] = t.y; xpre[u][2] = t.z; xpre[u][3] = t.w;
                } else {
                    const uint2 t = reinterpret_cast<const uint2 *>(xr)[f];
                    xpre[u][0] = __uint_as_float(t.x << 16); xpre[u][1] = __uint_as_float(t.x & 0xffff0000u);
                    xpre[u][2] = __uint_as_float(t.y << 16); xpre[u][3] = __uint_as_float(t.y & 0xffff0000u);
                }
            }
        }
    }

    // XS_REG: every lane reads its pieces' activations straight from memory
    // (L2 after the first workgroups), before the weights: no LDS for x, no
    // workgroup barrier.  The reads are 16-byte vectors at a stride of one
    // piece, so for short rows staging through LDS is cheaper.
    if constexpr (XS == XS_REG) {
#pragma unroll
        for (int s = 0; s < NPL; s++) {
            const uint32_t pg = b0 * T::P + min(c + 32u * s, pieces > 0 ? pieces - 1 : 0u);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const uint32_t f = T::unmap(pg, t);
                if constexpr (sizeof(XT) == 4) {
                    const float4 q = reinterpret_cast<const float4 *>(xr)[f];
                    xv[s][4 * t] = q.x; xv[s][4 * t + 1] = q.y; xv[s][4 * t + 2] = q.z; xv[s][4 * t + 3] = q.w;
                } else {
                    const uint2 q = reinterpret_cast<const uint2 *>(xr)[f];
                    xv[s][4 * t] = __uint_as_float(q.x << 16); xv[s][4 * t + 1] = __uint_as_float(q.x & 0xffff0000u);
                    xv[s][4 * t + 2] = __uint_as_float(q.y << 16); xv[s][4 * t + 3] = __uint_as_float(q.y & 0xffff0000u);
                }
            }
        }
    }

    const uint32_t G = gridDim.x, g0 = blockIdx.x;
    if constexpr (DIRECT) {
        if (g0 < a.ngroups) issue_direct(g0, da);
        if (g0 + G < a.ngroups) issue_direct(g0 + G, db);
        if (g0 + 2 * G < a.ngroups) issue_direct(g0 + 2 * G, dc);
    } else {
        if (g0 < a.ngroups) issue(g0, ra);
        if (g0 + G < a.ngroups) issue(g0 + G, rb);
    }

    // Staged: x (f32) to LDS in piece-major order, then the per-piece sums.  With a
    // fused norm, x is the bf16 row before normalisation: every workgroup
    // takes its inverse RMS (the same routine and order as oco_norm, so the
    // staged values equal oco_norm's output bit for bit) and normalises
    // while staging.
    if constexpr (XS != XS_REG) {
        float inv = 1.f;
        if constexpr (XS == XS_NORM || XS == XS_NORM_FULL) inv = block_inv_rms(reinterpret_cast<const uint16_t *>(xr), p.k, a.norm_eps, part);
        for (uint32_t f0 = threadIdx.x; f0 < p.k / 4; f0 += 4 * 256) {
            float v[4][4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t f = f0 + 256 * u;
                if (XS == XS_STAGED && f0 == threadIdx.x) {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[u][e] = xpre[u][e];
                } else if (f < p.k / 4) {
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
                    if constexpr (XS == XS_NORM || XS == XS_NORM_FULL) {
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
                            v[u][e] = bf16_bits_to_f32(norm_value_bits(v[u][e], inv, wn[e], XS == XS_NORM_FULL));
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
                float xt[32], st[NS];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    float4 q = xs4[t * PT + pp];
                    xt[4 * t] = q.x; xt[4 * t + 1] = q.y; xt[4 * t + 2] = q.z; xt[4 * t + 3] = q.w;
                }
                T::sums(xt, st);
#pragma unroll
                for (int j = 0; j < T::NSUM; j++) xsum[j * PT + pp] = st[j];
            }
        }
        __syncthreads();
    }
    if constexpr (XS == XS_REG) {
#pragma unroll
        for (int s = 0; s < NPL; s++) T::sums(xv[s], sv[s]);
    } else {
#pragma unroll
        for (int s = 0; s < NPL; s++) {
            const uint32_t pg = b0 * T::P + min(c + 32u * s, pieces > 0 ? pieces - 1 : 0u);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float4 q = xs4[t * PT + pg];
                xv[s][4 * t] = q.x; xv[s][4 * t + 1] = q.y; xv[s][4 * t + 2] = q.z; xv[s][4 * t + 3] = q.w;
            }
#pragma unroll
            for (int j = 0; j < T::NSUM; j++) sv[s][j] = xsum[j * PT + pg];
        }
    }

    uint8_t *tile = tiles + (size_t)wave * TILE;
    // One row group: its registers to this wavefront's LDS tile, the loads of
    // the group two ahead into the freed registers, then the decode.
    auto group = [&](uint32_t g, u32x4 *regs, typename T::Raw *dr) __attribute__((always_inline)) {
        float acc = 0.f;
        if constexpr (DIRECT) {
#pragma unroll
            for (int s = 0; s < NPL; s++) {
                const uint32_t pl = c + 32 * s;
                if (pl < pieces) acc += tile_dot<FMT>(dr[s], xv[s], sv[s], pl % T::P);
            }
            if (g + 3 * G < a.ngroups) issue_direct(g + 3 * G, dr);
        } else {
#pragma unroll
            for (int i = 0; i < ROWS * LPR; i++) reinterpret_cast<u32x4 *>(tile)[i * 64 + lane] = regs[i];
            const uint32_t rbase = half * LPR * 1024 + (row_offset(g, half) & 15u);
            if (g + 2 * G < a.ngroups) issue(g + 2 * G, regs);
#pragma unroll
            for (int s = 0; s < NPL; s++) {
                const uint32_t pl = c + 32 * s;
                if (pl < pieces) {
                    const uint32_t blk = pl / T::P, cc = pl % T::P;
                    typename T::Raw raw = T::load(tile + rbase + blk * T::BYTES, cc);
                    acc += tile_dot<FMT>(raw, xv[s], sv[s], cc);
                }
            }
        }
        acc = half_sum(acc);

        const uint32_t row = g * rows_per_group + set * ROWS + half;
        if (ks > 1) {
            if (c == 0) part[wave * 2 + half] = acc;
            __syncthreads();
            if (sl == 0) {
                float v = 0.f;
                for (uint32_t j = 0; j < ks; j++) v += part[(wave + j) * 2 + half];
                acc = v;
            }
            __syncthreads();
        }
        if (sl == 0 && c == 0 && row < p.n) {
            float v = acc;
            if (p.has_bias) v += round_bf16(a.bias[(uint64_t)expert * p.n + row] + (p.has_bias == 2 ? 1.0f : 0.0f));
            const uint64_t o = (uint64_t)route * p.n + row;
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(v);
            else
                reinterpret_cast<float *>(a.y)[o] = v;
        }
    };
    if constexpr (DIRECT) {
        for (uint32_t g = g0; g < a.ngroups; g += 3 * G) {
            group(g, ra, da);
            if (g + G < a.ngroups) group(g + G, rb, db);
            if (g + 2 * G < a.ngroups) group(g + 2 * G, ra, dc);
        }
    } else {
        for (uint32_t g = g0; g < a.ngroups; g += 2 * G) {
            group(g, ra, da);
            if (g + G < a.ngroups) group(g + G, rb, db);
        }
    }
}

typedef void (*StreamFn)(const uint8_t *, const void *, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
                         uint32_t, uint32_t, StreamArgs);

template <int FMT, typename XT, int XS, bool DIRECT>
static StreamFn stream_pick_npl_d(int npl) {
    switch (npl) {
    case 1: return stream_kernel<FMT, XT, 1, XS, DIRECT>;
    case 2: return stream_kernel<FMT, XT, 2, XS, DIRECT>;
    case 3: return stream_kernel<FMT, XT, 3, XS, DIRECT>;
    case 4: return stream_kernel<FMT, XT, 4, XS, DIRECT>;
    }
    return nullptr;
}
template <int FMT, typename XT, int XS>
static StreamFn stream_pick_npl(int npl, bool direct) {
    if constexpr (DirectOk<FMT>::value)
        if (direct) return stream_pick_npl_d<FMT, XT, XS, true>(npl);
    return stream_pick_npl_d<FMT, XT, XS, false>(npl);
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

// xs: an XS_* source of x; the fused norms only with bf16 rows.
template <typename XT>
static StreamFn stream_pick_format(uint32_t fmt, int xs, int npl, bool direct, int &lpr) {
    switch (fmt) {
#define F(FM)                                                                                   \
    case FM:                                                                                    \
        lpr = stream_lpr<FM>(npl);                                                              \
        if constexpr (sizeof(XT) == 2) {                                                        \
            if (xs == XS_NORM) return stream_pick_npl<FM, XT, XS_NORM>(npl, direct);            \
            if (xs == XS_NORM_FULL) return stream_pick_npl<FM, XT, XS_NORM_FULL>(npl, direct);  \
        }                                                                                       \
        if (xs == XS_REG) return stream_pick_npl<FM, XT, XS_REG>(npl, direct);                  \
        return xs == XS_STAGED ? stream_pick_npl<FM, XT, XS_STAGED>(npl, direct) : nullptr;
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
static StreamPlan stream_plan(uint32_t fmt, uint32_t k, uint32_t n, uint32_t m, bool fused_norm) {
    int32_t ov[4];
    if (plan_override(OCO_KNOB_STREAM_PLAN, ov) == 3 && ov[0] > 0) return {ov[0], ov[1], ov[2]};
    uint64_t row_bytes = oco_row_bytes(fmt, k);
    int ks = row_bytes > 6144 ? 4 : row_bytes > 3072 ? 2 : 1;
    // Q8_0 decodes at one conversion and one FMA per weight, so one
    // wavefront per row set holds up while its pieces fit a lane (k <= 4096;
    // measured, 4096 x 4096: 7.28 -> 6.55 us against a K split of 2).  The
    // K-quants lose without the split (lm_head 111 -> 148 us, Q4_K
    // 12288 x 4096 10.9 -> 14.5 us).
    if (fmt == OCO_Q8_0 && k / 32 <= 128) ks = 1;
    (void)m;
    // Workgroups per CU, measured: three pay off on long streams (the 510 MB
    // Q6_K lm_head 3.6 -> 4.2 TB/s) and for MXFP4 and Q4_K at every measured
    // size (the headline 5760 x 2880 5.30 -> 5.17 us, its 720 row groups one
    // per workgroup; Q4_K 12288 x 4096 10.86 -> 10.66 us); mid-size Q5_K and
    // Q6_K lose with three (12288 x 4096 13.6 -> 16.0 us, 4096 x 12288
    // 14.3 -> 15.7 us), and Q8_0 4096 x 4096 is level.  A fused norm, which
    // every workgroup repeats while staging, keeps two (Qwen3-8B's norm +
    // ffn_up + ffn_gate: 24.60 -> 24.17 us against three).
    const bool long_stream = (uint64_t)n * row_bytes > (128ull << 20);
    const int wg = long_stream || (!fused_norm && (fmt == OCO_MXFP4 || fmt == OCO_Q4_K)) ? 3 : 2;
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
    // The streaming kernel reads x in 16-byte (f32) or 8-byte (bf16) vectors.
    const bool x_vec = ((uintptr_t)x & (x_dtype == OCO_DT_F32 ? 15u : 7u)) == 0;
    if (streamable(format) && x_vec && !(plan_override(OCO_KNOB_MATVEC_PLAIN, plain) && plain[0])) {
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
        StreamPlan sp = stream_plan(format, p->k, p->n, p->m, norm != nullptr);
        if (sp.ks != 1 && sp.ks != 2 && sp.ks != 4) sp.ks = 1;
        uint32_t slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
        int npl = (int)((slice_blocks * P + 31) / 32);
        while (npl > 4 && sp.ks < 4) {  // widen the K split until a lane's pieces fit
            sp.ks *= 2;
            slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
            npl = (int)((slice_blocks * P + 31) / 32);
        }
        // Q4_K / Q5_K blocks are whole 16-byte chunks: on a 16-byte aligned
        // base every lane loads its own pieces (OCO_KNOB_STREAM_DIRECT 0 turns
        // this off).
        int32_t dov[4];
        const bool direct = (format == OCO_Q4_K || format == OCO_Q5_K) && ((uintptr_t)w & 15u) == 0 &&
                            !(plan_override(OCO_KNOB_STREAM_DIRECT, dov) && dov[0] == 0);
        // Direct loads hold three register sets of pieces: past two pieces per
        // lane that costs occupancy, so split K further (measured: Q4_K and
        // Q5_K 12288 x 4096, 14.7 -> 11.1 us).
        int32_t sov[4];
        while (direct && npl > 2 && sp.ks < 4 && plan_override(OCO_KNOB_STREAM_PLAN, sov) != 3) {
            sp.ks *= 2;
            slice_blocks = (nblocks + sp.ks - 1) / sp.ks;
            npl = (int)((slice_blocks * P + 31) / 32);
        }
        // Where the activations come from: a fused norm stages them through
        // LDS; otherwise rows past 8192 values read them straight into
        // registers, since staged x would take LDS that occupancy needs
        // (measured, Q6_K 4096 x 12288: 15.2 -> 14.5 us), while shorter rows
        // stage (MXFP4 5760 x 2880: 5.25 us staged, 7.7 us from registers).
        // OCO_KNOB_STREAM_DIRECT's second value, when given, picks: 0 staged,
        // 1 registers.
        int xs = norm ? (norm->full_layer ? XS_NORM_FULL : XS_NORM) : p->k > 8192 ? XS_REG : XS_STAGED;
        if (!norm && plan_override(OCO_KNOB_STREAM_DIRECT, dov) >= 2) xs = dov[1] ? XS_REG : XS_STAGED;
        int lpr = 0;
        StreamFn fn = npl > 4 ? nullptr
                    : x_dtype == OCO_DT_F32 ? stream_pick_format<float>(format, xs, npl, direct, lpr)
                                            : stream_pick_format<bf16_t>(format, xs, npl, direct, lpr);
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
            const uint32_t rows_per_group = (4 / sp.ks) * 2;
            a.ngroups = (p->n + rows_per_group - 1) / rows_per_group;
            const uint32_t nsum = (format == OCO_Q8_0 || format == OCO_Q4_0 || format == OCO_Q4_1) ? 1
                                  : (format == OCO_Q4_K || format == OCO_Q5_K)                    ? 2
                                  : format == OCO_Q6_K                                            ? 4
                                                                                                  : 0;
            const size_t tile = direct ? 0 : (size_t)2 * lpr * 1024;
            const size_t xbytes = xs != XS_REG ? (size_t)p->k * 4 + (size_t)nsum * (p->k / 32) * 4 : 0;
            const size_t lds = xbytes + 4 * tile + 32 * sizeof(float);
            if (lds > 160 * 1024)
                return fail(OCO_ERR_UNSUPPORTED, "oco_matvec: k=%u needs %zu bytes of LDS", p->k, lds);
            if (lds > 64 * 1024)
                OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn,
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                                  "hipFuncSetAttribute"));
            const uint32_t grid = std::min<uint32_t>(a.ngroups, (uint32_t)(cus * sp.wg_per_cu));
            if (a.p.routes > 0x7fffffffu) return fail(OCO_ERR_INVALID, "oco_matvec: routes=%u", a.p.routes);
            const uint32_t mode = sp.ks == 4 ? 2u : sp.ks == 2 ? 1u : 0u;
            hipLaunchKernelGGL(fn, dim3(grid, p->m), dim3(256), lds, (hipStream_t)stream, a.w, a.x,
                               (uint32_t)a.row_bytes, a.p.n, a.p.k, mode, a.slice_blocks, a.ngroups, a.p.experts,
                               a.p.routes | (a.p.route_major ? 0x80000000u : 0u), a);
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
