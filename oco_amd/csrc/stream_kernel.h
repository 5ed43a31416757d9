// The streaming matvec kernel (Q8_0, Q4_0, Q4_1, Q4_K, Q5_K, Q6_K, MXFP4),
// shared by the single-matrix entry points (matvec.hip) and the grouped
// form that streams several matrices over one activation row in one grid
// (matvec_group.hip).
#pragma once
#include "norm.h"
#include "stream.h"

namespace oco {

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
    // Grouped form (MULTI): nmat matrices of the same format and shape,
    // each with its own weights, output and bias; ngroups counts the row
    // groups of one matrix.  Matrix i's groups are i * ngroups ..
    // (i + 1) * ngroups - 1 of the grid's sequence.
    uint32_t nmat;
    const uint8_t *wm[OCO_MATVEC_GROUP_MAX];
    void *ym[OCO_MATVEC_GROUP_MAX];
    const float *bm[OCO_MATVEC_GROUP_MAX];
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

template <int FMT, typename XT, int NPL, int XS, bool DIRECT, bool MULTI>
__global__ __launch_bounds__(256) void stream_kernel(const uint8_t *w_, const void *x_, uint32_t row_bytes_,
                                                     uint32_t n_, uint32_t k_, uint32_t mode_, uint32_t slice_,
                                                     uint32_t ngroups_, uint32_t experts_, uint32_t routes_,
                                                     StreamArgs a) {
    a.w = w_;
    a.x = x_;
    a.row_bytes = row_bytes_;
    a.p.n = n_;
    a.p.k = k_;
    // mode_: bits 0-1 log2 of the K split, bit 2 relu² of x on load
    const uint32_t ks_log2 = mode_ & 3u;
    const bool rs = (mode_ >> 2) & 1u;
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
    // MULTI: group g of the grid's sequence is group local(g) of matrix
    // mat(g) (uniform values: scalar work).
    const uint32_t ng = a.ngroups;
    const uint32_t total = MULTI ? ng * a.nmat : ng;
    auto mat = [&](uint32_t g) -> uint32_t {
        if constexpr (MULTI)
            return (uint32_t)(g >= ng) + (uint32_t)(g >= 2 * ng) + (uint32_t)(g >= 3 * ng);
        else
            return 0u;
    };
    auto local = [&](uint32_t g) -> uint32_t { return MULTI ? g - mat(g) * ng : g; };
    // Entries of the per-matrix arrays by select, not by a dynamic index
    // (which would copy the argument block to scratch memory).
    auto pick = [&](auto const (&arr)[OCO_MATVEC_GROUP_MAX], uint32_t i) {
        return i == 0 ? arr[0] : i == 1 ? arr[1] : i == 2 ? arr[2] : arr[3];
    };
    auto mbase = [&](uint32_t g) -> const uint8_t * {
        if constexpr (MULTI)
            return pick(a.wm, mat(g));
        else
            return ebase;
    };

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
    // DIRECT: groups in flight per wavefront.  The grouped form runs longer
    // per workgroup and takes a fourth, at three workgroups per CU even with
    // the fused norm (norm + Qwen3-8B up + gate: 21.6 -> 20.8-21.3 us);
    // single matrices lose with it (Q4_K 12288 x 4096: 10.5 -> 11.0 us).
    constexpr int RD = MULTI ? 4 : 3;
    typename T::Raw da[DIRECT ? NPL : 1], db[DIRECT ? NPL : 1], dc[DIRECT ? NPL : 1], dd[DIRECT && RD > 3 ? NPL : 1];
    // DIRECT: one buffer resource over the matrix.  The range ends at a
    // whole dword: a block's dword-aligned span may end up to three bytes
    // past the tensor, and a dword that straddles the range end would read
    // as zero (the same page holds it).
    const uint64_t dbytes = ((uint64_t)p.n * a.row_bytes + 3) & ~3ull;
    auto direct_rsrc = [&](const uint8_t *base) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0,
                                                 (uint32_t)(dbytes > 0xffffffffull ? 0xffffffffull : dbytes), 0x00020000);
    };
    __amdgpu_buffer_rsrc_t rall;
    if constexpr (DIRECT && !MULTI) rall = direct_rsrc(ebase);
    // DIRECT: this half-wavefront's row of group g (rows past n read row n - 1
    // and are never stored), pieces past the slice read the last piece.
    auto issue_direct = [&](uint32_t g, typename T::Raw *dst) __attribute__((always_inline)) {
        if constexpr (DIRECT) {
            if constexpr (MULTI) rall = direct_rsrc(mbase(g));
            const uint32_t row = min(local(g) * rows_per_group + set * ROWS + half, p.n - 1);
            const uint32_t roff = row * (uint32_t)a.row_bytes;
#pragma unroll
            for (int s = 0; s < NPL; s++) {
                const uint32_t pl = min(c + 32u * s, pieces - 1), blk = b0 + pl / T::P, cc = pl % T::P;
                dst[s] = T::direct(rall, roff + blk * T::BYTES, cc);
            }
        }
    };
    // Byte offset of tile row i of group g from the 16-byte boundary at or
    // below its matrix's start.
    auto row_offset = [&](uint32_t g, int i) -> uint32_t {
        const uint32_t row = local(g) * rows_per_group + set * ROWS + i;
        const uint32_t shift = (uint32_t)((uintptr_t)mbase(g) & 15);
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
        const uintptr_t base_al = (uintptr_t)mbase(g) & ~(uintptr_t)15;
#pragma unroll
        for (int i = 0; i < ROWS; i++) {
            const uint32_t row = local(g) * rows_per_group + set * ROWS + i;
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
            if (rs) {
#pragma unroll
                for (int e = 0; e < 32; e++) xv[s][e] = relu_sqr(xv[s][e]);
            }
        }
    }

    const uint32_t G = gridDim.x, g0 = blockIdx.x;
    if constexpr (DIRECT) {
        if (g0 < total) issue_direct(g0, da);
        if (g0 + G < total) issue_direct(g0 + G, db);
        if (g0 + 2 * G < total) issue_direct(g0 + 2 * G, dc);
        if (RD > 3 && g0 + 3 * G < total) issue_direct(g0 + 3 * G, dd);
    } else {
        if (g0 < total) issue(g0, ra);
        if (g0 + G < total) issue(g0 + G, rb);
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
                    } else if (rs) {
#pragma unroll
                        for (int e = 0; e < 4; e++) v[u][e] = relu_sqr(v[u][e]);
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
            if (g + RD * G < total) issue_direct(g + RD * G, dr);
        } else {
#pragma unroll
            for (int i = 0; i < ROWS * LPR; i++) reinterpret_cast<u32x4 *>(tile)[i * 64 + lane] = regs[i];
            const uint32_t rbase = half * LPR * 1024 + (row_offset(g, half) & 15u);
            if (g + 2 * G < total) issue(g + 2 * G, regs);
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

        const uint32_t row = local(g) * rows_per_group + set * ROWS + half;
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
            const float *bias = a.bias;
            void *y = a.y;
            if constexpr (MULTI) {
                bias = pick(a.bm, mat(g));
                y = pick(a.ym, mat(g));
            }
            if (p.has_bias) v += round_bf16(bias[(uint64_t)expert * p.n + row] + (p.has_bias == 2 ? 1.0f : 0.0f));
            const uint64_t o = (uint64_t)route * p.n + row;
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(y)[o] = f32_to_bf16_bits(v);
            else
                reinterpret_cast<float *>(y)[o] = v;
        }
    };
    if constexpr (DIRECT) {
        for (uint32_t g = g0; g < total; g += RD * G) {
            group(g, ra, da);
            if (g + G < total) group(g + G, rb, db);
            if (g + 2 * G < total) group(g + 2 * G, ra, dc);
            if (RD > 3 && g + 3 * G < total) group(g + 3 * G, ra, dd);
        }
    } else {
        for (uint32_t g = g0; g < total; g += 2 * G) {
            group(g, ra, da);
            if (g + G < total) group(g + G, rb, db);
        }
    }
}

typedef void (*StreamFn)(const uint8_t *, const void *, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
                         uint32_t, uint32_t, StreamArgs);

template <int FMT, typename XT, int XS, bool DIRECT, bool MULTI>
StreamFn stream_pick_npl_d(int npl) {
    switch (npl) {
    case 1: return stream_kernel<FMT, XT, 1, XS, DIRECT, MULTI>;
    case 2: return stream_kernel<FMT, XT, 2, XS, DIRECT, MULTI>;
    case 3: return stream_kernel<FMT, XT, 3, XS, DIRECT, MULTI>;
    case 4: return stream_kernel<FMT, XT, 4, XS, DIRECT, MULTI>;
    }
    return nullptr;
}
template <int FMT, typename XT, int XS, bool MULTI>
StreamFn stream_pick_npl(int npl, bool direct) {
    if constexpr (DirectOk<FMT>::value)
        if (direct) return stream_pick_npl_d<FMT, XT, XS, true, MULTI>(npl);
    return stream_pick_npl_d<FMT, XT, XS, false, MULTI>(npl);
}

template <int FMT>
int stream_lpr(int npl) {
    switch (npl) {
    case 1: return StreamShape<FMT, 1>::LPR;
    case 2: return StreamShape<FMT, 2>::LPR;
    case 3: return StreamShape<FMT, 3>::LPR;
    case 4: return StreamShape<FMT, 4>::LPR;
    }
    return 0;
}

// xs: an XS_* source of x; the fused norms only with bf16 rows.
template <typename XT, bool MULTI>
StreamFn stream_pick_format(uint32_t fmt, int xs, int npl, bool direct, int &lpr) {
    switch (fmt) {
#define F(FM)                                                                                   \
    case FM:                                                                                    \
        lpr = stream_lpr<FM>(npl);                                                              \
        if constexpr (sizeof(XT) == 2) {                                                        \
            if (xs == XS_NORM) return stream_pick_npl<FM, XT, XS_NORM, MULTI>(npl, direct);            \
            if (xs == XS_NORM_FULL) return stream_pick_npl<FM, XT, XS_NORM_FULL, MULTI>(npl, direct);  \
        }                                                                                              \
        if (xs == XS_REG) return stream_pick_npl<FM, XT, XS_REG, MULTI>(npl, direct);                  \
        return xs == XS_STAGED ? stream_pick_npl<FM, XT, XS_STAGED, MULTI>(npl, direct) : nullptr;
        F(OCO_Q8_0) F(OCO_MXFP4) F(OCO_Q4_K) F(OCO_Q6_K) F(OCO_Q4_0) F(OCO_Q4_1) F(OCO_Q5_K)
#undef F
    }
    return nullptr;
}


}  // namespace oco
