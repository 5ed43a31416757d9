// Routed MXFP4 experts on the block-scaled FP8 x FP4 MFMA: the grouped
// expert GEMMs of expert_up_tensor / moe_activate / expert_down_tensor
// (projections.metal:192-376, routing.metal:44-64) and, at decode, the
// routed matvecs of expert_expand / matvec_mxfp4 (:78-182) -- with no weight
// decode at all: each GGUF block's 16 payload bytes are the B operand as
// stored and its E8M0 byte the B scale (the operand layout is described in
// mxmatmul.hip).
//
// Activations are split per row into TERMS E4M3 terms with E8M0 scales per
// 32-block (the split of mxmatmul.hip), stored row-major so that tiles can
// gather arbitrary rows: record (row, K step of 64) =
//     data [term][part 2][block 2][16 B]   (lane part p reads 32 bytes)
//     scales [block 2][4 bytes, byte t = term t] E8M0, padded to 16 bytes
// Two terms hold bf16 inputs exactly; f32 inputs (and the f32 activations
// between gate/up and down) take three: relL2 ~1.4e-5 of the product
// against ~6e-4 with two (numpy model, N(0,1) and SwiGLU-shaped rows).
#include "matmul.h"
#include "stream.h"

namespace oco {

typedef int mxe_i32x8 __attribute__((ext_vector_type(8)));
typedef float mxe_f32x16 __attribute__((ext_vector_type(16)));

__host__ __device__ constexpr uint32_t mxr_data(int terms) { return 64u * terms; }
__host__ __device__ constexpr uint32_t mxr_rec(int terms) { return 64u * terms + 16u; }

uint64_t mx_rows_bytes(uint32_t rows, uint32_t k, int terms) {
    return (uint64_t)rows * ((k + 63) / 64) * mxr_rec(terms);
}

// Smallest E with amax <= 448 * 2^E, as E (E8M0 byte E + 127); 128 (NaN byte)
// for a non-finite block.
__device__ __forceinline__ int mxe_scale_exp(float amax) {
    if (!(amax <= 3.402823466e38f)) return 128;
    if (amax == 0.f) return -127;
    const uint32_t b = __float_as_uint(amax);
    int e;
    uint32_t mant;
    if (b >> 23) {
        e = (int)(b >> 23) - 127;
        mant = b & 0x7fffffu;
    } else {
        const int lz = __builtin_clz(b) - 8;
        e = -126 - lz;
        mant = (b << lz) & 0x7fffffu;
    }
    const int E = mant <= 0x600000u ? e - 8 : e - 7;
    return E < -127 ? -127 : E;
}

// One thread per (row, K step, block): the block's two E4M3 terms, written
// in W's nibble order, and its two E8M0 scales.
template <typename XT, int TERMS>
__global__ __launch_bounds__(256) void mx_rows_split_kernel(const XT *x, uint8_t *rec, uint32_t rows, uint32_t k) {
    const uint32_t ksteps = (k + 63) / 64;
    const uint64_t item = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // (row, step, block)
    const uint32_t blk = (uint32_t)(item & 1);
    const uint64_t rs = item >> 1;
    if (rs >= (uint64_t)rows * ksteps) return;
    const uint32_t row = (uint32_t)(rs / ksteps), s = (uint32_t)(rs % ksteps);
    const uint32_t k0 = s * 64 + 32 * blk;
    float v[32];
    if (k0 < k) {
        const XT *src = x + (uint64_t)row * k + k0;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            if constexpr (sizeof(XT) == 4)
                v[i] = src[i];
            else
                v[i] = __uint_as_float((uint32_t)src[i] << 16);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = 0.f;
    }
    uint8_t *out = rec + ((uint64_t)row * ksteps + s) * mxr_rec(TERMS);
    uint32_t scales = 0;
#pragma unroll
    for (int t = 0; t < TERMS; t++) {
        float amax = 0.f;
        bool nan = false;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            amax = fmaxf(amax, fabsf(v[i]));
            nan |= v[i] != v[i];
        }
        if (nan) amax = __uint_as_float(0x7fc00000u);
        const int E = mxe_scale_exp(amax);
        scales |= (uint32_t)(E + 127) << (8 * t);
        const float inv = E == 128 ? 0.f : __builtin_ldexpf(1.f, -E), sc = E == 128 ? 0.f : __builtin_ldexpf(1.f, E);
        uint32_t codes[8];
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
        // part p, byte e of this block: value 8p + e / 2 + 16 (e & 1) (W's nibble order)
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
            *reinterpret_cast<uint4 *>(out + ((t * 2 + p) * 2 + blk) * 16) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    *reinterpret_cast<uint32_t *>(out + mxr_data(TERMS) + 4 * blk) = scales;
}

// Tile: one route-plan tile of up to TR routes (16 or 32: the plan's tile
// rows) and 32-column weight tiles, one per wavefront (gate/up: the first
// NW / 2 wavefronts take gate rows, the others the up rows of the same
// columns, and hand their sums over through LDS for the fused activation).
// The K loop runs in quads of
// four K steps (eight blocks, 136 bytes of each weight row):
//  - B: every weight row's quad is fetched as the 16-byte-aligned 160-byte
//    span holding it, 16 bytes per lane (whole lines per row and request --
//    reading 34 bytes per row per step reached well under half the HBM rate
//    of line-sized requests), and staged in this wavefront's LDS region;
//  - A: the tile's live rows' four split records, shared by the workgroup's
//    wavefronts, are fetched by all lanes into LDS.
// Both are loaded one quad ahead into registers and written to LDS at the
// top of the next quad, so one vmcnt(0) and two barriers per quad order
// everything.
template <int G, int NW, int TERMS, int TR>
__global__ __launch_bounds__(64 * NW) void mx_experts_kernel(MatmulArgs a, const uint8_t *xrec) {
    constexpr int NT = 1;                          // weight tiles per wavefront
    constexpr int WROWS = 32 * NT;                 // weight rows per wavefront
    constexpr int WLD = WROWS * 10 / 64;           // 16-byte loads per lane per quad (10 per row)
    constexpr int CT = G == MM_GATE_UP ? NW / 2 : NW;  // column tiles per workgroup
    constexpr uint32_t WSLOT = 176;                // LDS bytes per staged row (11 x 16)
    constexpr uint32_t AREC = mxr_rec(TERMS);
    constexpr uint32_t AROW = 4 * AREC + 16;       // LDS bytes per tile row of A (four records + pad)
    constexpr uint32_t APR = 4 * AREC / 16;        // 16-byte pieces per tile row and quad
    constexpr int ALD = (TR * APR + 64 * NW - 1) / (64 * NW);  // A loads per lane per quad (TR rows)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane & 31, part = lane >> 5;
    const uint32_t used = gridDim.x * min(a.plan[1], gridDim.y);
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, used);
    if (lin >= used) return;  // uniform: a surplus workgroup
    const uint32_t bx = lin % gridDim.x, y = lin / gridDim.x;
    const uint32_t expert = a.plan[6 + 2 * y], first = a.plan[7 + 2 * y];
    const uint64_t grouped = 6 + 2 * ((uint64_t)(a.routes + 15) / 16 + a.experts);
    const uint64_t list = grouped + (uint64_t)expert * (a.routes + 1);
    const uint64_t sorted = grouped + (uint64_t)a.experts * (a.routes + 1);
    const uint32_t rows = min((uint32_t)TR, a.plan[list] - first);
    const uint32_t sorted0 = a.plan[sorted + expert] + first;
    // Wavefronts past the last column still load (clamped rows) and join the
    // barriers; they store nothing.
    const bool upw = G == MM_GATE_UP && wave >= CT;  // an up wavefront
    const uint32_t col0 = (bx * CT + wave % CT) * 32;
    const uint32_t ksteps = (a.k + 63) / 64, nblk = a.k / 32, quads = (ksteps + 3) / 4;

    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t *alds = lds;                                           // [TR][AROW]
    uint8_t *wlds = lds + TR * AROW + wave * (WROWS * WSLOT);       // [WROWS][WSLOT]

    // A: piece p (16 bytes) of the quad = tile row p / APR, byte 16 (p % APR)
    // of its four consecutive records.
    const uint32_t xrows = G == MM_GATE_UP ? a.routes / a.topk : a.routes;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xrec), 0, (uint32_t)((uint64_t)xrows * ksteps * AREC), 0x00020000);
    const uint32_t pieces = rows * APR;
    uint32_t asrc[ALD], adst[ALD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t p = threadIdx.x + 64 * NW * i, r = min(p / APR, TR - 1u), q16 = p % APR;
        uint32_t xrow = 0;
        if (p < pieces) xrow = G == MM_GATE_UP ? a.plan[list + 1 + first + r] / a.topk : sorted0 + r;
        asrc[i] = xrow * ksteps * AREC + 16 * q16;
        adst[i] = r * AROW + 16 * q16;
    }
    // A fragments: this lane's tile row (rows past the tile read row 0: a
    // row of C depends on its own row of A only, and those rows are never
    // stored).
    const uint32_t arow = (uint32_t)c < rows ? c : 0u;
    const uint32_t afrag = arow * AROW + 32 * part, ascale = arow * AROW + mxr_data(TERMS) + 4 * part;

    // B: load i of a lane covers staged row f / 10, chunk f % 10 (f = lane +
    // 64 i); quad q's span of a row at byte R starts at
    //   (R + 136 q) & ~15 = ((R + 8 (q & 1)) & ~15) + 136 q - 8 (q & 1),
    // a per-lane offset fixed for each parity of q plus a uniform one.  The
    // buffer range returns zeros past the expert's matrix.
    __amdgpu_buffer_rsrc_t rw[NT];
    uint32_t rsh[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
        const uint8_t *eb = (upw ? a.w2 : a.w) + expert * a.expert_bytes;
        rsh[j] = (uint32_t)(uintptr_t)eb & 15u;
        const uint64_t span = (a.expert_bytes + rsh[j] + 160 + 15) & ~15ull;
        rw[j] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(eb - rsh[j]), 0,
                                                  (uint32_t)std::min<uint64_t>(span, 0xffffffffull), 0x00020000);
    }
    uint32_t boff[WLD][2], wdst[WLD];
#pragma unroll
    for (int i = 0; i < WLD; i++) {
        const uint32_t f = lane + 64 * i, row = f / 10, chunk = f % 10, j = row / 32;
        const uint32_t r = rsh[j] + min(col0 + row % 32, a.n - 1) * (uint32_t)a.row_bytes;
#pragma unroll
        for (int p = 0; p < 2; p++) boff[i][p] = ((r + 8 * p) & ~15u) + 16 * chunk;
        wdst[i] = row * WSLOT + 16 * chunk;
    }
    // B fragments: block 8 q + 2 s + part of this lane's row sits at byte
    // ((R + 8 (q & 1)) & 15) + 34 s + 17 part of the staged span (scale
    // byte, then 16 payload bytes).
    uint32_t fpay[NT][2];  // [tile][parity]: lds offset of the payload of step 0
#pragma unroll
    for (int j = 0; j < NT; j++) {
        const uint32_t r = rsh[j] + min(col0 + c, a.n - 1) * (uint32_t)a.row_bytes;
#pragma unroll
        for (int p = 0; p < 2; p++) fpay[j][p] = (j * 32 + c) * WSLOT + ((r + 8 * p) & 15u) + 17 * part + 1;
    }

    u32x4 wreg[WLD], areg[ALD];
    auto issue = [&](uint32_t q, int par) __attribute__((always_inline)) {
        const uint32_t sw = 136 * q - 8 * (q & 1), sa = 4 * q * AREC;
#pragma unroll
        for (int i = 0; i < WLD; i++)
            wreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rw[(lane + 64 * i) / 10 / 32], boff[i][par], sw, 0);
#pragma unroll
        for (int i = 0; i < ALD; i++)
            if (threadIdx.x + 64 * NW * i < pieces) areg[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, asrc[i], sa, 0);
    };
    mxe_f32x16 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) acc[j] = mxe_f32x16{};
    auto quad = [&](uint32_t q, int par) __attribute__((always_inline)) {
        __syncthreads();  // every wavefront is done with the previous quad's A
#pragma unroll
        for (int i = 0; i < WLD; i++) *reinterpret_cast<u32x4 *>(wlds + wdst[i]) = wreg[i];
#pragma unroll
        for (int i = 0; i < ALD; i++)
            if (threadIdx.x + 64 * NW * i < pieces) *reinterpret_cast<u32x4 *>(alds + adst[i]) = areg[i];
        __syncthreads();  // this quad's A is in place
        if (q + 1 < quads) issue(q + 1, par ^ 1);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t step = 4 * q + s;
            if (step >= ksteps) break;  // uniform
            // the lone last block's partner is zero with scale 1
            const bool live = 2 * step + part < nblk;
            u32x4 av[TERMS][2];
#pragma unroll
            for (int t = 0; t < TERMS; t++)
#pragma unroll
                for (int b = 0; b < 2; b++)
                    av[t][b] = *reinterpret_cast<const u32x4 *>(alds + afrag + s * AREC + 64 * t + 16 * b);
            const uint32_t sa = *reinterpret_cast<const uint32_t *>(alds + ascale + s * AREC);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const uint32_t pay = fpay[j][par] + 34 * s;
                const uint32_t *pw = reinterpret_cast<const uint32_t *>(wlds + (pay & ~3u));
                uint32_t w[5];
#pragma unroll
                for (int i = 0; i < 5; i++) w[i] = pw[i];
                uint32_t qd[4];
#pragma unroll
                for (int i = 0; i < 4; i++) qd[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], pay);
                const mxe_i32x8 bv =
                    live ? mxe_i32x8{(int)qd[0], (int)qd[1], (int)qd[2], (int)qd[3], 0, 0, 0, 0} : mxe_i32x8{};
                const int sb = live ? (int)wlds[pay - 1] : 127;
#pragma unroll
                for (int t = 0; t < TERMS; t++) {
                    const mxe_i32x8 avt{(int)av[t][0].x, (int)av[t][0].y, (int)av[t][0].z, (int)av[t][0].w,
                                        (int)av[t][1].x, (int)av[t][1].y, (int)av[t][1].z, (int)av[t][1].w};
                    if (t == 0)
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(avt, bv, acc[j], 0, 4, 0, (int)sa, 0, sb);
                    else if (t == 1)
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(avt, bv, acc[j], 0, 4, 1, (int)sa, 0, sb);
                    else
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(avt, bv, acc[j], 0, 4, 2, (int)sa, 0, sb);
                }
            }
        }
    };
    issue(0, 0);
    for (uint32_t q = 0; q < quads; q += 2) {
        quad(q, 0);
        if (q + 1 < quads) quad(q + 1, 1);
    }

    // C: lane l holds column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4.
    const uint32_t col = col0 + c;
    const uint64_t bi = (uint64_t)expert * a.n + min(col, a.n - 1);
    if constexpr (G == MM_GATE_UP) {
        // up sums to the gate wavefront of the same columns (the A region is free now)
        float *hand = reinterpret_cast<float *>(lds);  // [CT][16][64]
        __syncthreads();
        if (upw) {
#pragma unroll
            for (int v = 0; v < 16; v++) hand[((wave - CT) * 16 + v) * 64 + lane] = acc[0][v];
        }
        __syncthreads();
        if (upw || col >= a.n) return;
        const float bg = a.bias ? round_bf16(a.bias[bi]) : 0.f;
        const float bu = a.bias2 ? round_bf16(a.bias2[bi] + (a.up_one ? 1.0f : 0.0f)) : (a.up_one ? 1.0f : 0.0f);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const uint32_t r = 8 * (v / 4) + 4 * part + (v % 4);
            const float up = hand[(wave * 16 + v) * 64 + lane];
            if (r < rows)
                reinterpret_cast<float *>(a.y)[(uint64_t)(sorted0 + r) * a.n + col] =
                    expert_activation(a.act, acc[0][v] + bg, up + bu);
        }
    } else {
        if (col >= a.n) return;
        const float b = a.bias ? round_bf16(a.bias[bi]) : 0.f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const uint32_t r = 8 * (v / 4) + 4 * part + (v % 4);
            if (r >= rows) continue;
            const float val = acc[0][v] + b;
            const uint64_t o = (uint64_t)a.plan[list + 1 + first + r] * a.n + col;
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(val);
            else
                reinterpret_cast<float *>(a.y)[o] = val;
        }
    }
}

int mx_rows_split(const void *x, bool bf16, uint8_t *rec, uint32_t rows, uint32_t k, int terms, hipStream_t stream) {
    const uint64_t items = (uint64_t)rows * ((k + 63) / 64) * 2;
    const dim3 grid((unsigned)((items + 255) / 256));
    if (bf16 && terms == 2)
        hipLaunchKernelGGL((mx_rows_split_kernel<uint16_t, 2>), grid, dim3(256), 0, stream, (const uint16_t *)x, rec, rows, k);
    else if (!bf16 && terms == 3)
        hipLaunchKernelGGL((mx_rows_split_kernel<float, 3>), grid, dim3(256), 0, stream, (const float *)x, rec, rows, k);
    else
        return fail(OCO_ERR_UNSUPPORTED, "experts: MXFP4 split of %s rows into %d terms", bf16 ? "bf16" : "f32", terms);
    return launch_check("experts MXFP4 row split");
}

constexpr int MXE_NW = 4;

template <int G, int TERMS, int TR>
static int mx_experts_go(const MatmulArgs &a, const uint8_t *xrec, hipStream_t stream) {
    const size_t lds = TR * (4 * mxr_rec(TERMS) + 16) + (size_t)MXE_NW * 32 * 176;
    static_assert(TR * (4 * mxr_rec(2) + 16) >= MXE_NW / 2 * 16 * 64 * 4, "the up hand-over fits the A region");
    auto fn = mx_experts_kernel<G, MXE_NW, TERMS, TR>;
    OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                      "hipFuncSetAttribute"));
    const uint32_t cols = 32 * (G == MM_GATE_UP ? MXE_NW / 2 : MXE_NW);
    const dim3 grid((a.n + cols - 1) / cols, (a.routes + TR - 1) / TR + a.experts);
    hipLaunchKernelGGL(fn, grid, dim3(64 * MXE_NW), lds, stream, a, xrec);
    return OCO_OK;
}

template <int G, int TERMS>
static int mx_experts_go_tr(const MatmulArgs &a, const uint8_t *xrec, uint32_t tile_rows, hipStream_t stream) {
    return tile_rows == 16 ? mx_experts_go<G, TERMS, 16>(a, xrec, stream) : mx_experts_go<G, TERMS, 32>(a, xrec, stream);
}

int mx_experts_launch(int mode, const MatmulArgs &a, const uint8_t *xrec, int terms, uint32_t tile_rows,
                      hipStream_t stream) {
    if (a.k % 32) return fail(OCO_ERR_INVALID, "experts: MXFP4 rows need k %% 32 == 0 (k=%u)", a.k);
    if (tile_rows != 16 && tile_rows != 32) return fail(OCO_ERR_INVALID, "experts: MXFP4 plan tiles of %u rows", tile_rows);
    // Kernel offsets are 32-bit: the split rows and one expert's matrix each stay under 4 GiB.
    if (mx_rows_bytes(a.routes, a.k, terms) > 0xffffffffull || a.expert_bytes + 4 > 0xffffffffull)
        return fail(OCO_ERR_UNSUPPORTED, "experts: MXFP4 operands over 4 GiB (routes=%u k=%u)", a.routes, a.k);
    const int rc = mode == MM_GATE_UP ? (terms == 2 ? mx_experts_go_tr<MM_GATE_UP, 2>(a, xrec, tile_rows, stream)
                                                    : mx_experts_go_tr<MM_GATE_UP, 3>(a, xrec, tile_rows, stream))
                                      : (terms == 2 ? mx_experts_go_tr<MM_DOWN, 2>(a, xrec, tile_rows, stream)
                                                    : mx_experts_go_tr<MM_DOWN, 3>(a, xrec, tile_rows, stream));
    OCO_TRY(rc);
    return launch_check("experts MXFP4 grouped matmul");
}

}  // namespace oco
