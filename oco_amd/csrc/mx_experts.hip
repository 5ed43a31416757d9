// Routed MXFP4 experts on the block-scaled FP6 x FP4 MFMA: the grouped
// expert GEMMs of expert_up_tensor / moe_activate / expert_down_tensor
// (projections.metal:192-376, routing.metal:44-64) and, at decode, the
// routed matvecs of expert_expand / matvec_mxfp4 (:78-182) -- with no weight
// decode at all: each GGUF block's 16 payload bytes are the B operand as
// stored and its E8M0 byte the B scale (the operand layout is described in
// mxmatmul.hip).
//
// Activations come split per row into four E2M3 terms (mxsplit.h): the A
// operand is FP6, which issues at the FP4 rate.
#include "matmul.h"
#include "mxsplit.h"
#include "route.h"
#include "stream.h"

namespace oco {

typedef int mxe_i32x8 __attribute__((ext_vector_type(8)));
typedef float mxe_f32x16 __attribute__((ext_vector_type(16)));
typedef float mxe_f32x4 __attribute__((ext_vector_type(4)));

uint64_t mx_rows_bytes(uint32_t rows, uint32_t k) { return (uint64_t)rows * ((k + 63) / 64) * MXR_REC; }

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
template <int G, int NW, int TR, int KS>
__global__ __launch_bounds__(64 * NW) void mx_experts_kernel(KPRE_PARAMS, MatmulArgs a) {
    KPRE_APPLY(a);
    const uint8_t *xrec = reinterpret_cast<const uint8_t *>(a.x);
    const uint64_t expert_bytes = (uint64_t)a.n * a.row_bytes;
    constexpr int NT = 1;                          // weight tiles per wavefront
    constexpr int WROWS = 32 * NT;                 // weight rows per wavefront
    constexpr int WLD = WROWS * 10 / 64;           // 16-byte loads per lane per quad (10 per row)
    constexpr int WPK = NW / KS;                   // wavefronts per K part (KS parts split the quads)
    constexpr int CT = G == MM_GATE_UP ? WPK / 2 : WPK;  // column tiles per workgroup
    constexpr uint32_t WSLOT = 176;                // LDS bytes per staged row (11 x 16)
    constexpr uint32_t AREC = MXR_REC;
    constexpr uint32_t AROW = 4 * AREC + 16;       // LDS bytes per tile row of A (four records + pad)
    constexpr uint32_t APR = 4 * AREC / 16;        // 16-byte pieces per tile row and quad
    constexpr int ALD = (KS * TR * APR + 64 * NW - 1) / (64 * NW);  // A loads per lane per quad (TR rows per part)
    static_assert(NW % KS == 0 && (G == MM_DOWN || (NW / KS) % 2 == 0), "wavefronts split evenly into parts and tiles");
    static_assert((KS - 1) * (NW / KS) * 16 * 64 * 4 <= KS * TR * AROW, "the K-part sums fit the record region");
    static_assert(4 * SMALL_PLAN_WORDS <= TR * AROW && TR <= 64, "the in-workgroup plan fits the record region");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane & 31, part = lane >> 5;
    const int kh = wave / WPK, wsub = wave % WPK;  // K part, wavefront within it
    // The plan's tile count (word 1) spreads exactly the used tiles evenly
    // over the XCDs, each XCD a contiguous range of them (tile-major); then
    // the tile's descriptor: expert, rows, first sorted row, its route ids.
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint32_t expert, rows, sorted0, bx, y;
    const uint32_t *rid;
    if (G == MM_GATE_UP && a.small) {
        // the plan built here (in the A region, free until the first quad)
        uint32_t *psh = reinterpret_cast<uint32_t *>(lds);
        const bool store = blockIdx.x == 0 && blockIdx.y == 0;  // this workgroup records the plan
        const SmallPlan sp =
            small_plan<64 * NW, TR>(a.logits, a.ids, a.routes / a.topk, a.experts, a.topk, psh, store);
        if (store)
            small_plan_store<TR>(sp, a.routes, a.desc_out, a.plan_out, psh, a.logits ? a.ids_out : nullptr,
                                 a.probs_out);
        const uint32_t used = gridDim.x * min(small_tiles(sp), gridDim.y);
        const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, used);
        if (lin >= used) return;  // uniform: a surplus workgroup
        bx = lin % gridDim.x;
        y = lin / gridDim.x;
        const SmallTile t = small_tile<TR>(sp, y, psh);
        __syncthreads();  // the tile's route ids are in place
        expert = t.expert;
        rows = t.rows;
        sorted0 = t.sorted0;
        rid = sh_tile(psh);
    } else {
        const uint32_t used = gridDim.x * min(a.plan[1], gridDim.y);
        const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, used);
        if (lin >= used) return;  // uniform: a surplus workgroup
        bx = lin % gridDim.x;
        y = lin / gridDim.x;
        const uint32_t *dsc = a.desc + (uint64_t)y * (PLAN_DESC_HEAD + TR);
        const uint4 head = *reinterpret_cast<const uint4 *>(dsc);
        rid = dsc + PLAN_DESC_HEAD;
        expert = head.x;
        rows = head.y;
        sorted0 = head.z;
        if (rows == 0) return;  // uniform: an unused tile slot
    }
    // Wavefronts past the last column still load (clamped rows) and join the
    // barriers; they store nothing.
    const bool upw = G == MM_GATE_UP && wsub >= CT;  // an up wavefront
    const uint32_t col0 = (bx * CT + wsub % CT) * 32;
    const uint32_t ksteps = (a.k + 63) / 64, nblk = a.k / 32, quads = (ksteps + 3) / 4;
    // K part kh takes quads kh * qpart .. (an even count: both parts keep
    // the parity of their local quad index)
    const uint32_t qpart = KS == 1 ? quads : (quads + 2 * KS - 1) / (2 * KS) * 2, q0 = kh * qpart;

    uint8_t *alds = lds;                                           // [KS][TR][AROW]
    uint8_t *wlds = lds + KS * TR * AROW + wave * (WROWS * WSLOT);  // [WROWS][WSLOT]

    // A: piece p (16 bytes) of the quad = tile row p / APR, byte 16 (p % APR)
    // of its four consecutive records.
    const uint32_t xrows = G == MM_GATE_UP ? a.routes / a.topk : a.routes;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xrec), 0, (uint32_t)((uint64_t)xrows * ksteps * AREC), 0x00020000);
    // Piece p of the quad: K part p / (rows APR), then tile row and byte.
    const uint32_t pieces = KS * rows * APR;
    uint32_t asrc[ALD], adst[ALD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t p = threadIdx.x + 64 * NW * i, kp = min(p / (rows * APR), KS - 1u), pr = p - kp * rows * APR;
        const uint32_t r = min(pr / APR, TR - 1u), q16 = pr % APR;
        uint32_t xrow = 0;
        if (p < pieces) xrow = G == MM_GATE_UP ? rid[r] / a.topk : sorted0 + r;
        asrc[i] = xrow * ksteps * AREC + kp * qpart * 4 * AREC + 16 * q16;
        adst[i] = (kp * TR + r) * AROW + 16 * q16;
    }
    // A fragments: this lane's tile row (rows past the tile read row 0: a
    // row of C depends on its own row of A only, and those rows are never
    // stored).
    const uint32_t arow = (uint32_t)c < rows ? c : 0u;
    const uint32_t arow0 = (kh * TR + arow) * AROW;
    const uint32_t a16 = arow0 + 16 * part, a8 = arow0 + MXR_CODES8 + 8 * part, ascale = arow0 + MXR_SCALES + 4 * part;

    // B: load i of a lane covers staged row f / 10, chunk f % 10 (f = lane +
    // 64 i); quad q's span of a row at byte R starts at
    //   (R + 136 q) & ~15 = ((R + 8 (q & 1)) & ~15) + 136 q - 8 (q & 1),
    // a per-lane offset fixed for each parity of q plus a uniform one.  The
    // buffer range returns zeros past the expert's matrix.
    __amdgpu_buffer_rsrc_t rw[NT];
    uint32_t rsh[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
        const uint8_t *eb = (upw ? a.w2 : a.w) + expert * expert_bytes;
        rsh[j] = (uint32_t)(uintptr_t)eb & 15u;
        const uint64_t span = (expert_bytes + rsh[j] + 160 + 15) & ~15ull;
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
    // Tiles of 16 rows run v_mfma_scale_f32_16x16x128_f8f6f4 (16 rows, half
    // the MFMA of the 32-row shape): lane l takes row / column l % 16 and
    // block g = l / 16 of each 128-K chunk (K steps 2h + g / 2 of the quad,
    // block g % 2 of the step), the wavefront's 32 columns as two column
    // tiles ct; C holds column l % 16, rows 4 (l / 16) + v.
    constexpr bool S16 = TR == 16;
    const uint32_t l16 = lane & 15, g16 = lane >> 4;
    const uint32_t arow16 = l16 < rows ? l16 : 0u;
    const uint32_t a16b = (kh * TR + arow16) * AROW + (g16 >> 1) * AREC;  // + 2 h AREC per chunk
    uint32_t fpay16[2][2];  // [column tile][parity]: lds offset of the payload of chunk 0
#pragma unroll
    for (int ct = 0; ct < 2; ct++) {
        const uint32_t r = rsh[0] + min(col0 + 16 * ct + l16, a.n - 1) * (uint32_t)a.row_bytes;
#pragma unroll
        for (int p = 0; p < 2; p++) fpay16[ct][p] = (16 * ct + l16) * WSLOT + ((r + 8 * p) & 15u) + 17 * g16 + 1;
    }

    u32x4 wreg[WLD], areg[ALD];
    auto issue = [&](uint32_t q, int par) __attribute__((always_inline)) {
        const uint32_t qg = q0 + q, sw = 136 * qg - 8 * (qg & 1), sa = 4 * q * AREC;  // q: this part's quad
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
    mxe_f32x4 acc16[2] = {mxe_f32x4{}, mxe_f32x4{}};
    auto quad = [&](uint32_t q, int par) __attribute__((always_inline)) {
        __syncthreads();  // every wavefront is done with the previous quad's A
#pragma unroll
        for (int i = 0; i < WLD; i++) *reinterpret_cast<u32x4 *>(wlds + wdst[i]) = wreg[i];
#pragma unroll
        for (int i = 0; i < ALD; i++)
            if (threadIdx.x + 64 * NW * i < pieces) *reinterpret_cast<u32x4 *>(alds + adst[i]) = areg[i];
        __syncthreads();  // this quad's A is in place
        if (q + 1 < qpart) issue(q + 1, par ^ 1);
        if constexpr (S16) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if (4 * (q0 + q) + 2 * h >= ksteps) break;  // uniform per wavefront
                // this lane's block: global block 2 (its step) + g % 2; a dead
                // block (past k, or the lone last block's partner) multiplies
                // zeros at scale 1 on both sides
                const uint32_t gstep = 4 * (q0 + q) + 2 * h + (g16 >> 1);
                const bool live = 2 * gstep + (g16 & 1) < nblk;
                const uint32_t ab = a16b + 2 * h * AREC;
                u32x4 av16[MX_TERMS];
                u32x2 av8[MX_TERMS];
#pragma unroll
                for (int t = 0; t < MX_TERMS; t++) {
                    av16[t] = *reinterpret_cast<const u32x4 *>(alds + ab + 32 * t + 16 * (g16 & 1));
                    av8[t] = *reinterpret_cast<const u32x2 *>(alds + ab + MXR_CODES8 + 16 * t + 8 * (g16 & 1));
                }
                const uint32_t sa = live ? *reinterpret_cast<const uint32_t *>(alds + ab + MXR_SCALES + 4 * (g16 & 1))
                                         : 0x7f7f7f7fu;
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                    const uint32_t pay = fpay16[ct][par] + 68 * h;
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
                    for (int t = 0; t < MX_TERMS; t++) {
                        const mxe_i32x8 avt{(int)av16[t].x, (int)av16[t].y, (int)av16[t].z, (int)av16[t].w,
                                            (int)av8[t].x,  (int)av8[t].y,  0,                0};
                        if (t == 0)
                            acc16[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(avt, bv, acc16[ct], 2, 4, 0, (int)sa, 0, sb);
                        else if (t == 1)
                            acc16[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(avt, bv, acc16[ct], 2, 4, 1, (int)sa, 0, sb);
                        else if (t == 2)
                            acc16[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(avt, bv, acc16[ct], 2, 4, 2, (int)sa, 0, sb);
                        else
                            acc16[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(avt, bv, acc16[ct], 2, 4, 3, (int)sa, 0, sb);
                    }
                }
            }
            return;
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t step = 4 * (q0 + q) + s;
            if (step >= ksteps) break;  // uniform per wavefront
            // the lone last block's partner is zero with scale 1
            const bool live = 2 * step + part < nblk;
            // A: each term's 24 code bytes of this lane's block (16 + 8)
            u32x4 av16[MX_TERMS];
            u32x2 av8[MX_TERMS];
#pragma unroll
            for (int t = 0; t < MX_TERMS; t++) {
                av16[t] = *reinterpret_cast<const u32x4 *>(alds + a16 + s * AREC + 32 * t);
                av8[t] = *reinterpret_cast<const u32x2 *>(alds + a8 + s * AREC + 16 * t);
            }
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
                for (int t = 0; t < MX_TERMS; t++) {
                    const mxe_i32x8 avt{(int)av16[t].x, (int)av16[t].y, (int)av16[t].z, (int)av16[t].w,
                                        (int)av8[t].x,  (int)av8[t].y,  0,                0};
                    // cbsz 2: A in E2M3; blgp 4: B in E2M1; op_sel picks term t's scale byte
                    if (t == 0)
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(avt, bv, acc[j], 2, 4, 0, (int)sa, 0, sb);
                    else if (t == 1)
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(avt, bv, acc[j], 2, 4, 1, (int)sa, 0, sb);
                    else if (t == 2)
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(avt, bv, acc[j], 2, 4, 2, (int)sa, 0, sb);
                    else
                        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(avt, bv, acc[j], 2, 4, 3, (int)sa, 0, sb);
                }
            }
        }
    };
    issue(0, 0);
    for (uint32_t q = 0; q < qpart; q += 2) {
        quad(q, 0);
        if (q + 1 < qpart) quad(q + 1, 1);
    }
    // The lane's results as (row, column from col0, value): the 32x32 shape
    // holds column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4; the 16x16
    // shape column 16 ct + l % 16, rows 4 (l / 16) + v.
    constexpr int NV = S16 ? 8 : 16;
    float accv[NV];
    uint32_t rowv[NV], colv[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        if constexpr (S16) {
            accv[i] = acc16[i / 4][i % 4];
            rowv[i] = 4 * g16 + i % 4;
            colv[i] = 16 * (i / 4) + l16;
        } else {
            accv[i] = acc[0][i];
            rowv[i] = 8 * (i / 4) + 4 * part + (i % 4);
            colv[i] = c;
        }
    }
    if constexpr (KS > 1) {
        // the other K parts' sums to part 0 (the A region is free now)
        float *red = reinterpret_cast<float *>(lds);  // [KS - 1][WPK][NV][64]
        __syncthreads();
        if (kh > 0) {
#pragma unroll
            for (int i = 0; i < NV; i++) red[(((kh - 1) * WPK + wsub) * NV + i) * 64 + lane] = accv[i];
        }
        __syncthreads();
        if (kh > 0) return;
#pragma unroll
        for (int k2 = 0; k2 < KS - 1; k2++)
#pragma unroll
            for (int i = 0; i < NV; i++) accv[i] += red[((k2 * WPK + wsub) * NV + i) * 64 + lane];
    }

    if constexpr (G == MM_GATE_UP) {
        // up sums to the gate wavefront of the same columns (the A region is free now)
        float *hand = reinterpret_cast<float *>(lds);  // [CT][NV][64]
        __syncthreads();
        if (upw) {
#pragma unroll
            for (int i = 0; i < NV; i++) hand[((wsub - CT) * NV + i) * 64 + lane] = accv[i];
        }
        __syncthreads();
        if (upw || col0 >= a.n) return;  // uniform per wavefront
        float actv[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint64_t bi = (uint64_t)expert * a.n + min(col0 + colv[i], a.n - 1);
            const float bg = a.bias ? round_bf16(a.bias[bi]) : 0.f;
            const float bu = a.bias2 ? round_bf16(a.bias2[bi] + (a.up_one ? 1.0f : 0.0f)) : (a.up_one ? 1.0f : 0.0f);
            actv[i] = expert_activation(a.act, accv[i] + bg, hand[(wsub * NV + i) * 64 + lane] + bu);
        }
        if (!a.yrec) {
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const uint32_t r = rowv[i], col = col0 + colv[i];
                if (r < rows && col < a.n) reinterpret_cast<float *>(a.y)[(uint64_t)(sorted0 + r) * a.n + col] = actv[i];
            }
            return;
        }
        // The 32 columns are one block of each activation row (n % 32 == 0).
        // The block goes through this wavefront's weight staging region (free
        // now), transposed so that lane r holds row r's 32 values, and each
        // live row's lane splits it into the down projection's record (and,
        // for a lone last block, zeros the partner).
        constexpr uint32_t TRS = 36;  // floats per transposed row (16-byte aligned rows)
        static_assert(32 * TRS * 4 <= WROWS * WSLOT, "the transposed block fits the staging region");
        float *tr = reinterpret_cast<float *>(wlds);
#pragma unroll
        for (int i = 0; i < NV; i++) tr[rowv[i] * TRS + colv[i]] = actv[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if ((uint32_t)lane < rows) {
            const uint32_t blk = col0 / 32, dsteps = (a.n + 63) / 64;
            float v[32];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 f = *reinterpret_cast<const float4 *>(tr + lane * TRS + 4 * q);
                v[4 * q] = f.x;
                v[4 * q + 1] = f.y;
                v[4 * q + 2] = f.z;
                v[4 * q + 3] = f.w;
            }
            uint8_t *rec = a.yrec + ((uint64_t)(sorted0 + lane) * dsteps + blk / 2) * MXR_REC;
            mx6_split_block(v, rec, blk & 1);
            if (!(blk & 1) && blk + 1 == a.n / 32) mx6_zero_block(rec, 1);  // a lone last block
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t r = rowv[i], col = col0 + colv[i];
            if (r >= rows || col >= a.n) continue;
            const float val = accv[i] + (a.bias ? round_bf16(a.bias[(uint64_t)expert * a.n + col]) : 0.f);
            const uint64_t o = (uint64_t)rid[r] * a.n + col;
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[o] = f32_to_bf16_bits(val);
            else
                reinterpret_cast<float *>(a.y)[o] = val;
        }
    }
}

constexpr int MXE_NW = 4;

template <int G, int TR, int KS>
static int mx_experts_go(const MatmulArgs &a, const uint8_t *xrec, hipStream_t stream) {
    const size_t lds = KS * TR * (4 * MXR_REC + 16) + (size_t)MXE_NW * 32 * 176;
    static_assert(TR * (4 * MXR_REC + 16) >= MXE_NW / 2 * 16 * 64 * 4, "the up hand-over fits the A region");
    auto fn = mx_experts_kernel<G, MXE_NW, TR, KS>;
    OCO_TRY(hip_check(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                      "hipFuncSetAttribute"));
    const uint32_t cols = 32 * (G == MM_GATE_UP ? MXE_NW / 2 : MXE_NW) / KS;
    const dim3 grid((a.n + cols - 1) / cols, (a.routes + TR - 1) / TR + a.experts);
    MatmulArgs b = a;
    b.x = xrec;
    hipLaunchKernelGGL(fn, grid, dim3(64 * MXE_NW), lds, stream, KPRE_ARGS(b), b);
    return OCO_OK;
}

template <int G>
static int mx_experts_go_tr(const MatmulArgs &a, const uint8_t *xrec, uint32_t tile_rows, hipStream_t stream) {
    if (tile_rows == 32) return mx_experts_go<G, 32, 1>(a, xrec, stream);
    if constexpr (G == MM_DOWN) {
        // The down tiles can split each tile's K over two halves of the
        // workgroup (OCO_KNOB_MX_EXPERTS_KS 2).  With the four-term
        // activations it no longer pays at any decode batch (gpt-oss, same
        // box: B = 4 72.0 -> 70.2 us without it, B = 6/8/12 81.5/97.3/113.7
        // against 85.7/102.3/119.2 with it), so it runs only when forced.
        int32_t ov[4];
        if (plan_override(OCO_KNOB_MX_EXPERTS_KS, ov) && ov[0] == 2) return mx_experts_go<G, 16, 2>(a, xrec, stream);
    }
    return mx_experts_go<G, 16, 1>(a, xrec, stream);
}

int mx_experts_launch(int mode, const MatmulArgs &a, const uint8_t *xrec, uint32_t tile_rows, hipStream_t stream) {
    if (a.k % 32) return fail(OCO_ERR_INVALID, "experts: MXFP4 rows need k %% 32 == 0 (k=%u)", a.k);
    if (tile_rows != 16 && tile_rows != 32) return fail(OCO_ERR_INVALID, "experts: MXFP4 plan tiles of %u rows", tile_rows);
    // Kernel offsets are 32-bit: the split rows and one expert's matrix each stay under 4 GiB.
    if (mx_rows_bytes(a.routes, a.k) > 0xffffffffull || a.expert_bytes + 4 > 0xffffffffull)
        return fail(OCO_ERR_UNSUPPORTED, "experts: MXFP4 operands over 4 GiB (routes=%u k=%u)", a.routes, a.k);
    const int rc = mode == MM_GATE_UP ? mx_experts_go_tr<MM_GATE_UP>(a, xrec, tile_rows, stream)
                                      : mx_experts_go_tr<MM_DOWN>(a, xrec, tile_rows, stream);
    OCO_TRY(rc);
    return launch_check("experts MXFP4 grouped matmul");
}

}  // namespace oco
