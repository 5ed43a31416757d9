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

// Tile: one route-plan tile of up to 32 routes; each wavefront owns one
// 32-column tile (gate/up: the 32 gate rows and the same 32 up rows, the
// activation fused in-lane).  A (the routes' split rows) and B (the GGUF
// bytes, each used by this wavefront only) are loaded straight into
// registers, D K steps ahead.
template <int G, int NW, int D, int TERMS>
__global__ __launch_bounds__(64 * NW) void mx_experts_kernel(MatmulArgs a, const uint8_t *xrec) {
    constexpr int NT = G == MM_GATE_UP ? 2 : 1;  // weight tiles per wavefront
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane & 31, part = lane >> 5;
    const uint32_t used = gridDim.x * min(a.plan[1], gridDim.y);
    const uint32_t lin = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, used);
    if (lin >= used) return;  // uniform: a surplus workgroup
    const uint32_t bx = lin % gridDim.x, y = lin / gridDim.x;
    const uint32_t expert = a.plan[6 + 2 * y], first = a.plan[7 + 2 * y];
    const uint64_t grouped = 6 + 2 * ((uint64_t)(a.routes + 15) / 16 + a.experts);
    const uint64_t list = grouped + (uint64_t)expert * (a.routes + 1);
    const uint64_t sorted = grouped + (uint64_t)a.experts * (a.routes + 1);
    const uint32_t rows = min(32u, a.plan[list] - first);
    const uint32_t sorted0 = a.plan[sorted + expert] + first;
    const uint32_t col0 = (bx * NW + wave) * 32;
    if (col0 >= a.n) return;  // uniform per wavefront; no barrier below
    const uint32_t ksteps = (a.k + 63) / 64, nblk = a.k / 32;

    // A: this lane's row (c) of the tile; rows past the tile read row 0 and are zeroed.
    const bool alive = (uint32_t)c < rows;
    const uint32_t amask = alive ? 0xffffffffu : 0u;
    uint32_t arow = 0;
    if (alive) arow = G == MM_GATE_UP ? a.plan[list + 1 + first + c] / a.topk : sorted0 + c;
    const uint8_t *ar = xrec + (uint64_t)arow * ksteps * mxr_rec(TERMS);
    // B: each wavefront stages its own weight rows' bytes for the step
    // through a private LDS region.  Per tile, row (32) x the step's two
    // blocks (34 bytes) are fetched as the dword-aligned span holding them,
    // ten consecutive lanes per row (coalesced; per-lane block loads would
    // touch 32-64 cache lines per instruction and saturate address
    // processing).  Slots are 11 dwords (odd: conflict-free fragment reads).
    constexpr int SLOT = 44, BU = 5 * NT;  // 32 rows x 10 dwords = 5 wavefront loads per tile
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t *wlds = lds + wave * (NT * 32 * SLOT);
    const uint8_t *bbase[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) bbase[j] = (j ? a.w2 : a.w) + expert * a.expert_bytes;
    uint32_t boff[BU];  // row offset within the expert's matrix (< 4 GiB)
#pragma unroll
    for (int u = 0; u < 5; u++) {
        const int row = (lane + 64 * u) / 10;
        boff[u] = min(col0 + row, a.n - 1) * (uint32_t)a.row_bytes;
#pragma unroll
        for (int j = 1; j < NT; j++) boff[5 * j + u] = boff[u];
    }
    uint32_t wlow[NT];  // this lane's row address mod 4 (the span alignment)
#pragma unroll
    for (int j = 0; j < NT; j++)
        wlow[j] = (uint32_t)(uintptr_t)((j ? a.w2 : a.w) + expert * a.expert_bytes +
                                        (uint64_t)min(col0 + c, a.n - 1) * a.row_bytes) & 3u;

    // Loads land in a stage untouched; masks apply when the stage is used,
    // so no load is waited for before its step comes round.
    struct Stage {
        uint4 a[TERMS][2];  // [term][block]
        uint32_t sa;
        uint32_t rb[BU];  // raw weight dwords
        uint32_t s;       // the K step held
    };
    auto load = [&](Stage &st, uint32_t s) __attribute__((always_inline)) {
        s = min(s, ksteps - 1);
        st.s = s;
        const uint8_t *r = ar + (uint64_t)s * mxr_rec(TERMS);
#pragma unroll
        for (int t = 0; t < TERMS; t++) {
            const uint4 *d = reinterpret_cast<const uint4 *>(r + (t * 2 + part) * 32);
            st.a[t][0] = d[0];
            st.a[t][1] = d[1];
        }
        st.sa = *reinterpret_cast<const uint32_t *>(r + mxr_data(TERMS) + 4 * part);
        const uint32_t len = 2 * s + 1 < nblk ? 34 : 17;
#pragma unroll
        for (int u = 0; u < BU; u++) {
            const uint32_t d = (lane + 64 * (u % 5)) % 10;
            const uint8_t *pb = bbase[u / 5] + boff[u] + s * 34;
            const uint32_t lo = (uint32_t)(uintptr_t)pb & 3u, last = (lo + len - 1) / 4;
            // only dwords holding bytes of this step's blocks
            st.rb[u] = *reinterpret_cast<const uint32_t *>(pb - lo + 4 * min(d, last));
        }
    };
    mxe_f32x16 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) acc[j] = mxe_f32x16{};
    auto step = [&](const Stage &st) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < BU; u++) {
            const uint32_t f = lane + 64 * (u % 5);
            *reinterpret_cast<uint32_t *>(wlds + ((u / 5) * 32 + f / 10) * SLOT + (f % 10) * 4) = st.rb[u];
        }
        // dead rows of the tile contribute zeros; the lone last block's
        // partner is zero with scale 1
        const bool live = 2 * st.s + part < nblk;
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const uint8_t *row = wlds + (j * 32 + c) * SLOT;
            const uint32_t off = ((wlow[j] + 34 * st.s) & 3u) + 17 * part;  // scale byte of block 2s + part
            uint32_t q[4];
            lds_bytes<16>(row + off + 1, q);
            const mxe_i32x8 bv = live ? mxe_i32x8{(int)q[0], (int)q[1], (int)q[2], (int)q[3], 0, 0, 0, 0} : mxe_i32x8{};
            const int sb = live ? (int)row[off] : 127;
#pragma unroll
            for (int t = 0; t < TERMS; t++) {
                const mxe_i32x8 av{(int)(st.a[t][0].x & amask), (int)(st.a[t][0].y & amask),
                                   (int)(st.a[t][0].z & amask), (int)(st.a[t][0].w & amask),
                                   (int)(st.a[t][1].x & amask), (int)(st.a[t][1].y & amask),
                                   (int)(st.a[t][1].z & amask), (int)(st.a[t][1].w & amask)};
                if (t == 0)
                    acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[j], 0, 4, 0, (int)st.sa, 0, sb);
                else if (t == 1)
                    acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[j], 0, 4, 1, (int)st.sa, 0, sb);
                else
                    acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[j], 0, 4, 2, (int)st.sa, 0, sb);
            }
        }
    };
    Stage st[D];
#pragma unroll
    for (int u = 0; u < D; u++) load(st[u], u);
    uint32_t s = 0;
    for (; s + D <= ksteps; s += D) {  // whole rounds: no branch between a load and its use
#pragma unroll
        for (int u = 0; u < D; u++) {
            step(st[u]);
            load(st[u], s + u + D);
        }
    }
#pragma unroll
    for (int u = 0; u < D; u++)
        if (s + u < ksteps) step(st[u]);

    // C: lane l holds column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4.
    const uint32_t col = col0 + c;
    if (col >= a.n) return;
    const uint64_t bi = (uint64_t)expert * a.n + col;
    if constexpr (G == MM_GATE_UP) {
        const float bg = a.bias ? round_bf16(a.bias[bi]) : 0.f;
        const float bu = a.bias2 ? round_bf16(a.bias2[bi] + (a.up_one ? 1.0f : 0.0f)) : (a.up_one ? 1.0f : 0.0f);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const uint32_t r = 8 * (v / 4) + 4 * part + (v % 4);
            if (r < rows)
                reinterpret_cast<float *>(a.y)[(uint64_t)(sorted0 + r) * a.n + col] =
                    expert_activation(a.act, acc[0][v] + bg, acc[1][v] + bu);
        }
    } else {
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

constexpr int MXE_NW = 4, MXE_D = 2;

template <int G, int TERMS>
static void mx_experts_go(const MatmulArgs &a, const uint8_t *xrec, dim3 grid, hipStream_t stream) {
    const size_t lds = (size_t)MXE_NW * (G == MM_GATE_UP ? 2 : 1) * 32 * 44;
    hipLaunchKernelGGL((mx_experts_kernel<G, MXE_NW, MXE_D, TERMS>), grid, dim3(64 * MXE_NW), lds, stream, a, xrec);
}

int mx_experts_launch(int mode, const MatmulArgs &a, const uint8_t *xrec, int terms, hipStream_t stream) {
    if (a.k % 32) return fail(OCO_ERR_INVALID, "experts: MXFP4 rows need k %% 32 == 0 (k=%u)", a.k);
    const uint32_t cols = 32 * MXE_NW;
    const dim3 grid((a.n + cols - 1) / cols, (a.routes + 31) / 32 + a.experts);
    if (mode == MM_GATE_UP)
        terms == 2 ? mx_experts_go<MM_GATE_UP, 2>(a, xrec, grid, stream) : mx_experts_go<MM_GATE_UP, 3>(a, xrec, grid, stream);
    else
        terms == 2 ? mx_experts_go<MM_DOWN, 2>(a, xrec, grid, stream) : mx_experts_go<MM_DOWN, 3>(a, xrec, grid, stream);
    return launch_check("experts MXFP4 grouped matmul");
}

}  // namespace oco
