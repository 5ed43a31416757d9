// Shared by the prefill matmul and the routed-expert prefill path.
#pragma once

#include "common.h"

namespace oco {

// The first 56 bytes arrive in SGPRs (KPre): the fields the tiles' first
// loads depend on come first.
struct MatmulArgs {
    const uint32_t *desc;  // MXFP4 expert tiles: the route plan's tile descriptors (route.h)
    const uint32_t *plan;  // grouped (routed-expert) mode: route plan with tile_rows = BM
    const uint8_t *w;
    const uint8_t *w2;     // up weights (gate/up mode)
    const void *x;         // activations (MXFP4 expert tiles: their E2M3 split records)
    uint32_t n, k;
    uint32_t row_bytes;    // bytes of one weight row (< 4 GiB)
    uint32_t routes, experts, topk;
    uint64_t expert_bytes; // bytes of one expert's matrix
    void *y;
    const float *bias;
    uint32_t m;
    uint32_t x_f16, y_bf16;
    const float *bias2;    // up bias (gate/up mode)
    uint32_t act, up_one;
    uint32_t *rowmax;      // [routes] max |activation| bits per expert-sorted row (gate/up writes, down reads)
    uint8_t *yrec;         // MXFP4 gate/up: the activations' E2M3 split records in place of f32 rows (or null)
    // MXFP4 gate/up at small decode batches (route.h's in-workgroup plan):
    // `small` set, the plan is built from `logits` (selection; ids_out and
    // probs_out receive it) or from `ids`, and written to desc_out / plan_out
    // for the down launch
    uint32_t small;
    const float *logits;
    const uint32_t *ids;
    uint32_t *ids_out;
    float *probs_out;
    uint32_t *desc_out, *plan_out;
};

// Power of two that brings a row with max |value| `bits` (f32 bits) into
// [2^14, 2^15) -- f16 range with its full precision; 1 for zero or
// non-finite rows.
__device__ __forceinline__ float row_gain(uint32_t bits) {
    if (bits == 0 || bits >= 0x7f800000u) return 1.0f;
    const int e = (int)(bits >> 23) - 127;  // floor(log2(max)), subnormals count as 2^-127
    return __builtin_ldexpf(1.0f, max(-100, min(100, 14 - e)));
}

// Four weights from the nibbles of one dword (one per byte, high nibbles
// clear), rounded to f16 as a * q - m (the reference's scale * value -
// minimum, then half(); a * q is exact in f32):
//   - a byte c < 16 read as E4M3 is c * 2^-9 (exponent 0: c/8 * 2^-6;
//     exponent 1: (8 + c - 8)/8 * 2^-6), so v_cvt_scalef32_pk_f32_fp8 with
//     scale 2^9 gives two exact f32 codes per instruction;
//   - v_fma_f32 gives fl32(a q - m); v_cvt_pk_f16_f32 rounds a pair to f16.
// Measured on gfx950, this costs about two thirds of v_cvt_f32_ubyte +
// v_fma_mix{lo,hi}_f16 per weight (the mixed-precision FMA issues at a
// fraction of the full rate).
typedef float q4f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void q4_four(uint32_t n, float a, float m, uint32_t &p01, uint32_t &p23) {
    const q4f32x2 c01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(n, 512.0f, false);
    const q4f32x2 c23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(n, 512.0f, true);
    const float f0 = __builtin_fmaf(a, c01[0], -m), f1 = __builtin_fmaf(a, c01[1], -m);
    const float f2 = __builtin_fmaf(a, c23[0], -m), f3 = __builtin_fmaf(a, c23[1], -m);
    // inline asm keeps the compiler from folding each FMA and its conversion
    // back into a mixed-precision FMA
    asm volatile("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(p01) : "v"(f0), "v"(f1));
    asm volatile("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(p23) : "v"(f2), "v"(f3));
}

// Grouped modes of matmul_kernel.
constexpr int MM_DENSE = 0;  // Y = X W^T
constexpr int MM_GATE_UP = 1;  // per expert tile: act = f(X W_gate^T, X W_up^T), f32 at expert-sorted rows
constexpr int MM_DOWN = 2;     // per expert tile: routed[route] = act W_down^T (+ bias), f32

// Expert activations (projections.metal:4-13 clipped SwiGLU; elementwise.metal:
// 70-88 SwiGLU), in f32; non-finite inputs give NaN.
__device__ __forceinline__ float expert_activation(uint32_t act, float g, float u) {
    if ((__float_as_uint(g) & 0x7f800000u) == 0x7f800000u || (__float_as_uint(u) & 0x7f800000u) == 0x7f800000u)
        return __uint_as_float(0x7fc00000u);
    float scale = 1.0f;
    if (act == OCO_ACT_SWIGLU_CLIPPED) {
        g = fminf(g, 7.0f);
        u = fminf(fmaxf(u, -6.0f), 8.0f);
        scale = 1.702f;
    }
    const float e = expf(-fabsf(g) * scale);
    const float sig = (g < 0 ? e : 1.0f) / (1.0f + e);
    return sig * g * u;
}

// One grouped GEMM over a route plan built with tile_rows = bm (32 or 64):
// MM_GATE_UP writes f32 activations at expert-sorted rows and each row's
// max |activation| (rowmax, zeroed by the caller); MM_DOWN reads them with
// a per-row power-of-two gain into f16 and writes f32 (or bf16) route rows.
int grouped_matmul_launch(int mode, uint32_t fmt, const MatmulArgs &a, uint32_t bm, hipStream_t stream);

// The same for Q4_K banks with weights decoded in registers (route plan with
// tile_rows = bm: 32, 48 or 64).
int moe_q4k_launch(int mode, const MatmulArgs &a, uint32_t bm, hipStream_t stream);

// MXFP4 banks on the block-scaled MFMA: activations split per row into three
// E2M3 terms (mxsplit.h; mx_rows_bytes each matrix) -- the inputs beside the
// router or the route plan, the activations by the gate/up tiles -- route
// plan with tile_rows = 16 or 32.
uint64_t mx_rows_bytes(uint32_t rows, uint32_t k);
int mx_experts_launch(int mode, const MatmulArgs &a, const uint8_t *xrec, uint32_t tile_rows, hipStream_t stream);

}  // namespace oco
