// Per-row split of activations into block-scaled FP6 (E2M3) terms for the
// MXFP4 expert tiles' MFMA (v_mfma_scale_f32_32x32x64_f8f6f4 with A in E2M3,
// B the GGUF E2M1 payload), stored row-major so that tiles can gather
// arbitrary rows.  Record (row, K step of 64), 208 bytes:
//     codes16 [term 4][block 2][16 B]   bytes 0..15 of the block's 24-byte codes
//     codes8  [term 4][block 2][8 B]    bytes 16..23
//     scales  [block 2][4 B]            byte t = term t's E8M0 scale
//     pad to 208
// Lane (row, block b) of the MFMA's A operand holds block b as 24 bytes,
// element e in bits 6e .. 6e + 5, element e being block column e / 2 for
// even e and 16 + e / 2 for odd e (the GGUF nibble order of the B payload).
// Four terms x = s1 q1 + s2 q2 + s3 q3 + s4 q4, each with its own E8M0
// scale, leave at most 1/50625 of the block maximum per value (measured
// relative L2 ~1.1e-6 on the expert layers, inside the 1e-5 bar of fp32
// activations; three terms measured 3-5e-5).
#pragma once
#include "common.h"

namespace oco {

constexpr int MX_TERMS = 4;
static_assert(MX_TERMS >= 1 && MX_TERMS <= 4, "one E8M0 scale byte per term in a 32-bit word");
constexpr uint32_t MXR_CODES8 = 32u * MX_TERMS;          // offset of the 8-byte parts
constexpr uint32_t MXR_SCALES = MXR_CODES8 + 16u * MX_TERMS;  // offset of the scale words
constexpr uint32_t MXR_REC = MXR_SCALES + 16u;           // record bytes (a multiple of 16)
static_assert(MXR_REC % 16 == 0, "records are whole 16-byte pieces");

typedef float mx_f32x16 __attribute__((ext_vector_type(16)));
typedef float mx_f32x32 __attribute__((ext_vector_type(32)));
typedef int mx_i32x6 __attribute__((ext_vector_type(6)));

// Smallest E with amax <= 7.5 * 2^E (7.5 = 1.875 * 2^2, the largest E2M3
// value), as E; 128 (the NaN byte) for a non-finite block, -127 at least.
// amax_bits: |x| as f32 bits (NaN and Inf order above every finite value).
__device__ __forceinline__ int mx6_scale_exp(uint32_t amax_bits) {
    if (amax_bits >= 0x7f800000u) return 128;
    if (amax_bits == 0) return -127;
    int e;
    uint32_t mant;
    if (amax_bits >> 23) {
        e = (int)(amax_bits >> 23) - 127;
        mant = amax_bits & 0x7fffffu;
    } else {  // subnormal amax: normalise
        const int lz = __builtin_clz(amax_bits) - 8;
        e = -126 - lz;
        mant = (amax_bits << lz) & 0x7fffffu;
    }
    const int E = mant <= 0x700000u ? e - 2 : e - 1;  // m <= 1.875 <=> m * 2^e <= 7.5 * 2^(e - 2)
    return E < -127 ? -127 : E;
}

// E2M3 codes of 32 values: position 2i takes lo[i], 2i + 1 hi[i] (measured
// on gfx950).  The asm statement keeps the sources live until the result
// exists: hipcc otherwise may give the result registers that overlap the
// sources, and the instruction then reads inputs it has already overwritten
// (seen: v_cvt_scalef32_2xpk16_fp6_f32 v[34:39], v[32:47], v[0:15]).
__device__ __forceinline__ mx_i32x6 fp6_pack(const mx_f32x16 &lo, const mx_f32x16 &hi) {
    mx_i32x6 c = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(lo, hi, 1.0f);
    asm volatile("" ::"v"(lo), "v"(hi), "v"(c));
    return c;
}
// The 32 values of E2M3 codes, in position order (same register rule).
__device__ __forceinline__ mx_f32x32 fp6_unpack(const mx_i32x6 &c) {
    mx_f32x32 d = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(c, 1.0f);
    asm volatile("" ::"v"(c), "v"(d));
    return d;
}

// One block (32 values v, block column order) into block b of record rec,
// by one lane: per term, the block's E8M0 scale s (the smallest power of two
// with max |v| / s <= 7.5), the codes of v / s, and the residual v - s q,
// exact in f32, carried to the next term.  A non-finite block gets the NaN
// scale byte in every term.
__device__ __forceinline__ void mx6_split_block(float v[32], uint8_t *rec, uint32_t b) {
    uint32_t scales = 0;
#pragma unroll
    for (int t = 0; t < MX_TERMS; t++) {
        // |x| bit patterns order like the values, with Inf above every finite
        // value and NaN above Inf: the integer maximum carries both (a tree:
        // five dependent steps, not 31).
        uint32_t mt[16];
#pragma unroll
        for (int i = 0; i < 16; i++) mt[i] = max(__float_as_uint(v[i]) & 0x7fffffffu, __float_as_uint(v[16 + i]) & 0x7fffffffu);
#pragma unroll
        for (int w = 8; w > 0; w >>= 1)
#pragma unroll
            for (int i = 0; i < w; i++) mt[i] = max(mt[i], mt[i + w]);
        const int E = mx6_scale_exp(mt[0]);
        scales |= (uint32_t)(E + 127) << (8 * t);
        const float inv = E == 128 ? 0.f : __builtin_ldexpf(1.f, -E), sc = E == 128 ? 0.f : __builtin_ldexpf(1.f, E);
        mx_f32x16 lo, hi;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            lo[i] = v[i] * inv;
            hi[i] = v[16 + i] * inv;
        }
        const mx_i32x6 c = fp6_pack(lo, hi);
        *reinterpret_cast<u32x4 *>(rec + 32 * t + 16 * b) = u32x4{(uint32_t)c[0], (uint32_t)c[1], (uint32_t)c[2], (uint32_t)c[3]};
        *reinterpret_cast<u32x2 *>(rec + MXR_CODES8 + 16 * t + 8 * b) = u32x2{(uint32_t)c[4], (uint32_t)c[5]};
        if (t + 1 < MX_TERMS) {
            const mx_f32x32 d = fp6_unpack(c);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                v[i] -= d[2 * i] * sc;
                v[16 + i] -= d[2 * i + 1] * sc;
            }
        }
    }
    *reinterpret_cast<uint32_t *>(rec + MXR_SCALES + 4 * b) = scales;
}

// Block b of record rec as zeros (codes 0, scale bytes 0): the partner of a
// row's lone last block.
__device__ __forceinline__ void mx6_zero_block(uint8_t *rec, uint32_t b) {
#pragma unroll
    for (int t = 0; t < MX_TERMS; t++) {
        *reinterpret_cast<u32x4 *>(rec + 32 * t + 16 * b) = u32x4{0, 0, 0, 0};
        *reinterpret_cast<u32x2 *>(rec + MXR_CODES8 + 16 * t + 8 * b) = u32x2{0, 0};
    }
    *reinterpret_cast<uint32_t *>(rec + MXR_SCALES + 4 * b) = 0;
}

// Item `item` = (row, K step, block) of k-wide rows x, split by one lane
// into the records rec [rows][K steps]; values past k are zero.
template <typename XT>
__device__ __forceinline__ void mx6_split_item(const XT *x, uint8_t *rec, uint32_t k, uint64_t item) {
    const uint32_t ksteps = (k + 63) / 64, b = (uint32_t)(item & 1);
    const uint64_t rs = item >> 1;
    const uint64_t row = rs / ksteps;
    const uint32_t s = (uint32_t)(rs % ksteps), k0 = s * 64 + 32 * b;
    float v[32];
    if (k0 < k && ((uintptr_t)x & 15u)) {  // rows off a 16-byte boundary: element loads
#pragma unroll
        for (int i = 0; i < 32; i++) {
            if constexpr (sizeof(XT) == 4)
                v[i] = reinterpret_cast<const float *>(x)[row * k + k0 + i];
            else
                v[i] = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(x)[row * k + k0 + i] << 16);
        }
    } else if (k0 < k) {  // k % 32 == 0: the whole block is in the row
        if constexpr (sizeof(XT) == 4) {
            const auto src = gp(reinterpret_cast<const u32x4 *>(x + row * k + k0));
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const u32x4 u = src[q];
                v[4 * q] = __uint_as_float(u.x);
                v[4 * q + 1] = __uint_as_float(u.y);
                v[4 * q + 2] = __uint_as_float(u.z);
                v[4 * q + 3] = __uint_as_float(u.w);
            }
        } else {
            const auto src = gp(reinterpret_cast<const u32x4 *>(x + row * k + k0));
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const u32x4 u = src[q];
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    v[8 * q + 2 * j] = __uint_as_float(w[j] << 16);
                    v[8 * q + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = 0.f;
    }
    uint8_t *r = rec + (row * ksteps + s) * MXR_REC;
    if (k0 < k)
        mx6_split_block(v, r, b);
    else
        mx6_zero_block(r, b);
}

}  // namespace oco
