// Per-row split of activations into E4M3 terms for the block-scaled MFMA
// (the split of mxmatmul.hip), stored row-major so that tiles can gather
// arbitrary rows: record (row, K step of 64) =
//     data [term][part 2][block 2][16 B]   (lane part p reads 32 bytes)
//     scales [block 2][4 bytes, byte t = term t] E8M0, padded to 16 bytes
// Two terms hold bf16 inputs exactly; f32 inputs (and the f32 activations
// between gate/up and down) take three: relL2 ~1.4e-5 of the product
// against ~6e-4 with two (numpy model, N(0,1) and SwiGLU-shaped rows).
#pragma once
#include "common.h"

namespace oco {

__host__ __device__ constexpr uint32_t mxr_data(int terms) { return 64u * terms; }
__host__ __device__ constexpr uint32_t mxr_rec(int terms) { return 64u * terms + 16u; }

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

// Max over each half wavefront (lanes 32h .. 32h + 31, all active): DPP
// within rows of 16, then a swap of rows 0 <-> 1 and 2 <-> 3.
__device__ __forceinline__ float half_wave_max(float v) {
    v = fmaxf(v, __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0xB1, 0xf, 0xf, false)));
    v = fmaxf(v, __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0x4E, 0xf, 0xf, false)));
    v = fmaxf(v, __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0x128, 0xf, 0xf, false)));
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// One block (32 values) of a row's K step into its record `rec` (the step's
// record; blk = which of its two blocks), split by 32 lanes together (lanes
// 32h .. 32h + 31, all active), lane i holding value i: per term, the block's
// E8M0 scale (the smallest with amax <= 448 * scale), each value's E4M3 code
// in W's nibble order, and the residual carried to the next term; one byte
// per lane and term.
template <int TERMS>
__device__ __forceinline__ void mx_split_lanes(float x, uint8_t *rec, uint32_t blk) {
    const uint32_t i = threadIdx.x & 31;
    // value i sits at byte e = 2 (i & 7) + i / 16 of part p = (i & 15) / 8
    uint8_t *dst = rec + (((i & 15) >> 3) * 2 + blk) * 16 + 2 * (i & 7) + (i >> 4);
    uint32_t scales = 0;
#pragma unroll
    for (int t = 0; t < TERMS; t++) {
        float amax = half_wave_max(fabsf(x));
        const uint64_t nan = __ballot(x != x) >> (threadIdx.x & 32);
        if ((uint32_t)nan) amax = __uint_as_float(0x7fc00000u);
        const int E = mxe_scale_exp(amax);
        scales |= (uint32_t)(E + 127) << (8 * t);
        const float inv = E == 128 ? 0.f : __builtin_ldexpf(1.f, -E), sc = E == 128 ? 0.f : __builtin_ldexpf(1.f, E);
        const uint32_t code = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x * inv, 0.f, 0, false) & 0xffu;
        x -= __builtin_amdgcn_cvt_f32_fp8((int)code, 0) * sc;
        dst[t * 64] = (uint8_t)code;
    }
    if (i == 0) *reinterpret_cast<uint32_t *>(rec + mxr_data(TERMS) + 4 * blk) = scales;
}


// Item `item` = (row, K step, block) split by the 32 lanes of a half
// wavefront (all active), lane i loading value i.
template <typename XT, int TERMS>
__device__ __forceinline__ void mx_split_item_lanes(const XT *x, uint8_t *rec, uint32_t k, uint64_t item) {
    const uint32_t ksteps = (k + 63) / 64, blk = (uint32_t)(item & 1);
    const uint64_t rs = item >> 1;
    const uint64_t row = rs / ksteps;
    const uint32_t s = (uint32_t)(rs % ksteps), k0 = s * 64 + 32 * blk, i = threadIdx.x & 31;
    float v = 0.f;
    if (k0 < k) {
        if constexpr (sizeof(XT) == 4)
            v = x[row * k + k0 + i];
        else
            v = __uint_as_float((uint32_t)x[row * k + k0 + i] << 16);
    }
    mx_split_lanes<TERMS>(v, rec + (row * ksteps + s) * mxr_rec(TERMS), blk);
}

}  // namespace oco
