// RMS normalisation pieces shared by the standalone norm kernels and the
// streaming matvec's fused-norm staging (elementwise.metal:6-58).
#pragma once
#include "common.h"

namespace oco {

// 1 / sqrt(mean(x^2) + epsilon) of one bf16 row, by a 256-thread workgroup
// (every thread gets the value).  Fixed order: thread t accumulates, with
// fmaf, the 8-element runs t, t + 256, t + 512, ... (elements 8 c .. 8 c + 7
// of run c, read as one 16-byte load when the row is 16-byte aligned); each
// wavefront reduces with wave_sum; the four wavefront sums are added in
// order.  `partial` is 4 floats of LDS.  Ends with a barrier, so `partial`
// may be reused right after.
__device__ __forceinline__ float block_inv_rms(const uint16_t *xr, uint32_t n, float epsilon, float *partial) {
    float s = 0.f;
    const bool vec = ((uintptr_t)xr & 15u) == 0;
    for (uint32_t c = threadIdx.x; 8 * c < n; c += 256) {
        float v[8];
        if (vec && 8 * c + 8 <= n) {
            const uint4 u = *reinterpret_cast<const uint4 *>(xr + 8 * c);
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[2 * j] = __uint_as_float(w4[j] << 16);
                v[2 * j + 1] = __uint_as_float(w4[j] & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 8 * c + j < n ? bf16_bits_to_f32(xr[8 * c + j]) : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) s = fmaf(v[j], v[j], s);
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = s;
    __syncthreads();
    const float total = ((partial[0] + partial[1]) + partial[2]) + partial[3];
    __syncthreads();
    return 1.0f / sqrtf(total / (float)n + epsilon);
}

// One normalised element, rounded as the reference does
// (elementwise.metal:24-26): full_layer: bf16(x inv w); else
// bf16(bf16(x inv) * bf16(w)).
__device__ __forceinline__ uint16_t norm_value_bits(float x, float inv, float w, uint32_t full_layer) {
    const float t = x * inv;
    return full_layer ? f32_to_bf16_bits(t * w) : f32_to_bf16_bits(round_bf16(t) * round_bf16(w));
}

}  // namespace oco
