// Shared device and host helpers of the gfx950 matrix path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/oco_hip.h"

// ---- host-side status plumbing ---------------------------------------------
namespace oco {
int fail(int code, const char *fmt, ...);   // records the message, returns code
int hip_check(hipError_t e, const char *what);
int launch_check(const char *what);        // hipGetLastError after a launch
// Kernel-choice override set through oco_plan_override (tests and tuning
// runs); copies up to 4 values into vals and returns their count, 0 when the
// knob is not overridden (the built-in choice table applies).
int plan_override(uint32_t knob, int32_t *vals);
// Resolve the device address of the experts' static scratch array on
// `device` (the current device), once per device.
int experts_scratch_init(int device);
}  // namespace oco

#define OCO_TRY(expr)              \
    do {                           \
        int _rc = (expr);          \
        if (_rc != OCO_OK) return _rc; \
    } while (0)

// ---- device helpers ----------------------------------------------------------
namespace oco {

typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bits_f32(uint32_t u) { return __uint_as_float(u); }

// IEEE half -> float (denormals kept: f16 denormals are enabled on gfx950).
__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
    _Float16 v;
    uint16_t b = (uint16_t)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// A pointer in the global address space.  Pointers unpacked from the
// preloaded argument words (KPRE_APPLY) are generic to the compiler, so
// their loads and stores become FLAT operations, which count in lgkmcnt as
// well as vmcnt: every LDS wait behind them then also waits for memory
// (measured: a store loop with an LDS read per iteration went from ~700 to
// a few clocks per iteration as global stores).
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T *gp(T *p) {
    return (__attribute__((address_space(1))) T *)p;
}

// A buffer resource the compiler keeps in SGPRs: every field goes through
// readfirstlane (the values are uniform; without this a resource built next
// to divergent code may land in VGPRs and every load becomes a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void *p, uint32_t bytes) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(uintptr_t)(((uint64_t)hi << 32) | lo), 0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// float -> bf16 bits, round to nearest even, NaN stays quiet.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Unaligned little-endian loads from GGUF byte streams (gfx950 global
// loads accept any byte alignment; the compiler emits single dword loads).
__device__ __forceinline__ uint32_t ld_u8(const uint8_t *p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint2 ld_u64(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

// The same loads through global-address-space pointers (gp below): global
// instructions instead of FLAT ones.  A FLAT load counts in lgkmcnt as well
// as vmcnt, so in a kernel that also uses LDS every wait for an LDS read
// waits for the FLAT loads issued before it -- weight prefetches included.
#define GLOBAL __attribute__((address_space(1)))
typedef const GLOBAL uint8_t *gbytes;
typedef uint16_t u16_u __attribute__((aligned(1)));
typedef uint32_t u32_u __attribute__((aligned(1)));
typedef uint32_t u32x2_u __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32x4_u __attribute__((ext_vector_type(4), aligned(1)));
__device__ __forceinline__ uint32_t ld_u8(gbytes p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16(gbytes p) { return *(const GLOBAL u16_u *)p; }
__device__ __forceinline__ uint32_t ld_u32(gbytes p) { return *(const GLOBAL u32_u *)p; }
__device__ __forceinline__ uint2 ld_u64(gbytes p) {
    const u32x2_u v = *(const GLOBAL u32x2_u *)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint4 ld_u128(gbytes p) {
    const u32x4_u v = *(const GLOBAL u32x4_u *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Streamed weight bytes are read through a buffer resource: loads carry the
// nontemporal hint (read once per call, so they should not displace the
// activations from L2/MALL), accept any byte offset, and return zero past
// `bytes` (so tail rows need no clamping).  Offsets are 32-bit: one
// resource covers at most 4 GiB, so kernels build one per row group.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
struct WSrc {
    __amdgpu_buffer_rsrc_t r;
    __device__ __forceinline__ WSrc(const uint8_t *base, uint64_t bytes) {
        uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
        r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, n, 0x00020000);
    }
    static constexpr int NT = 2;  // cache policy: nontemporal
    __device__ __forceinline__ uint32_t u8(uint32_t off) const {
        return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, NT);
    }
    __device__ __forceinline__ uint32_t u16(uint32_t off) const {
        return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, NT);
    }
    __device__ __forceinline__ uint32_t u32(uint32_t off) const {
        return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, NT);
    }
    __device__ __forceinline__ uint2 u64(uint32_t off) const {
        u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, NT);
        return make_uint2(v.x, v.y);
    }
    __device__ __forceinline__ uint4 u128(uint32_t off) const {
        u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, NT);
        return make_uint4(v.x, v.y, v.z, v.w);
    }
};

// Kernel arguments in preloaded SGPRs.  The command processor preloads the
// leading scalar (and vector) kernel arguments into SGPRs when the code is
// built with -amdgpu-kernarg-preload-count, but not a struct passed by
// value, whose fields the waves then fetch from the kernarg segment before
// anything that depends on them can start.  Kernels that take a parameter
// struct therefore also take its first 56 bytes as four vector arguments
// (KPRE_PARAMS), launched with KPRE_ARGS(s), and overwrite the struct's
// head with them (kpre_apply), so the fields laid out first in each struct
// are read from SGPRs.
struct KPre {
    u32x4 a, b, c;
    u32x2 d;
};
constexpr size_t KPRE_BYTES = 56;
template <class S>
inline KPre kpre(const S &s) {
    KPre k;
    memset(&k, 0, sizeof k);
    memcpy(&k, &s, sizeof(S) < KPRE_BYTES ? sizeof(S) : KPRE_BYTES);
    return k;
}
template <class S>
__device__ __forceinline__ void kpre_apply(S &s, u32x4 a, u32x4 b, u32x4 c, u32x2 d) {
    const uint32_t w[14] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, d.x, d.y};
    __builtin_memcpy(&s, w, sizeof(S) < KPRE_BYTES ? sizeof(S) : KPRE_BYTES);
}
#define KPRE_PARAMS u32x4 kpre_a, u32x4 kpre_b, u32x4 kpre_c, u32x2 kpre_d
#define KPRE_APPLY(s) kpre_apply(s, kpre_a, kpre_b, kpre_c, kpre_d)
#define KPRE_ARGS(s) kpre(s).a, kpre(s).b, kpre(s).c, kpre(s).d

// E8M0 shared exponent: finite powers exact, 0 -> 2^-127, 255 -> NaN
// (projections.metal:19-23).
__device__ __forceinline__ float e8m0_scale(uint32_t e) {
    float s = e == 0 ? bits_f32(0x00400000u) : bits_f32(e << 23);
    return e == 255 ? bits_f32(0x7fc00000u) : s;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// Full wave64 sum, result in every lane: DPP butterflies inside each
// 16-lane row (quad_perm [1,0,3,2], [2,3,0,1], row_ror 4, row_ror 8), then
// gfx950's permlane16/32 swaps across rows.  All VALU, no LDS round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x124>(v);
    v += dpp_f32<0x128>(v);
    auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
    auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
}

// Activation element loads, f32 or bf16 (bits in uint16_t).
struct bf16_t {
    uint16_t bits;
};

template <typename XT>
struct XLoad;
// The relu² input transform of the vector kernels (weights.metal:22-24,
// vector.metal:120-123): the positive part of x, squared in f32.  max
// returns its non-NaN operand, so NaN inputs become 0, as Metal's max does.
__device__ __forceinline__ float relu_sqr(float v) {
    const float r = fmaxf(v, 0.f);
    return r * r;
}

template <>
struct XLoad<float> {
    // n contiguous values starting at p (n multiple of 4, p 16-byte aligned
    // whenever k is a multiple of 4), squared positive parts when rs.
    template <int N>
    __device__ __forceinline__ static void run(const float *p, float *out, bool rs = false) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            float4 v = *reinterpret_cast<const float4 *>(p + i);
            out[i] = v.x;
            out[i + 1] = v.y;
            out[i + 2] = v.z;
            out[i + 3] = v.w;
        }
        if (rs) {
#pragma unroll
            for (int i = 0; i < N; i++) out[i] = relu_sqr(out[i]);
        }
    }
    __device__ __forceinline__ static float one(const float *p, uint64_t i) { return p[i]; }
};
template <>
struct XLoad<bf16_t> {
    template <int N>
    __device__ __forceinline__ static void run(const bf16_t *p, float *out, bool rs = false) {
#pragma unroll
        for (int i = 0; i < N; i += 8) {
            uint4 v = *reinterpret_cast<const uint4 *>(p + i);
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                out[i + 2 * j] = __uint_as_float(w[j] << 16);
                out[i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            }
        }
        if (rs) {
#pragma unroll
            for (int i = 0; i < N; i++) out[i] = relu_sqr(out[i]);
        }
    }
    __device__ __forceinline__ static float one(const bf16_t *p, uint64_t i) {
        return bf16_bits_to_f32(p[i].bits);
    }
};

// XCD-aware workgroup order.  MI355X dispatches workgroup p (linear id) to
// XCD p % 8, and each XCD has its own L2.  xcd_order(p, used) renumbers the
// first `used` logical ids so that XCD x runs one contiguous range of them,
// evenly split: workgroups that share operands, when numbered consecutively,
// then share one L2.  Surplus workgroups (grids sized for a bound known only
// on the device) get `used` and exit.
constexpr uint32_t XCDS = 8;
__device__ __forceinline__ uint32_t xcd_order(uint32_t p, uint32_t used) {
    const uint32_t q = used / XCDS, r = used % XCDS, x = p % XCDS, slot = p / XCDS;
    return slot < q + (x < r ? 1u : 0u) ? x * q + min(x, r) + slot : used;
}

}  // namespace oco
