// GGUF block formats on gfx950: exact scalar decode (dequantization) and the
// per-lane "piece" decoders the matvec kernels stream through.
//
// A row of k coefficients is k/BLOCK consecutive GGUF blocks of BYTES bytes
// (src/tensor.rs:24-38).  In the matvec kernels P lanes share one block, each
// lane decoding one piece of E = BLOCK/P coefficients with a single wide
// load, so a wavefront step covers 64/P consecutive blocks of a row in one
// contiguous span (coalesced 8- or 16-byte loads; MXFP4/Q8_0/Q6_K blocks are
// not 4-byte aligned and rely on gfx950's unaligned global loads).
//
// Piece decoders factor the block's affine terms out of the dot product:
// sum_i (a q_i - b) x_i = a sum_i q_i x_i - b sum_i x_i, with the activation
// sums computed once per lane and shared by every row that lane visits.
// Integer codes convert exactly; products accumulate in fp32.
#pragma once
#include "common.h"

namespace oco {

// ---------------------------------------------------------------------------
// Exact scalar decode of element j of one block: weights.metal:48-85.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void kquant_scale_min(const uint8_t *scales, uint32_t s, uint32_t &sc,
                                                 uint32_t &mn) {
    if (s < 4) {
        sc = scales[s] & 63u;
        mn = scales[s + 4] & 63u;
    } else {
        sc = (scales[s + 4] & 15u) | ((scales[s - 4] >> 6) << 4);
        mn = (scales[s + 4] >> 4) | ((scales[s] >> 6) << 4);
    }
}

__device__ __forceinline__ float decode_scalar(uint32_t fmt, const uint8_t *b, uint32_t j) {
    switch (fmt) {
    case OCO_F32: return __uint_as_float(ld_u32(b));
    case OCO_F16: return half_bits_to_f32(ld_u16(b));
    case OCO_BF16: return bf16_bits_to_f32(ld_u16(b));
    case OCO_Q4_0: {
        uint32_t q = (b[2 + j % 16] >> (j / 16 * 4)) & 15u;
        return half_bits_to_f32(ld_u16(b)) * (float)((int)q - 8);
    }
    case OCO_Q4_1: {
        uint32_t q = (b[4 + j % 16] >> (j / 16 * 4)) & 15u;
        return __fadd_rn(__fmul_rn(half_bits_to_f32(ld_u16(b)), (float)q),
                         half_bits_to_f32(ld_u16(b + 2)));
    }
    case OCO_Q8_0: return half_bits_to_f32(ld_u16(b)) * (float)(int8_t)b[2 + j];
    case OCO_MXFP4: {
        uint32_t q = (b[1 + j % 16] >> (j / 16 * 4)) & 15u;
        const float mag[8] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
        float v = (q & 8) ? -mag[q & 7] : mag[q & 7];
        return v * e8m0_scale(b[0]);
    }
    case OCO_Q4_K:
    case OCO_Q5_K: {
        uint32_t s = j / 32, sc, mn;
        kquant_scale_min(b + 4, s, sc, mn);
        uint32_t q = (b[(fmt == OCO_Q4_K ? 16 : 48) + j / 64 * 32 + j % 32] >> (s % 2 * 4)) & 15u;
        if (fmt == OCO_Q5_K) q |= ((b[16 + j % 32] >> s) & 1u) << 4;
        float a = __fmul_rn(half_bits_to_f32(ld_u16(b)), (float)sc);
        float m = __fmul_rn(half_bits_to_f32(ld_u16(b + 2)), (float)mn);
        return __fsub_rn(__fmul_rn(a, (float)q), m);
    }
    case OCO_Q6_K: {
        uint32_t h = j / 128, q = j % 128 / 32, l = j % 32;
        uint32_t lo = (b[h * 64 + (q % 2) * 32 + l] >> (q / 2 * 4)) & 15u;
        uint32_t hi = (b[128 + h * 32 + l] >> (q * 2)) & 3u;
        int sc = (int8_t)b[192 + j / 16];
        return __fmul_rn(__fmul_rn(half_bits_to_f32(ld_u16(b + 208)), (float)sc),
                         (float)((int)(lo | (hi << 4)) - 32));
    }
    }
    return __uint_as_float(0x7fc00000u);
}

// ---------------------------------------------------------------------------
// Piece decoders for the streaming matvec.
// ---------------------------------------------------------------------------
// Converts byte i of w (unsigned) to float exactly with one
// v_cvt_f32_ubyte{0..3}.  i must be a constant after unrolling.  Written as
// asm because the compiler otherwise folds the caller's nibble mask into a
// v_bfe_u32 and converts byte 0, two instructions per weight.
__device__ __forceinline__ float ub(uint32_t w, int i) {
    float f;
    switch (i) {
    case 0: asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(w)); break;
    case 1: asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(w)); break;
    case 2: asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(w)); break;
    default: asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(w)); break;
    }
    return f;
}

template <int FMT>
struct Piece;

// Q8_0: 34-byte blocks {f16 d, int8 q[32]}; 4 lanes per block, 8 codes each.
template <>
struct Piece<OCO_Q8_0> {
    static constexpr int BLOCK = 32, BYTES = 34, P = 4, E = 8;
    struct X {
        float v[8];
    };
    template <typename XT>
    __device__ __forceinline__ static void load_x(const XT *xr, uint32_t block, int piece, X &x, bool rs = false) {
        XLoad<XT>::template run<8>(xr + block * 32 + piece * 8, x.v, rs);
    }
    __device__ __forceinline__ static float dot(const WSrc &w, uint32_t b, int piece, const X &x) {
        uint2 q = w.u64(b + 2 + piece * 8);
        float d = half_bits_to_f32(w.u16(b));
        // each code straight from its sign-extended byte
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s0 = fmaf((float)(int8_t)(q.x >> (8 * i)), x.v[i], s0);
            s1 = fmaf((float)(int8_t)(q.y >> (8 * i)), x.v[4 + i], s1);
        }
        return d * (s0 + s1);
    }
};

// MXFP4: 17-byte blocks {E8M0 e, 16 bytes of E2M1 pairs}; 2 lanes per block,
// each lane 8 code bytes = 16 values (low nibbles: columns 8h+i, high
// nibbles: columns 16+8h+i).  gfx950's v_cvt_scalef32_pk_f32_fp4 decodes
// two E2M1 values per instruction; the block's power of two applies once to
// the piece's sum (exact: scaling by 2^e commutes with fp32 rounding away
// from the subnormal range).
template <>
struct Piece<OCO_MXFP4> {
    static constexpr int BLOCK = 32, BYTES = 17, P = 2, E = 16;
    struct X {
        float lo[8], hi[8];
    };
    template <typename XT>
    __device__ __forceinline__ static void load_x(const XT *xr, uint32_t block, int piece, X &x, bool rs = false) {
        XLoad<XT>::template run<8>(xr + block * 32 + piece * 8, x.lo, rs);
        XLoad<XT>::template run<8>(xr + block * 32 + 16 + piece * 8, x.hi, rs);
    }
    template <int I>
    __device__ __forceinline__ static void pair(uint32_t w, const X &x, int base, float &s0, float &s1) {
        f32x2 v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, I);
        s0 = fmaf(v.x, x.lo[base + I], s0);
        s1 = fmaf(v.y, x.hi[base + I], s1);
    }
    __device__ __forceinline__ static float dot(const WSrc &w, uint32_t b, int piece, const X &x) {
        uint32_t e = w.u8(b);
        uint2 q = w.u64(b + 1 + piece * 8);
        float s0 = 0.f, s1 = 0.f;
        pair<0>(q.x, x, 0, s0, s1);
        pair<1>(q.x, x, 0, s0, s1);
        pair<2>(q.x, x, 0, s0, s1);
        pair<3>(q.x, x, 0, s0, s1);
        pair<0>(q.y, x, 4, s0, s1);
        pair<1>(q.y, x, 4, s0, s1);
        pair<2>(q.y, x, 4, s0, s1);
        pair<3>(q.y, x, 4, s0, s1);
        return (s0 + s1) * e8m0_scale(e);
    }
};

// Q4_K: 144-byte blocks {f16 d, f16 dmin, 12 bytes of 6-bit (scale, min),
// 128 bytes of nibbles}; 8 lanes per block, lane c reading 16 code bytes
// (bytes 16c..16c+15 of qs): low nibbles are columns 64g + 16(c%2) + i of
// sub-block 2g, high nibbles columns 64g + 32 + 16(c%2) + i of sub-block
// 2g+1, g = c/2.
template <int FMT>
struct KQuant4 {
    static constexpr int BLOCK = 256, P = 8, E = 32;
    static constexpr int BYTES = FMT == OCO_Q4_K ? 144 : 176;
    struct X {
        float lo[16], hi[16];
        float sum_lo, sum_hi;
    };
    template <typename XT>
    __device__ __forceinline__ static void load_x(const XT *xr, uint32_t block, int piece, X &x, bool rs = false) {
        int g = piece >> 1, l0 = (piece & 1) * 16;
        XLoad<XT>::template run<16>(xr + block * 256 + g * 64 + l0, x.lo, rs);
        XLoad<XT>::template run<16>(xr + block * 256 + g * 64 + 32 + l0, x.hi, rs);
        float a = 0.f, c = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            a += x.lo[i];
            c += x.hi[i];
        }
        x.sum_lo = a;
        x.sum_hi = c;
    }
    __device__ __forceinline__ static float dot(const WSrc &w, uint32_t b, int piece, const X &x) {
        int g = piece >> 1, l0 = (piece & 1) * 16;
        uint4 hdr = w.u128(b);
        uint4 qs = w.u128(b + (FMT == OCO_Q4_K ? 16 : 48) + 16 * piece);
        uint4 qh;
        if (FMT == OCO_Q5_K) qh = w.u128(b + 16 + l0);
        // scales[12] = bytes 4..15 of the block = hdr.y, hdr.z, hdr.w.
        uint32_t s0 = 2 * g, s1 = 2 * g + 1;
        uint32_t sc0, mn0, sc1, mn1;
        {
            uint32_t sb[12];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sb[i] = byte_of(hdr.y, i);
                sb[4 + i] = byte_of(hdr.z, i);
                sb[8 + i] = byte_of(hdr.w, i);
            }
            // s0 is even, s1 = s0 + 1: select from constant indices to keep the
            // bytes in registers.
            uint32_t sc[8], mn[8];
#pragma unroll
            for (int s = 0; s < 8; s++) {
                if (s < 4) {
                    sc[s] = sb[s] & 63u;
                    mn[s] = sb[s + 4] & 63u;
                } else {
                    sc[s] = (sb[s + 4] & 15u) | ((sb[s - 4] >> 6) << 4);
                    mn[s] = (sb[s + 4] >> 4) | ((sb[s] >> 6) << 4);
                }
            }
            sc0 = sc[0]; mn0 = mn[0]; sc1 = sc[1]; mn1 = mn[1];
#pragma unroll
            for (int s = 2; s < 8; s += 2) {
                if (s0 == (uint32_t)s) {
                    sc0 = sc[s]; mn0 = mn[s]; sc1 = sc[s + 1]; mn1 = mn[s + 1];
                }
            }
        }
        float d = half_bits_to_f32(hdr.x & 0xffffu), dmin = half_bits_to_f32(hdr.x >> 16);
        uint32_t c[4] = {qs.x, qs.y, qs.z, qs.w};
        float a0 = 0.f, a1 = 0.f;
        if (FMT == OCO_Q4_K) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t lo = c[j] & 0x0f0f0f0fu, hi = (c[j] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    a0 = fmaf(ub(lo, i), x.lo[4 * j + i], a0);
                    a1 = fmaf(ub(hi, i), x.hi[4 * j + i], a1);
                }
            }
        } else {
            uint32_t h[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t lo = (c[j] & 0x0f0f0f0fu) | (((h[j] >> s0) & 0x01010101u) << 4);
                uint32_t hi = ((c[j] >> 4) & 0x0f0f0f0fu) | (((h[j] >> s1) & 0x01010101u) << 4);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    a0 = fmaf(ub(lo, i), x.lo[4 * j + i], a0);
                    a1 = fmaf(ub(hi, i), x.hi[4 * j + i], a1);
                }
            }
        }
        float r = (d * (float)sc0) * a0 - (dmin * (float)mn0) * x.sum_lo;
        return fmaf(d * (float)sc1, a1, fmaf(-(dmin * (float)mn1), x.sum_hi, r));
    }
};
template <>
struct Piece<OCO_Q4_K> : KQuant4<OCO_Q4_K> {};
template <>
struct Piece<OCO_Q5_K> : KQuant4<OCO_Q5_K> {};

// Q6_K: 210-byte blocks {ql[128], qh[64], int8 sc[16], f16 d}; 8 lanes per
// block, lane c covering half h = c/4 and columns l0 = 8(c%4) .. l0+7 of each
// of the four 32-column quarters q (coefficient h*128 + q*32 + l).
template <>
struct Piece<OCO_Q6_K> {
    static constexpr int BLOCK = 256, BYTES = 210, P = 8, E = 32;
    struct X {
        float v[4][8];
        float sum[4];
    };
    template <typename XT>
    __device__ __forceinline__ static void load_x(const XT *xr, uint32_t block, int piece, X &x, bool rs = false) {
        int h = piece >> 2, l0 = (piece & 3) * 8;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            XLoad<XT>::template run<8>(xr + block * 256 + h * 128 + q * 32 + l0, x.v[q], rs);
            x.sum[q] = ((x.v[q][0] + x.v[q][1]) + (x.v[q][2] + x.v[q][3])) +
                       ((x.v[q][4] + x.v[q][5]) + (x.v[q][6] + x.v[q][7]));
        }
    }
    __device__ __forceinline__ static float dot(const WSrc &w, uint32_t b, int piece, const X &x) {
        int h = piece >> 2, l0 = (piece & 3) * 8;
        uint2 ql0 = w.u64(b + h * 64 + l0);       // quarters 0 (low) and 2 (high)
        uint2 ql1 = w.u64(b + h * 64 + 32 + l0);  // quarters 1 (low) and 3 (high)
        uint2 qh = w.u64(b + 128 + h * 32 + l0);
        uint2 scw = w.u64(b + 192 + h * 8 + (l0 >> 4));  // scales of quarters at bytes 0,2,4,6
        float d = half_bits_to_f32(w.u16(b + 208));
        float r = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint2 src = (q & 1) ? ql1 : ql0;
            int shift = (q >> 1) * 4;
            float a = 0.f;
#pragma unroll
            for (int half = 0; half < 2; half++) {
                uint32_t lw = half ? src.y : src.x, hw = half ? qh.y : qh.x;
                uint32_t code = ((lw >> shift) & 0x0f0f0f0fu) | (((hw >> (2 * q)) & 0x03030303u) << 4);
#pragma unroll
                for (int i = 0; i < 4; i++) a = fmaf(ub(code, i), x.v[q][4 * half + i], a);
            }
            uint32_t sw = q < 2 ? scw.x : scw.y;
            float sc = (float)(int8_t)((sw >> (16 * (q & 1))) & 0xffu);
            r = fmaf(sc, fmaf(-32.f, x.sum[q], a), r);
        }
        return d * r;
    }
};

// Q4_0 / Q4_1: 18/20-byte blocks; 2 lanes per block, each 8 code bytes.
template <int FMT>
struct Q4Legacy {
    static constexpr int BLOCK = 32, P = 2, E = 16;
    static constexpr int BYTES = FMT == OCO_Q4_0 ? 18 : 20;
    static constexpr int CODES = FMT == OCO_Q4_0 ? 2 : 4;
    struct X {
        float lo[8], hi[8];
        float sum;
    };
    template <typename XT>
    __device__ __forceinline__ static void load_x(const XT *xr, uint32_t block, int piece, X &x, bool rs = false) {
        XLoad<XT>::template run<8>(xr + block * 32 + piece * 8, x.lo, rs);
        XLoad<XT>::template run<8>(xr + block * 32 + 16 + piece * 8, x.hi, rs);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) s += x.lo[i] + x.hi[i];
        x.sum = s;
    }
    __device__ __forceinline__ static float dot(const WSrc &w, uint32_t b, int piece, const X &x) {
        uint2 q = w.u64(b + CODES + piece * 8);
        float d = half_bits_to_f32(w.u16(b));
        uint32_t c[2] = {q.x, q.y};
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            uint32_t lo = c[j] & 0x0f0f0f0fu, hi = (c[j] >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a = fmaf(ub(lo, i), x.lo[4 * j + i], a);
                a = fmaf(ub(hi, i), x.hi[4 * j + i], a);
            }
        }
        if (FMT == OCO_Q4_0) return d * fmaf(-8.f, x.sum, a);
        return fmaf(d, a, half_bits_to_f32(w.u16(b + 2)) * x.sum);
    }
};
template <>
struct Piece<OCO_Q4_0> : Q4Legacy<OCO_Q4_0> {};
template <>
struct Piece<OCO_Q4_1> : Q4Legacy<OCO_Q4_1> {};

// Plain F32 / F16 / BF16 rows: one lane per 16-byte piece.
template <int FMT>
struct Plain {
    static constexpr int E = FMT == OCO_F32 ? 4 : 8;
    static constexpr int BLOCK = E, P = 1, BYTES = 16;
    struct X {
        float v[E];
    };
    template <typename XT>
    __device__ __forceinline__ static void load_x(const XT *xr, uint32_t block, int, X &x, bool rs = false) {
        XLoad<XT>::template run<E>(xr + block * E, x.v, rs);
    }
    __device__ __forceinline__ static float dot(const WSrc &w, uint32_t b, int, const X &x) {
        uint4 q = w.u128(b);
        uint32_t c[4] = {q.x, q.y, q.z, q.w};
        float a = 0.f;
        if (FMT == OCO_F32) {
#pragma unroll
            for (int i = 0; i < 4; i++) a = fmaf(__uint_as_float(c[i]), x.v[i], a);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float lo = FMT == OCO_F16 ? half_bits_to_f32(c[i] & 0xffffu) : __uint_as_float(c[i] << 16);
                float hi = FMT == OCO_F16 ? half_bits_to_f32(c[i] >> 16) : __uint_as_float(c[i] & 0xffff0000u);
                a = fmaf(lo, x.v[2 * i], a);
                a = fmaf(hi, x.v[2 * i + 1], a);
            }
        }
        return a;
    }
};
template <>
struct Piece<OCO_F32> : Plain<OCO_F32> {};
template <>
struct Piece<OCO_F16> : Plain<OCO_F16> {};
template <>
struct Piece<OCO_BF16> : Plain<OCO_BF16> {};

}  // namespace oco
