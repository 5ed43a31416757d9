// Tile decoders for the streaming matvec: GGUF blocks decoded from an LDS
// copy of the weight rows, against activations staged in LDS.
//
// Every format here splits a row into 32-coefficient pieces (a piece is one
// lane's unit of work: a whole Q8_0/MXFP4 block, or one eighth of a Q4_K /
// Q6_K super-block).  Activations are staged once per workgroup in
// piece-major order: run t (4 floats) of piece p lives at float4 index
// t * PT + p, PT = pieces per row, so the 32 lanes of a half-wavefront, which
// hold consecutive pieces, read consecutive 16-byte words (no bank
// conflicts), and the two halves, which hold different rows of the same
// pieces, read identical words (broadcast).  Per-piece activation sums the
// affine terms need are staged beside them.
#pragma once
#include "formats.h"

namespace oco {

// N bytes (N a multiple of 4) from an LDS address of any alignment.  gfx950
// serves a ds_read that is not naturally aligned about ten times slower than
// an aligned one, so this reads the covering dwords aligned (the compiler
// pairs them into ds_read2_b32) and realigns them with v_alignbyte_b32.
template <int N>
__device__ __forceinline__ void lds_bytes(const uint8_t *p, uint32_t *out) {
    const uint32_t a = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t *d = reinterpret_cast<const uint32_t *>(p - a);
    uint32_t w[N / 4 + 1];
#pragma unroll
    for (int i = 0; i <= N / 4; i++) w[i] = d[i];
#pragma unroll
    for (int i = 0; i < N / 4; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], a);
}
__device__ __forceinline__ uint4 lds_u128(const uint8_t *p) {
    uint32_t o[4];
    lds_bytes<16>(p, o);
    return make_uint4(o[0], o[1], o[2], o[3]);
}
__device__ __forceinline__ uint2 lds_u64(const uint8_t *p) {
    uint32_t o[2];
    lds_bytes<8>(p, o);
    return make_uint2(o[0], o[1]);
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t *p) {
    uint32_t o[1];
    lds_bytes<4>(p, o);
    return o[0] & 0xffffu;
}

template <int FMT>
struct Tile;

// Two nibble codes at once: byte c < 16 read as E4M3 is exactly c * 2^-9,
// so v_cvt_scalef32_pk_f32_fp8 on a dword of masked nibbles (bytes 0-1 or
// 2-3 by HI) with the scale 2^9 gives c0 and c1 as floats.  (The scale
// operand acts as a power of two: only its exponent is applied.)
template <bool HI>
__device__ __forceinline__ f32x2 nib2(uint32_t masked) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)masked, 512.f, HI);
}

// MXFP4: piece = block {e, 16 code bytes}; code byte i holds columns i (low
// nibble) and 16 + i (high nibble) of the block.  gfx950's
// v_cvt_scalef32_pk_f32_fp4 decodes two E2M1 codes per instruction.
template <>
struct Tile<OCO_MXFP4> {
    static constexpr int BLOCK = 32, BYTES = 17, P = 1, NSUM = 0;
    struct Raw {
        uint4 q;
        uint32_t e;
    };
    __device__ __forceinline__ static void map(uint32_t f, uint32_t &p, uint32_t &t) {
        p = f >> 3;
        t = f & 7;
    }
    // float4 index of run t of piece p (the inverse of map)
    __device__ __forceinline__ static uint32_t unmap(uint32_t p, uint32_t t) { return p * 8 + t; }
    __device__ __forceinline__ static void sums(const float *, float *) {}
    __device__ __forceinline__ static Raw load(const uint8_t *blk, int) {
        Raw r;
        r.e = blk[0];
        r.q = lds_u128(blk + 1);
        return r;
    }
    template <int I>
    __device__ __forceinline__ static void pair(uint32_t w, const float *x, int j, float &s0, float &s1) {
        f32x2 v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, I);
        s0 = fmaf(v.x, x[4 * j + I], s0);
        s1 = fmaf(v.y, x[16 + 4 * j + I], s1);
    }
    __device__ __forceinline__ static float dot(const Raw &r, const float *x, const float *) {
        float s0 = 0.f, s1 = 0.f;
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            pair<0>(w[j], x, j, s0, s1);
            pair<1>(w[j], x, j, s0, s1);
            pair<2>(w[j], x, j, s0, s1);
            pair<3>(w[j], x, j, s0, s1);
        }
        return (s0 + s1) * e8m0_scale(r.e);
    }
};

// Q8_0: piece = block {f16 d, int8 q[32]}.  Each code converts straight
// from its sign-extended byte (v_cvt_f32_i32 with a byte select), so the
// block needs no activation sum.
template <>
struct Tile<OCO_Q8_0> {
    static constexpr int BLOCK = 32, BYTES = 34, P = 1, NSUM = 0;
    struct Raw {
        uint4 a, b;
        uint32_t d;
    };
    __device__ __forceinline__ static void map(uint32_t f, uint32_t &p, uint32_t &t) {
        p = f >> 3;
        t = f & 7;
    }
    // float4 index of run t of piece p (the inverse of map)
    __device__ __forceinline__ static uint32_t unmap(uint32_t p, uint32_t t) { return p * 8 + t; }
    __device__ __forceinline__ static void sums(const float *, float *) {}
    __device__ __forceinline__ static Raw load(const uint8_t *blk, int) {
        Raw r;
        r.d = lds_u16(blk);
        uint32_t o[8];
        lds_bytes<32>(blk + 2, o);
        r.a = make_uint4(o[0], o[1], o[2], o[3]);
        r.b = make_uint4(o[4], o[5], o[6], o[7]);
        return r;
    }
    __device__ __forceinline__ static float dot(const Raw &r, const float *x, const float *) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a0 = fmaf((float)(int8_t)(w[j] >> (8 * i)), x[4 * j + i], a0);
                a1 = fmaf((float)(int8_t)(w[j + 1] >> (8 * i)), x[4 * j + 4 + i], a1);
            }
        }
        return half_bits_to_f32(r.d) * (a0 + a1);
    }
};

// (scale, min) of sub-blocks 2g and 2g + 1 of a Q4_K / Q5_K super-block
// (get_scale_min_k4, weights.metal:67-77) as the bytes [sc0, sc1, mn0, mn1]
// of one word, from scales[12] = hdr.y (bytes 0..3), hdr.z (4..7), hdr.w
// (8..11).  Sub-block j < 4 has sc = scales[j] & 63, mn = scales[j + 4] & 63;
// j >= 4 has sc = (scales[j + 4] & 15) | (scales[j - 4] >> 6) << 4 and mn =
// (scales[j + 4] >> 4) | (scales[j] >> 6) << 4.  Both forms read bytes b,
// b + 1 (b = 2 (g & 1)) of hdr.y and hdr.z, the second also of hdr.w, so two
// byte permutes gather them (the byte conversions v_cvt_f32_ubyte0..3 then
// take each value straight from the word).
__device__ __forceinline__ uint32_t k_scale_min(const uint4 &hdr, uint32_t g) {
    const uint32_t b = 2u * (g & 1u);
    const uint32_t sel = b | ((b + 1) << 8) | ((b + 4) << 16) | ((b + 5) << 24);
    const uint32_t yz = __builtin_amdgcn_perm(hdr.z, hdr.y, sel);  // y_b, y_b1, z_b, z_b1
    const uint32_t ww = __builtin_amdgcn_perm(hdr.w, hdr.w, (sel & 0xffffu) | ((sel & 0xffffu) << 16));  // w_b, w_b1, w_b, w_b1
    return g < 2 ? yz & 0x3f3f3f3fu : (ww & 0x00000f0fu) | ((ww >> 4) & 0x0f0f0000u) | ((yz >> 2) & 0x30303030u);
}

// Q4_K: piece c of a super-block = qs bytes 16c..16c+15; low nibbles are
// columns 64g + 16(c&1) + i of sub-block 2g, high nibbles columns
// 64g + 32 + 16(c&1) + i of sub-block 2g+1 (g = c/2).  The 16-byte header
// (d, dmin, 6-bit scales/mins) is read by all eight lanes of the block.
template <>
struct Tile<OCO_Q4_K> {
    static constexpr int BLOCK = 256, BYTES = 144, P = 8, NSUM = 2;
    struct Raw {
        uint4 hdr, qs;
    };
    __device__ __forceinline__ static void map(uint32_t f, uint32_t &p, uint32_t &t) {
        uint32_t b = f >> 6, rem = f & 63, g = rem >> 4, w = rem & 15;
        uint32_t odd = (w & 7) >> 2;
        p = b * 8 + 2 * g + odd;
        t = (w >> 3) * 4 + (w & 3);
    }
    __device__ __forceinline__ static uint32_t unmap(uint32_t p, uint32_t t) {
        const uint32_t c = p & 7;
        return (p >> 3) * 64 + (c >> 1) * 16 + (t >> 2) * 8 + (c & 1) * 4 + (t & 3);
    }
    __device__ __forceinline__ static void sums(const float *x, float *s) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            a += x[i];
            b += x[16 + i];
        }
        s[0] = a;
        s[1] = b;
    }
    __device__ __forceinline__ static Raw load(const uint8_t *blk, int c) {
        Raw r;
        r.hdr = lds_u128(blk);
        r.qs = lds_u128(blk + 16 + 16 * c);
        return r;
    }
    // Piece c of the block at byte `off` straight from memory (16-byte
    // aligned blocks: 144 is a multiple of 16).
    static constexpr bool DIRECT = true;
    __device__ __forceinline__ static Raw direct(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t c) {
        Raw r;
        const u32x4 h = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 2);
        const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 + 16 * c, 0, 2);
        r.hdr = make_uint4(h.x, h.y, h.z, h.w);
        r.qs = make_uint4(q.x, q.y, q.z, q.w);
        return r;
    }
    __device__ __forceinline__ static float dot(const Raw &r, const float *x, const float *s, int c) {
        const uint32_t g = (uint32_t)c >> 1;
        const uint32_t scm = k_scale_min(r.hdr, g);
        const float sc0 = ub(scm, 0), sc1 = ub(scm, 1), mn0 = ub(scm, 2), mn1 = ub(scm, 3);
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        const float d = half_bits_to_f32(r.hdr.x & 0xffffu), dmin = half_bits_to_f32(r.hdr.x >> 16);
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t lo = w[j] & 0x0f0f0f0fu, hi = (w[j] >> 4) & 0x0f0f0f0fu;
            const f32x2 l0 = nib2<false>(lo), l1 = nib2<true>(lo);
            const f32x2 h0 = nib2<false>(hi), h1 = nib2<true>(hi);
            a0 = fmaf(l0.x, x[4 * j], a0);
            a1 = fmaf(h0.x, x[16 + 4 * j], a1);
            a0 = fmaf(l0.y, x[4 * j + 1], a0);
            a1 = fmaf(h0.y, x[16 + 4 * j + 1], a1);
            a0 = fmaf(l1.x, x[4 * j + 2], a0);
            a1 = fmaf(h1.x, x[16 + 4 * j + 2], a1);
            a0 = fmaf(l1.y, x[4 * j + 3], a0);
            a1 = fmaf(h1.y, x[16 + 4 * j + 3], a1);
        }
        const float v = fmaf(d * sc0, a0, -(dmin * mn0) * s[0]);
        return fmaf(d * sc1, a1, fmaf(-(dmin * mn1), s[1], v));
    }
};

// Q6_K: piece c covers half h = c/4 and columns l0 = 8(c&3) .. l0+7 of each
// 32-column quarter q (coefficient 128h + 32q + l).
template <>
struct Tile<OCO_Q6_K> {
    static constexpr int BLOCK = 256, BYTES = 210, P = 8, NSUM = 4;
    struct Raw {
        uint2 ql0, ql1, qh, sc;
        uint32_t d;
    };
    __device__ __forceinline__ static void map(uint32_t f, uint32_t &p, uint32_t &t) {
        uint32_t b = f >> 6, rem = f & 63, h = rem >> 5, r2 = rem & 31, q = r2 >> 3, w = r2 & 7;
        p = b * 8 + 4 * h + (w >> 1);
        t = 2 * q + (w & 1);
    }
    __device__ __forceinline__ static uint32_t unmap(uint32_t p, uint32_t t) {
        const uint32_t c = p & 7;
        return (p >> 3) * 64 + (c >> 2) * 32 + (t >> 1) * 8 + (c & 3) * 2 + (t & 1);
    }
    __device__ __forceinline__ static void sums(const float *x, float *s) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) a += x[8 * q + i];
            s[q] = a;
        }
    }
    // The piece's fields sit at offsets from the block that are multiples of
    // 4 (ql, qh, d) or not (the scales): one aligned base and one shift
    // serve the first group, with the lane's field offsets folded into two
    // adds and the reads' immediate offsets.
    __device__ __forceinline__ static Raw load(const uint8_t *blk, int c) {
        const int h = c >> 2, l0 = (c & 3) * 8;
        const uint32_t a = (uint32_t)(uintptr_t)blk & 3u;
        const uint8_t *b = blk - a;
        const uint32_t *q = reinterpret_cast<const uint32_t *>(b + h * 64 + l0);
        const uint32_t *qh = reinterpret_cast<const uint32_t *>(b + 128 + h * 32 + l0);
        const uint32_t *dp = reinterpret_cast<const uint32_t *>(b + 208);
        Raw r;
        r.ql0 = make_uint2(__builtin_amdgcn_alignbyte(q[1], q[0], a), __builtin_amdgcn_alignbyte(q[2], q[1], a));
        r.ql1 = make_uint2(__builtin_amdgcn_alignbyte(q[9], q[8], a), __builtin_amdgcn_alignbyte(q[10], q[9], a));
        r.qh = make_uint2(__builtin_amdgcn_alignbyte(qh[1], qh[0], a), __builtin_amdgcn_alignbyte(qh[2], qh[1], a));
        r.d = __builtin_amdgcn_alignbyte(dp[1], dp[0], a) & 0xffffu;
        r.sc = lds_u64(blk + 192 + h * 8 + (l0 >> 4));
        return r;
    }
    __device__ __forceinline__ static float dot(const Raw &r, const float *x, const float *s, int) {
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint2 src = (q & 1) ? r.ql1 : r.ql0;
            const int shift = (q >> 1) * 4;
            float a = 0.f;
#pragma unroll
            for (int half = 0; half < 2; half++) {
                uint32_t lw = half ? src.y : src.x, hw = half ? r.qh.y : r.qh.x;
                uint32_t code = ((lw >> shift) & 0x0f0f0f0fu) | (((hw >> (2 * q)) & 0x03030303u) << 4);
#pragma unroll
                for (int i = 0; i < 4; i++) a = fmaf(ub(code, i), x[8 * q + 4 * half + i], a);
            }
            uint32_t sw = q < 2 ? r.sc.x : r.sc.y;
            float sc = (float)(int8_t)((sw >> (16 * (q & 1))) & 0xffu);
            acc = fmaf(sc, fmaf(-32.f, s[q], a), acc);
        }
        return half_bits_to_f32(r.d) * acc;
    }
};

// Q4_0: piece = block {f16 d, 16 code bytes}; byte i holds columns i (low
// nibble) and 16 + i (high nibble); w = d (q - 8) (weights.metal:55-59),
// computed as d (sum q x - 8 sum x).
template <>
struct Tile<OCO_Q4_0> {
    static constexpr int BLOCK = 32, BYTES = 18, P = 1, NSUM = 1;
    struct Raw {
        uint4 q;
        uint32_t d;
    };
    __device__ __forceinline__ static void map(uint32_t f, uint32_t &p, uint32_t &t) {
        p = f >> 3;
        t = f & 7;
    }
    // float4 index of run t of piece p (the inverse of map)
    __device__ __forceinline__ static uint32_t unmap(uint32_t p, uint32_t t) { return p * 8 + t; }
    __device__ __forceinline__ static void sums(const float *x, float *s) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) a += x[i];
        s[0] = a;
    }
    __device__ __forceinline__ static Raw load(const uint8_t *blk, int) {
        Raw r;
        r.d = lds_u16(blk);
        r.q = lds_u128(blk + 2);
        return r;
    }
    // sum of code * x over the block
    __device__ __forceinline__ static float nibble_dot(const uint4 &q, const float *x) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t lo = w[j] & 0x0f0f0f0fu, hi = (w[j] >> 4) & 0x0f0f0f0fu;
            const f32x2 l0 = nib2<false>(lo), l1 = nib2<true>(lo);
            const f32x2 h0 = nib2<false>(hi), h1 = nib2<true>(hi);
            a0 = fmaf(l0.x, x[4 * j], a0);
            a1 = fmaf(h0.x, x[16 + 4 * j], a1);
            a0 = fmaf(l0.y, x[4 * j + 1], a0);
            a1 = fmaf(h0.y, x[16 + 4 * j + 1], a1);
            a0 = fmaf(l1.x, x[4 * j + 2], a0);
            a1 = fmaf(h1.x, x[16 + 4 * j + 2], a1);
            a0 = fmaf(l1.y, x[4 * j + 3], a0);
            a1 = fmaf(h1.y, x[16 + 4 * j + 3], a1);
        }
        return a0 + a1;
    }
    __device__ __forceinline__ static float dot(const Raw &r, const float *x, const float *s) {
        return half_bits_to_f32(r.d) * fmaf(-8.f, s[0], nibble_dot(r.q, x));
    }
};

// Q4_1: piece = block {f16 d, f16 m, 16 code bytes}; w = d q + m
// (weights.metal:55-59), computed as d sum q x + m sum x.
template <>
struct Tile<OCO_Q4_1> {
    static constexpr int BLOCK = 32, BYTES = 20, P = 1, NSUM = 1;
    struct Raw {
        uint4 q;
        uint32_t dm;
    };
    __device__ __forceinline__ static void map(uint32_t f, uint32_t &p, uint32_t &t) {
        p = f >> 3;
        t = f & 7;
    }
    // float4 index of run t of piece p (the inverse of map)
    __device__ __forceinline__ static uint32_t unmap(uint32_t p, uint32_t t) { return p * 8 + t; }
    __device__ __forceinline__ static void sums(const float *x, float *s) { Tile<OCO_Q4_0>::sums(x, s); }
    __device__ __forceinline__ static Raw load(const uint8_t *blk, int) {
        Raw r;
        uint32_t o[5];
        lds_bytes<20>(blk, o);
        r.dm = o[0];
        r.q = make_uint4(o[1], o[2], o[3], o[4]);
        return r;
    }
    __device__ __forceinline__ static float dot(const Raw &r, const float *x, const float *s) {
        return fmaf(half_bits_to_f32(r.dm & 0xffffu), Tile<OCO_Q4_0>::nibble_dot(r.q, x),
                    half_bits_to_f32(r.dm >> 16) * s[0]);
    }
};

// Q5_K: the Q4_K piece (qs at byte 48 instead of 16) plus the fifth bit of
// each code from qh[32] at byte 16: column j takes bit j / 32 of qh[j % 32]
// (weights.metal:67-77).  Piece c's low-nibble columns (sub-block 2g) and
// high-nibble columns (sub-block 2g + 1) share the qh bytes 16 (c & 1) ..
// + 15, bits 2g and 2g + 1.
template <>
struct Tile<OCO_Q5_K> {
    static constexpr int BLOCK = 256, BYTES = 176, P = 8, NSUM = 2;
    struct Raw {
        uint4 hdr, qh, qs;
    };
    __device__ __forceinline__ static void map(uint32_t f, uint32_t &p, uint32_t &t) { Tile<OCO_Q4_K>::map(f, p, t); }
    __device__ __forceinline__ static uint32_t unmap(uint32_t p, uint32_t t) { return Tile<OCO_Q4_K>::unmap(p, t); }
    __device__ __forceinline__ static void sums(const float *x, float *s) { Tile<OCO_Q4_K>::sums(x, s); }
    __device__ __forceinline__ static Raw load(const uint8_t *blk, int c) {
        Raw r;
        r.hdr = lds_u128(blk);
        r.qh = lds_u128(blk + 16 + 16 * (c & 1));
        r.qs = lds_u128(blk + 48 + 16 * c);
        return r;
    }
    // Piece c of the block at byte `off` straight from memory (176 is a
    // multiple of 16).
    static constexpr bool DIRECT = true;
    __device__ __forceinline__ static Raw direct(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t c) {
        Raw r;
        const u32x4 h = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 2);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 + 16 * (c & 1), 0, 2);
        const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 48 + 16 * c, 0, 2);
        r.hdr = make_uint4(h.x, h.y, h.z, h.w);
        r.qh = make_uint4(b.x, b.y, b.z, b.w);
        r.qs = make_uint4(q.x, q.y, q.z, q.w);
        return r;
    }
    __device__ __forceinline__ static float dot(const Raw &r, const float *x, const float *s, int c) {
        const uint32_t g = (uint32_t)c >> 1;
        const uint32_t scm = k_scale_min(r.hdr, g);
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        const uint32_t hb[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t lo = (w[j] & 0x0f0f0f0fu) | (((hb[j] >> (2 * g)) & 0x01010101u) << 4);
            const uint32_t hi = ((w[j] >> 4) & 0x0f0f0f0fu) | (((hb[j] >> (2 * g + 1)) & 0x01010101u) << 4);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a0 = fmaf(ub(lo, i), x[4 * j + i], a0);
                a1 = fmaf(ub(hi, i), x[16 + 4 * j + i], a1);
            }
        }
        const float d = half_bits_to_f32(r.hdr.x & 0xffffu), dmin = half_bits_to_f32(r.hdr.x >> 16);
        const float v = fmaf(d * ub(scm, 0), a0, -(dmin * ub(scm, 2)) * s[0]);
        return fmaf(d * ub(scm, 1), a1, fmaf(-(dmin * ub(scm, 3)), s[1], v));
    }
};

// Uniform call shape for formats whose dot ignores the piece index.
template <int FMT>
__device__ __forceinline__ float tile_dot(const typename Tile<FMT>::Raw &r, const float *x,
                                          const float *s, int c) {
    if constexpr (FMT == OCO_Q4_K || FMT == OCO_Q5_K || FMT == OCO_Q6_K)
        return Tile<FMT>::dot(r, x, s, c);
    else
        return Tile<FMT>::dot(r, x, s);
}

// Sum over each 32-lane half of the wavefront (both halves independently).
__device__ __forceinline__ float half_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x124>(v);
    v += dpp_f32<0x128>(v);
    auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
}

}  // namespace oco
