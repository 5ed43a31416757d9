/*
 * CPU oracle for the quantized-weight matrix path.  TEST INFRASTRUCTURE ONLY:
 * this file is the checker that the HIP library is compared against, and the
 * scalar "port" CPU baseline that bench.py times.  Nothing in the product
 * library links, loads or calls it.
 *
 * Every function restates one piece of the reference (xhjkl/oco) in plain C;
 * each cites the reference file:line whose behaviour it follows.  Paths are
 * relative to the reference checkout.
 *
 * Pinning (what checks each function beyond re-typing its formula):
 *   - oo_dequant: round trip against the reference's own independent GGUF
 *     packers (src/weights/dispatch_tests/matrix_precision.rs:145-287,
 *     mxfp4.rs:46-81 and 283-307) restated in tests/golden/packers.py: the
 *     packers record every coefficient in fp64 from the codes they choose, and
 *     the decode here must reproduce them exactly (tests/test_oracle.py).
 *     Special cases: fp16 subnormal/Inf/NaN scales, E8M0 0 and 255, Q6_K
 *     code 0 -> -32, checked against closed forms.
 *   - oo_matvec_f64 / oo_matvec_f32: all-ones weights with x = 1 and 2 give
 *     y = K and 2K exactly (compute/tests.rs:40-80), linearity in x, brute
 *     force on tiny K against numpy float64, and the reference's roundoff
 *     bound gamma_{2K+8} * sum|w x| (matrix_precision.rs:136-142).
 *   - oo_select_experts: known answer logits_selecting([3,0,2,1])
 *     (mxfp4.rs:38-44), brute force over all 4-subsets on random logits,
 *     tie rule (lowest index), non-finite -> NaN probabilities.
 *   - oo_route_plan: brute force reconstruction of every route from the
 *     plan, tile coverage, the ids pattern of mxfp4.rs:345-347.
 *   - oo_swiglu_clipped: closed form in fp64 (mxfp4.rs:139-147) and the
 *     NaN/Inf propagation rules.
 *   - oo_moe_sum: hand-computed cases and the bf16 rounding points.
 *   - oo_argmax_f32: the reference's own known answers
 *     (src/weights/dispatch_tests/numerics.rs:14-69: every non-finite class
 *     at index 2049 of 2051, signed zeros, ties at 31/32, 1023/1024,
 *     1024/2048) and brute force against numpy's argmax on finite data.
 *   - oo_norm / oo_add_norm: the fp64 closed form checked against numpy
 *     (rms of a constant row is the constant; scaling x leaves y unchanged up
 *     to rounding; full_layer 0 and 1 differ only in the rounding point).
 * The fp32 summation order of the Metal kernels is not reproducible without
 * Metal; it is bounded, not pinned (the tests use relative L2 and the bound).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* GGUF format codes: src/tensor.rs:9-20. */
enum {
    OO_F32 = 0, OO_F16 = 1, OO_Q4_0 = 2, OO_Q4_1 = 3, OO_Q8_0 = 8,
    OO_Q4_K = 12, OO_Q5_K = 13, OO_Q6_K = 14, OO_BF16 = 30, OO_MXFP4 = 39
};
enum { OO_DT_F32 = 0, OO_DT_BF16 = 1, OO_DT_F16 = 2 };

/* Matrix parameter block: shaders/matrix/weights.metal:87-89. */
typedef struct {
    uint32_t k, n, m, route_major, routes, experts, has_bias;
} oo_matrix;

/* (elements, bytes) per block: src/tensor.rs:24-38. */
int oo_block_layout(uint32_t fmt, uint32_t *elements, uint32_t *bytes) {
    uint32_t e, b;
    switch (fmt) {
    case OO_F32: e = 1; b = 4; break;
    case OO_F16: case OO_BF16: e = 1; b = 2; break;
    case OO_Q4_0: e = 32; b = 18; break;
    case OO_Q4_1: e = 32; b = 20; break;
    case OO_Q8_0: e = 32; b = 34; break;
    case OO_Q4_K: e = 256; b = 144; break;
    case OO_Q5_K: e = 256; b = 176; break;
    case OO_Q6_K: e = 256; b = 210; break;
    case OO_MXFP4: e = 32; b = 17; break;
    default: return -1;
    }
    *elements = e;
    *bytes = b;
    return 0;
}

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* IEEE binary16 -> binary32, exact for every input including subnormals,
 * infinities and NaN (the `float(half)` conversion of weights.metal:35-37). */
float oo_fp16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 31, man = h & 1023;
    if (exp == 31)
        return bits_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        /* subnormal: man * 2^-24, exact in binary32 */
        float v = (float)man * 0x1p-24f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112) << 23) | (man << 13));
}

float oo_bf16(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* binary32 -> bfloat16, round to nearest even; NaN stays a quiet NaN
 * (Metal's `bfloat(float)` used by store_result, weights.metal:28-33). */
uint16_t oo_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1);
    return (uint16_t)(u >> 16);
}

/* binary32 -> binary16, round to nearest even with subnormals; the `half(x)`
 * operand conversion of the reference's tiled kernels (projections.metal:226-233). */
uint16_t oo_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u)
        return sign | 0x7e00u;
    if (a >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return sign | 0x7c00u;
    if (a < 0x38800000u) { /* below 2^-14: subnormal half */
        /* value = a_float; quantum 2^-24 */
        float v = bits_f32(a);
        float q = v * 0x1p24f; /* exact scaling */
        float r = rintf(q);    /* default rounding mode: nearest even */
        return sign | (uint16_t)r;
    }
    uint32_t e = (a >> 23) - 112, m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1)))
        h++;
    return sign | (uint16_t)h;
}

static float ld_f16(const uint8_t *p) { return oo_fp16((uint16_t)(p[0] | (p[1] << 8))); }

/* E8M0 shared exponent of an MXFP4 block.  Finite powers decode exactly, 0
 * is 2^-127 (0x00400000) and 255 is NaN: projections.metal:19-23.  (The
 * generic weight() at weights.metal:44 would yield +Inf for 255; this build
 * follows the expert kernels' NaN, the OCP MX convention.) */
static float e8m0(uint8_t e) {
    if (e == 255)
        return bits_f32(0x7fc00000u);
    return e == 0 ? bits_f32(0x00400000u) : bits_f32((uint32_t)e << 23);
}

static const float kE2M1[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f,
                                -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};

/* Decode element j of one block: weights.metal:48-85 (and mxfp4() at :40-46). */
static float decode(uint32_t fmt, const uint8_t *b, uint32_t j) {
    switch (fmt) {
    case OO_F32: { float v; memcpy(&v, b, 4); return v; }
    case OO_F16: return ld_f16(b);
    case OO_BF16: return oo_bf16((uint16_t)(b[0] | (b[1] << 8)));
    case OO_Q4_0: {
        uint32_t q = (b[2 + j % 16] >> (j / 16 * 4)) & 15;
        return ld_f16(b) * (float)((int)q - 8);
    }
    case OO_Q4_1: {
        uint32_t q = (b[4 + j % 16] >> (j / 16 * 4)) & 15;
        /* d*q + m, two roundings as written at weights.metal:58 */
        float dq = ld_f16(b) * (float)q;
        return dq + ld_f16(b + 2);
    }
    case OO_Q8_0: return ld_f16(b) * (float)(int8_t)b[2 + j];
    case OO_MXFP4: {
        uint32_t q = (b[1 + j % 16] >> (j / 16 * 4)) & 15;
        return kE2M1[q] * e8m0(b[0]);
    }
    case OO_Q4_K: case OO_Q5_K: {
        uint32_t s = j / 32;
        const uint8_t *sc = b + 4;
        uint32_t scale = s < 4 ? (sc[s] & 63u) : ((sc[s + 4] & 15u) | ((sc[s - 4] >> 6) << 4));
        uint32_t mn = s < 4 ? (sc[s + 4] & 63u) : ((uint32_t)(sc[s + 4] >> 4) | ((uint32_t)(sc[s] >> 6) << 4));
        uint32_t q = (b[(fmt == OO_Q4_K ? 16 : 48) + j / 64 * 32 + j % 32] >> (s % 2 * 4)) & 15u;
        if (fmt == OO_Q5_K)
            q |= ((b[16 + j % 32] >> s) & 1u) << 4;
        /* d*sc and d*sc*q and dmin*mn are exact in binary32 (<= 22 significant
         * bits); the subtraction rounds once, so fused and unfused agree. */
        float a = ld_f16(b) * (float)scale;
        float m = ld_f16(b + 2) * (float)mn;
        return a * (float)q - m;
    }
    case OO_Q6_K: {
        uint32_t h = j / 128, q = j % 128 / 32, l = j % 32;
        uint32_t lo = (b[h * 64 + (q % 2) * 32 + l] >> (q / 2 * 4)) & 15u;
        uint32_t hi = (b[128 + h * 32 + l] >> (q * 2)) & 3u;
        int sc = (int8_t)b[192 + j / 16];
        return ld_f16(b + 208) * (float)sc * (float)((int)(lo | (hi << 4)) - 32);
    }
    }
    return NAN;
}

/* Dequantize `count` consecutive coefficients starting at block 0 of `w`.
 * `count` must be a multiple of the block's element count. */
int oo_dequant(uint32_t fmt, const uint8_t *w, uint64_t count, float *out) {
    uint32_t be, bb;
    if (oo_block_layout(fmt, &be, &bb))
        return -1;
    if (count % be)
        return -2;
    for (uint64_t i = 0; i < count; i++)
        out[i] = decode(fmt, w + (i / be) * bb, (uint32_t)(i % be));
    return 0;
}

/* Token rows (embed, weights.metal:90-109): row r is bf16 of the decoded
 * row ids[r] of a [vocab][k] tensor; native BF16 copies the stored bits;
 * ids >= vocab splice feature row (id - vocab), and ids past the
 * feature_rows give a row of quiet NaN (0x7fc0), this build's rule for the
 * case the reference leaves unchecked. */
int oo_embed(uint32_t fmt, const uint8_t *w, uint32_t k, uint32_t vocab, const uint32_t *ids, uint32_t rows,
             const uint16_t *features, uint32_t feature_rows, uint16_t *out) {
    uint32_t be, bb;
    if (oo_block_layout(fmt, &be, &bb) || k % be) return -1;
    const uint64_t row_bytes = (uint64_t)(k / be) * bb;
    for (uint32_t r = 0; r < rows; r++) {
        const uint32_t id = ids[r];
        uint16_t *o = out + (uint64_t)r * k;
        for (uint32_t c = 0; c < k; c++) {
            if (id >= vocab) {
                o[c] = features && id - vocab < feature_rows ? features[(uint64_t)(id - vocab) * k + c] : 0x7fc0;
                continue;
            }
            const uint8_t *blk = w + (uint64_t)id * row_bytes + (uint64_t)(c / be) * bb;
            if (fmt == 30) {
                o[c] = (uint16_t)(blk[0] | (blk[1] << 8));
            } else {
                o[c] = oo_f32_to_bf16(decode(fmt, blk, c % be));
            }
        }
    }
    return 0;
}

static double load_x(const void *x, int dt, uint64_t i) {
    if (dt == OO_DT_F32) return ((const float *)x)[i];
    if (dt == OO_DT_BF16) return oo_bf16(((const uint16_t *)x)[i]);
    return oo_fp16(((const uint16_t *)x)[i]);
}

/* Row address and input/output indexing of the vector kernels:
 * expert = experts>1 ? ids[route] : 0, input = experts>1 && !route_major ?
 * route/routes : route (vector.metal:76-78); output at route*n + row.  */
static void route_geometry(const oo_matrix *p, const uint32_t *ids, uint32_t route,
                           uint32_t *expert, uint32_t *input) {
    *expert = p->experts > 1 ? ids[route] : 0;
    *input = (p->experts > 1 && !p->route_major) ? route / p->routes : route;
}

/* Bias epilogue of every matrix kernel: bf16(bias + (has_bias == 2 ? 1 : 0))
 * added in fp32 (vector.metal:140-142). */
static float bias_term(const oo_matrix *p, const float *bias, uint32_t expert, uint32_t row) {
    if (!p->has_bias) return 0.f;
    float b = bias[(uint64_t)expert * p->n + row] + (p->has_bias == 2 ? 1.0f : 0.0f);
    return oo_bf16(oo_f32_to_bf16(b));
}

/* fp64 reference of y = W x + b for every (route, row), before output
 * storage rounding, plus sum |w x| + |b| for the roundoff bound
 * (matrix_precision.rs:119-142).  Rows are routes * n long. */
int oo_matvec_f64(uint32_t fmt, const uint8_t *w, const void *x, int x_dtype,
                  const float *bias, const uint32_t *ids, const oo_matrix *p,
                  double *y, double *magnitude) {
    uint32_t be, bb;
    if (oo_block_layout(fmt, &be, &bb) || p->k % be)
        return -1;
    uint64_t row_bytes = (uint64_t)p->k / be * bb;
    float *row = (float *)malloc(sizeof(float) * p->k);
    if (!row) return -3;
    for (uint32_t route = 0; route < p->m; route++) {
        uint32_t expert, input;
        route_geometry(p, ids, route, &expert, &input);
        for (uint32_t r = 0; r < p->n; r++) {
            oo_dequant(fmt, w + ((uint64_t)expert * p->n + r) * row_bytes, p->k, row);
            double s = 0, mag = 0;
            for (uint32_t i = 0; i < p->k; i++) {
                double t = (double)row[i] * load_x(x, x_dtype, (uint64_t)input * p->k + i);
                s += t;
                mag += fabs(t);
            }
            double b = bias_term(p, bias, expert, r);
            y[(uint64_t)route * p->n + r] = s + b;
            if (magnitude) magnitude[(uint64_t)route * p->n + r] = mag + fabs(b);
        }
    }
    free(row);
    return 0;
}

/* Scalar fp32 dequantize-then-dot: the CPU baseline ("port") and the
 * storage-rounding model of the reference (store_result, weights.metal:28-33;
 * f32 routed output when experts > 1 && !route_major, vector.metal:142-146).
 * `threads` > 1 splits rows with OpenMP. */
int oo_matvec_f32(uint32_t fmt, const uint8_t *w, const void *x, int x_dtype,
                  const float *bias, const uint32_t *ids, const oo_matrix *p,
                  void *y, int y_dtype, int threads) {
    uint32_t be, bb;
    if (oo_block_layout(fmt, &be, &bb) || p->k % be)
        return -1;
    uint64_t row_bytes = (uint64_t)p->k / be * bb;
    int f32_out = y_dtype == OO_DT_F32 || (p->experts > 1 && !p->route_major);
    for (uint32_t route = 0; route < p->m; route++) {
        uint32_t expert, input;
        route_geometry(p, ids, route, &expert, &input);
        float *xf = (float *)malloc(sizeof(float) * p->k);
        if (!xf) return -3;
        for (uint32_t i = 0; i < p->k; i++)
            xf[i] = (float)load_x(x, x_dtype, (uint64_t)input * p->k + i);
#ifdef _OPENMP
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
#endif
        {
            float *row = (float *)malloc(sizeof(float) * p->k);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int64_t r = 0; r < (int64_t)p->n; r++) {
                const uint8_t *src = w + ((uint64_t)expert * p->n + (uint64_t)r) * row_bytes;
                for (uint32_t i = 0; i < p->k; i++)
                    row[i] = decode(fmt, src + (i / be) * bb, i % be);
                float s = 0.f;
                for (uint32_t i = 0; i < p->k; i++)
                    s = fmaf(row[i], xf[i], s);
                s += bias_term(p, bias, expert, (uint32_t)r);
                uint64_t o = (uint64_t)route * p->n + (uint64_t)r;
                if (f32_out) ((float *)y)[o] = s;
                else ((uint16_t *)y)[o] = oo_f32_to_bf16(s);
            }
            free(row);
        }
        free(xf);
    }
    (void)threads;
    return 0;
}

/* Top-k expert selection for one token (routing.metal:71-94, generalised
 * from 4-of-32 to k-of-E): repeatedly take the maximum, ties to the lowest
 * index; the chosen logits are rounded to bf16; probabilities are
 * bf16(exp(c_r - c_0) / sum_j exp(c_j - c_0)) over the k chosen.  Any
 * non-finite logit (or non-finite chosen value) gives NaN probabilities while
 * the ids stay valid (non-finite logits rank as -inf). */
int oo_select_experts(const float *logits, uint32_t experts, uint32_t k,
                      uint32_t *ids, float *probs) {
    if (k == 0 || k > experts || k > 64) return -1;
    int invalid = 0;
    uint8_t taken[1024];
    if (experts > 1024) return -1;
    memset(taken, 0, experts);
    float chosen[64];
    for (uint32_t e = 0; e < experts; e++)
        if ((f32_bits(logits[e]) & 0x7f800000u) == 0x7f800000u) invalid = 1;
    for (uint32_t r = 0; r < k; r++) {
        float mx = -INFINITY;
        for (uint32_t e = 0; e < experts; e++) {
            float v = (f32_bits(logits[e]) & 0x7f800000u) == 0x7f800000u ? -INFINITY : logits[e];
            if (!taken[e] && v > mx) mx = v;
        }
        uint32_t id = 0xffffffffu;
        for (uint32_t e = 0; e < experts; e++) {
            float v = (f32_bits(logits[e]) & 0x7f800000u) == 0x7f800000u ? -INFINITY : logits[e];
            if (!taken[e] && v == mx) { id = e; break; }
        }
        ids[r] = id;
        if (id < experts) taken[id] = 1;
        chosen[r] = oo_bf16(oo_f32_to_bf16(mx));
    }
    for (uint32_t r = 0; r < k; r++)
        if ((f32_bits(chosen[r]) & 0x7f800000u) == 0x7f800000u) invalid = 1;
    if (invalid) {
        for (uint32_t r = 0; r < k; r++) probs[r] = bits_f32(0x7fc00000u);
        return 0;
    }
    float sum = 0.f;
    for (uint32_t r = 0; r < k; r++) sum += expf(chosen[r] - chosen[0]);
    for (uint32_t r = 0; r < k; r++)
        probs[r] = oo_bf16(oo_f32_to_bf16(expf(chosen[r] - chosen[0]) / sum));
    return 0;
}

/* Clipped SwiGLU of gpt-oss: projections.metal:4-13 (and moe_activate,
 * routing.metal:44-64).  Non-finite operands give NaN before clipping. */
float oo_swiglu_clipped(float g, float u) {
    if ((f32_bits(g) & 0x7f800000u) == 0x7f800000u || (f32_bits(u) & 0x7f800000u) == 0x7f800000u)
        return bits_f32(0x7fc00000u);
    g = fminf(g, 7.0f);
    u = fminf(fmaxf(u, -6.0f), 8.0f);
    float e = expf(-fabsf(g) * 1.702f);
    float sigmoid = (g < 0 ? e : 1.0f) / (1.0f + e);
    return sigmoid * g * u;
}

/* Words in a route plan for R routes over E experts: dispatch arguments (6),
 * tile pairs 2*(ceil(R/16)+E), per-expert lists E*(R+1), expert-sorted first
 * rows E, then each route's sorted row R (gpt_oss.rs:63-74). */
uint64_t oo_route_plan_words(uint32_t routes, uint32_t experts) {
    return 6 + 2 * ((uint64_t)(routes + 15) / 16 + experts) + (uint64_t)experts * (routes + 1) +
           experts + routes;
}

/* Route plan: routing.metal:4-39 (route_plan_64), generalised to E experts
 * and any tile height as route_plan_n does (nemotron.metal:238-273).
 * Layout: [0..5] two dispatch grids (up_tiles, tiles, 1, down_tiles, tiles, 1);
 * [6..] (expert, first list row) per tile; lists at 6+2*(ceil(R/16)+E): per
 * expert a count then the route indices in route order; then each expert's
 * first row in expert-sorted order; then each route's sorted row. */
uint64_t oo_route_plan(const uint32_t *ids, uint32_t routes, uint32_t experts, uint32_t tile_rows,
                       uint32_t up_tiles, uint32_t down_tiles, uint32_t *plan) {
    if (tile_rows < 16) /* the tile area holds ceil(routes/16) + experts tiles */
        return (uint64_t)-1;
    uint64_t grouped = 6 + 2 * ((uint64_t)(routes + 15) / 16 + experts);
    uint64_t sorted = grouped + (uint64_t)experts * (routes + 1);
    uint32_t tiles = 0, offset = 0;
    for (uint32_t e = 0; e < experts; e++) {
        uint64_t base = grouped + (uint64_t)e * (routes + 1);
        uint32_t count = 0;
        for (uint32_t i = 0; i < routes; i++)
            if (ids[i] == e) plan[base + 1 + count++] = i;
        plan[base] = count;
    }
    for (uint32_t e = 0; e < experts; e++) {
        uint32_t routed = plan[grouped + (uint64_t)e * (routes + 1)];
        plan[sorted + e] = offset;
        for (uint32_t i = 0; i < routed; i++)
            plan[sorted + experts + plan[grouped + (uint64_t)e * (routes + 1) + 1 + i]] = offset + i;
        offset += routed;
        for (uint32_t begin = 0; begin < routed; begin += tile_rows) {
            plan[6 + 2 * (uint64_t)tiles] = e;
            plan[6 + 2 * (uint64_t)tiles + 1] = begin;
            tiles++;
        }
    }
    plan[0] = up_tiles; plan[1] = tiles; plan[2] = 1;
    plan[3] = down_tiles; plan[4] = tiles; plan[5] = 1;
    return tiles;
}

/* Weighted combine with residual: routing.metal:157-168, k routes per token:
 * out = bf16(out + bf16(sum_r route_r * p_r)), the sum in route order. */
void oo_moe_sum(const uint16_t *routes, const float *probs, uint16_t *out,
                uint32_t hidden, uint32_t batch, uint32_t k) {
    for (uint64_t i = 0; i < (uint64_t)hidden * batch; i++) {
        uint64_t t = i / hidden, d = i % hidden;
        float s = 0.f;
        for (uint32_t r = 0; r < k; r++)
            s += oo_bf16(routes[(t * k + r) * hidden + d]) * probs[t * k + r];
        out[i] = oo_f32_to_bf16(oo_bf16(out[i]) + oo_bf16(oo_f32_to_bf16(s)));
    }
}

/* Greedy token selection: shaders/argmax.metal:1-47.  Finite logits order as
 * integers after folding the sign (-0 counts as +0); ties go to the lowest
 * index; any Inf or NaN makes the answer 0xffffffff, as does n == 0. */
uint32_t oo_argmax_f32(const float *logits, uint32_t n) {
    uint32_t val = 0, id = 0xffffffffu;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t bits;
        memcpy(&bits, &logits[i], 4);
        if ((bits & 0x7f800000u) == 0x7f800000u) return 0xffffffffu;
        bits = (bits & 0x7fffffffu) == 0 ? 0u : bits;
        const uint32_t v = bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
        if (v > val) {
            val = v;
            id = i;
        }
    }
    return id;
}

/* RMS normalisation of bf16 rows: elementwise.metal:6-28.
 * inv = 1 / sqrt(mean(x^2) + epsilon) in fp64; y = bf16(x inv w) when
 * full_layer, else bf16(bf16(x inv) * bf16(w)) (the two rounding points of
 * the reference).  Returns the f64 row values before the final rounding in
 * `exact` (may be NULL) so tests can bound the rounding. */
void oo_norm(const uint16_t *x, const float *w, uint16_t *y, double *exact, uint32_t rows, uint32_t n,
             float epsilon, int full_layer) {
    for (uint32_t r = 0; r < rows; r++) {
        const uint16_t *xr = x + (uint64_t)r * n;
        double s = 0;
        for (uint32_t i = 0; i < n; i++) {
            const double v = oo_bf16(xr[i]);
            s += v * v;
        }
        const double inv = 1.0 / sqrt(s / n + (double)epsilon);
        for (uint32_t i = 0; i < n; i++) {
            const double t = oo_bf16(xr[i]) * inv;
            const double v = full_layer ? t * (double)w[i]
                                        : (double)oo_bf16(oo_f32_to_bf16((float)t)) * oo_bf16(oo_f32_to_bf16(w[i]));
            if (exact) exact[(uint64_t)r * n + i] = v;
            y[(uint64_t)r * n + i] = oo_f32_to_bf16((float)v);
        }
    }
}

/* Residual add then normalisation: elementwise.metal:32-58.  x (the
 * residual stream, bf16) becomes bf16(x + y); out is its normalised form. */
void oo_add_norm(uint16_t *x, const uint16_t *y, const float *w, uint16_t *out, double *exact, uint32_t rows,
                 uint32_t n, float epsilon, int full_layer) {
    for (uint64_t i = 0; i < (uint64_t)rows * n; i++) x[i] = oo_f32_to_bf16(oo_bf16(x[i]) + oo_bf16(y[i]));
    oo_norm(x, w, out, exact, rows, n, epsilon, full_layer);
}
