/* Self-test driver for the oracle under ASan/UBSan (test infrastructure).
 * Runs every oracle entry point over random bytes of every format so the
 * sanitizers see each code path; exits non-zero on any failed call. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

typedef struct { uint32_t k, n, m, route_major, routes, experts, has_bias; } oo_matrix;
int oo_block_layout(uint32_t, uint32_t *, uint32_t *);
int oo_dequant(uint32_t, const uint8_t *, uint64_t, float *);
int oo_matvec_f64(uint32_t, const uint8_t *, const void *, int, const float *, const uint32_t *,
                  const oo_matrix *, double *, double *);
int oo_matvec_f32(uint32_t, const uint8_t *, const void *, int, const float *, const uint32_t *,
                  const oo_matrix *, void *, int, int);
int oo_select_experts(const float *, uint32_t, uint32_t, uint32_t *, float *);
float oo_swiglu_clipped(float, float);
uint64_t oo_route_plan_words(uint32_t, uint32_t);
uint64_t oo_route_plan(const uint32_t *, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t *);
void oo_moe_sum(const uint16_t *, const float *, uint16_t *, uint32_t, uint32_t, uint32_t);
uint32_t oo_argmax_f32(const float *, uint32_t);
void oo_norm(const uint16_t *, const float *, uint16_t *, double *, uint32_t, uint32_t, float, int);
void oo_add_norm(uint16_t *, const uint16_t *, const float *, uint16_t *, double *, uint32_t, uint32_t, float, int);

int main(void) {
    const uint32_t fmts[] = {0, 1, 2, 3, 8, 12, 13, 14, 30, 39};
    uint32_t k = 512, n = 5, E = 3;
    srand(1);
    for (unsigned f = 0; f < sizeof fmts / sizeof *fmts; f++) {
        uint32_t be, bb;
        if (oo_block_layout(fmts[f], &be, &bb)) return 1;
        size_t bytes = (size_t)E * n * (k / be) * bb;
        uint8_t *w = malloc(bytes);
        for (size_t i = 0; i < bytes; i++) w[i] = (uint8_t)rand();
        float *out = malloc(sizeof(float) * E * n * k);
        if (oo_dequant(fmts[f], w, (uint64_t)E * n * k, out)) return 2;
        float x[2 * 512], bias[3 * 5];
        for (int i = 0; i < 2 * 512; i++) x[i] = (float)rand() / RAND_MAX - 0.5f;
        for (int i = 0; i < 15; i++) bias[i] = (float)i;
        uint32_t ids[4] = {2, 0, 1, 2};
        oo_matrix p = {k, n, 4, 0, 2, E, 2};
        double y[4 * 5], mag[4 * 5];
        float y32[4 * 5];
        if (oo_matvec_f64(fmts[f], w, x, 0, bias, ids, &p, y, mag)) return 3;
        if (oo_matvec_f32(fmts[f], w, x, 0, bias, ids, &p, y32, 0, 2)) return 4;
        free(w);
        free(out);
    }
    float logits[128];
    uint32_t sel[8];
    float probs[8];
    for (int i = 0; i < 128; i++) logits[i] = (float)rand() / RAND_MAX;
    if (oo_select_experts(logits, 128, 8, sel, probs)) return 5;
    (void)oo_swiglu_clipped(3.f, -9.f);
    uint32_t routes = 68, ids[68];
    for (uint32_t i = 0; i < routes; i++) ids[i] = (uint32_t)rand() % 32;
    uint32_t *plan = calloc(oo_route_plan_words(routes, 32), 4);
    oo_route_plan(ids, routes, 32, 64, 1, 1, plan);
    free(plan);
    uint16_t r16[4 * 2 * 3] = {0}, o16[2 * 3] = {0};
    float pr[8] = {.25f, .25f, .25f, .25f, .5f, .5f, 0, 0};
    oo_moe_sum(r16, pr, o16, 3, 2, 4);
    if (oo_argmax_f32(logits, 128) >= 128 || oo_argmax_f32(logits, 0) != 0xffffffffu) return 6;
    uint16_t xb[2 * 96], yb[2 * 96], nb[2 * 96];
    float nw[96];
    double ex[2 * 96];
    for (int i = 0; i < 2 * 96; i++) {
        xb[i] = (uint16_t)(0x3f00 + rand() % 256);
        yb[i] = (uint16_t)(0xbf00 + rand() % 256);
    }
    for (int i = 0; i < 96; i++) nw[i] = 1.0f + (float)i / 96;
    oo_norm(xb, nw, nb, ex, 2, 96, 1e-6f, 0);
    oo_add_norm(xb, yb, nw, nb, NULL, 2, 96, 1e-6f, 1);
    puts("oracle selftest ok");
    return 0;
}
