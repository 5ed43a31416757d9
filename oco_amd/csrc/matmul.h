// Shared by the prefill matmul and the routed-expert prefill path.
#pragma once

#include "common.h"

namespace oco {

struct MatmulArgs {
    const uint8_t *w;
    const void *x;
    void *y;
    const float *bias;
    uint32_t m, n, k;
    uint64_t row_bytes;
    uint32_t x_f16, y_bf16;
    // Grouped (routed-expert) mode: tiles come from a route plan.
    const uint32_t *plan;  // route plan with tile_rows = BM
    const uint8_t *w2;     // up weights (gate/up mode)
    const float *bias2;    // up bias (gate/up mode)
    uint64_t expert_bytes; // bytes of one expert's matrix
    uint32_t routes, experts, topk, act, up_one;
    uint32_t *rowmax;      // [routes] max |activation| bits per expert-sorted row (gate/up writes, down reads)
};

// Grouped modes of matmul_kernel.
constexpr int MM_DENSE = 0;  // Y = X W^T
constexpr int MM_GATE_UP = 1;  // per expert tile: act = f(X W_gate^T, X W_up^T), f32 at expert-sorted rows
constexpr int MM_DOWN = 2;     // per expert tile: routed[route] = act W_down^T (+ bias), f32

// One grouped GEMM over a route plan built with tile_rows = bm (32 or 64):
// MM_GATE_UP writes f32 activations at expert-sorted rows and each row's
// max |activation| (rowmax, zeroed by the caller); MM_DOWN reads them with
// a per-row power-of-two gain into f16 and writes f32 (or bf16) route rows.
int grouped_matmul_launch(int mode, uint32_t fmt, const MatmulArgs &a, uint32_t bm, hipStream_t stream);

// The same for Q4_K banks with weights decoded in registers (route plan with
// tile_rows = bm: 32, 48 or 64).
int moe_q4k_launch(int mode, const MatmulArgs &a, uint32_t bm, hipStream_t stream);

}  // namespace oco
