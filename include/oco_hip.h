/*
 * oco_hip.h -- C ABI of the MI355X (gfx950) quantized-weight matrix path.
 *
 * Drop-in for the Metal kernels and operator seams of xhjkl/oco:
 *   - GGUF block dequantization fused into decode matvec (shaders/matrix),
 *   - the top-k routed expert path (shaders/experts),
 *   - prefill matmul on MFMA,
 * behind plain-C entry points: pointers and sizes only, no C++ or torch types.
 *
 * Conventions (mirroring the reference's seam, src/gpu/dispatch.rs:211-285 and
 * src/error.rs:9-27):
 *   - every entry point returns an int status, OCO_OK (0) on success; the
 *     message of the last failure on the calling thread is oco_last_error();
 *   - no C++ exception crosses the ABI;
 *   - device pointers are plain `void *` in device memory (oco_buffer_alloc or
 *     any hipMalloc'd memory); weights are read-only and may sit at any byte
 *     offset (GGUF guarantees only 1-byte alignment for MXFP4 blocks);
 *   - calls are ordered on the given stream (NULL = the default stream) and
 *     never synchronise the host except oco_stream_sync and the transfer
 *     helpers marked "blocking";
 *   - kernels never report data errors: NaN is the in-band failure signal
 *     (E8M0 exponent 255, non-finite router inputs), as in the reference.
 *
 * Each declaration cites the reference interface it replaces (file:line,
 * relative to the oco checkout).
 */
#ifndef OCO_HIP_H
#define OCO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
enum {
    OCO_OK = 0,
    OCO_ERR_INVALID = 1,     /* bad argument or geometry (Error::Request)      */
    OCO_ERR_UNSUPPORTED = 2, /* format/variant without a kernel               */
    OCO_ERR_HIP = 3,         /* HIP runtime failure (Error::Gpu)              */
    OCO_ERR_MEMORY = 4,      /* allocation failure                            */
    OCO_ERR_CHECKPOINT = 5   /* malformed or unsupported GGUF (Error::Checkpoint) */
};

/* GGUF format codes: src/tensor.rs:9-20 (WeightFormat). */
typedef enum oco_format {
    OCO_F32 = 0,
    OCO_F16 = 1,
    OCO_Q4_0 = 2,
    OCO_Q4_1 = 3,
    OCO_Q8_0 = 8,
    OCO_Q4_K = 12,
    OCO_Q5_K = 13,
    OCO_Q6_K = 14,
    OCO_BF16 = 30,
    OCO_MXFP4 = 39
} oco_format;

/* Activation / output element types.  The reference's kernels read bf16 and
 * store bf16 unless `output_f32` is specialised (weights.metal:24-33). */
typedef enum oco_dtype { OCO_DT_F32 = 0, OCO_DT_BF16 = 1, OCO_DT_F16 = 2 } oco_dtype;

/* Kernel parameter block: shaders/matrix/weights.metal:87-89 and
 * src/weights/compute/matrix.rs:10-20 (Matrix).
 *   k, n       : input width, output rows (GGUF shape [k, n(, experts)])
 *   m          : routes (vector rows); for oco_matmul the activation rows
 *   route_major: routed input is indexed by route, not route/routes
 *   routes     : routes per token (top-k)
 *   experts    : experts in the bank; > 1 selects rows through ids[route]
 *   has_bias   : 0 none, 1 add bf16(bias), 2 add bf16(bias + 1) (gpt-oss up)
 * Routed rows: expert = experts > 1 ? ids[route] : 0, input =
 * experts > 1 && !route_major ? route / routes : route, output at
 * route * n + row, and f32 output whenever experts > 1 && !route_major
 * (vector.metal:76-78, 142-146). */
typedef struct oco_matrix {
    uint32_t k, n, m, route_major, routes, experts, has_bias;
} oco_matrix;

typedef void *oco_stream; /* hipStream_t; NULL = default stream */
typedef void *oco_event;  /* hipEvent_t */

/* Thread-local message of the last failed call on this thread ("" if none). */
const char *oco_last_error(void);

/* Kernel-choice overrides.  No counterpart in the reference, whose kernel
 * choice tables are fixed at pipeline build time (src/weights/pipelines.rs:
 * 227-355, compute/matrix.rs:130-379); here the same tables run unless a
 * knob is set, so that parity tests can reach every kernel variant and
 * tuning runs can compare them.  count == 0 clears the knob.  Not
 * synchronised with launches on other threads: set knobs before launching. */
typedef enum oco_knob {
    OCO_KNOB_STREAM_PLAN = 0,     /* streaming matvec: 1 (reserved), K split (1|2|4), WGs per CU */
    OCO_KNOB_MATVEC_PLAN = 1,     /* plain matvec (F32/F16/BF16): rows per wave, K split */
    OCO_KNOB_MATVEC_PLAIN = 2,    /* value 1: quantized formats take the plain matvec, not the streaming one */
    OCO_KNOB_MX_TILE = 3,         /* reserved (the MXFP4 prefill has a single tile: 128 x 96) */
    OCO_KNOB_MX_PREFILL_OFF = 4,  /* value 1: MXFP4 prefill takes the f16 MFMA tiles instead of the FP4 ones */
    OCO_KNOB_MATMUL_TILE = 5,     /* f16 MFMA prefill tile choice index */
    OCO_KNOB_MOE_MX_TOKENS = 6,   /* MXFP4 banks take the block-scaled MFMA tiles from this many tokens */
    OCO_KNOB_MOE_MFMA_TOKENS = 7, /* other banks take the grouped MFMA tiles from this many tokens */
    OCO_KNOB_MOE_Q4_ROWS = 8,     /* Q4_K grouped tiles: rows per tile (32|48|64), value 0: the f16 LDS tiles */
    OCO_KNOB_MOE_WG = 9,          /* routed decode kernel: workgroups per CU */
    OCO_KNOB_MX_EXPERTS_KS = 10,  /* MXFP4 expert down tiles of 16 rows: K split (1|2) */
    OCO_KNOB_STREAM_DIRECT = 11,  /* value 0: Q4_K/Q5_K streaming matvec through the LDS tile even when aligned;
                                     second value (optional): activations 0 staged in LDS, 1 in registers */
    OCO_KNOB_MATMUL_VENDOR = 12,  /* f16-operand prefill: value 0 the fused f16 MFMA tiles, 1 the dequantize pass
                                     and the vendor GEMM (default: the vendor GEMM from 32 activation rows) */
    OCO_KNOB_COUNT = 13
} oco_knob;
int oco_plan_override(uint32_t knob, const int32_t *values, uint32_t count);

/* (elements, bytes) per GGUF block: src/tensor.rs:24-38 (block_layout). */
int oco_block_layout(uint32_t format, uint32_t *elements, uint32_t *bytes);

/* Bytes of one row of `k` coefficients; 0 when k is not block aligned. */
uint64_t oco_row_bytes(uint32_t format, uint32_t k);

/* ---- device, memory, streams: src/gpu.rs:34-117, src/gpu/buffer.rs,
 *      src/gpu/dispatch.rs, src/weights/compute/submission.rs ------------- */

/* Select device `ordinal` for this thread and report its compute units.
 * Replaces Gpu::new (src/gpu.rs:41-50). */
int oco_device_open(int ordinal, int *compute_units);

/* Device allocations (MappedRegions / Arena storage, src/gpu/buffer.rs:145-297,
 * src/gpu/arena.rs:19-125). */
int oco_buffer_alloc(size_t bytes, void **out);
int oco_buffer_free(void *ptr);
/* Blocking host<->device copies (the reference's BufferView reads/writes). */
int oco_buffer_upload(void *dst, const void *src, size_t bytes);
int oco_buffer_download(void *dst, const void *src, size_t bytes);
/* Device-to-device copy on a stream. */
int oco_buffer_copy(void *dst, const void *src, size_t bytes, oco_stream stream);
/* Fill `words` 32-bit words with `pattern` by a kernel (guard sentinels,
 * dispatch_tests.rs:12-13); safe inside captured graphs. */
int oco_buffer_fill32(void *dst, uint32_t pattern, size_t words, oco_stream stream);

/* Diagnostic exports: no counterpart in the reference and not part of the
 * matrix path.  oco_buffer_xor32 XORs `words` 32-bit words at src (16-byte
 * aligned, words a multiple of 4, at most OCO_XOR32_MAX_BYTES bytes) into
 * OCO_XOR32_SLOTS words of device memory at out: the XOR of
 * out[0 .. OCO_XOR32_SLOTS - 1] is the XOR of the words (each workgroup
 * stores its share; all slots are written).  It is an integrity check of
 * weights made resident, and the plain HBM read stream that the matvec
 * kernels are measured against.  oco_buffer_xor32_geometry reports the
 * launch it would make (16 KiB rounds; workgroups), or OCO_ERR_INVALID past
 * the size limit, without touching a device. */
#define OCO_XOR32_SLOTS 1024u
#define OCO_XOR32_MAX_BYTES (0xffffffffull - 32768ull)
int oco_buffer_xor32(const void *src, size_t words, uint32_t *out, oco_stream stream);
int oco_buffer_xor32_geometry(uint64_t words, uint64_t *rounds, uint64_t *workgroups);

/* One queue per session (src/weights/compute.rs:36-55). */
int oco_stream_create(oco_stream *out);
int oco_stream_sync(oco_stream stream);
int oco_stream_destroy(oco_stream stream);

/* Timestamps (OCO_PROFILE stamps, src/gpu/profile.rs:33-46). */
int oco_event_create(oco_event *out);
int oco_event_record(oco_event event, oco_stream stream);
int oco_event_elapsed_ms(oco_event start, oco_event stop, float *ms);
int oco_event_destroy(oco_event event);

/* Stream capture into a replayable HIP graph, for launch-bound sequences of
 * short kernels (the reference encodes a whole token's dispatches into one
 * command buffer, src/weights/compute/submission.rs:21-107).  Calls between
 * begin and end are recorded, not run; the library records no memset nodes. */
typedef void *oco_graph;
int oco_graph_begin(oco_stream stream);
int oco_graph_end(oco_stream stream, oco_graph *out);
int oco_graph_launch(oco_graph graph, oco_stream stream);
int oco_graph_destroy(oco_graph graph);

/* ---- dequantization ----------------------------------------------------- */

/* Decode `count` coefficients (a multiple of the block's elements) of a GGUF
 * tensor starting at `w` into f32: the `weight()` decoder of
 * shaders/matrix/weights.metal:48-85 (mxfp4 at :40-46).  Bit-exact:
 * Q8_0, Q6_K, Q4_0, MXFP4, F16, BF16 are exact; Q4_K/Q5_K/Q4_1 round once.
 * MXFP4 exponent 255 decodes to NaN (projections.metal:19-23). */
int oco_dequant(uint32_t format, const void *w, uint64_t count, float *out, oco_stream stream);

/* Token embedding rows: out[r] = bf16 of row ids[r] of a GGUF tensor of
 * `vocabulary` rows of `k` coefficients, decoded as oco_dequant does (native
 * BF16 rows are copied as bits).  Ids >= vocabulary take row (id -
 * vocabulary) of `features` (bf16 [feature_rows, k], may be NULL when
 * feature_rows == 0): the spliced audio feature rows of the reference.  Ids
 * past those rows too get a NaN row (the reference reads them unchecked).
 * out: bf16 [rows, k].  Replaces `embed` (shaders/matrix/weights.metal:90-109,
 * pipeline Builder::embedding, src/weights/pipelines.rs:180-193, dispatched
 * by Compute::embed, src/weights/compute/matrix.rs:487-516). */
int oco_embed(uint32_t format, const void *w, uint32_t k, uint32_t vocabulary, const uint32_t *ids, uint32_t rows,
              const uint16_t *features, uint32_t feature_rows, uint16_t *out, oco_stream stream);

/* ---- decode matvec ------------------------------------------------------ */

/* y = W x (+ bias) for every route in p->m, fp32 accumulation.
 * Replaces the vector kernels `matvec`, `matvec_q8_split`, `matvec_q6k`,
 * `matvec_q5k`, `matvec_q4`, `matvec_split` (shaders/matrix/vector.metal:66,
 * 155, 232, 292, 370; q8-dot.metal:39) as chosen by Builder::vector_kernel
 * (src/weights/pipelines.rs:227-265) and dispatched by
 * DenseMatrix::apply_row / Bindings::output (compute/matrix.rs:63, 519).
 *   x: p->m (or tokens, for routed input) rows of p->k elements of x_dtype
 *   y: p->m * p->n elements of y_dtype (forced f32 when routed non-route-major)
 *   bias: f32 [experts * n] or NULL when has_bias == 0
 *   ids: u32 [m] expert per route, or NULL when experts <= 1 */
int oco_matvec(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
               oco_dtype y_dtype, const float *bias, const uint32_t *ids, const oco_matrix *p,
               oco_stream stream);

/* oco_matvec with relu^2 applied to every input element on load:
 * x -> max(x, 0)^2 in f32 (a NaN element reads as 0), before the dot
 * products.  Replaces the vector kernels specialised with `input_relu_sqr`
 * (shaders/matrix/weights.metal:22-24, vector.metal:120-123, 185-190,
 * q8-dot.metal:12-15, 59-64) as Builder::vector_kernel(kind, output,
 * relu_sqr = true, ..) builds them (src/weights/pipelines.rs:227-254) for
 * Nemotron's relu^2 feed-forward down projection (nemotron/load.rs:408).
 * Same arguments and rules as oco_matvec. */
int oco_matvec_relu_sqr(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                        oco_dtype y_dtype, const float *bias, const uint32_t *ids, const oco_matrix *p,
                        oco_stream stream);

/* ---- prefill matmul ----------------------------------------------------- */

/* Y[m, n] = X[m, k] W^T (+ bias) on MFMA with fp32 accumulation.
 * Replaces DenseMatrix::apply's tiled plans (compute/matrix.rs:130-379,
 * `matmul`/`matmul_q4*`/`matmul_tensor_*`, batch.metal:24-79, tensor.metal:9-102).
 * Operands: formats other than MXFP4 decode to f16 (the reference's
 * half(w), tile.metal:16-80) with activations converted to f16; from 32
 * rows (n % 4 == 0) that decode is one pass into a workspace and the
 * product a vendor (hipBLASLt) f16 GEMM, below it fused MFMA tiles.  X is
 * bf16 or f16 row-major; Y f32 or bf16.  MXFP4 runs the block-scaled FP6 x
 * FP4 MFMA on the GGUF bytes as stored, with each 32-block of X split into
 * two E2M3 terms with their own E8M0 scales (at most 1/225 of the block
 * maximum per value; relative L2 of the product a few 1e-4, inside the 2e-3
 * bound for bf16-activation MFMA prefill), also through a workspace.
 * oco_matmul takes workspaces from the stream-ordered pool (hipMallocAsync).
 * With bf16 X, up to Builder::dense's vector_rows rows (pipelines.rs:271-283:
 * 1; 4 for Q4_0/Q4_1 and three Q5_K/Q8_0 shapes; 128 for Q8_0 2880 -> 512;
 * every m for F32 with n <= 128) run oco_matvec instead, exact weights and
 * fp32, as DenseMatrix::apply does; Q4_0/Q4_1 with n > 1024 scale each
 * activation row by the reference's power-of-two gain before the f16
 * rounding (matmul_q4_half). */
int oco_matmul(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
               oco_dtype y_dtype, const float *bias, const oco_matrix *p, oco_stream stream);

/* Workspace bytes oco_matmul_ws needs for this call (0: none).  The
 * reference draws such scratch from the session Arena (src/gpu/arena.rs). */
uint64_t oco_matmul_workspace(uint32_t format, oco_dtype x_dtype, const oco_matrix *p);

/* oco_matmul with caller-owned workspace (no allocation; graph-capturable).
 * Calls sharing one workspace must be ordered on one stream. */
int oco_matmul_ws(uint32_t format, const void *w, const void *x, oco_dtype x_dtype, void *y,
                  oco_dtype y_dtype, const float *bias, const oco_matrix *p, void *workspace,
                  uint64_t workspace_bytes, oco_stream stream);

/* The norm -> MXFP4 prefill pair in two launches instead of three: the RMS
 * norm of oco_norm (same rounding) whose workgroups also split each output
 * row into the E2M3 records the MXFP4 prefill reads, bit for bit the records
 * oco_matmul would make from oco_norm's output.  `split`: at least
 * oco_matmul_workspace(OCO_MXFP4, OCO_DT_BF16, {k = n, m = rows}) bytes; `y`
 * (optional, may be null) receives the bf16 output rows too; n % 32 == 0.
 * Replaces prepare_norm_scales + apply_norm (the batch norm folded into the
 * matrix's input: feed_forward.rs:99-101, compute/matrix.rs:429-441). */
int oco_norm_mx_split(const void *x, const float *norm_w, void *y, uint32_t rows, uint32_t n, float epsilon,
                      int full_layer, void *split, uint64_t split_bytes, oco_stream stream);

/* oco_add_norm (x = bf16(x + y) in place, then the norm; `out` optional)
 * writing the same split records: the residual add -> norm -> MXFP4 prefill
 * of a layer step in two launches.  Replaces add_norm
 * (elementwise.metal:32-58) feeding apply_norm (compute/matrix.rs:429-441). */
int oco_add_norm_mx_split(void *x, const void *y, const float *norm_w, void *out, uint32_t rows, uint32_t n,
                          float epsilon, int full_layer, void *split, uint64_t split_bytes, oco_stream stream);

/* oco_matmul for MXFP4 weights from rows already split by oco_norm_mx_split
 * or oco_add_norm_mx_split (the same m and k): equal to the norm then
 * oco_matmul, bit for bit, from two rows on (one row takes oco_matmul's
 * matvec; this entry always runs the block-scaled MFMA). */
int oco_matmul_mx_split(const void *w, const void *split, uint64_t split_bytes, void *y, oco_dtype y_dtype,
                        const float *bias, const oco_matrix *p, oco_stream stream);

/* ---- routing ------------------------------------------------------------ */

/* Per token: top-k of `experts` logits (ties to the lowest index, non-finite
 * ranks as -inf), chosen logits rounded to bf16, probabilities bf16 of the
 * softmax over the chosen k; any non-finite input -> NaN probabilities.
 * Replaces select_expert_values (shaders/experts/routing.metal:71-94),
 * generalised to experts <= 256, k <= 8.  ids/probs: [tokens, k]. */
int oco_route_select(const float *logits, uint32_t tokens, uint32_t experts, uint32_t k,
                     uint32_t *ids, float *probs, oco_stream stream);

/* Router logits = bf16(x) . bf16(W) + bf16(bias) over `experts` rows of f32
 * weights [experts, hidden], then oco_route_select.  Replaces `router` and
 * `router_logits` (routing.metal:96-146).  `logits` (may be NULL) receives
 * [tokens, experts] f32. */
int oco_router(const void *x, oco_dtype x_dtype, const float *w, const float *bias,
               uint32_t tokens, uint32_t hidden, uint32_t experts, uint32_t k, float *logits,
               uint32_t *ids, float *probs, oco_stream stream);

/* Words of a route plan for `routes` routes over `experts` experts
 * (src/weights/gpt_oss.rs:63-74). */
uint64_t oco_route_plan_words(uint32_t routes, uint32_t experts);

/* Per-expert route lists, (expert, first row) tiles of `tile_rows`, two
 * dispatch grids at words 0-5, expert-sorted offsets and each route's sorted
 * row: route_plan_64 (routing.metal:4-39) and route_plan_n
 * (nemotron.metal:238-273).  ids: u32 [routes].  The tile area holds
 * ceil(routes/16) + experts tiles, so tile_rows must be >= 16.  Words not
 * listed above (unused tile slots, list entries past each count) are left
 * untouched, as in the reference. */
int oco_route_plan(const uint32_t *ids, uint32_t routes, uint32_t experts, uint32_t tile_rows,
                   uint32_t up_tiles, uint32_t down_tiles, uint32_t *plan, oco_stream stream);

/* ---- routed experts ----------------------------------------------------- */

/* Activation applied between the gate/up and down projections. */
typedef enum oco_activation {
    OCO_ACT_SWIGLU_CLIPPED = 0, /* gpt-oss: sigmoid(1.702 g') g' u', g' = min(g,7),
                                   u' = clamp(u,-6,8) (projections.metal:4-13) */
    OCO_ACT_SWIGLU = 1          /* silu(g) * u, the dense `gate` kernel
                                   (elementwise.metal:70-88), in f32 */
} oco_activation;

/* One expert bank (src/weights/gpt_oss/load.rs:20-40, operands.rs ExpertWeight):
 * gate/up [experts][ffn][hidden] and down [experts][hidden][ffn] GGUF rows,
 * f32 biases [experts * rows] or NULL. */
typedef struct oco_experts {
    uint32_t format;        /* oco_format of gate/up/down */
    uint32_t hidden, ffn;   /* model width, expert width */
    uint32_t experts, k;    /* bank size, routes per token */
    uint32_t activation;    /* oco_activation */
    uint32_t up_bias_one;   /* 1: up bias carries +1 (has_bias == 2, gpt-oss) */
    const void *gate, *up, *down;
    const float *gate_bias, *up_bias, *down_bias;
} oco_experts;

/* Workspace bytes oco_experts_apply needs for `tokens` tokens. */
uint64_t oco_experts_workspace(const oco_experts *w, uint32_t tokens);

/* out[t] = bf16(out[t] + bf16(sum_r p[t,r] * down_{e_r}(act(gate_{e_r} x_t, up_{e_r} x_t)))).
 * Replaces Bindings::experts (src/weights/compute/feed_forward.rs:107-275):
 * router outputs (ids, probs [tokens, k]) are inputs here, as produced by
 * oco_router/oco_route_select; each selected expert's weights are streamed
 * once per call however many tokens chose it.  x: [tokens, hidden] of
 * x_dtype; out: [tokens, hidden] bf16 residual (read and written);
 * `routed` (may be NULL) receives the per-route f32 down outputs
 * [tokens*k, hidden] before the combine.  workspace: oco_experts_workspace bytes.
 * From 32 tokens on (prefill) the layer runs as grouped MFMA tiles over the
 * route plan -- expert_up_tensor / moe_activate / expert_down_tensor
 * (projections.metal:192-376, routing.metal:44-64) -- on f16 operands as the
 * reference's half tiles do; activation rows enter the down tiles with a
 * power-of-two gain into f16 range (the reference's q4_input_scales idea),
 * so large activations do not overflow. */
int oco_experts_apply(const oco_experts *w, const void *x, oco_dtype x_dtype,
                      const uint32_t *ids, const float *probs, uint32_t tokens, uint16_t *out,
                      float *routed, void *workspace, uint64_t workspace_bytes, oco_stream stream);

/* The whole routed layer from the router on, as Bindings::experts runs it
 * (src/weights/compute/feed_forward.rs:107-275): router logits =
 * bf16(x) . bf16(router_w) + bf16(router_bias) over `experts` f32 rows
 * [experts, hidden] (router_logits / router, routing.metal:96-146), top-k
 * selection with softmax over the chosen (select_expert_values, :71-94) --
 * at one token inside the gate/up kernel as expert_expand does
 * (projections.metal:78-137), else by its own launch -- then everything
 * oco_experts_apply does.  ids/probs [tokens, k] receive the selection
 * (routing.ids / routing.prob of the reference); workspace:
 * oco_experts_workspace bytes (the logits live at its end). */
int oco_experts_forward(const oco_experts *w, const float *router_w, const float *router_bias, const void *x,
                        oco_dtype x_dtype, uint32_t tokens, uint16_t *out, uint32_t *ids, float *probs,
                        float *routed, void *workspace, uint64_t workspace_bytes, oco_stream stream);

/* oco_experts_forward without a workspace argument and without any
 * allocation: no counterpart in the reference.  It is for callers that
 * cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Its workspace is a
 * static device array of OCO_EXPERTS_SCRATCH_BYTES per GPU (held until the
 * process ends; gpt-oss-20b needs 2.3 MB of it at 16 tokens and fits up to
 * 57); calls whose oco_experts_workspace(w, tokens) exceeds it fail with
 * OCO_ERR_INVALID.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (two streams, two threads) race and must be ordered by the caller.
 * Nothing in it needs to start at zero; it keeps the last call's contents.
 * Its device address is resolved by oco_device_open, or on the first call
 * on a device. */
#define OCO_EXPERTS_SCRATCH_BYTES (8ull << 20)
int oco_experts_forward_static(const oco_experts *w, const float *router_w, const float *router_bias, const void *x,
                               oco_dtype x_dtype, uint32_t tokens, uint16_t *out, uint32_t *ids, float *probs,
                               float *routed, oco_stream stream);

/* Single-token fused expansion: select the top-k experts from `logits`
 * [experts], then gate and up projections of the selected experts with the
 * activation applied; up_out/act_out [k, ffn] f32; ids/probs [k].
 * Replaces expert_expand (projections.metal:78-137). */
int oco_expert_expand(const oco_experts *w, const void *x, oco_dtype x_dtype,
                      const float *logits, uint32_t *ids, float *probs, float *up_out,
                      float *act_out, oco_stream stream);

/* Weighted combine with residual: out = bf16(out + bf16(sum_r route_r p_r)).
 * routes: [tokens*k, hidden] of routes_dtype (bf16 in the reference; f32
 * route values are rounded to bf16 before weighting, as stored there).
 * k <= 8 (the expert banks' limit); OCO_ERR_INVALID beyond.
 * Replaces moe_sum (routing.metal:157-168). */
int oco_moe_sum(const void *routes, oco_dtype routes_dtype, const float *probs, uint16_t *out,
                uint32_t hidden, uint32_t tokens, uint32_t k, oco_stream stream);

/* ---- the steps either side of the decode matvec -------------------------- */

/* RMS normalisation of `rows` bf16 rows of n: y = bf16(x * inv * w) with
 * inv = 1/sqrt(mean(x^2) + epsilon); full_layer == 0 rounds x * inv and w to
 * bf16 before the product, as the reference does.  w: f32 [n].
 * Replaces Compute::norm / the norm kernel (elementwise.metal:6-28). */
int oco_norm(const void *x, const float *w, void *y, uint32_t rows, uint32_t n, float epsilon,
             int full_layer, oco_stream stream);

/* Residual add then normalisation: x = bf16(x + y) (x is updated in place,
 * the residual stream), out = norm(x).  Replaces add_norm
 * (elementwise.metal:32-58). */
int oco_add_norm(void *x, const void *y, const float *w, void *out, uint32_t rows, uint32_t n,
                 float epsilon, int full_layer, oco_stream stream);

/* oco_matvec whose bf16 input rows are RMS-normalised on the way in (the
 * norm fused into the matvec's activation staging): the result equals
 * oco_norm followed by oco_matvec with bf16 x, bit for bit, without the
 * normalised row ever reaching memory.  Replaces the norm -> matvec pair of
 * the reference's layer step (elementwise.metal:6-28 feeding
 * vector.metal:66-394). */
int oco_matvec_norm(uint32_t format, const void *w, const void *x, const float *norm_w, float epsilon,
                    int full_layer, void *y, oco_dtype y_dtype, const float *bias,
                    const uint32_t *ids, const oco_matrix *p, oco_stream stream);

/* Several matrices of one format and shape -- `count` (1..4) weights w[i]
 * into outputs y[i] with biases bias[i] (bias may be NULL when
 * p->has_bias == 0) -- over the same input rows x, in one grid: the
 * projections that share an input (ffn_gate and ffn_up) stream back to
 * back with no launch between them, and the input row and its optional
 * RMS norm (norm_w != NULL: x is the bf16 row before normalisation, as in
 * oco_matvec_norm) are staged once per workgroup for all of them.  Each
 * y[i] equals oco_matvec (or oco_matvec_norm) of w[i] bit for bit.  Dense
 * matrices only (p->experts <= 1).  Replaces the concurrent pair of the
 * reference's feed-forward entry (Compute::feed_forward): apply_norm for
 * `gate`, then apply_norm_concurrent for `up`, which skips the barrier
 * between the two dispatches (src/weights/compute/feed_forward.rs:97-104,
 * compute/matrix.rs:127-146, src/gpu/dispatch.rs:235-259). */
#define OCO_MATVEC_GROUP_MAX 4u
int oco_matvec_group(uint32_t format, uint32_t count, const void *const *w, const void *x, oco_dtype x_dtype,
                     const float *norm_w, float epsilon, int full_layer, void *const *y, oco_dtype y_dtype,
                     const float *const *bias, const oco_matrix *p, oco_stream stream);

/* Greedy token selection over n f32 logits: out[0] = index of the largest
 * value (ties: lowest index; -0 == +0), or 0xffffffff if any logit is Inf or
 * NaN or n == 0.  Replaces Compute::argmax / argmax_f32
 * (compute.rs:132-140, argmax.metal:1-47). */
int oco_argmax_f32(const float *logits, uint32_t n, uint32_t *out, oco_stream stream);
/* Workspace form: the partial results of large n live in caller memory of
 * oco_argmax_workspace(n) bytes (0: none needed). */
uint64_t oco_argmax_workspace(uint32_t n);
int oco_argmax_f32_ws(const float *logits, uint32_t n, uint32_t *out, void *workspace,
                      uint64_t workspace_bytes, oco_stream stream);

/* ---- GGUF checkpoints and residency (src/gguf.rs) ------------------------- */

/* An open GGUF v3 file: memory-mapped, metadata structurally validated,
 * the requested keys indexed.  Replaces Gguf::open (gguf.rs:108-150). */
typedef struct oco_gguf oco_gguf;
int oco_gguf_open(const char *path, const char *const *keep, uint32_t nkeep, oco_gguf **out);
int oco_gguf_close(oco_gguf *gguf);

/* Typed metadata reads (gguf.rs:239-348); strings point into the mapping
 * (valid until oco_gguf_close) and are not NUL-terminated. */
int oco_gguf_has(const oco_gguf *gguf, const char *key);
int oco_gguf_text(const oco_gguf *gguf, const char *key, const char **text, size_t *len);
int oco_gguf_number(const oco_gguf *gguf, const char *key, double *out);
int oco_gguf_boolean(const oco_gguf *gguf, const char *key, int *out);
int oco_gguf_unsigned(const oco_gguf *gguf, const char *key, uint64_t *out);
int oco_gguf_array(const oco_gguf *gguf, const char *key, uint32_t *element_kind, uint64_t *count);
int oco_gguf_array_string(const oco_gguf *gguf, const char *key, uint64_t index, const char **text,
                          size_t *len);
int oco_gguf_array_unsigned(const oco_gguf *gguf, const char *key, uint64_t *out, uint64_t capacity);

/* Tensor directory entry: shape (GGUF order, shape[0] is the row width),
 * GGUF type code, absolute byte offset in the file and the extent up to the
 * next tensor.  Replaces Entry (gguf.rs:24-33). */
typedef struct oco_gguf_entry {
    uint64_t shape[4];
    uint32_t rank;
    uint32_t code;
    uint64_t offset;
    uint64_t extent;
} oco_gguf_entry;

/* Build and check the directory (alignment, overlap, bounds): gguf.rs:156-237. */
int oco_gguf_directory(oco_gguf *gguf, uint64_t *count);
int oco_gguf_entry_at(const oco_gguf *gguf, uint64_t index, const char **name, oco_gguf_entry *out);
int oco_gguf_find(const oco_gguf *gguf, const char *name, oco_gguf_entry *out);

/* A tensor checked for execution (format alignment, whole blocks, index
 * range, payload inside its extent): Entry::select / Tensor (gguf.rs:17-87). */
typedef struct oco_gguf_tensor {
    uint32_t format;
    uint32_t rank;
    uint64_t shape[4];
    uint64_t offset;
    uint64_t bytes;
} oco_gguf_tensor;
int oco_gguf_select(const oco_gguf_entry *entry, oco_gguf_tensor *out);

/* Host view of a selected tensor's bytes in the mapping (NULL if outside). */
const void *oco_gguf_data(const oco_gguf *gguf, const oco_gguf_tensor *tensor);

/* Device residency: copy a selected tensor once into device memory `dst`
 * (>= tensor->bytes), blocking until done.  Replaces the zero-copy Metal
 * views over the mapping (buffer.rs:145-297): here the weights live in HBM. */
int oco_gguf_upload(const oco_gguf *gguf, const oco_gguf_tensor *tensor, void *dst, oco_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* OCO_HIP_H */
