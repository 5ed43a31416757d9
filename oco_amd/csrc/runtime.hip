// Runtime seam: status strings, device selection, device memory, streams and
// events.  Replaces oco's Metal device/buffer/queue layer (src/gpu.rs,
// src/gpu/buffer.rs, src/gpu/dispatch.rs, src/gpu/profile.rs) with HIP.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace oco {

static thread_local char g_error[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return code;
}

int hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return OCO_OK;
    return fail(e == hipErrorOutOfMemory ? OCO_ERR_MEMORY : OCO_ERR_HIP, "%s: %s", what,
                hipGetErrorString(e));
}

int launch_check(const char *what) { return hip_check(hipGetLastError(), what); }

// Override table of oco_plan_override: a count of 0 means "not set".
static int32_t g_knob_vals[OCO_KNOB_COUNT][4];
static uint32_t g_knob_count[OCO_KNOB_COUNT];

int plan_override(uint32_t knob, int32_t *vals) {
    if (knob >= OCO_KNOB_COUNT) return 0;
    const uint32_t n = __atomic_load_n(&g_knob_count[knob], __ATOMIC_ACQUIRE);
    for (uint32_t i = 0; i < n; i++) vals[i] = g_knob_vals[knob][i];
    return (int)n;
}

// XOR of all 32-bit words: each thread keeps four 16-byte nontemporal loads
// in flight per round (the shape of a plain HBM stream); workgroup b stores
// its XOR to out[b] (an atomic per workgroup into one word costs
// microseconds of contention), workgroup 0 zeroes the slots no workgroup
// owns.  XOR is order-independent: exact.
// The round count is precomputed on the host, so the loop ends after
// `rounds` rounds whatever the size; offsets stay below 2^32 because the
// host caps bytes at XOR32_MAX_BYTES.
__global__ __launch_bounds__(256) void xor32_kernel(const uint8_t *src, uint32_t bytes, uint32_t rounds, uint32_t *out) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src), 0, bytes, 0x00020000);
    constexpr int U = 4;
    uint32_t acc = 0;
    for (uint32_t round = blockIdx.x; round < rounds; round += gridDim.x) {
        const uint32_t base = round * 256u * U * 16u;
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, base + (u * 256 + threadIdx.x) * 16, 0, 2);
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    __shared__ uint32_t part[4];
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
    if (blockIdx.x == 0)
        for (uint32_t i = gridDim.x + threadIdx.x; i < OCO_XOR32_SLOTS; i += 256) out[i] = 0;
}

// Size limit and launch geometry of xor32_kernel: 16 KiB per workgroup
// round, one workgroup per round up to OCO_XOR32_SLOTS.  The last round
// starts below XOR32_MAX_BYTES and reads at most 16 KiB past its start, so
// every buffer offset fits 32 bits.
constexpr uint64_t XOR32_MAX_BYTES = OCO_XOR32_MAX_BYTES;
bool xor32_geometry(uint64_t words, uint64_t *rounds, uint64_t *grid) {
    if (words > XOR32_MAX_BYTES / 4) return false;
    *rounds = (words * 4 + 16383u) / 16384u;
    *grid = *rounds < OCO_XOR32_SLOTS ? *rounds : OCO_XOR32_SLOTS;
    return true;
}

__global__ void fill32_kernel(uint32_t *dst, uint32_t pattern, size_t words) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < words; i += stride) dst[i] = pattern;
}

}  // namespace oco

using namespace oco;

extern "C" {

const char *oco_last_error(void) { return g_error; }

int oco_plan_override(uint32_t knob, const int32_t *values, uint32_t count) {
    if (knob >= OCO_KNOB_COUNT) return fail(OCO_ERR_INVALID, "oco_plan_override: unknown knob %u", knob);
    if (count > 4 || (count && !values)) return fail(OCO_ERR_INVALID, "oco_plan_override: 0..4 values");
    __atomic_store_n(&g_knob_count[knob], 0u, __ATOMIC_RELEASE);
    for (uint32_t i = 0; i < count; i++) g_knob_vals[knob][i] = values[i];
    __atomic_store_n(&g_knob_count[knob], count, __ATOMIC_RELEASE);
    return OCO_OK;
}

int oco_block_layout(uint32_t format, uint32_t *elements, uint32_t *bytes) {
    uint32_t e, b;
    switch (format) {
    case OCO_F32: e = 1; b = 4; break;
    case OCO_F16:
    case OCO_BF16: e = 1; b = 2; break;
    case OCO_Q4_0: e = 32; b = 18; break;
    case OCO_Q4_1: e = 32; b = 20; break;
    case OCO_Q8_0: e = 32; b = 34; break;
    case OCO_Q4_K: e = 256; b = 144; break;
    case OCO_Q5_K: e = 256; b = 176; break;
    case OCO_Q6_K: e = 256; b = 210; break;
    case OCO_MXFP4: e = 32; b = 17; break;
    default: return fail(OCO_ERR_UNSUPPORTED, "unknown GGUF format %u", format);
    }
    if (elements) *elements = e;
    if (bytes) *bytes = b;
    return OCO_OK;
}

uint64_t oco_row_bytes(uint32_t format, uint32_t k) {
    uint32_t e, b;
    if (oco_block_layout(format, &e, &b) != OCO_OK || k % e) return 0;
    return (uint64_t)(k / e) * b;
}

int oco_device_open(int ordinal, int *compute_units) {
    int count = 0;
    OCO_TRY(hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount"));
    if (ordinal < 0 || ordinal >= count)
        return fail(OCO_ERR_INVALID, "device %d out of range (%d devices)", ordinal, count);
    OCO_TRY(hip_check(hipSetDevice(ordinal), "hipSetDevice"));
    // The static experts scratch is resolved here when the ordinal has a
    // slot; devices beyond the table still open (the static entry point
    // then reports them), and a failure here is retried on its first call.
    if (ordinal < 64) (void)experts_scratch_init(ordinal);
    if (compute_units) {
        int cu = 0;
        OCO_TRY(hip_check(hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, ordinal),
                          "hipDeviceGetAttribute"));
        *compute_units = cu;
    }
    return OCO_OK;
}

int oco_buffer_alloc(size_t bytes, void **out) {
    if (!out) return fail(OCO_ERR_INVALID, "oco_buffer_alloc: null out");
    *out = nullptr;
    return hip_check(hipMalloc(out, bytes ? bytes : 1), "hipMalloc");
}

int oco_buffer_free(void *ptr) { return hip_check(hipFree(ptr), "hipFree"); }

int oco_buffer_upload(void *dst, const void *src, size_t bytes) {
    return hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

int oco_buffer_download(void *dst, const void *src, size_t bytes) {
    return hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

int oco_buffer_copy(void *dst, const void *src, size_t bytes, oco_stream stream) {
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream),
                     "hipMemcpyAsync D2D");
}

int oco_buffer_fill32(void *dst, uint32_t pattern, size_t words, oco_stream stream) {
    if (!words) return OCO_OK;
    if (!dst) return fail(OCO_ERR_INVALID, "oco_buffer_fill32: null destination");
    size_t blocks = (words + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill32_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (uint32_t *)dst, pattern, words);
    return launch_check("fill32");
}

int oco_buffer_xor32(const void *src, size_t words, uint32_t *out, oco_stream stream) {
    if (!words) return OCO_OK;
    if (!src || !out) return fail(OCO_ERR_INVALID, "oco_buffer_xor32: null pointer");
    if (((uintptr_t)src & 15u) || words % 4) return fail(OCO_ERR_INVALID, "oco_buffer_xor32: needs 16-byte aligned whole chunks");
    uint64_t rounds64 = 0, grid64 = 0;
    if (!xor32_geometry(words, &rounds64, &grid64))
        return fail(OCO_ERR_INVALID, "oco_buffer_xor32: %zu words is over the %llu-byte limit", words,
                    (unsigned long long)XOR32_MAX_BYTES);
    hipLaunchKernelGGL(xor32_kernel, dim3((uint32_t)grid64), dim3(256), 0, (hipStream_t)stream, (const uint8_t *)src,
                       (uint32_t)(words * 4), (uint32_t)rounds64, out);
    return launch_check("xor32");
}

int oco_buffer_xor32_geometry(uint64_t words, uint64_t *rounds, uint64_t *workgroups) {
    if (!rounds || !workgroups) return fail(OCO_ERR_INVALID, "oco_buffer_xor32_geometry: null pointer");
    if (!xor32_geometry(words, rounds, workgroups))
        return fail(OCO_ERR_INVALID, "oco_buffer_xor32_geometry: over the size limit");
    return OCO_OK;
}

int oco_stream_create(oco_stream *out) {
    hipStream_t s;
    OCO_TRY(hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate"));
    *out = (oco_stream)s;
    return OCO_OK;
}

int oco_stream_sync(oco_stream stream) {
    return hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int oco_stream_destroy(oco_stream stream) {
    return hip_check(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
}

int oco_event_create(oco_event *out) {
    hipEvent_t e;
    OCO_TRY(hip_check(hipEventCreate(&e), "hipEventCreate"));
    *out = (oco_event)e;
    return OCO_OK;
}

int oco_event_record(oco_event event, oco_stream stream) {
    return hip_check(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
}

int oco_event_elapsed_ms(oco_event start, oco_event stop, float *ms) {
    OCO_TRY(hip_check(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize"));
    return hip_check(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop),
                     "hipEventElapsedTime");
}

int oco_event_destroy(oco_event event) {
    return hip_check(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
}

int oco_graph_begin(oco_stream stream) {
    if (!stream) return fail(OCO_ERR_INVALID, "oco_graph_begin: capture needs a created stream");
    return hip_check(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal),
                     "hipStreamBeginCapture");
}

int oco_graph_end(oco_stream stream, oco_graph *out) {
    hipGraph_t g;
    OCO_TRY(hip_check(hipStreamEndCapture((hipStream_t)stream, &g), "hipStreamEndCapture"));
    hipGraphExec_t exec;
    int rc = hip_check(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    hipGraphDestroy(g);
    if (rc != OCO_OK) return rc;
    *out = (oco_graph)exec;
    return OCO_OK;
}

int oco_graph_launch(oco_graph graph, oco_stream stream) {
    return hip_check(hipGraphLaunch((hipGraphExec_t)graph, (hipStream_t)stream), "hipGraphLaunch");
}

int oco_graph_destroy(oco_graph graph) {
    return hip_check(hipGraphExecDestroy((hipGraphExec_t)graph), "hipGraphExecDestroy");
}

}  // extern "C"
