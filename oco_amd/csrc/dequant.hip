// Dequantization of GGUF tensors to f32: the `weight()` decoder of
// shaders/matrix/weights.metal:48-85 (and `embed`'s decode, :93-109),
// bit-exact with the scalar definition.  One thread per coefficient; a
// grid-stride loop keeps the grid bounded for any tensor size.
#include "formats.h"

namespace oco {

template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *w, uint64_t count, float *out) {
    constexpr uint32_t BE = FMT == OCO_F32 || FMT == OCO_F16 || FMT == OCO_BF16 ? 1
                            : (FMT == OCO_Q4_K || FMT == OCO_Q5_K || FMT == OCO_Q6_K) ? 256 : 32;
    constexpr uint32_t BB = FMT == OCO_F32 ? 4 : (FMT == OCO_F16 || FMT == OCO_BF16) ? 2
                            : FMT == OCO_Q4_0 ? 18 : FMT == OCO_Q4_1 ? 20 : FMT == OCO_Q8_0 ? 34
                            : FMT == OCO_Q4_K ? 144 : FMT == OCO_Q5_K ? 176 : FMT == OCO_Q6_K ? 210 : 17;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (; i < count; i += stride) out[i] = decode_scalar(FMT, w + (i / BE) * BB, (uint32_t)(i % BE));
}

}  // namespace oco

using namespace oco;

extern "C" int oco_dequant(uint32_t format, const void *w, uint64_t count, float *out,
                           oco_stream stream) {
    uint32_t e, b;
    OCO_TRY(oco_block_layout(format, &e, &b));
    if (count % e) return fail(OCO_ERR_INVALID, "oco_dequant: count %llu not a multiple of %u",
                               (unsigned long long)count, e);
    if (!count) return OCO_OK;
    if (!w || !out) return fail(OCO_ERR_INVALID, "oco_dequant: null pointer");
    uint64_t blocks = (count + 255) / 256;
    unsigned grid = (unsigned)(blocks < 262144 ? blocks : 262144);
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *wp = (const uint8_t *)w;
    switch (format) {
#define CASE(F) \
    case F: hipLaunchKernelGGL(dequant_kernel<F>, dim3(grid), dim3(256), 0, s, wp, count, out); break;
        CASE(OCO_F32) CASE(OCO_F16) CASE(OCO_BF16) CASE(OCO_Q4_0) CASE(OCO_Q4_1) CASE(OCO_Q8_0)
        CASE(OCO_Q4_K) CASE(OCO_Q5_K) CASE(OCO_Q6_K) CASE(OCO_MXFP4)
#undef CASE
    default: return fail(OCO_ERR_UNSUPPORTED, "oco_dequant: format %u", format);
    }
    return launch_check("oco_dequant");
}
