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

// ---- token embedding rows ----------------------------------------------------
// embed (weights.metal:90-109): out[r] = bf16(row ids[r] of the GGUF tensor
// [vocabulary rows of k]), through the same scalar decoder as oco_dequant;
// native BF16 rows are copied as bits.  Ids at or past the vocabulary take
// row (id - vocabulary) of the caller's bf16 feature rows; ids past those
// too get a NaN row (the reference does not check them).  Grid: (column
// chunks of 2048, rows); each thread writes 8 consecutive values.
namespace oco {

template <int FMT>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t *w, const uint32_t *ids, uint16_t *out,
                                                    const uint16_t *features, uint32_t k, uint32_t vocab,
                                                    uint32_t feature_rows, uint64_t row_bytes) {
    constexpr uint32_t BE = FMT == OCO_F32 || FMT == OCO_F16 || FMT == OCO_BF16 ? 1
                            : (FMT == OCO_Q4_K || FMT == OCO_Q5_K || FMT == OCO_Q6_K) ? 256 : 32;
    constexpr uint32_t BB = FMT == OCO_F32 ? 4 : (FMT == OCO_F16 || FMT == OCO_BF16) ? 2
                            : FMT == OCO_Q4_0 ? 18 : FMT == OCO_Q4_1 ? 20 : FMT == OCO_Q8_0 ? 34
                            : FMT == OCO_Q4_K ? 144 : FMT == OCO_Q5_K ? 176 : FMT == OCO_Q6_K ? 210 : 17;
    const uint32_t r = blockIdx.y;
    const uint32_t id = ids[r];
    uint16_t *o = out + (uint64_t)r * k;
    const uint32_t c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (c0 >= k) return;
    const uint32_t cn = min(8u, k - c0);
    if (id >= vocab) {
        const bool have = features && id - vocab < feature_rows;
        const uint16_t *f = have ? features + (uint64_t)(id - vocab) * k : nullptr;
        for (uint32_t j = 0; j < cn; j++) o[c0 + j] = have ? f[c0 + j] : (uint16_t)0x7fc0u;
        return;
    }
    const uint8_t *row = w + (uint64_t)id * row_bytes;
    for (uint32_t j = 0; j < cn; j++) {
        const uint32_t c = c0 + j;
        const uint8_t *blk = row + (uint64_t)(c / BE) * BB;
        if constexpr (FMT == OCO_BF16)
            o[c] = (uint16_t)ld_u16(blk);
        else
            o[c] = f32_to_bf16_bits(decode_scalar(FMT, blk, c % BE));
    }
}

}  // namespace oco

extern "C" int oco_embed(uint32_t format, const void *w, uint32_t k, uint32_t vocabulary, const uint32_t *ids,
                         uint32_t rows, const uint16_t *features, uint32_t feature_rows, uint16_t *out,
                         oco_stream stream) {
    uint32_t e, b;
    OCO_TRY(oco_block_layout(format, &e, &b));
    if (k == 0 || k % e) return fail(OCO_ERR_INVALID, "oco_embed: width %u is not whole blocks of %u", k, e);
    if (!rows) return OCO_OK;
    if (rows > 65535) return fail(OCO_ERR_INVALID, "oco_embed: %u rows exceed 65535", rows);
    if (!w || !ids || !out) return fail(OCO_ERR_INVALID, "oco_embed: null pointer");
    if (feature_rows && !features) return fail(OCO_ERR_INVALID, "oco_embed: feature_rows without features");
    const uint64_t row_bytes = oco_row_bytes(format, k);
    const dim3 grid((k + 2047) / 2048, rows);
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *wp = (const uint8_t *)w;
    switch (format) {
#define CASE(F)                                                                                                 \
    case F:                                                                                                     \
        hipLaunchKernelGGL(embed_kernel<F>, grid, dim3(256), 0, s, wp, ids, out, features, k, vocabulary,     \
                           feature_rows, row_bytes);                                                            \
        break;
        CASE(OCO_F32) CASE(OCO_F16) CASE(OCO_BF16) CASE(OCO_Q4_0) CASE(OCO_Q4_1) CASE(OCO_Q8_0)
        CASE(OCO_Q4_K) CASE(OCO_Q5_K) CASE(OCO_Q6_K) CASE(OCO_MXFP4)
#undef CASE
    default: return fail(OCO_ERR_UNSUPPORTED, "oco_embed: format %u", format);
    }
    return launch_check("oco_embed");
}
