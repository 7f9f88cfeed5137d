// Host-side launch interface of the gfx950 kernels (the library's internal
// HIP table). Every launcher validates nothing beyond what its kernel needs
// to stay in bounds; the public entry points validate shapes and dtypes first.
// All launchers enqueue on `stream` and return the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "safetensors.h"

namespace icsdk {
namespace k {

enum class Unary { Silu, Gelu, Relu, Copy };
enum class Binary { Add, Mul, SiluMul, GeluMul };

// y[i] = op(x[i]) / op(a[i], b[i]); T is float or f16 (uint16_t storage).
hipError_t unary_f32(Unary op, const float *x, float *y, size_t n, hipStream_t s);
hipError_t unary_f16(Unary op, const uint16_t *x, uint16_t *y, size_t n, hipStream_t s);
hipError_t binary_f32(Binary op, const float *a, const float *b, float *y, size_t n,
                      hipStream_t s);
hipError_t binary_f16(Binary op, const uint16_t *a, const uint16_t *b, uint16_t *y,
                      size_t n, hipStream_t s);

// y[r, c] = x[r, c] + bias[c] (optionally GELU'd).
hipError_t bias_add_f32(const float *x, const float *bias, float *y, size_t rows,
                        size_t width, bool gelu, hipStream_t s);
hipError_t bias_add_f16(const uint16_t *x, const uint16_t *bias, uint16_t *y,
                        size_t rows, size_t width, bool gelu, hipStream_t s);

// Row normalisation over the last dimension. For rms_norm_f16 a non-null
// `residual` makes it the fused residual+RMSNorm: sum = f16(x + residual) is
// written to `sum_out` and normalised.
hipError_t rms_norm_f32(const float *x, const float *w, float *y, size_t rows,
                        size_t width, float eps, hipStream_t s);
hipError_t rms_norm_f16(const uint16_t *x, const uint16_t *residual, uint16_t *sum_out,
                        const uint16_t *w, uint16_t *y, size_t rows, size_t width,
                        float eps, hipStream_t s);
hipError_t layer_norm_f32(const float *x, const float *scale, const float *bias,
                          float *y, size_t rows, size_t width, float eps,
                          hipStream_t s);
hipError_t layer_norm_f16(const uint16_t *x, const uint16_t *scale,
                          const uint16_t *bias, uint16_t *y, size_t rows,
                          size_t width, float eps, hipStream_t s);

// Row softmax; q_len == 0: no mask, else causal with query = row % q_len.
hipError_t softmax_f32(const float *x, float *y, size_t rows, size_t width,
                       size_t q_len, hipStream_t s);
hipError_t softmax_f16(const uint16_t *x, uint16_t *y, size_t rows, size_t width,
                       size_t q_len, hipStream_t s);

// Row sum / max into f32 outputs.
hipError_t row_sum_f32(const float *x, float *y, size_t rows, size_t width, hipStream_t s);
hipError_t row_sum_f16(const uint16_t *x, float *y, size_t rows, size_t width,
                       hipStream_t s);
hipError_t row_max_f32(const float *x, float *y, size_t rows, size_t width, hipStream_t s);
hipError_t row_max_f16(const uint16_t *x, float *y, size_t rows, size_t width,
                       hipStream_t s);

// Two-pass grid reductions. `partials` is device scratch of at least
// grid_reduce_scratch_bytes() bytes.
size_t grid_reduce_scratch_bytes();
hipError_t sum_max_f32(const float *x, size_t n, double *sum_out, float *max_out,
                       void *partials, hipStream_t s);
// Bytes of partials sum_max_f32 writes for n elements (at most
// grid_reduce_scratch_bytes()).
size_t sum_max_partials_bytes(size_t n);
// The allocation-free variant's partials: a file-scope device array of
// no_alloc_scratch_bytes() bytes in k_global.hip. no_alloc_scratch() returns
// its address on the current device (looked up once per device);
// sum_max_f32_no_alloc() runs sum_max_f32 with it and refuses a launch whose
// partials would not fit in scratch_bytes.
size_t no_alloc_scratch_bytes();
// Linear of at most kGemvMaxRows input rows as a GEMV over the weights
// (k_linear.hip): hipErrorNotSupported when the shape or alignment does not
// qualify (the caller then uses the GEMM library).
constexpr size_t kGemvMaxRows = 4;
hipError_t linear_gemv(bool f32, const void *x, const void *w, const void *bias, void *y,
                       size_t rows, size_t in, size_t out, hipStream_t s);
hipError_t no_alloc_scratch(void **ptr);
hipError_t sum_max_f32_no_alloc(const float *x, size_t n, double *sum_out, float *max_out,
                                void *scratch_ptr, size_t scratch_bytes, hipStream_t s);
hipError_t argmax_f32(const float *x, size_t n, uint32_t *index_out, void *partials,
                      hipStream_t s);
hipError_t argmax_f16(const uint16_t *x, size_t n, uint32_t *index_out, void *partials,
                      hipStream_t s);

// In-place split-half RoPE on q [seq, qh, dim] and k [seq, kh, dim].
// Shapes whose half row is a multiple of the 16-byte vector (<= 128 pairs,
// aligned tensors) need no scratch; others need `table`, device scratch of
// rope_table_bytes(...) bytes (the per-call cos/sin table). 0 = none needed.
size_t rope_table_bytes(size_t seq, size_t qh, size_t kh, size_t dim, size_t elem,
                        const void *q, const void *k);
hipError_t rope_f32(float *q, float *k, size_t seq, size_t qh, size_t kh, size_t dim,
                    double theta, size_t offset, void *table, hipStream_t s);
hipError_t rope_f16(uint16_t *q, uint16_t *k, size_t seq, size_t qh, size_t kh,
                    size_t dim, double theta, size_t offset, void *table, hipStream_t s);

// Strided view (x + addend) * mult -> contiguous y. Shapes/strides in
// elements; addend/mult shapes broadcast (1 or equal), either may be null.
struct ViewArgs {
    int rank;
    uint64_t shape[8];
    int64_t strides[8];
    uint64_t offset;
    uint64_t addend_shape[8];
    uint64_t mult_shape[8];
};
hipError_t view_add_mul_f32(const float *x, const ViewArgs &v, const float *addend,
                            const float *mult, float *y, hipStream_t s);
hipError_t view_add_mul_f16(const uint16_t *x, const ViewArgs &v, const uint16_t *addend,
                            const uint16_t *mult, uint16_t *y, hipStream_t s);

// Embedding lookup: out[i, :] = table[ids[i], :] (rows of row_bytes bytes,
// elements of elem_bytes = 2 or 4). ids are I16/U16/I32/U32/I64/U64; an id
// that is negative or >= table_rows gives a zero row. embedding_check writes
// 1 to `flag` (pinned host memory) and to the device word `skip` when any id
// is such, else 0 (one block); embedding_gather writes nothing when `skip`
// (may be null) holds a non-zero word.
bool embedding_index_type(TensorDType dtype);
hipError_t embedding_check(TensorDType index_dtype, const void *ids, size_t count,
                           uint64_t table_rows, uint32_t *flag, uint32_t *skip, hipStream_t s);
hipError_t embedding_gather(TensorDType index_dtype, const void *table, uint64_t table_rows,
                            size_t row_bytes, size_t elem_bytes, const void *ids, size_t count,
                            void *out, const uint32_t *skip, hipStream_t s);

// Scaled dot-product attention with the accelerator semantics of the
// reference (q [B,Hq,Lq,D], k [B,Hkv,Lkv,D], v [B,Hkv,Lkv,Dv], mask [Lq,Lkv]
// or null, out [B,Hq,Lq,Dv]). D and Dv up to 512.
struct SdpaShape {
    size_t batch, q_heads, kv_heads, q_len, kv_len, head_dim, value_dim;
};
// `workspace` (may be null) lets the flash path split the key range of long
// query blocks over several blocks: sdpa_workspace_bytes(shape, f32, causal)
// bytes, 0 when the shape would not split.
size_t sdpa_workspace_bytes(const SdpaShape &shape, bool f32, bool causal);
hipError_t sdpa_f32(const float *q, const float *k, const float *v, const float *mask,
                    float *out, const SdpaShape &shape, float scale, bool causal,
                    void *workspace, size_t workspace_bytes, hipStream_t s);
hipError_t sdpa_f16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                    const uint16_t *mask, uint16_t *out, const SdpaShape &shape, float scale,
                    bool causal, void *workspace, size_t workspace_bytes, hipStream_t s);

// Quantized linear y[rows, out] = x[rows, in] * dequant(w)^T with w packed
// [out, in/32, 34] (Q8_0) or [out, in/32, 18] (Q4_0); in % 32 == 0.
hipError_t linear_q8_0_f16(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                           size_t in, size_t out, hipStream_t s);
hipError_t linear_q4_0_f16(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                           size_t in, size_t out, hipStream_t s);
// Packs total_blocks 32-weight f16 blocks (16-byte aligned) into Q8_0 / Q4_0
// blocks; a non-finite weight sets *bad to 1.
hipError_t quantize_f16(bool q8, const uint16_t *weight, uint8_t *packed, uint32_t *bad,
                        size_t total_blocks, hipStream_t s);

// Synthetic inputs (counter-based splitmix64).
hipError_t fill_uniform(TensorDType dtype, void *y, size_t n, uint64_t seed,
                        uint64_t stream, float low, float high, hipStream_t s);
hipError_t fill_normal(TensorDType dtype, void *y, size_t n, uint64_t seed,
                       uint64_t stream, float mean, float std_dev, hipStream_t s);

// dtype conversion among F32 / F16 / BF16 with the reference's bit rules.
hipError_t convert(TensorDType from, const void *x, TensorDType to, void *y, size_t n,
                   hipStream_t s);

}  // namespace k
}  // namespace icsdk
