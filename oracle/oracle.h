/* CPU oracle for the tensor-ops hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain C11 restatement of the reference's portable semantics, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker. Nothing in the product library (inference_c_amd/) links or calls
 * it. Each function names the reference file:line it follows; functions for
 * ops the reference lacks are closed forms.
 *
 * Build: oracle/Makefile -> oracle/liboracle.so, compiled -O3 -std=c11 with
 * -ffp-contract=off (the reference's gcc -std=c11 default: no a*b+c
 * contraction), so float expressions evaluate exactly as in the reference.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   conversions        exhaustive f16, dense f32 sweep vs oracle/_ref
 *                      (reference build) and the reference's known answers
 *   add/mul/bias       closed form (one IEEE op) + reference known answers
 *   silu/gelu/swiglu   bit-exact vs oracle/_ref (silu) / known answers +
 *                      double-precision evaluation of the same formula
 *   rms/layer norm     bit-exact vs oracle/_ref + known answers
 *   softmax            bit-exact vs oracle/_ref tensor_sdpa_f32 with identity
 *                      K and V + reference known answers + special rows
 *   row/global reduce  closed form vs numpy float64
 *   rope               known answers + norm preservation + position 0 identity
 *   view add/mul       brute-force index math on tiny shapes (numpy)
 *   embedding lookup   known answers + accept/reject and rows bit-exact vs
 *                      oracle/_ref for every index dtype + numpy.take
 *   sdpa               known answers + vs oracle/_ref tensor_sdpa_f32 within
 *                      a few roundings of sum p|v| + special-row closed forms
 *   matmul / linear    bit-exact vs oracle/_ref tensor_matmul_* /
 *                      tensor_linear_* (host path) + known answers
 *   quantize           bit-exact vs oracle/_ref
 *                      tensor_quantize_linear_weight_f16 + known answers
 *   quantized linear   known answer (the reference test's own check) + a
 *                      double-precision dot product of the dequantized
 *                      weights within the f32 rounding bound
 */
#ifndef INFERENCE_ORACLE_H
#define INFERENCE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* conversions: src/common/tensor_f16.c:17-85, src/common/tensor_buffer.c:40-51 */
float orc_f16_to_f32(uint16_t value);
uint16_t orc_f32_to_f16(float value);
float orc_bf16_to_f32(uint16_t value);
uint16_t orc_f32_to_bf16(float value);
void orc_f16_to_f32_array(const uint16_t *x, float *y, size_t n);
void orc_f32_to_f16_array(const float *x, uint16_t *y, size_t n);
void orc_f32_to_bf16_array(const float *x, uint16_t *y, size_t n);

/* synthetic inputs (the generator behind tensor_fill_uniform/normal) */
uint64_t orc_rng_bits(uint64_t seed, uint64_t stream, uint64_t index);
void orc_fill_uniform_f32(float *y, size_t n, uint64_t seed, uint64_t stream,
                          uint64_t first, float low, float high);
void orc_fill_uniform_f16(uint16_t *y, size_t n, uint64_t seed, uint64_t stream,
                          uint64_t first, float low, float high);
void orc_fill_normal_f32(float *y, size_t n, uint64_t seed, uint64_t stream,
                         uint64_t first, float mean, float std_dev);
void orc_fill_normal_f16(uint16_t *y, size_t n, uint64_t seed, uint64_t stream,
                         uint64_t first, float mean, float std_dev);

/* elementwise */
void orc_add_f32(const float *a, const float *b, float *y, size_t n);
void orc_mul_f32(const float *a, const float *b, float *y, size_t n);
void orc_add_f16(const uint16_t *a, const uint16_t *b, uint16_t *y, size_t n);
void orc_mul_f16(const uint16_t *a, const uint16_t *b, uint16_t *y, size_t n);
void orc_silu_f32(const float *x, float *y, size_t n);
void orc_silu_f16(const uint16_t *x, uint16_t *y, size_t n);
float orc_gelu_scalar(float x);
double orc_gelu_scalar_f64(double x);
void orc_gelu_f32(const float *x, float *y, size_t n);
void orc_gelu_f16(const uint16_t *x, uint16_t *y, size_t n);
void orc_gelu_f64(const double *x, double *y, size_t n);
void orc_gelu_multiply_f16(const uint16_t *x, const uint16_t *gate, uint16_t *y,
                           size_t n);
void orc_relu_f16(const uint16_t *x, uint16_t *y, size_t n);
void orc_silu_multiply_f32(const float *gate, const float *up, float *y, size_t n);
void orc_silu_multiply_f16(const uint16_t *gate, const uint16_t *up, uint16_t *y,
                           size_t n);
void orc_bias_add_f32(const float *x, const float *bias, float *y, size_t rows,
                      size_t width, int gelu);
void orc_bias_add_f16(const uint16_t *x, const uint16_t *bias, uint16_t *y,
                      size_t rows, size_t width, int gelu);

/* row reductions */
void orc_rms_norm_f32(const float *x, const float *w, float *y, size_t rows,
                      size_t width, float eps);
void orc_rms_norm_f16(const uint16_t *x, const uint16_t *w, uint16_t *y,
                      size_t rows, size_t width, float eps);
void orc_layer_norm_f32(const float *x, const float *scale, const float *bias,
                        float *y, size_t rows, size_t width, float eps);
void orc_layer_norm_f16(const uint16_t *x, const uint16_t *scale,
                        const uint16_t *bias, uint16_t *y, size_t rows,
                        size_t width, float eps);
void orc_residual_rms_norm_f16(const uint16_t *x, const uint16_t *r,
                               const uint16_t *w, uint16_t *sum, uint16_t *y,
                               size_t rows, size_t width, float eps);
void orc_softmax_f32(const float *x, float *y, size_t rows, size_t width,
                     size_t q_len);
void orc_softmax_f16(const uint16_t *x, uint16_t *y, size_t rows, size_t width,
                     size_t q_len);
void orc_row_sum_f32(const float *x, double *sum, double *abs_sum, size_t rows,
                     size_t width);
void orc_row_sum_f16(const uint16_t *x, double *sum, double *abs_sum,
                     size_t rows, size_t width);
void orc_row_max_f32(const float *x, float *y, size_t rows, size_t width);
void orc_row_max_f16(const uint16_t *x, float *y, size_t rows, size_t width);

/* whole-tensor reductions */
void orc_sum_max_f32(const float *x, size_t n, double *sum, double *abs_sum,
                     float *max);
uint32_t orc_argmax_f32(const float *x, size_t n);
uint32_t orc_argmax_f16(const uint16_t *x, size_t n);

/* rope (in place) */
void orc_rope_f32(float *q, float *k, size_t seq, size_t qh, size_t kh,
                  size_t dim, double theta, size_t offset);
void orc_rope_f16(uint16_t *q, uint16_t *k, size_t seq, size_t qh, size_t kh,
                  size_t dim, double theta, size_t offset);

/* strided view (x + addend) * multiplier, contiguous output; addend and
   multiplier are broadcast (shape dims 1 or equal), NULL = skipped */
void orc_view_add_mul_f16(const uint16_t *x, size_t rank, const uint64_t *shape,
                          const int64_t *strides, uint64_t offset,
                          const uint16_t *addend, const uint64_t *addend_shape,
                          const uint16_t *mult, const uint64_t *mult_shape,
                          uint16_t *y);
void orc_view_add_mul_f32(const float *x, size_t rank, const uint64_t *shape,
                          const int64_t *strides, uint64_t offset,
                          const float *addend, const uint64_t *addend_shape,
                          const float *mult, const uint64_t *mult_shape,
                          float *y);

/* embedding lookup: returns 1, or 0 (output untouched) when an index is
   unreadable for its dtype (TensorDType numbering), negative or outside the
   table; the compute-table variant zero-fills rows of out-of-range ids */
int orc_embedding_lookup(const void *table, size_t table_rows, size_t row_bytes,
                         const void *indices, int index_dtype, size_t count, void *out);
void orc_embedding_gather_u32(const void *table, size_t table_rows, size_t row_bytes,
                              const uint32_t *ids, size_t count, void *out);

/* scaled dot-product attention with the accelerator backend's semantics
   (q [B,Hq,Lq,D], k [B,Hkv,Lkv,D], v [B,Hkv,Lkv,Dv], mask [Lq,Lkv] or NULL,
   out [B,Hq,Lq,Dv]); scores = caller scratch of Lkv floats */
void orc_sdpa_f32(const float *q, const float *k, const float *v, const float *mask, float *out,
                  size_t batch, size_t qh, size_t kvh, size_t ql, size_t kl, size_t dim,
                  size_t vdim, float scale, int causal, float *scores);
void orc_sdpa_f16(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *mask,
                  uint16_t *out, size_t batch, size_t qh, size_t kvh, size_t ql, size_t kl,
                  size_t dim, size_t vdim, float scale, int causal, float *scores);
void orc_sdpa_abs_weight(const void *q, const void *k, const void *v, const void *mask,
                         double *out, int f16, size_t batch, size_t qh, size_t kvh, size_t ql,
                         size_t kl, size_t dim, size_t vdim, float scale, int causal,
                         float *scores);

/* matmul y[rows,cols] = a[rows,inner] b[inner,cols]; linear y[rows,out] =
   x[rows,in] w[out,in]^T (+ bias[out]) -- the reference's host loops */
void orc_matmul_f32(const float *a, const float *b, float *y, size_t rows, size_t inner,
                    size_t cols);
void orc_matmul_f16(const uint16_t *a, const uint16_t *b, uint16_t *y, size_t rows,
                    size_t inner, size_t cols);
void orc_linear_f32(const float *x, const float *w, const float *bias, float *y, size_t rows,
                    size_t in, size_t out);
void orc_linear_f16(const uint16_t *x, const uint16_t *w, const uint16_t *bias, uint16_t *y,
                    size_t rows, size_t in, size_t out);

/* Q8_0 (format 1, 34-byte blocks) / Q4_0 (format 2, 18-byte blocks) */
uint16_t orc_quant_scale_to_f16(float value);
int orc_quantize_f16(const uint16_t *weight, size_t out, size_t in, int format, uint8_t *dst);
void orc_linear_quant_f16(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                          size_t in, size_t out, int q8);
void orc_linear_quant_abs_weight(const uint16_t *x, const uint8_t *w, double *y, size_t rows,
                                 size_t in, size_t out, int q8);

#ifdef __cplusplus
}
#endif

#endif
