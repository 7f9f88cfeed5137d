/* Public tensor operations.
 *
 * Same 13 declarations as include/tensor_ops.h:8-49 of the reference.
 * Each returns 1 on success and 0 on failure, writing a message into
 * (error, error_capacity) when error is not NULL; outputs are preallocated by
 * the caller, and every operand is validated before any work is queued.
 *
 * In this library every elementwise and normalisation op runs on the GPU:
 *   - operands in device storage: the kernel is enqueued on the SDK stream and
 *     the call returns at once (synchronize before host-side reads);
 *   - operands in host storage: they are staged through device memory and the
 *     call returns when the host output has been written.
 * All operands of one call must share one storage kind.
 *
 * matmul and linear also run on the GPU (hipBLASLt, f32 or f16 with f32
 * accumulation; the linear's bias is added inside the GEMM before its one
 * rounding). Device-storage linears go through the compute table returned by
 * tensor_compute_preferred_backend(), as the reference does, so a
 * TENSOR_BACKEND naming another backend makes them fail. The embedding
 * lookups check every index before any row is written (host indices on the
 * host; device indices by a one-block kernel whose verdict the call waits
 * for), then gather the rows on the GPU.
 *
 * Without a HIP device every compute entry point fails with a message
 * beginning "HIP device unavailable"; there is no CPU arithmetic path.
 */
#ifndef TENSOR_OPS_H
#define TENSOR_OPS_H

#include "tensor_buffer.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/tensor_ops.h:8-13 (src/common/tensor_ops.c:163-222) */
int tensor_matmul_f32(const TensorBuffer *left, const TensorBuffer *right,
                      TensorBuffer *output, char *error,
                      size_t error_capacity);
int tensor_matmul_f16(const TensorBuffer *left, const TensorBuffer *right,
                      TensorBuffer *output, char *error,
                      size_t error_capacity);
/* reference :14-19 (tensor_ops.c:224-398) */
int tensor_linear_f32(const TensorBuffer *input, const TensorBuffer *weight,
                      const TensorBuffer *bias, TensorBuffer *output,
                      char *error, size_t error_capacity);
int tensor_linear_f16(const TensorBuffer *input, const TensorBuffer *weight,
                      const TensorBuffer *bias, TensorBuffer *output,
                      char *error, size_t error_capacity);
/* reference :20-27 (tensor_ops.c:86-161) */
int tensor_embedding_lookup_f32(const TensorBuffer *table,
                                const TensorBuffer *indices,
                                TensorBuffer *output, char *error,
                                size_t error_capacity);
int tensor_embedding_lookup_f16(const TensorBuffer *table,
                                const TensorBuffer *indices,
                                TensorBuffer *output, char *error,
                                size_t error_capacity);
/* reference :28-33 (tensor_ops.c:400-459): y = x * (1/sqrtf(mean(x^2)+eps)) * w
   over the last dimension; eps must be finite and >= 0. */
int tensor_rms_norm_f32(const TensorBuffer *input, const TensorBuffer *weight,
                        float epsilon, TensorBuffer *output, char *error,
                        size_t error_capacity);
int tensor_rms_norm_f16(const TensorBuffer *input, const TensorBuffer *weight,
                        float epsilon, TensorBuffer *output, char *error,
                        size_t error_capacity);
/* reference :34-41 (tensor_ops.c:461-543); scale and bias may be NULL. */
int tensor_layer_norm_f32(const TensorBuffer *input, const TensorBuffer *scale,
                          const TensorBuffer *bias, float epsilon,
                          TensorBuffer *output, char *error,
                          size_t error_capacity);
int tensor_layer_norm_f16(const TensorBuffer *input, const TensorBuffer *scale,
                          const TensorBuffer *bias, float epsilon,
                          TensorBuffer *output, char *error,
                          size_t error_capacity);
/* reference :42-45 (tensor_ops.c:545-573): y = x / (1 + exp(-x)) */
int tensor_silu_f32(const TensorBuffer *input, TensorBuffer *output,
                    char *error, size_t error_capacity);
int tensor_silu_f16(const TensorBuffer *input, TensorBuffer *output,
                    char *error, size_t error_capacity);
/* reference :46-49 (tensor_ops.c:575-622): y = f16(f32(a) + f32(b)).
   Device-buffer calls enqueue GPU work; synchronize before host-side reads. */
int tensor_residual_add_f16(const TensorBuffer *left, const TensorBuffer *right,
                            TensorBuffer *output, char *error,
                            size_t error_capacity);

#ifdef __cplusplus
}
#endif

#endif
