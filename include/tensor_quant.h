/* Q8_0 / Q4_0 quantized weights.
 *
 * reference include/tensor_quant.h:10-36, unchanged. The HIP library
 * computes the packing on the GPU (bit-identical to the reference's
 * src/common/tensor_quant.c:48-100) and runs the quantized linear with a
 * dequantizing GEMV kernel.
 */
#ifndef TENSOR_QUANT_H
#define TENSOR_QUANT_H

#include "tensor_buffer.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TENSOR_WEIGHT_Q8_0 = 1,
    TENSOR_WEIGHT_Q4_0 = 2
} TensorWeightQuantization;

/* Quantize an [output, input] FP16 matrix into GGML-compatible Q*_0 blocks
 * (Q8_0: f16 scale + 32 int8; Q4_0: f16 scale + 16 bytes of nibbles). The
 * input width must be a multiple of 32. The returned U8 tensor has shape
 * [output, input/32, block_bytes] and is host resident.
 * reference include/tensor_quant.h:15-24 */
int tensor_quantize_linear_weight_f16(const uint16_t *weight,
                                      size_t output_width,
                                      size_t input_width,
                                      TensorWeightQuantization format,
                                      TensorBuffer **result,
                                      char *error, size_t error_capacity);

/* Device-only quantized linear: input [..., in] and output [..., out] are
 * FP16 device tensors, the weight is the packed U8 tensor above on the
 * device. reference include/tensor_quant.h:26-34 */
int tensor_linear_q8_0_f16(const TensorBuffer *input,
                           const TensorBuffer *packed_weight,
                           TensorBuffer *output, char *error,
                           size_t error_capacity);
int tensor_linear_q4_0_f16(const TensorBuffer *input,
                           const TensorBuffer *packed_weight,
                           TensorBuffer *output, char *error,
                           size_t error_capacity);

#ifdef __cplusplus
}
#endif
#endif
