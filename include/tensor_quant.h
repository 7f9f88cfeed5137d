/* Weight-quantization formats named by the compute vtable.
 *
 * Only the enum of include/tensor_quant.h:10-13 of the reference is declared:
 * quantized GEMMs are contractions and are not part of the HIP tensor-ops
 * library. The values are ABI and match the reference.
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

#ifdef __cplusplus
}
#endif

#endif
