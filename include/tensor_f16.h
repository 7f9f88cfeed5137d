/* Scalar IEEE binary16 / bfloat16 conversions (host functions).
 *
 * Replaces include/tensor_f16.h:6-8 of the reference (implemented there in
 * src/common/tensor_f16.c:17-85). Semantics: f32->f16 rounds to nearest even,
 * keeps subnormals, overflows to infinity, and keeps a NaN's sign and top ten
 * payload bits (forcing a nonzero payload); f16->f32 and bf16->f32 are exact.
 * The GPU kernels of this library use the same rounding.
 */
#ifndef TENSOR_F16_H
#define TENSOR_F16_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t tensor_f32_to_f16(float value);
float tensor_f16_to_f32(uint16_t value);
float tensor_bf16_to_f32(uint16_t value);

#ifdef __cplusplus
}
#endif

#endif
