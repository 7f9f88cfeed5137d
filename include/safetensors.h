/* Element types shared by every TensorBuffer.
 *
 * Only the dtype part of the reference header is declared here: the
 * safetensors file reader itself is not part of the HIP tensor-ops library.
 * The enumerator order (and therefore every numeric value) is the ABI and is
 * kept identical to include/safetensors.h:11-28 of the reference, so a
 * TensorDType produced by reference code means the same thing here.
 */
#ifndef SAFETENSORS_H
#define SAFETENSORS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TENSOR_DTYPE_UNKNOWN,   /* 0 */
    TENSOR_DTYPE_BOOL,      /* 1 */
    TENSOR_DTYPE_U8,        /* 2 */
    TENSOR_DTYPE_I8,        /* 3 */
    TENSOR_DTYPE_I16,       /* 4 */
    TENSOR_DTYPE_U16,       /* 5 */
    TENSOR_DTYPE_I32,       /* 6 */
    TENSOR_DTYPE_U32,       /* 7 */
    TENSOR_DTYPE_I64,       /* 8 */
    TENSOR_DTYPE_U64,       /* 9 */
    TENSOR_DTYPE_F8_E4M3,   /* 10 */
    TENSOR_DTYPE_F8_E5M2,   /* 11 */
    TENSOR_DTYPE_F16,       /* 12 */
    TENSOR_DTYPE_BF16,      /* 13 */
    TENSOR_DTYPE_F32,       /* 14 */
    TENSOR_DTYPE_F64        /* 15 */
} TensorDType;

/* One tensor's metadata in a safetensors file or store (reference
 * include/safetensors.h:30-37, layout kept: tensor_buffer_load reads dtype,
 * rank, shape and byte_length from the record the store returns). */
typedef struct {
    const char *name;
    TensorDType dtype;
    size_t rank;
    const uint64_t *shape;
    uint64_t data_offset;
    uint64_t byte_length;
} SafeTensorInfo;

/* Replaces src/common/safetensors.c's tensor_dtype_name / tensor_dtype_size
 * (declared at include/safetensors.h:41-42 of the reference). Unknown dtypes
 * have size 0 and name "UNKNOWN". */
const char *tensor_dtype_name(TensorDType dtype);
size_t tensor_dtype_size(TensorDType dtype);

#ifdef __cplusplus
}
#endif

#endif
