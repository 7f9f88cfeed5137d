/* Opaque handle for a weight store.
 *
 * The safetensors/sharded store (src/common/tensor_store.c of the reference)
 * is outside the HIP tensor-ops library. The type is declared only because
 * tensor_buffer_load (include/tensor_buffer.h:29-31 of the reference) names
 * it; in this library that entry point reports that no store is linked.
 * Reference declaration: include/tensor_store.h:8.
 */
#ifndef TENSOR_STORE_H
#define TENSOR_STORE_H

#include "safetensors.h"

typedef struct TensorStore TensorStore;

#endif
