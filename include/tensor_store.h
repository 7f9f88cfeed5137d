/* Opaque handle for a weight store.
 *
 * The safetensors/sharded store (src/common/tensor_store.c of the reference)
 * is not part of the HIP tensor-ops library: it stays in the program that
 * links this library (the reference's own tensor_store.c). The handle and the
 * two lookups tensor_buffer_load needs are declared here; the library
 * references them weakly, so they resolve to the program's store code when it
 * is linked, and tensor_buffer_load reports an error when it is not.
 * Reference declarations: include/tensor_store.h:8,19-23.
 */
#ifndef TENSOR_STORE_H
#define TENSOR_STORE_H

#include "safetensors.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct TensorStore TensorStore;

/* reference include/tensor_store.h:19-20 (defined by tensor_store.c) */
const SafeTensorInfo *tensor_store_find(const TensorStore *store,
                                        const char *tensor_name);
/* reference include/tensor_store.h:21-23 (defined by tensor_store.c) */
int tensor_store_read_raw(const TensorStore *store, const char *tensor_name,
                          void *destination, size_t capacity,
                          char *error, size_t error_capacity);

#ifdef __cplusplus
}
#endif

#endif
