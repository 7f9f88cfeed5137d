/* Host- or device-resident contiguous tensors.
 *
 * Same declarations, ownership and storage rules as
 * include/tensor_buffer.h:14-58 of the reference (implementation
 * src/common/tensor_buffer.c:142-409): rank <= 16, row-major contiguous
 * bytes, host storage owns a heap block, device storage owns a
 * TensorDeviceBuffer (none for zero-byte tensors), and tensor_buffer_data()
 * returns NULL for device tensors.
 */
#ifndef TENSOR_BUFFER_H
#define TENSOR_BUFFER_H

#include "safetensors.h"
#include "tensor_store.h"

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct TensorBuffer TensorBuffer;
typedef struct TensorWorkspace TensorWorkspace;

typedef enum {
    TENSOR_BUFFER_STORAGE_HOST,
    TENSOR_BUFFER_STORAGE_DEVICE
} TensorBufferStorage;

/* reference include/tensor_buffer.h:21-23 */
int tensor_buffer_create(TensorDType dtype, const uint64_t *shape, size_t rank,
                         TensorBuffer **result, char *error,
                         size_t error_capacity);
/* reference :24-26 */
int tensor_buffer_create_device(TensorDType dtype, const uint64_t *shape,
                                size_t rank, TensorBuffer **result,
                                char *error, size_t error_capacity);
/* reference :27-30. The host data comes from the program's workspace arena
   (the reference's tensor_workspace.c, reached through a weak reference);
   without that code linked the call fails with a message. */
int tensor_buffer_create_in_workspace(TensorDType dtype, const uint64_t *shape,
                                      size_t rank, TensorWorkspace *workspace,
                                      TensorBuffer **result, char *error,
                                      size_t error_capacity);
/* reference :31-33. Reads through the program's tensor store (the
   reference's tensor_store.c, reached through weak references); without that
   code linked the call fails with a message. */
int tensor_buffer_load(const TensorStore *store, const char *tensor_name,
                       TensorBuffer **result, char *error,
                       size_t error_capacity);
/* reference :34-36 (host only there, tensor_buffer.c:274-298). Here the
   conversion runs on the GPU for host and device sources alike; the result
   has the source's storage. */
int tensor_buffer_convert(const TensorBuffer *source, TensorDType target_dtype,
                          TensorBuffer **result, char *error,
                          size_t error_capacity);
/* reference :37-43 */
void tensor_buffer_free(TensorBuffer *buffer);
TensorDType tensor_buffer_dtype(const TensorBuffer *buffer);
size_t tensor_buffer_rank(const TensorBuffer *buffer);
const uint64_t *tensor_buffer_shape(const TensorBuffer *buffer);
size_t tensor_buffer_element_count(const TensorBuffer *buffer);
size_t tensor_buffer_byte_length(const TensorBuffer *buffer);
TensorBufferStorage tensor_buffer_storage(const TensorBuffer *buffer);
/* reference :44-46 */
int tensor_buffer_upload(TensorBuffer *buffer, size_t byte_offset,
                         const void *source, size_t byte_length,
                         char *error, size_t error_capacity);
/* reference :47-49 */
int tensor_buffer_download(const TensorBuffer *buffer, size_t byte_offset,
                           void *destination, size_t byte_length,
                           char *error, size_t error_capacity);
/* reference :50-55. Enqueues a device-to-device copy; synchronize before
   dependent host access. */
int tensor_buffer_copy_device(TensorBuffer *destination,
                              size_t destination_offset,
                              const TensorBuffer *source, size_t source_offset,
                              size_t byte_length, char *error,
                              size_t error_capacity);
/* reference :56-57 */
const void *tensor_buffer_data(const TensorBuffer *buffer);
void *tensor_buffer_data_mut(TensorBuffer *buffer);

/* Raw device address of a device tensor, NULL for host tensors.
   Reference: src/common/tensor_buffer_internal.h:9 (internal there). */
void *tensor_buffer_device_handle_internal(const TensorBuffer *buffer);

#ifdef __cplusplus
}
#endif

#endif
