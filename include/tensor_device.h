/* Device buffers on the HIP backend (MI355X / gfx950).
 *
 * Same declarations and contract as include/tensor_device.h:10-37 of the
 * reference (CUDA implementation: src/platform/cuda/tensor_device_cuda.cu:33-129).
 * All work is ordered on one per-process SDK stream:
 *   - uploads have consumed the host source when they return;
 *   - downloads wait for all earlier SDK work and for the copy itself;
 *   - device-to-device copies and kernels are enqueued and return at once;
 *   - tensor_device_synchronize waits for everything enqueued so far.
 * Every function returns 1 on success and 0 on failure, with a message
 * written to (error, error_capacity) when error is not NULL.
 */
#ifndef TENSOR_DEVICE_H
#define TENSOR_DEVICE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct TensorDeviceBuffer TensorDeviceBuffer;

/* reference include/tensor_device.h:13 */
int tensor_device_available(void);
/* reference :14-16; a zero-byte buffer is an error, as in
   tensor_device_cuda.cu:42-44 */
int tensor_device_buffer_create(size_t byte_length,
                                TensorDeviceBuffer **result,
                                char *error, size_t error_capacity);
/* reference :17 */
void tensor_device_buffer_free(TensorDeviceBuffer *buffer);
/* reference :18 */
size_t tensor_device_buffer_size(const TensorDeviceBuffer *buffer);
/* reference :24-27 */
int tensor_device_buffer_upload(TensorDeviceBuffer *destination,
                                size_t destination_offset,
                                const void *source, size_t byte_length,
                                char *error, size_t error_capacity);
/* reference :28-31 */
int tensor_device_buffer_download(const TensorDeviceBuffer *source,
                                  size_t source_offset, void *destination,
                                  size_t byte_length, char *error,
                                  size_t error_capacity);
/* reference :32-36 */
int tensor_device_buffer_copy(TensorDeviceBuffer *destination,
                              size_t destination_offset,
                              const TensorDeviceBuffer *source,
                              size_t source_offset, size_t byte_length,
                              char *error, size_t error_capacity);
/* reference :37 */
int tensor_device_synchronize(char *error, size_t error_capacity);

/* Raw device address of a buffer (hipMalloc pointer), or NULL.
   Reference: src/common/tensor_device_internal.h:9, which the reference keeps
   internal; it is exported here so host code above the C ABI can hand the
   address to other HIP code. */
void *tensor_device_buffer_native_handle(const TensorDeviceBuffer *buffer);

#ifdef __cplusplus
}
#endif

#endif
