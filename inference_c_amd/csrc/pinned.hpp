// Host <-> device transfers of caller memory through pinned staging chunks.
//
// Caller memory is ordinary pageable memory, which the DMA engines cannot
// read at full rate (measured on MI355X: pageable 30 GB/s host-to-device and
// 18 GB/s device-to-host, pinned 57 GB/s both ways). Each transfer is cut
// into pieces of one pinned chunk; host threads copy a piece between the
// caller's memory and a chunk while the DMA of the previous piece runs.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>

namespace icsdk {

// Enqueues `bytes` from host memory `src` into device memory `dst` on
// `stream` (after the work already there). Returns once `src` has been
// read: the host may reuse it; the device copy completes in stream order.
bool pinned_to_device(void *dst, const void *src, size_t bytes, hipStream_t stream,
                      char *error, size_t capacity);

// Copies `bytes` from device memory `src` (after the work already on
// `stream`) into host memory `dst`; returns once every byte is in `dst`.
bool pinned_to_host(void *dst, const void *src, size_t bytes, hipStream_t stream, char *error,
                    size_t capacity);

// Frees the idle pinned chunks (release_cache); chunks in use are kept.
void pinned_release();

}  // namespace icsdk
