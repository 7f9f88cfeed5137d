// Internal host-side services of the HIP tensor-ops library: error text,
// the per-process SDK device/stream, the device staging pool and the
// grid-reduction scratch.
#pragma once

#include <hip/hip_runtime_api.h>

#include <mutex>
#include <stddef.h>
#include <stdint.h>

namespace icsdk {

void set_error(char *error, size_t capacity, const char *format, ...)
    __attribute__((format(printf, 3, 4)));

// Lazily initialises the SDK device (the device current on first use) and
// its stream, once per process. Returns false with a message when no HIP
// device is usable.
bool sdk_ready(char *error, size_t capacity);
hipStream_t sdk_stream();
int sdk_device();
// Makes the SDK device current on the calling thread (host threads other
// than the initialising one may start on another device).
void bind_device();

// status == hipSuccess, or a message "<what>: <hip error text>".
bool hip_ok(hipError_t status, const char *what, char *error, size_t capacity);

// Device staging memory for host-storage operands, reused across calls.
// Blocks are cached by size class until scratch_clear().
void *scratch_acquire(size_t bytes);
void scratch_release(void *ptr, size_t bytes);
void scratch_clear();

// Device copies of host tables passed to the compute-table slots, keyed by
// host address like the CUDA backend's weight cache
// (src/platform/cuda/tensor_compute_cuda.cu:24-50): the first call uploads
// `bytes` bytes (enqueued on the SDK stream), later calls with the same
// address reuse the copy, a call with the same address and another size
// fails (nullptr), and weight_cache_clear() frees them (release_cache).
void *weight_cache_get(const void *host, size_t bytes);
void weight_cache_clear();

// Words of pinned (page-locked, device-mapped) host memory that a kernel
// writes and the host reads after waiting for the stream: a verdict without
// a device-to-host copy. nullptr when none can be allocated.
uint32_t *host_word_acquire();
void host_word_release(uint32_t *word);

class HostWord {
public:
    HostWord() : word_(host_word_acquire()) {}
    HostWord(const HostWord &) = delete;
    HostWord &operator=(const HostWord &) = delete;
    ~HostWord() { host_word_release(word_); }
    uint32_t *get() const { return word_; }
    uint32_t read() const { return *static_cast<volatile uint32_t *>(word_); }

private:
    uint32_t *word_;
};

// A pool block held for the duration of one call (none for zero bytes).
// Returning it to the pool right after the launches is safe: every later
// user of the block enqueues on the same SDK stream, after this call's
// kernels.
class ScratchBlock {
public:
    explicit ScratchBlock(size_t bytes)
        : bytes_(bytes), ptr_(bytes == 0 ? nullptr : scratch_acquire(bytes)) {}
    ScratchBlock(const ScratchBlock &) = delete;
    ScratchBlock &operator=(const ScratchBlock &) = delete;
    ~ScratchBlock() {
        if (ptr_ != nullptr) scratch_release(ptr_, bytes_);
    }
    void *get() const { return ptr_; }

private:
    size_t bytes_;
    void *ptr_;
};

// Partial-result buffer of the two-pass grid reductions. The launches of one
// reduction must be enqueued under grid_reduce_mutex() so that two host
// threads never interleave their passes on the shared buffer.
std::mutex &grid_reduce_mutex();
void *grid_reduce_partials(char *error, size_t capacity);

}  // namespace icsdk
