// SDK device state and the tensor_device.h contract on HIP.
//
// Reference: include/tensor_device.h:10-37 and the CUDA implementation
// src/platform/cuda/tensor_device_cuda.cu:33-129 (cudaMalloc, blocking
// cudaMemcpy on the legacy stream, cudaDeviceSynchronize). Here every copy
// and kernel is ordered on one non-blocking SDK stream created at first use;
// uploads and downloads synchronise that stream before returning, D2D copies
// only enqueue, and tensor_device_synchronize waits for the stream.
#include "pinned.hpp"
#include "sdk.hpp"

#include "kernels.hpp"
#include "tensor_device.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <vector>

struct TensorDeviceBuffer {
    void *data;
    size_t byte_length;
};

namespace icsdk {

void set_error(char *error, size_t capacity, const char *format, ...) {
    if (error == nullptr || capacity == 0) return;
    va_list args;
    va_start(args, format);
    std::vsnprintf(error, capacity, format, args);
    va_end(args);
}

bool hip_ok(hipError_t status, const char *what, char *error, size_t capacity) {
    if (status == hipSuccess) return true;
    set_error(error, capacity, "%s: %s", what, hipGetErrorString(status));
    return false;
}

namespace {

struct SdkState {
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    char reason[192] = "HIP runtime not initialised";
};

SdkState &state() {
    static SdkState s;
    static std::once_flag once;
    std::call_once(once, [] {
        int count = 0;
        hipError_t status = hipGetDeviceCount(&count);
        if (status != hipSuccess || count <= 0) {
            std::snprintf(s.reason, sizeof s.reason, "no HIP device is available (%s)",
                          status != hipSuccess ? hipGetErrorString(status) : "0 devices");
            return;
        }
        if ((status = hipGetDevice(&s.device)) != hipSuccess ||
            (status = hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking)) != hipSuccess) {
            std::snprintf(s.reason, sizeof s.reason, "HIP device initialisation failed (%s)",
                          hipGetErrorString(status));
            return;
        }
        s.ready = true;
    });
    return s;
}

// ---- staging pool ------------------------------------------------------------

constexpr size_t kScratchGranule = size_t{1} << 16;

size_t size_class(size_t bytes) {
    size_t c = kScratchGranule;
    while (c < bytes) c <<= 1;
    return c;
}

std::mutex pool_mutex;
std::multimap<size_t, void *> pool;

}  // namespace

bool sdk_ready(char *error, size_t capacity) {
    SdkState &s = state();
    if (!s.ready) {
        set_error(error, capacity, "HIP device unavailable: %s", s.reason);
        return false;
    }
    bind_device();
    return true;
}

hipStream_t sdk_stream() { return state().stream; }
int sdk_device() { return state().device; }

void bind_device() {
    const int want = state().device;
    int current = -1;
    if (want >= 0 && (hipGetDevice(&current) != hipSuccess || current != want))
        (void)hipSetDevice(want);
}

void *scratch_acquire(size_t bytes) {
    const size_t c = size_class(bytes);
    {
        std::lock_guard<std::mutex> lock(pool_mutex);
        auto found = pool.find(c);
        if (found != pool.end()) {
            void *p = found->second;
            pool.erase(found);
            return p;
        }
    }
    void *p = nullptr;
    if (hipMalloc(&p, c) != hipSuccess) return nullptr;
    return p;
}

void scratch_release(void *ptr, size_t bytes) {
    if (ptr == nullptr) return;
    std::lock_guard<std::mutex> lock(pool_mutex);
    pool.emplace(size_class(bytes), ptr);
}

void scratch_clear() {
    std::vector<void *> blocks;
    {
        std::lock_guard<std::mutex> lock(pool_mutex);
        for (auto &entry : pool) blocks.push_back(entry.second);
        pool.clear();
    }
    if (blocks.empty() || !state().ready) return;
    bind_device();
    (void)hipStreamSynchronize(state().stream);
    for (void *p : blocks) (void)hipFree(p);
}

namespace {
std::mutex weights_mutex;
std::map<const void *, std::pair<void *, size_t>> weights;
}  // namespace

void *weight_cache_get(const void *host, size_t bytes) {
    if (host == nullptr || bytes == 0 || !state().ready) return nullptr;
    std::lock_guard<std::mutex> lock(weights_mutex);
    auto found = weights.find(host);
    if (found != weights.end())
        return found->second.second == bytes ? found->second.first : nullptr;
    bind_device();
    void *device = nullptr;
    if (hipMalloc(&device, bytes) != hipSuccess) return nullptr;
    if (!pinned_to_device(device, host, bytes, state().stream, nullptr, 0)) {
        (void)hipStreamSynchronize(state().stream);
        (void)hipFree(device);
        return nullptr;
    }
    weights.emplace(host, std::make_pair(device, bytes));
    return device;
}

void weight_cache_clear() {
    std::vector<void *> blocks;
    {
        std::lock_guard<std::mutex> lock(weights_mutex);
        for (auto &entry : weights) blocks.push_back(entry.second.first);
        weights.clear();
    }
    if (blocks.empty() || !state().ready) return;
    bind_device();
    (void)hipStreamSynchronize(state().stream);
    for (void *p : blocks) (void)hipFree(p);
}

namespace {
std::mutex words_mutex;
std::vector<uint32_t *> free_words;
constexpr size_t kWordsPerSlab = 1024;  // one 4 KiB page of pinned memory
}  // namespace

uint32_t *host_word_acquire() {
    std::lock_guard<std::mutex> lock(words_mutex);
    if (free_words.empty()) {
        if (!state().ready) return nullptr;
        bind_device();
        void *slab = nullptr;
        // coherent: a kernel's store is not held in a device cache; slabs stay
        // allocated for the life of the process
        if (hipHostMalloc(&slab, kWordsPerSlab * sizeof(uint32_t),
                          hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
            return nullptr;
        for (size_t i = 0; i < kWordsPerSlab; ++i)
            free_words.push_back(static_cast<uint32_t *>(slab) + i);
    }
    uint32_t *word = free_words.back();
    free_words.pop_back();
    return word;
}

void host_word_release(uint32_t *word) {
    if (word == nullptr) return;
    std::lock_guard<std::mutex> lock(words_mutex);
    free_words.push_back(word);
}

std::mutex &grid_reduce_mutex() {
    static std::mutex m;
    return m;
}

void *grid_reduce_partials(char *error, size_t capacity) {
    static void *partials = nullptr;
    static std::once_flag once;
    static hipError_t status = hipSuccess;
    std::call_once(once, [] { status = hipMalloc(&partials, k::grid_reduce_scratch_bytes()); });
    if (status != hipSuccess) {
        hip_ok(status, "hipMalloc (grid reduction partials)", error, capacity);
        return nullptr;
    }
    return partials;
}

}  // namespace icsdk

using namespace icsdk;

namespace {
bool valid_range(size_t total, size_t offset, size_t length) {
    return offset <= total && length <= total - offset;
}
}  // namespace

extern "C" int tensor_device_available(void) { return state().ready ? 1 : 0; }

extern "C" int tensor_device_buffer_create(size_t byte_length, TensorDeviceBuffer **result,
                                           char *error, size_t error_capacity) {
    if (result != nullptr) *result = nullptr;
    if (result == nullptr || byte_length == 0) {
        set_error(error, error_capacity, "device buffer size must be nonzero");
        return 0;
    }
    if (!sdk_ready(error, error_capacity)) return 0;
    auto *buffer = static_cast<TensorDeviceBuffer *>(std::calloc(1, sizeof(TensorDeviceBuffer)));
    if (buffer == nullptr) {
        set_error(error, error_capacity, "out of memory creating device buffer");
        return 0;
    }
    if (!hip_ok(hipMalloc(&buffer->data, byte_length), "hipMalloc", error, error_capacity)) {
        std::free(buffer);
        return 0;
    }
    buffer->byte_length = byte_length;
    *result = buffer;
    return 1;
}

extern "C" void tensor_device_buffer_free(TensorDeviceBuffer *buffer) {
    if (buffer == nullptr) return;
    if (buffer->data != nullptr) {
        bind_device();
        // queued kernels may still read or write the block
        (void)hipStreamSynchronize(sdk_stream());
        (void)hipFree(buffer->data);
    }
    std::free(buffer);
}

extern "C" size_t tensor_device_buffer_size(const TensorDeviceBuffer *buffer) {
    return buffer == nullptr ? 0 : buffer->byte_length;
}

extern "C" void *tensor_device_buffer_native_handle(const TensorDeviceBuffer *buffer) {
    return buffer == nullptr ? nullptr : buffer->data;
}

extern "C" int tensor_device_buffer_upload(TensorDeviceBuffer *destination,
                                           size_t destination_offset, const void *source,
                                           size_t byte_length, char *error,
                                           size_t error_capacity) {
    if (destination == nullptr || (byte_length > 0 && source == nullptr) ||
        !valid_range(destination->byte_length, destination_offset, byte_length)) {
        set_error(error, error_capacity, "invalid device upload range or pointer");
        return 0;
    }
    if (byte_length == 0) return 1;
    if (!sdk_ready(error, error_capacity)) return 0;
    // the source has been read into pinned chunks when this returns; the
    // device copy completes in stream order
    return pinned_to_device(static_cast<char *>(destination->data) + destination_offset, source,
                            byte_length, sdk_stream(), error, error_capacity);
}

extern "C" int tensor_device_buffer_download(const TensorDeviceBuffer *source,
                                             size_t source_offset, void *destination,
                                             size_t byte_length, char *error,
                                             size_t error_capacity) {
    if (source == nullptr || (byte_length > 0 && destination == nullptr) ||
        !valid_range(source->byte_length, source_offset, byte_length)) {
        set_error(error, error_capacity, "invalid device download range or pointer");
        return 0;
    }
    if (byte_length == 0) return 1;
    if (!sdk_ready(error, error_capacity)) return 0;
    return pinned_to_host(destination, static_cast<const char *>(source->data) + source_offset,
                          byte_length, sdk_stream(), error, error_capacity);
}

extern "C" int tensor_device_buffer_copy(TensorDeviceBuffer *destination,
                                         size_t destination_offset,
                                         const TensorDeviceBuffer *source, size_t source_offset,
                                         size_t byte_length, char *error,
                                         size_t error_capacity) {
    if (destination == nullptr || source == nullptr ||
        !valid_range(destination->byte_length, destination_offset, byte_length) ||
        !valid_range(source->byte_length, source_offset, byte_length)) {
        set_error(error, error_capacity, "invalid device-to-device copy range");
        return 0;
    }
    if (byte_length == 0) return 1;
    if (!sdk_ready(error, error_capacity)) return 0;
    return hip_ok(hipMemcpyAsync(static_cast<char *>(destination->data) + destination_offset,
                                 static_cast<const char *>(source->data) + source_offset,
                                 byte_length, hipMemcpyDeviceToDevice, sdk_stream()),
                  "hipMemcpyAsync device-to-device", error, error_capacity);
}

extern "C" int tensor_device_synchronize(char *error, size_t error_capacity) {
    if (!sdk_ready(error, error_capacity)) return 0;
    return hip_ok(hipStreamSynchronize(sdk_stream()), "hipStreamSynchronize", error,
                  error_capacity);
}
