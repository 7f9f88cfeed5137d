// TensorBuffer, dtype helpers and the scalar f16 conversions.
//
// TensorBuffer follows include/tensor_buffer.h:14-58 of the reference and the
// rules of src/common/tensor_buffer.c:142-409: rank <= 16, shape copied,
// element/byte counts checked for overflow, host data zero-initialised (one
// byte for empty tensors), device storage allocated only for non-empty
// tensors, data() NULL for device tensors, range-checked upload / download /
// device copy. tensor_buffer_convert runs on the GPU (ops.cpp).
//
// Workspace arenas and weight stores are the program's, not this library's:
// tensor_buffer_create_in_workspace and tensor_buffer_load call the
// reference's tensor_workspace_allocate / tensor_store_find /
// tensor_store_read_raw through weak references. A program that holds a
// TensorWorkspace or TensorStore has linked the code that made it, so the
// references resolve; otherwise they stay null and the call reports it.
#include "sdk.hpp"

#include "tensor_buffer.h"
#include "tensor_device.h"
#include "tensor_f16.h"
#include "tensor_store.h"

#include <cstdint>
#include <cstdlib>
#include <cstring>

struct TensorBuffer {
    TensorDType dtype;
    size_t rank;
    uint64_t *shape;
    size_t element_count;
    size_t byte_length;
    void *data;                       // host storage
    TensorDeviceBuffer *device;       // device storage (NULL when empty)
    TensorBufferStorage storage;
    bool owns_data;                   // false for workspace-backed host data
};

// reference include/tensor_workspace.h:17-19 (defined by tensor_workspace.c)
extern "C" void *tensor_workspace_allocate(TensorWorkspace *workspace, size_t size,
                                           size_t alignment, char *error,
                                           size_t error_capacity) __attribute__((weak));
extern "C" const SafeTensorInfo *tensor_store_find(const TensorStore *store,
                                                   const char *tensor_name)
    __attribute__((weak));
extern "C" int tensor_store_read_raw(const TensorStore *store, const char *tensor_name,
                                     void *destination, size_t capacity, char *error,
                                     size_t error_capacity) __attribute__((weak));

using icsdk::set_error;

namespace {

constexpr size_t kMaxRank = 16;

// workspace: host storage comes from the arena (reference
// tensor_buffer.c:183-186, alignment _Alignof(max_align_t)), not the heap.
int create(TensorDType dtype, const uint64_t *shape, size_t rank, bool host,
           TensorWorkspace *workspace, TensorBuffer **result, char *error,
           size_t capacity) {
    if (result != nullptr) *result = nullptr;
    const size_t element_size = tensor_dtype_size(dtype);
    if (result == nullptr || element_size == 0 || rank > kMaxRank ||
        (rank > 0 && shape == nullptr)) {
        set_error(error, capacity, "invalid tensor buffer dtype, rank, or shape");
        return 0;
    }
    size_t elements = 1;
    for (size_t d = 0; d < rank; ++d) {
        if (shape[d] > SIZE_MAX || (shape[d] != 0 && elements > SIZE_MAX / (size_t)shape[d])) {
            set_error(error, capacity, "tensor shape exceeds addressable size");
            return 0;
        }
        elements *= (size_t)shape[d];
    }
    if (elements > SIZE_MAX / element_size) {
        set_error(error, capacity, "tensor byte length exceeds addressable size");
        return 0;
    }
    auto *buffer = static_cast<TensorBuffer *>(std::calloc(1, sizeof(TensorBuffer)));
    if (buffer == nullptr) {
        set_error(error, capacity, "out of memory creating tensor buffer");
        return 0;
    }
    if (rank > 0) {
        buffer->shape = static_cast<uint64_t *>(std::malloc(rank * sizeof(uint64_t)));
        if (buffer->shape == nullptr) {
            std::free(buffer);
            set_error(error, capacity, "out of memory copying tensor shape");
            return 0;
        }
        std::memcpy(buffer->shape, shape, rank * sizeof(uint64_t));
    }
    const size_t bytes = elements * element_size;
    buffer->dtype = dtype;
    buffer->rank = rank;
    buffer->element_count = elements;
    buffer->byte_length = bytes;
    buffer->storage = host ? TENSOR_BUFFER_STORAGE_HOST : TENSOR_BUFFER_STORAGE_DEVICE;
    if (host) {
        buffer->data = workspace == nullptr
                           ? std::calloc(bytes == 0 ? 1 : bytes, 1)
                           : tensor_workspace_allocate(workspace, bytes, alignof(max_align_t),
                                                       error, capacity);
        buffer->owns_data = workspace == nullptr;
        if (buffer->data == nullptr) {
            std::free(buffer->shape);
            std::free(buffer);
            set_error(error, capacity, "out of memory allocating tensor data");
            return 0;
        }
    } else if (bytes > 0 &&
               !tensor_device_buffer_create(bytes, &buffer->device, error, capacity)) {
        std::free(buffer->shape);
        std::free(buffer);
        return 0;
    }
    *result = buffer;
    return 1;
}

bool valid_range(const TensorBuffer *buffer, size_t offset, size_t length) {
    return buffer != nullptr && offset <= buffer->byte_length &&
           length <= buffer->byte_length - offset;
}

uint32_t bits_of(float value) {
    uint32_t bits;
    std::memcpy(&bits, &value, sizeof bits);
    return bits;
}

float float_of(uint32_t bits) {
    float value;
    std::memcpy(&value, &bits, sizeof value);
    return value;
}

}  // namespace

extern "C" {

// reference src/common/safetensors.c:317-336
const char *tensor_dtype_name(TensorDType dtype) {
    static const char *const names[] = {"UNKNOWN", "BOOL", "U8",      "I8",      "I16",
                                        "U16",     "I32",  "U32",     "I64",     "U64",
                                        "F8_E4M3", "F8_E5M2", "F16",  "BF16",    "F32",
                                        "F64"};
    const unsigned index = (unsigned)dtype;
    return index < sizeof(names) / sizeof(names[0]) ? names[index] : "UNKNOWN";
}

// reference src/common/safetensors.c:338-360
size_t tensor_dtype_size(TensorDType dtype) {
    switch (dtype) {
        case TENSOR_DTYPE_BOOL: case TENSOR_DTYPE_U8: case TENSOR_DTYPE_I8:
        case TENSOR_DTYPE_F8_E4M3: case TENSOR_DTYPE_F8_E5M2:
            return 1;
        case TENSOR_DTYPE_I16: case TENSOR_DTYPE_U16: case TENSOR_DTYPE_F16:
        case TENSOR_DTYPE_BF16:
            return 2;
        case TENSOR_DTYPE_I32: case TENSOR_DTYPE_U32: case TENSOR_DTYPE_F32:
            return 4;
        case TENSOR_DTYPE_I64: case TENSOR_DTYPE_U64: case TENSOR_DTYPE_F64:
            return 8;
        default:
            return 0;
    }
}

// Scalar conversions (reference src/common/tensor_f16.c:17-85). Exact widening;
// narrowing rounds to nearest even on the 2^-24 grid below 2^-14, overflows at
// 65520, and keeps a NaN's sign and top ten payload bits (zero payload -> 1).
float tensor_f16_to_f32(uint16_t value) {
    const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    const uint32_t exponent = (value >> 10) & 0x1fu;
    const uint32_t mantissa = value & 0x3ffu;
    if (exponent == 0x1fu) return float_of(sign | 0x7f800000u | (mantissa << 13));
    if (exponent != 0) return float_of(sign | ((exponent + 112u) << 23) | (mantissa << 13));
    const float magnitude = (float)mantissa * 0x1p-24f;
    return sign ? -magnitude : magnitude;
}

uint16_t tensor_f32_to_f16(float value) {
    const uint32_t bits = bits_of(value);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t magnitude = bits & 0x7fffffffu;
    if (magnitude > 0x7f800000u) {
        const uint16_t payload = (uint16_t)((magnitude >> 13) & 0x3ffu);
        return (uint16_t)(sign | 0x7c00u | (payload ? payload : 1u));
    }
    if (magnitude >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (magnitude >= 0x38800000u) {
        const uint32_t rebased = magnitude - 0x38000000u;
        return (uint16_t)(sign | ((rebased + 0x0fffu + ((rebased >> 13) & 1u)) >> 13));
    }
    if (magnitude <= 0x33000000u) return sign;
    const uint32_t shift = 126u - (magnitude >> 23);
    const uint32_t significand = (magnitude & 0x7fffffu) | 0x800000u;
    uint32_t quotient = significand >> shift;
    const uint32_t remainder = significand & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (remainder > half || (remainder == half && (quotient & 1u))) quotient++;
    return (uint16_t)(sign | quotient);
}

float tensor_bf16_to_f32(uint16_t value) { return float_of((uint32_t)value << 16); }

int tensor_buffer_create(TensorDType dtype, const uint64_t *shape, size_t rank,
                         TensorBuffer **result, char *error, size_t error_capacity) {
    return create(dtype, shape, rank, true, nullptr, result, error, error_capacity);
}

int tensor_buffer_create_device(TensorDType dtype, const uint64_t *shape, size_t rank,
                                TensorBuffer **result, char *error, size_t error_capacity) {
    if (result != nullptr) *result = nullptr;
    if (result == nullptr) {
        set_error(error, error_capacity, "device tensor result pointer is required");
        return 0;
    }
    return create(dtype, shape, rank, false, nullptr, result, error, error_capacity);
}

// reference src/common/tensor_buffer.c:235-246
int tensor_buffer_create_in_workspace(TensorDType dtype, const uint64_t *shape, size_t rank,
                                      TensorWorkspace *workspace, TensorBuffer **result,
                                      char *error, size_t error_capacity) {
    if (workspace == nullptr) {
        if (result != nullptr) *result = nullptr;
        set_error(error, error_capacity, "workspace-backed tensor requires a workspace");
        return 0;
    }
    if (tensor_workspace_allocate == nullptr) {
        if (result != nullptr) *result = nullptr;
        set_error(error, error_capacity,
                  "workspace-backed tensor requires tensor_workspace.c linked into the program");
        return 0;
    }
    return create(dtype, shape, rank, true, workspace, result, error, error_capacity);
}

// reference src/common/tensor_buffer.c:248-271: a host tensor of the stored
// dtype and shape, filled with the stored bytes.
int tensor_buffer_load(const TensorStore *store, const char *tensor_name,
                       TensorBuffer **result, char *error, size_t error_capacity) {
    if (result != nullptr) *result = nullptr;
    if (tensor_store_find == nullptr || tensor_store_read_raw == nullptr) {
        set_error(error, error_capacity,
                  "tensor_buffer_load requires tensor_store.c linked into the program");
        return 0;
    }
    const SafeTensorInfo *info = tensor_store_find(store, tensor_name);
    if (info == nullptr || result == nullptr) {
        set_error(error, error_capacity, "tensor metadata was not found");
        return 0;
    }
    TensorBuffer *buffer = nullptr;
    if (!tensor_buffer_create(info->dtype, info->shape, info->rank, &buffer, error,
                              error_capacity))
        return 0;
    if (buffer->byte_length != info->byte_length ||
        !tensor_store_read_raw(store, tensor_name, buffer->data, buffer->byte_length, error,
                               error_capacity)) {
        tensor_buffer_free(buffer);
        if (error != nullptr && error_capacity > 0 && error[0] == '\0')
            set_error(error, error_capacity, "tensor metadata byte length mismatch");
        return 0;
    }
    *result = buffer;
    return 1;
}

void tensor_buffer_free(TensorBuffer *buffer) {
    if (buffer == nullptr) return;
    if (buffer->owns_data) std::free(buffer->data);
    tensor_device_buffer_free(buffer->device);
    std::free(buffer->shape);
    std::free(buffer);
}

TensorDType tensor_buffer_dtype(const TensorBuffer *buffer) {
    return buffer == nullptr ? TENSOR_DTYPE_UNKNOWN : buffer->dtype;
}

size_t tensor_buffer_rank(const TensorBuffer *buffer) { return buffer == nullptr ? 0 : buffer->rank; }

const uint64_t *tensor_buffer_shape(const TensorBuffer *buffer) {
    return buffer == nullptr ? nullptr : buffer->shape;
}

size_t tensor_buffer_element_count(const TensorBuffer *buffer) {
    return buffer == nullptr ? 0 : buffer->element_count;
}

size_t tensor_buffer_byte_length(const TensorBuffer *buffer) {
    return buffer == nullptr ? 0 : buffer->byte_length;
}

TensorBufferStorage tensor_buffer_storage(const TensorBuffer *buffer) {
    return buffer == nullptr ? TENSOR_BUFFER_STORAGE_HOST : buffer->storage;
}

void *tensor_buffer_device_handle_internal(const TensorBuffer *buffer) {
    if (buffer == nullptr || buffer->storage != TENSOR_BUFFER_STORAGE_DEVICE) return nullptr;
    return tensor_device_buffer_native_handle(buffer->device);
}

int tensor_buffer_upload(TensorBuffer *buffer, size_t byte_offset, const void *source,
                         size_t byte_length, char *error, size_t error_capacity) {
    if (!valid_range(buffer, byte_offset, byte_length) || (byte_length > 0 && source == nullptr)) {
        set_error(error, error_capacity, "invalid tensor upload range or pointer");
        return 0;
    }
    if (byte_length == 0) return 1;
    if (buffer->storage == TENSOR_BUFFER_STORAGE_DEVICE)
        return tensor_device_buffer_upload(buffer->device, byte_offset, source, byte_length,
                                           error, error_capacity);
    std::memcpy(static_cast<unsigned char *>(buffer->data) + byte_offset, source, byte_length);
    return 1;
}

int tensor_buffer_download(const TensorBuffer *buffer, size_t byte_offset, void *destination,
                           size_t byte_length, char *error, size_t error_capacity) {
    if (!valid_range(buffer, byte_offset, byte_length) ||
        (byte_length > 0 && destination == nullptr)) {
        set_error(error, error_capacity, "invalid tensor download range or pointer");
        return 0;
    }
    if (byte_length == 0) return 1;
    if (buffer->storage == TENSOR_BUFFER_STORAGE_DEVICE)
        return tensor_device_buffer_download(buffer->device, byte_offset, destination,
                                             byte_length, error, error_capacity);
    std::memcpy(destination, static_cast<const unsigned char *>(buffer->data) + byte_offset,
                byte_length);
    return 1;
}

int tensor_buffer_copy_device(TensorBuffer *destination, size_t destination_offset,
                              const TensorBuffer *source, size_t source_offset,
                              size_t byte_length, char *error, size_t error_capacity) {
    if (!valid_range(destination, destination_offset, byte_length) ||
        !valid_range(source, source_offset, byte_length) ||
        destination->storage != TENSOR_BUFFER_STORAGE_DEVICE ||
        source->storage != TENSOR_BUFFER_STORAGE_DEVICE) {
        set_error(error, error_capacity, "tensor device copy requires valid device-resident ranges");
        return 0;
    }
    if (byte_length == 0) return 1;
    return tensor_device_buffer_copy(destination->device, destination_offset, source->device,
                                     source_offset, byte_length, error, error_capacity);
}

const void *tensor_buffer_data(const TensorBuffer *buffer) {
    return buffer == nullptr || buffer->storage != TENSOR_BUFFER_STORAGE_HOST ? nullptr
                                                                              : buffer->data;
}

void *tensor_buffer_data_mut(TensorBuffer *buffer) {
    return buffer == nullptr || buffer->storage != TENSOR_BUFFER_STORAGE_HOST ? nullptr
                                                                              : buffer->data;
}

}  // extern "C"
