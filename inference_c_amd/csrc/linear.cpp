// Linear, matmul and the Q8_0 / Q4_0 weight functions
// (include/tensor_ops.h, include/tensor_quant.h).
//
// Validation order and messages are the reference's
// (src/common/tensor_ops.c:163-398, src/common/tensor_quant.c:48-141). The
// arithmetic runs on the GPU for host and device storage alike:
//   matmul, linear   hipBLASLt GEMM with f32 accumulation; a linear's bias is
//                    fused into the GEMM (one rounding, like the reference's
//                    host loop, which starts each sum at the bias);
//   quantize         k_quant.hip's quantizer, bit-for-bit the reference's
//                    rounding, on the uploaded weights;
//   quantized linear k_quant.hip's dequantizing GEMV.
// A device linear goes through tensor_compute_preferred_backend() like the
// reference (a missing backend or slot fails the same way); the GEMM itself
// is enqueued with the bias fused rather than as two slot calls.
#include "gemm.hpp"
#include "kernels.hpp"
#include "sdk.hpp"
#include "staging.hpp"

#include "tensor_buffer.h"
#include "tensor_compute_backend.h"
#include "tensor_ops.h"
#include "tensor_quant.h"

#include <climits>
#include <cstring>

using namespace icsdk;

namespace {

using Buf = const TensorBuffer *;

bool host_of(Buf t, TensorDType dtype) {
    return t != nullptr && tensor_buffer_storage(t) == TENSOR_BUFFER_STORAGE_HOST &&
           tensor_buffer_dtype(t) == dtype;
}

bool device_of(Buf t, TensorDType dtype) {
    return t != nullptr && tensor_buffer_storage(t) == TENSOR_BUFFER_STORAGE_DEVICE &&
           tensor_buffer_dtype(t) == dtype;
}

bool on_device(Buf t) {
    return t != nullptr && tensor_buffer_storage(t) == TENSOR_BUFFER_STORAGE_DEVICE;
}

const void *handle(Buf t) { return t ? tensor_buffer_device_handle_internal(t) : nullptr; }

int fail(char *error, size_t capacity, const char *message) {
    set_error(error, capacity, "%s", message);
    return 0;
}

// tensor_ops.c:163-215 (host storage only, as in the reference)
int matmul(TensorDType dtype, Buf left, Buf right, TensorBuffer *output, char *error,
           size_t capacity) {
    if (!host_of(left, dtype) || !host_of(right, dtype) || !host_of(output, dtype) ||
        tensor_buffer_rank(left) != 2 || tensor_buffer_rank(right) != 2 ||
        tensor_buffer_rank(output) != 2) {
        set_error(error, capacity, "matmul requires rank-2 %s tensors",
                  dtype == TENSOR_DTYPE_F32 ? "F32" : "F16");
        return 0;
    }
    const uint64_t *ls = tensor_buffer_shape(left), *rs = tensor_buffer_shape(right);
    const uint64_t *os = tensor_buffer_shape(output);
    if (ls[1] != rs[0] || os[0] != ls[0] || os[1] != rs[1])
        return fail(error, capacity, "matmul tensor dimensions do not match");
    const size_t rows = ls[0], inner = ls[1], cols = rs[1];
    if (rows == 0 || cols == 0) return 1;
    Staging st("matmul", true, error, capacity);
    if (!st.begin()) return 0;
    const void *pa = st.in(tensor_buffer_data(left), tensor_buffer_byte_length(left));
    const void *pb = st.in(tensor_buffer_data(right), tensor_buffer_byte_length(right));
    void *py = st.out(tensor_buffer_data_mut(output), tensor_buffer_byte_length(output));
    if (st.failed()) return 0;
    if (inner == 0)  // every sum is empty: zeros
        return st.finish(k::fill_uniform(dtype, py, rows * cols, 0, 0, 0.0f, 0.0f, st.stream()))
                   ? 1 : 0;
    if (!gemm(GemmKind::kMatmul, dtype, pa, pb, nullptr, py, rows, inner, cols, st.stream(),
              error, capacity))
        return 0;
    return st.finish(hipSuccess) ? 1 : 0;
}

// tensor_ops.c:217-398
int linear(TensorDType dtype, Buf input, Buf weight, Buf bias, TensorBuffer *output,
           char *error, size_t capacity) {
    const char *type = dtype == TENSOR_DTYPE_F32 ? "F32" : "F16";
    if (on_device(input) || on_device(weight) || on_device(bias) || on_device(output)) {
        if (!device_of(input, dtype) || !device_of(weight, dtype) || !device_of(output, dtype) ||
            (bias != nullptr && !device_of(bias, dtype)) || tensor_buffer_rank(input) == 0 ||
            tensor_buffer_rank(weight) != 2 ||
            tensor_buffer_rank(output) != tensor_buffer_rank(input) ||
            (bias != nullptr && tensor_buffer_rank(bias) != 1)) {
            set_error(error, capacity, "device linear requires all operands on one device with "
                      "%s dtype and compatible ranks", type);
            return 0;
        }
        const size_t rank = tensor_buffer_rank(input);
        const uint64_t *is = tensor_buffer_shape(input), *ws = tensor_buffer_shape(weight);
        const uint64_t *os = tensor_buffer_shape(output);
        const size_t iw = is[rank - 1], ow = ws[0];
        if (iw == 0 || ow == 0 || ws[1] != iw || os[rank - 1] != ow ||
            (bias != nullptr && tensor_buffer_shape(bias)[0] != ow))
            return fail(error, capacity, "device linear dimensions do not match");
        for (size_t d = 0; d + 1 < rank; ++d)
            if (is[d] != os[d])
                return fail(error, capacity, "device linear leading dimensions do not match");
        const size_t rows = tensor_buffer_element_count(input) / iw;
        const TensorComputeBackend *backend = tensor_compute_preferred_backend();
        const bool slot = backend != nullptr &&
                          (dtype == TENSOR_DTYPE_F32 ? backend->linear_f32_device != nullptr
                                                     : backend->linear_f16_device != nullptr) &&
                          (bias == nullptr ||
                           (dtype == TENSOR_DTYPE_F32 ? backend->bias_add_f32_device != nullptr
                                                      : backend->bias_add_f16_device != nullptr));
        // the CUDA slot refuses empty and > INT_MAX dimensions
        if (!slot || rows == 0 || rows > INT_MAX || iw > INT_MAX || ow > INT_MAX ||
            !sdk_ready(nullptr, 0) ||
            !gemm(GemmKind::kLinear, dtype, handle(input), handle(weight), handle(bias),
                  tensor_buffer_device_handle_internal(output), rows, iw, ow, sdk_stream(),
                  nullptr, 0))
            return fail(error, capacity, "device linear backend operation failed");
        return 1;
    }
    if (!host_of(input, dtype) || !host_of(weight, dtype) || !host_of(output, dtype) ||
        tensor_buffer_rank(input) == 0 || tensor_buffer_rank(weight) != 2 ||
        tensor_buffer_rank(output) != tensor_buffer_rank(input) ||
        (bias != nullptr && (!host_of(bias, dtype) || tensor_buffer_rank(bias) != 1))) {
        set_error(error, capacity, "linear requires %s input, rank-2 weight, optional rank-1 "
                  "bias, and matching output rank", type);
        return 0;
    }
    const size_t rank = tensor_buffer_rank(input);
    const uint64_t *is = tensor_buffer_shape(input), *ws = tensor_buffer_shape(weight);
    const uint64_t *os = tensor_buffer_shape(output);
    const size_t iw = is[rank - 1], ow = ws[0];
    if (iw == 0 || ow == 0 || ws[1] != iw || os[rank - 1] != ow ||
        (bias != nullptr && tensor_buffer_shape(bias)[0] != ow))
        return fail(error, capacity,
                    "linear input, weight, bias, and output dimensions do not match");
    for (size_t d = 0; d + 1 < rank; ++d)
        if (is[d] != os[d])
            return fail(error, capacity, "linear output leading dimensions must match input");
    const size_t rows = tensor_buffer_element_count(input) / iw;
    if (rows == 0) return 1;
    Staging st("linear", true, error, capacity);
    if (!st.begin()) return 0;
    const void *px = st.in(tensor_buffer_data(input), tensor_buffer_byte_length(input));
    const void *pw = st.in(tensor_buffer_data(weight), tensor_buffer_byte_length(weight));
    const void *pb = bias ? st.in(tensor_buffer_data(bias), tensor_buffer_byte_length(bias))
                          : nullptr;
    void *py = st.out(tensor_buffer_data_mut(output), tensor_buffer_byte_length(output));
    if (st.failed()) return 0;
    if (!gemm(GemmKind::kLinear, dtype, px, pw, pb, py, rows, iw, ow, st.stream(), error,
              capacity))
        return 0;
    return st.finish(hipSuccess) ? 1 : 0;
}

// tensor_quant.c:102-141
int linear_quantized(bool q8, Buf input, Buf weight, TensorBuffer *output, char *error,
                     size_t capacity) {
    const size_t block_bytes = q8 ? 34 : 18;
    if (!device_of(input, TENSOR_DTYPE_F16) || !device_of(weight, TENSOR_DTYPE_U8) ||
        !device_of(output, TENSOR_DTYPE_F16) || tensor_buffer_rank(input) == 0 ||
        tensor_buffer_rank(weight) != 3 || tensor_buffer_rank(output) != tensor_buffer_rank(input))
        return fail(error, capacity, "quantized linear requires device-resident FP16 "
                    "input/output and packed U8 weights");
    const size_t rank = tensor_buffer_rank(input);
    const uint64_t *is = tensor_buffer_shape(input), *ws = tensor_buffer_shape(weight);
    const uint64_t *os = tensor_buffer_shape(output);
    const size_t iw = is[rank - 1], ow = ws[0];
    if (ws[1] != iw / 32 || iw % 32 || ws[2] != block_bytes || os[rank - 1] != ow)
        return fail(error, capacity, "quantized linear shapes are incompatible");
    for (size_t d = 0; d + 1 < rank; ++d)
        if (is[d] != os[d])
            return fail(error, capacity, "quantized linear leading dimensions do not match");
    const TensorComputeBackend *backend = tensor_compute_preferred_backend();
    int (*operation)(const void *, const void *, void *, size_t, size_t, size_t) = nullptr;
    if (backend)
        operation = q8 ? backend->linear_q8_0_f16_device : backend->linear_q4_0_f16_device;
    // an empty input width reaches the slot as a refusal (no rows to count)
    const size_t rows = iw == 0 ? 0 : tensor_buffer_element_count(input) / iw;
    if (operation == nullptr || handle(input) == nullptr || handle(weight) == nullptr ||
        handle(output) == nullptr ||
        !operation(handle(input), handle(weight), tensor_buffer_device_handle_internal(output),
                   rows, iw, ow))
        return fail(error, capacity, "quantized linear GPU kernel is unavailable");
    return 1;
}

}  // namespace

extern "C" {

int tensor_matmul_f32(Buf left, Buf right, TensorBuffer *output, char *error, size_t capacity) {
    return matmul(TENSOR_DTYPE_F32, left, right, output, error, capacity);
}
int tensor_matmul_f16(Buf left, Buf right, TensorBuffer *output, char *error, size_t capacity) {
    return matmul(TENSOR_DTYPE_F16, left, right, output, error, capacity);
}
int tensor_linear_f32(Buf input, Buf weight, Buf bias, TensorBuffer *output, char *error,
                      size_t capacity) {
    return linear(TENSOR_DTYPE_F32, input, weight, bias, output, error, capacity);
}
int tensor_linear_f16(Buf input, Buf weight, Buf bias, TensorBuffer *output, char *error,
                      size_t capacity) {
    return linear(TENSOR_DTYPE_F16, input, weight, bias, output, error, capacity);
}

// tensor_quant.c:48-100; the blocks are computed on the GPU and the packed
// tensor is returned host resident, as in the reference.
int tensor_quantize_linear_weight_f16(const uint16_t *weight, size_t output_width,
                                      size_t input_width, TensorWeightQuantization format,
                                      TensorBuffer **result, char *error, size_t capacity) {
    if (result) *result = nullptr;
    const size_t block_bytes = format == TENSOR_WEIGHT_Q8_0 ? 34
                               : format == TENSOR_WEIGHT_Q4_0 ? 18 : 0;
    const char *invalid =
        "quantized linear weight requires a valid format and input width divisible by 32";
    if (!weight || !result || !output_width || !input_width || input_width % 32 ||
        !block_bytes || output_width > SIZE_MAX / (input_width / 32) / block_bytes ||
        output_width > SIZE_MAX / input_width / sizeof(uint16_t))
        return fail(error, capacity, invalid);
    const uint64_t shape[3] = {output_width, input_width / 32, block_bytes};
    if (!tensor_buffer_create(TENSOR_DTYPE_U8, shape, 3, result, error, capacity)) return 0;
    uint32_t bad = 0;
    bool ok;
    {
        Staging st("quantize", true, error, capacity);
        ok = st.begin();
        if (ok) {
            const void *pw = st.in(weight, output_width * input_width * sizeof(uint16_t));
            void *pp = st.out(tensor_buffer_data_mut(*result), tensor_buffer_byte_length(*result));
            void *pf = st.inout(&bad, sizeof bad);
            ok = !st.failed() &&
                 st.finish(k::quantize_f16(format == TENSOR_WEIGHT_Q8_0,
                                           static_cast<const uint16_t *>(pw),
                                           static_cast<uint8_t *>(pp), static_cast<uint32_t *>(pf),
                                           output_width * (input_width / 32), st.stream()));
        }
    }
    if (ok && bad != 0) {
        ok = false;
        set_error(error, capacity, "quantized weights must contain only finite values");
    }
    if (!ok) {
        tensor_buffer_free(*result);
        *result = nullptr;
        return 0;
    }
    return 1;
}

int tensor_linear_q8_0_f16(Buf input, Buf packed_weight, TensorBuffer *output, char *error,
                           size_t capacity) {
    return linear_quantized(true, input, packed_weight, output, error, capacity);
}
int tensor_linear_q4_0_f16(Buf input, Buf packed_weight, TensorBuffer *output, char *error,
                           size_t capacity) {
    return linear_quantized(false, input, packed_weight, output, error, capacity);
}

}  // extern "C"
