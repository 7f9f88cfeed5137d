// The "hip" TensorComputeBackend and backend selection.
//
// Reference: include/tensor_compute_backend.h:49-130, the CUDA table
// src/platform/cuda/tensor_compute_cuda.cu:714-834 and the selector
// src/common/backend_dispatch.c:10-35.
//
// Host-pointer slots are synchronous: operands are staged through the device
// pool (reused across calls, released by release_cache), the kernel runs on
// the SDK stream and the outputs are copied back before the slot returns.
// The embedding slots keep their table uploaded per host address, as the
// CUDA backend does, until release_cache.
// *_device slots take raw device addresses and only enqueue. Argument checks
// mirror the CUDA wrappers (non-null pointers, nonzero sizes, no size_t
// overflow); a failed check returns 0.
#include "kernels.hpp"
#include "sdk.hpp"
#include "staging.hpp"

#include "tensor_compute_backend.h"
#include "tensor_device.h"

#include <cstdlib>
#include <cstring>

using namespace icsdk;

namespace {

bool product(size_t a, size_t b, size_t *out) {
    if (b != 0 && a > SIZE_MAX / b) return false;
    *out = a * b;
    return true;
}

template <typename T> bool count_ok(size_t n) { return n > 0 && n <= SIZE_MAX / sizeof(T); }

int hip_available(void) { return tensor_device_available(); }

template <typename T>
int host_unary(k::Unary op, const T *x, T *y, size_t n) {
    if (x == nullptr || y == nullptr || !count_ok<T>(n)) return 0;
    Staging st("hip backend", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *px = st.in(x, n * sizeof(T));
    void *py = st.out(y, n * sizeof(T));
    if (st.failed()) return 0;
    hipError_t status;
    if constexpr (sizeof(T) == 4)
        status = k::unary_f32(op, static_cast<const float *>(px), static_cast<float *>(py), n,
                              st.stream());
    else
        status = k::unary_f16(op, static_cast<const uint16_t *>(px), static_cast<uint16_t *>(py),
                              n, st.stream());
    return st.finish(status) ? 1 : 0;
}

template <typename T>
int host_binary(k::Binary op, const T *a, const T *b, T *y, size_t n) {
    if (a == nullptr || b == nullptr || y == nullptr || !count_ok<T>(n)) return 0;
    Staging st("hip backend", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *pa = st.in(a, n * sizeof(T));
    const void *pb = st.in(b, n * sizeof(T));
    void *py = st.out(y, n * sizeof(T));
    if (st.failed()) return 0;
    hipError_t status;
    if constexpr (sizeof(T) == 4)
        status = k::binary_f32(op, static_cast<const float *>(pa), static_cast<const float *>(pb),
                               static_cast<float *>(py), n, st.stream());
    else
        status = k::binary_f16(op, static_cast<const uint16_t *>(pa),
                               static_cast<const uint16_t *>(pb), static_cast<uint16_t *>(py), n,
                               st.stream());
    return st.finish(status) ? 1 : 0;
}

template <typename T>
int host_norm(const T *x, const T *scale, const T *bias, T *y, size_t rows, size_t width,
              float eps, bool layer) {
    size_t n;
    if (x == nullptr || scale == nullptr || y == nullptr || rows == 0 || width == 0 ||
        !product(rows, width, &n) || !count_ok<T>(n))
        return 0;
    Staging st("hip backend", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *px = st.in(x, n * sizeof(T));
    const void *ps = st.in(scale, width * sizeof(T));
    const void *pb = bias ? st.in(bias, width * sizeof(T)) : nullptr;
    void *py = st.out(y, n * sizeof(T));
    if (st.failed()) return 0;
    hipError_t status;
    if constexpr (sizeof(T) == 4) {
        auto *fx = static_cast<const float *>(px);
        auto *fs = static_cast<const float *>(ps);
        status = layer ? k::layer_norm_f32(fx, fs, static_cast<const float *>(pb),
                                           static_cast<float *>(py), rows, width, eps, st.stream())
                       : k::rms_norm_f32(fx, fs, static_cast<float *>(py), rows, width, eps,
                                         st.stream());
    } else {
        auto *hx = static_cast<const uint16_t *>(px);
        auto *hs = static_cast<const uint16_t *>(ps);
        status = layer ? k::layer_norm_f16(hx, hs, static_cast<const uint16_t *>(pb),
                                           static_cast<uint16_t *>(py), rows, width, eps,
                                           st.stream())
                       : k::rms_norm_f16(hx, nullptr, nullptr, hs, static_cast<uint16_t *>(py),
                                         rows, width, eps, st.stream());
    }
    return st.finish(status) ? 1 : 0;
}

template <typename T>
int host_bias(const T *x, const T *b, T *y, size_t rows, size_t width) {
    size_t n;
    if (x == nullptr || b == nullptr || y == nullptr || rows == 0 || width == 0 ||
        !product(rows, width, &n) || !count_ok<T>(n))
        return 0;
    Staging st("hip backend", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *px = st.in(x, n * sizeof(T));
    const void *pb = st.in(b, width * sizeof(T));
    void *py = st.out(y, n * sizeof(T));
    if (st.failed()) return 0;
    hipError_t status;
    if constexpr (sizeof(T) == 4)
        status = k::bias_add_f32(static_cast<const float *>(px), static_cast<const float *>(pb),
                                 static_cast<float *>(py), rows, width, false, st.stream());
    else
        status = k::bias_add_f16(static_cast<const uint16_t *>(px),
                                 static_cast<const uint16_t *>(pb), static_cast<uint16_t *>(py),
                                 rows, width, false, st.stream());
    return st.finish(status) ? 1 : 0;
}

template <typename T>
int host_rope(T *q, T *k, size_t seq, size_t qh, size_t kh, size_t dim, double theta,
              size_t offset) {
    size_t qn, kn;
    if (q == nullptr || k == nullptr || seq == 0 || qh == 0 || kh == 0 || dim == 0 ||
        dim % 2 != 0 || dim > 65536 || qh > (1u << 20) || kh > (1u << 20) ||
        !product(seq, qh * dim, &qn) || !product(seq, kh * dim, &kn) || !count_ok<T>(qn) ||
        !count_ok<T>(kn) || seq * (dim / 2) > 0xffffffffu)
        return 0;
    Staging st("hip backend", true, nullptr, 0);
    if (!st.begin()) return 0;
    void *pq = st.inout(q, qn * sizeof(T));
    void *pk = st.inout(k, kn * sizeof(T));
    if (st.failed()) return 0;
    const size_t table_bytes = k::rope_table_bytes(seq, qh, kh, dim, sizeof(T), pq, pk);
    ScratchBlock table(table_bytes);
    if (table_bytes != 0 && table.get() == nullptr) return 0;
    hipError_t status;
    if constexpr (sizeof(T) == 4)
        status = k::rope_f32(static_cast<float *>(pq), static_cast<float *>(pk), seq, qh, kh, dim,
                             theta, offset, table.get(), st.stream());
    else
        status = k::rope_f16(static_cast<uint16_t *>(pq), static_cast<uint16_t *>(pk), seq, qh,
                             kh, dim, theta, offset, table.get(), st.stream());
    return st.finish(status) ? 1 : 0;
}

template <typename T>
int host_argmax(const T *x, size_t n, uint32_t *result) {
    if (x == nullptr || result == nullptr || n == 0 || n > 0xffffffffu) return 0;
    Staging st("hip backend", true, nullptr, 0);
    if (!st.begin()) return 0;
    void *partials = grid_reduce_partials(nullptr, 0);
    if (partials == nullptr) return 0;
    const void *px = st.in(x, n * sizeof(T));
    void *pr = st.out(result, sizeof(uint32_t));
    if (st.failed()) return 0;
    hipError_t status;
    {
        std::lock_guard<std::mutex> lock(grid_reduce_mutex());
        if constexpr (sizeof(T) == 4)
            status = k::argmax_f32(static_cast<const float *>(px), n, static_cast<uint32_t *>(pr),
                                   partials, st.stream());
        else
            status = k::argmax_f16(static_cast<const uint16_t *>(px), n,
                                   static_cast<uint32_t *>(pr), partials, st.stream());
    }
    return st.finish(status) ? 1 : 0;
}

// ---- slot functions --------------------------------------------------------

int rms16(const uint16_t *x, const uint16_t *s, uint16_t *y, size_t r, size_t w, float e) {
    return host_norm(x, s, (const uint16_t *)nullptr, y, r, w, e, false);
}
int layer16(const uint16_t *x, const uint16_t *s, const uint16_t *b, uint16_t *y, size_t r,
            size_t w, float e) {
    return host_norm(x, s, b, y, r, w, e, true);
}
int rms32(const float *x, const float *s, float *y, size_t r, size_t w, float e) {
    return host_norm(x, s, (const float *)nullptr, y, r, w, e, false);
}
int layer32(const float *x, const float *s, const float *b, float *y, size_t r, size_t w,
            float e) {
    return host_norm(x, s, b, y, r, w, e, true);
}
int bias16(const uint16_t *x, const uint16_t *b, uint16_t *y, size_t r, size_t w) {
    return host_bias(x, b, y, r, w);
}
int bias32(const float *x, const float *b, float *y, size_t r, size_t w) {
    return host_bias(x, b, y, r, w);
}
int gelu16(const uint16_t *x, uint16_t *y, size_t n) { return host_unary(k::Unary::Gelu, x, y, n); }
int gelu32(const float *x, float *y, size_t n) { return host_unary(k::Unary::Gelu, x, y, n); }
int relu16(const uint16_t *x, uint16_t *y, size_t n) { return host_unary(k::Unary::Relu, x, y, n); }
int gelu_mul16(const uint16_t *x, const uint16_t *g, uint16_t *y, size_t n) {
    return host_binary(k::Binary::GeluMul, x, g, y, n);
}
int silu_mul16(const uint16_t *g, const uint16_t *u, uint16_t *y, size_t n) {
    return host_binary(k::Binary::SiluMul, g, u, y, n);
}
int silu_mul32(const float *g, const float *u, float *y, size_t n) {
    return host_binary(k::Binary::SiluMul, g, u, y, n);
}
int residual16(const uint16_t *a, const uint16_t *b, uint16_t *y, size_t n) {
    return host_binary(k::Binary::Add, a, b, y, n);
}
int residual32(const float *a, const float *b, float *y, size_t n) {
    return host_binary(k::Binary::Add, a, b, y, n);
}
int rope16(uint16_t *q, uint16_t *k, size_t s, size_t qh, size_t kh, size_t d, double t,
           size_t p) {
    return host_rope(q, k, s, qh, kh, d, t, p);
}
int rope32(float *q, float *k, size_t s, size_t qh, size_t kh, size_t d, double t) {
    return host_rope(q, k, s, qh, kh, d, t, 0);
}
int argmax16(const uint16_t *x, size_t n, uint32_t *r) { return host_argmax(x, n, r); }
int argmax32(const float *x, size_t n, uint32_t *r) { return host_argmax(x, n, r); }

// Compute-table embedding slots (CUDA: tensor_compute_cuda.cu:484-495): the
// table is uploaded once per host address (weight cache), the ids and the
// output are staged; an id at or past table_rows gives a zero row.
template <typename T>
int host_embedding(const T *table, const uint32_t *ids, T *out, size_t rows, size_t width,
                   size_t table_rows) {
    size_t n, table_n;
    if (table == nullptr || ids == nullptr || out == nullptr || rows == 0 || width == 0 ||
        table_rows == 0 || !product(rows, width, &n) || !product(table_rows, width, &table_n) ||
        !count_ok<T>(n) || !count_ok<T>(table_n) || !count_ok<uint32_t>(rows))
        return 0;
    Staging st("hip backend", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *device_table = weight_cache_get(table, table_n * sizeof(T));
    if (device_table == nullptr) return 0;
    const void *pi = st.in(ids, rows * sizeof(uint32_t));
    void *po = st.out(out, n * sizeof(T));
    if (st.failed()) return 0;
    return st.finish(k::embedding_gather(TENSOR_DTYPE_U32, device_table, table_rows,
                                         width * sizeof(T), sizeof(T), pi, rows, po,
                                         st.stream()))
               ? 1
               : 0;
}
int embedding16(const uint16_t *t, const uint32_t *ids, uint16_t *o, size_t r, size_t w,
                size_t tr) {
    return host_embedding(t, ids, o, r, w, tr);
}
int embedding32(const float *t, const uint32_t *ids, float *o, size_t r, size_t w, size_t tr) {
    return host_embedding(t, ids, o, r, w, tr);
}

void release_cache(void) {
    scratch_clear();
    weight_cache_clear();
}

// Device-resident slots: raw device addresses, enqueue only.
int bias32_device(const void *x, const void *b, void *y, size_t rows, size_t width) {
    size_t n;
    if (x == nullptr || b == nullptr || y == nullptr || rows == 0 || width == 0 ||
        !product(rows, width, &n) || !sdk_ready(nullptr, 0))
        return 0;
    return k::bias_add_f32(static_cast<const float *>(x), static_cast<const float *>(b),
                           static_cast<float *>(y), rows, width, false, sdk_stream()) == hipSuccess;
}
int bias16_device(const void *x, const void *b, void *y, size_t rows, size_t width) {
    size_t n;
    if (x == nullptr || b == nullptr || y == nullptr || rows == 0 || width == 0 ||
        !product(rows, width, &n) || !sdk_ready(nullptr, 0))
        return 0;
    return k::bias_add_f16(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(b),
                           static_cast<uint16_t *>(y), rows, width, false,
                           sdk_stream()) == hipSuccess;
}
int residual16_device(const void *a, const void *b, void *y, size_t n) {
    if (a == nullptr || b == nullptr || y == nullptr || n == 0 || !sdk_ready(nullptr, 0)) return 0;
    return k::binary_f16(k::Binary::Add, static_cast<const uint16_t *>(a),
                         static_cast<const uint16_t *>(b), static_cast<uint16_t *>(y), n,
                         sdk_stream()) == hipSuccess;
}

int unavailable(void) { return 0; }

}  // namespace

extern "C" const TensorComputeBackend *tensor_compute_hip_backend(void) {
    static const TensorComputeBackend backend = [] {
        TensorComputeBackend b;
        std::memset(&b, 0, sizeof b);
        b.name = "hip";
        b.is_available = hip_available;
        b.rms_norm_f16 = rms16;
        b.layer_norm_f16 = layer16;
        b.bias_add_f16 = bias16;
        b.gelu_f16 = gelu16;
        b.gelu_multiply_f16 = gelu_mul16;
        b.relu_f16 = relu16;
        b.rope_f16 = rope16;
        b.silu_multiply_f16 = silu_mul16;
        b.residual_add_f16 = residual16;
        b.argmax_f16 = argmax16;
        b.embedding_f16 = embedding16;
        b.rms_norm_f32 = rms32;
        b.layer_norm_f32 = layer32;
        b.bias_add_f32 = bias32;
        b.gelu_f32 = gelu32;
        b.rope_f32 = rope32;
        b.silu_multiply_f32 = silu_mul32;
        b.residual_add_f32 = residual32;
        b.argmax_f32 = argmax32;
        b.embedding_f32 = embedding32;
        b.release_cache = release_cache;
        b.bias_add_f32_device = bias32_device;
        b.bias_add_f16_device = bias16_device;
        b.residual_add_f16_device = residual16_device;
        return b;
    }();
    return &backend;
}

// reference src/platform/cuda/tensor_compute_cuda_stub.c:7-12 and the Metal stub
extern "C" const TensorComputeBackend *tensor_compute_cuda_backend(void) {
    static const TensorComputeBackend backend = [] {
        TensorComputeBackend b;
        std::memset(&b, 0, sizeof b);
        b.name = "cuda";
        b.is_available = unavailable;
        return b;
    }();
    return &backend;
}

extern "C" const TensorComputeBackend *tensor_compute_metal_backend(void) {
    static const TensorComputeBackend backend = [] {
        TensorComputeBackend b;
        std::memset(&b, 0, sizeof b);
        b.name = "metal";
        b.is_available = unavailable;
        return b;
    }();
    return &backend;
}

// TENSOR_BACKEND is read on every call, as in the reference: unset, empty,
// "auto" or "hip" select the HIP table when a device is present; "cuda",
// "metal", "qnn" and any other value select nothing in a HIP build.
extern "C" const TensorComputeBackend *tensor_compute_preferred_backend(void) {
    const char *requested = std::getenv("TENSOR_BACKEND");
    if (requested == nullptr || requested[0] == '\0' || std::strcmp(requested, "auto") == 0 ||
        std::strcmp(requested, "hip") == 0) {
        const TensorComputeBackend *hip = tensor_compute_hip_backend();
        return hip->is_available() ? hip : nullptr;
    }
    return nullptr;
}
