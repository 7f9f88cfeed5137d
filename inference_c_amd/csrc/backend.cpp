// The "hip" TensorComputeBackend and backend selection.
//
// Reference: include/tensor_compute_backend.h:49-130, the CUDA table
// src/platform/cuda/tensor_compute_cuda.cu:714-834 and the selector
// src/common/backend_dispatch.c:10-35.
//
// Host-pointer slots are synchronous: operands are staged through the device
// pool (reused across calls, released by release_cache), the kernel runs on
// the SDK stream and the outputs are copied back before the slot returns.
// The embedding, linear and quantized-linear slots keep their table / weight
// uploaded per host address, as the CUDA backend does, until release_cache.
// *_device slots take raw device addresses and only enqueue. Argument checks
// mirror the CUDA wrappers (non-null pointers, nonzero sizes, no size_t
// overflow); a failed check returns 0.
#include "gemm.hpp"
#include "kernels.hpp"
#include "pinned.hpp"
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
                                         width * sizeof(T), sizeof(T), pi, rows, po, nullptr,
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

// ---- GEMM-adjacent slots ----------------------------------------------------
// CUDA: linear / linear_resident (tensor_compute_cuda.cu:174-214, :399-427),
// quantized linear (:216-265, :695-713), rms_norm_linear_f32, mlp_f16 and
// qkv_f16 (:769-786). Dimensions above INT_MAX are refused as cuBLAS does.

template <typename T> constexpr TensorDType dtype_of() {
    return sizeof(T) == 4 ? TENSOR_DTYPE_F32 : TENSOR_DTYPE_F16;
}

bool linear_dims_ok(size_t rows, size_t in, size_t out, size_t elem) {
    constexpr size_t kIntMax = 2147483647;
    size_t a, b, c;
    return rows != 0 && in != 0 && out != 0 && rows <= kIntMax && in <= kIntMax &&
           out <= kIntMax && product(rows, in, &a) && product(out, in, &b) &&
           product(rows, out, &c) && a <= SIZE_MAX / elem && b <= SIZE_MAX / elem &&
           c <= SIZE_MAX / elem;
}

// y[rows][out] = x[rows][in] w[out][in]^T: host pointers, w cached per address
template <typename T>
int host_linear(const T *x, const T *w, T *y, size_t rows, size_t in, size_t out) {
    if (x == nullptr || w == nullptr || y == nullptr || !linear_dims_ok(rows, in, out, sizeof(T)))
        return 0;
    Staging st("hip linear", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *dw = weight_cache_get(w, out * in * sizeof(T));
    if (dw == nullptr) return 0;
    const void *px = st.in(x, rows * in * sizeof(T));
    void *py = st.out(y, rows * out * sizeof(T));
    if (st.failed() ||
        !gemm(GemmKind::kLinear, dtype_of<T>(), px, dw, nullptr, py, rows, in, out, st.stream(),
              nullptr, 0))
        return 0;
    return st.finish(hipSuccess) ? 1 : 0;
}
int linear32(const float *x, const float *w, float *y, size_t r, size_t i, size_t o) {
    return host_linear(x, w, y, r, i, o);
}
int linear16(const uint16_t *x, const uint16_t *w, uint16_t *y, size_t r, size_t i, size_t o) {
    return host_linear(x, w, y, r, i, o);
}

template <typename T>
int device_linear(const void *x, const void *w, void *y, size_t rows, size_t in, size_t out) {
    if (x == nullptr || w == nullptr || y == nullptr || !linear_dims_ok(rows, in, out, sizeof(T)) ||
        !sdk_ready(nullptr, 0))
        return 0;
    return gemm(GemmKind::kLinear, dtype_of<T>(), x, w, nullptr, y, rows, in, out, sdk_stream(),
                nullptr, 0) ? 1 : 0;
}
int linear32_device(const void *x, const void *w, void *y, size_t r, size_t i, size_t o) {
    return device_linear<float>(x, w, y, r, i, o);
}
int linear16_device(const void *x, const void *w, void *y, size_t r, size_t i, size_t o) {
    return device_linear<uint16_t>(x, w, y, r, i, o);
}

bool quant_dims_ok(bool q8, size_t rows, size_t in, size_t out) {
    size_t a, b;
    return rows != 0 && in != 0 && out != 0 && in % 32 == 0 && product(rows, in, &a) &&
           product(rows, out, &b) && a <= SIZE_MAX / 2 && b <= SIZE_MAX / 2 &&
           out <= SIZE_MAX / (in / 32) / (q8 ? 34u : 18u);
}

hipError_t quant_launch(bool q8, const void *x, const void *w, void *y, size_t rows, size_t in,
                        size_t out, hipStream_t s) {
    auto *hx = static_cast<const uint16_t *>(x);
    auto *pw = static_cast<const uint8_t *>(w);
    auto *hy = static_cast<uint16_t *>(y);
    return q8 ? k::linear_q8_0_f16(hx, pw, hy, rows, in, out, s)
              : k::linear_q4_0_f16(hx, pw, hy, rows, in, out, s);
}

int quant_device(bool q8, const void *x, const void *w, void *y, size_t rows, size_t in,
                 size_t out) {
    if (x == nullptr || w == nullptr || y == nullptr || !quant_dims_ok(q8, rows, in, out) ||
        !sdk_ready(nullptr, 0))
        return 0;
    return quant_launch(q8, x, w, y, rows, in, out, sdk_stream()) == hipSuccess;
}
int q8_device(const void *x, const void *w, void *y, size_t r, size_t i, size_t o) {
    return quant_device(true, x, w, y, r, i, o);
}
int q4_device(const void *x, const void *w, void *y, size_t r, size_t i, size_t o) {
    return quant_device(false, x, w, y, r, i, o);
}

int quant_host(bool q8, const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
               size_t in, size_t out) {
    if (x == nullptr || w == nullptr || y == nullptr || !quant_dims_ok(q8, rows, in, out))
        return 0;
    Staging st("hip quantized linear", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *dw = weight_cache_get(w, out * (in / 32) * (q8 ? 34u : 18u));
    if (dw == nullptr) return 0;
    const void *px = st.in(x, rows * in * sizeof(uint16_t));
    void *py = st.out(y, rows * out * sizeof(uint16_t));
    if (st.failed()) return 0;
    return st.finish(quant_launch(q8, px, dw, py, rows, in, out, st.stream())) ? 1 : 0;
}
int q8_host(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t r, size_t i, size_t o) {
    return quant_host(true, x, w, y, r, i, o);
}
int q4_host(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t r, size_t i, size_t o) {
    return quant_host(false, x, w, y, r, i, o);
}

// norm = RMSNorm(x) * scale, y = norm w^T; both outputs written back
int rms_linear32(const float *x, const float *scale, float *norm, const float *w, float *y,
                 size_t rows, size_t in, size_t out, float eps) {
    if (x == nullptr || scale == nullptr || norm == nullptr || w == nullptr || y == nullptr ||
        !linear_dims_ok(rows, in, out, sizeof(float)))
        return 0;
    Staging st("hip rms_norm_linear", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *dw = weight_cache_get(w, out * in * sizeof(float));
    if (dw == nullptr) return 0;
    const void *px = st.in(x, rows * in * sizeof(float));
    const void *ps = st.in(scale, in * sizeof(float));
    void *pn = st.out(norm, rows * in * sizeof(float));
    void *py = st.out(y, rows * out * sizeof(float));
    if (st.failed()) return 0;
    const hipError_t status =
        k::rms_norm_f32(static_cast<const float *>(px), static_cast<const float *>(ps),
                        static_cast<float *>(pn), rows, in, eps, st.stream());
    if (status != hipSuccess ||
        !gemm(GemmKind::kLinear, TENSOR_DTYPE_F32, pn, dw, nullptr, py, rows, in, out,
              st.stream(), nullptr, 0))
        return 0;
    return st.finish(hipSuccess) ? 1 : 0;
}

// y = (gelu(x w1^T + b1)) w2^T + b2 (CUDA: linear, bias+GELU, linear, bias)
int mlp16(const uint16_t *x, const uint16_t *w1, const uint16_t *b1, const uint16_t *w2,
          const uint16_t *b2, uint16_t *y, size_t rows, size_t in, size_t mid, size_t out) {
    if (x == nullptr || w1 == nullptr || b1 == nullptr || w2 == nullptr || b2 == nullptr ||
        y == nullptr || !linear_dims_ok(rows, in, mid, 2) || !linear_dims_ok(rows, mid, out, 2))
        return 0;
    Staging st("hip mlp", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *dw1 = weight_cache_get(w1, mid * in * 2);
    const void *dw2 = weight_cache_get(w2, out * mid * 2);
    if (dw1 == nullptr || dw2 == nullptr) return 0;
    const void *px = st.in(x, rows * in * 2);
    const void *pb1 = st.in(b1, mid * 2);
    const void *pb2 = st.in(b2, out * 2);
    void *py = st.out(y, rows * out * 2);
    ScratchBlock raw(rows * mid * 2), act(rows * mid * 2);
    if (st.failed() || raw.get() == nullptr || act.get() == nullptr) return 0;
    auto *hraw = static_cast<uint16_t *>(raw.get());
    auto *hact = static_cast<uint16_t *>(act.get());
    if (!gemm(GemmKind::kLinear, TENSOR_DTYPE_F16, px, dw1, nullptr, hraw, rows, in, mid,
              st.stream(), nullptr, 0) ||
        k::bias_add_f16(hraw, static_cast<const uint16_t *>(pb1), hact, rows, mid, true,
                        st.stream()) != hipSuccess ||
        !gemm(GemmKind::kLinear, TENSOR_DTYPE_F16, hact, dw2, pb2, py, rows, mid, out,
              st.stream(), nullptr, 0))
        return 0;
    return st.finish(hipSuccess) ? 1 : 0;
}

// q/k/v = x w^T (+ bias); biases optional
int qkv16(const uint16_t *x, const uint16_t *wq, const uint16_t *wk, const uint16_t *wv,
          const uint16_t *bq, const uint16_t *bk, const uint16_t *bv, uint16_t *q, uint16_t *k,
          uint16_t *v, size_t rows, size_t in, size_t out) {
    if (x == nullptr || wq == nullptr || wk == nullptr || wv == nullptr || q == nullptr ||
        k == nullptr || v == nullptr || !linear_dims_ok(rows, in, out, 2))
        return 0;
    Staging st("hip qkv", true, nullptr, 0);
    if (!st.begin()) return 0;
    const uint16_t *weights[3] = {wq, wk, wv};
    const uint16_t *biases[3] = {bq, bk, bv};
    uint16_t *outs[3] = {q, k, v};
    const void *px = st.in(x, rows * in * 2);
    for (int i = 0; i < 3; ++i) {
        const void *dw = weight_cache_get(weights[i], out * in * 2);
        const void *pb = biases[i] ? st.in(biases[i], out * 2) : nullptr;
        void *py = st.out(outs[i], rows * out * 2);
        if (dw == nullptr || st.failed() ||
            !gemm(GemmKind::kLinear, TENSOR_DTYPE_F16, px, dw, pb, py, rows, in, out,
                  st.stream(), nullptr, 0))
            return 0;
    }
    return st.finish(hipSuccess) ? 1 : 0;
}

void release_cache(void) {
    scratch_clear();
    weight_cache_clear();
    gemm_release();
    pinned_release();
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
        b.linear_f32 = linear32;
        b.linear_f16 = linear16;
        b.linear_f32_device = linear32_device;
        b.linear_f16_device = linear16_device;
        b.linear_q8_0_f16_device = q8_device;
        b.linear_q4_0_f16_device = q4_device;
        b.linear_q8_0_f16 = q8_host;
        b.linear_q4_0_f16 = q4_host;
        b.rms_norm_linear_f32 = rms_linear32;
        b.mlp_f16 = mlp16;
        b.qkv_f16 = qkv16;
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
