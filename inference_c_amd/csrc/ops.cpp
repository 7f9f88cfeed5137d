// Public tensor operations (include/tensor_ops.h, include/tensor_ops_ext.h,
// tensor_buffer_convert).
//
// Each entry point validates its operands first (dtype, shape, one storage
// kind), with the reference's messages where the reference has the op
// (src/common/tensor_ops.c), then binds the operands -- device tensors in
// place, host tensors staged through device memory -- and enqueues the
// kernel on the SDK stream. Device calls return after the launch; host calls
// return once the host output is written. There is no host arithmetic path:
// without a HIP device every compute call fails with a message.
#include "kernels.hpp"
#include "sdk.hpp"
#include "staging.hpp"

#include "tensor_buffer.h"
#include "tensor_compute_backend.h"
#include "tensor_ops.h"
#include "tensor_ops_ext.h"

#include <cmath>
#include <cstring>
#include <initializer_list>
#include <mutex>

using namespace icsdk;

namespace {

using Buf = const TensorBuffer *;

bool same_shape(Buf a, Buf b) {
    if (tensor_buffer_rank(a) != tensor_buffer_rank(b)) return false;
    for (size_t d = 0; d < tensor_buffer_rank(a); ++d)
        if (tensor_buffer_shape(a)[d] != tensor_buffer_shape(b)[d]) return false;
    return true;
}

bool is(Buf t, TensorDType dtype) { return t != nullptr && tensor_buffer_dtype(t) == dtype; }

// True when every non-null operand has the same storage; *host receives it.
bool common_storage(std::initializer_list<Buf> operands, bool *host) {
    bool seen = false, first_host = true;
    for (Buf t : operands) {
        if (t == nullptr) continue;
        const bool h = tensor_buffer_storage(t) == TENSOR_BUFFER_STORAGE_HOST;
        if (!seen) {
            first_host = h;
            seen = true;
        } else if (h != first_host) {
            return false;
        }
    }
    *host = first_host;
    return true;
}

size_t last_dim(Buf t) {
    const size_t rank = tensor_buffer_rank(t);
    return rank == 0 ? 1 : (size_t)tensor_buffer_shape(t)[rank - 1];
}

const void *src(Staging &st, Buf t) {
    if (t == nullptr) return nullptr;
    return st.host() ? st.in(tensor_buffer_data(t), tensor_buffer_byte_length(t))
                     : tensor_buffer_device_handle_internal(t);
}

void *dst(Staging &st, TensorBuffer *t) {
    if (t == nullptr) return nullptr;
    return st.host() ? st.out(tensor_buffer_data_mut(t), tensor_buffer_byte_length(t))
                     : tensor_buffer_device_handle_internal(t);
}

void *srcdst(Staging &st, TensorBuffer *t) {
    if (t == nullptr) return nullptr;
    return st.host() ? st.inout(tensor_buffer_data_mut(t), tensor_buffer_byte_length(t))
                     : tensor_buffer_device_handle_internal(t);
}

int storage_error(const char *op, char *error, size_t capacity) {
    set_error(error, capacity, "%s operands must use the same storage type", op);
    return 0;
}

template <typename T> const T *as(const void *p) { return static_cast<const T *>(p); }
template <typename T> T *as(void *p) { return static_cast<T *>(p); }

// ---- elementwise drivers -------------------------------------------------

int unary(const char *op, const char *message, TensorDType dtype, k::Unary kind, Buf x,
          TensorBuffer *y, char *error, size_t capacity) {
    if (!is(x, dtype) || !is(y, dtype) || !same_shape(x, y)) {
        set_error(error, capacity, "%s", message);
        return 0;
    }
    bool host;
    if (!common_storage({x, y}, &host)) return storage_error(op, error, capacity);
    const size_t n = tensor_buffer_element_count(x);
    if (n == 0) return 1;
    Staging st(op, host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    const hipError_t status =
        dtype == TENSOR_DTYPE_F32
            ? k::unary_f32(kind, as<float>(px), as<float>(py), n, st.stream())
            : k::unary_f16(kind, as<uint16_t>(px), as<uint16_t>(py), n, st.stream());
    return st.finish(status) ? 1 : 0;
}

int binary(const char *op, const char *message, TensorDType dtype, k::Binary kind, Buf a,
           Buf b, TensorBuffer *y, char *error, size_t capacity) {
    if (!is(a, dtype) || !is(b, dtype) || !is(y, dtype) || !same_shape(a, b) ||
        !same_shape(a, y)) {
        set_error(error, capacity, "%s", message);
        return 0;
    }
    bool host;
    if (!common_storage({a, b, y}, &host)) return storage_error(op, error, capacity);
    const size_t n = tensor_buffer_element_count(a);
    if (n == 0) return 1;
    Staging st(op, host, error, capacity);
    if (!st.begin()) return 0;
    const void *pa = src(st, a);
    const void *pb = src(st, b);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    const hipError_t status =
        dtype == TENSOR_DTYPE_F32
            ? k::binary_f32(kind, as<float>(pa), as<float>(pb), as<float>(py), n, st.stream())
            : k::binary_f16(kind, as<uint16_t>(pa), as<uint16_t>(pb), as<uint16_t>(py), n,
                            st.stream());
    return st.finish(status) ? 1 : 0;
}

int bias(const char *op, TensorDType dtype, bool gelu, Buf x, Buf b, TensorBuffer *y,
         char *error, size_t capacity) {
    if (!is(x, dtype) || !is(b, dtype) || !is(y, dtype) || tensor_buffer_rank(x) == 0 ||
        tensor_buffer_rank(b) != 1 || !same_shape(x, y) ||
        tensor_buffer_shape(b)[0] != last_dim(x) || last_dim(x) == 0) {
        set_error(error, capacity,
                  "%s requires an input of rank >= 1, a rank-1 bias matching its last "
                  "dimension, and a same-shaped output of one dtype", op);
        return 0;
    }
    bool host;
    if (!common_storage({x, b, y}, &host)) return storage_error(op, error, capacity);
    const size_t width = last_dim(x);
    const size_t rows = tensor_buffer_element_count(x) / width;
    if (rows == 0) return 1;
    Staging st(op, host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    const void *pb = src(st, b);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    const hipError_t status =
        dtype == TENSOR_DTYPE_F32
            ? k::bias_add_f32(as<float>(px), as<float>(pb), as<float>(py), rows, width, gelu,
                              st.stream())
            : k::bias_add_f16(as<uint16_t>(px), as<uint16_t>(pb), as<uint16_t>(py), rows,
                              width, gelu, st.stream());
    return st.finish(status) ? 1 : 0;
}

// ---- normalisation drivers --------------------------------------------------

int rms(TensorDType dtype, Buf x, Buf w, float eps, TensorBuffer *y, char *error,
        size_t capacity) {
    const bool f32 = dtype == TENSOR_DTYPE_F32;
    if (!is(x, dtype) || !is(w, dtype) || !is(y, dtype) || tensor_buffer_rank(x) == 0 ||
        tensor_buffer_rank(w) != 1 || !same_shape(x, y) || !std::isfinite(eps) || eps < 0.0f) {
        set_error(error, capacity, f32
                  ? "RMSNorm requires compatible F32 tensors and nonnegative epsilon"
                  : "RMSNorm requires compatible F16 tensors and nonnegative epsilon");
        return 0;
    }
    const size_t width = last_dim(x);
    if (width == 0 || tensor_buffer_shape(w)[0] != width) {
        set_error(error, capacity, "RMSNorm weight width does not match input");
        return 0;
    }
    bool host;
    if (!common_storage({x, w, y}, &host)) return storage_error("RMSNorm", error, capacity);
    const size_t rows = tensor_buffer_element_count(x) / width;
    if (rows == 0) return 1;
    Staging st("RMSNorm", host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    const void *pw = src(st, w);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    const hipError_t status =
        f32 ? k::rms_norm_f32(as<float>(px), as<float>(pw), as<float>(py), rows, width, eps,
                              st.stream())
            : k::rms_norm_f16(as<uint16_t>(px), nullptr, nullptr, as<uint16_t>(pw),
                              as<uint16_t>(py), rows, width, eps, st.stream());
    return st.finish(status) ? 1 : 0;
}

int layer(TensorDType dtype, Buf x, Buf scale, Buf bias_t, float eps, TensorBuffer *y,
          char *error, size_t capacity) {
    const bool f32 = dtype == TENSOR_DTYPE_F32;
    if (!is(x, dtype) || !is(y, dtype) || tensor_buffer_rank(x) == 0 || !same_shape(x, y) ||
        !std::isfinite(eps) || eps < 0.0f ||
        (scale != nullptr && (!is(scale, dtype) || tensor_buffer_rank(scale) != 1)) ||
        (bias_t != nullptr && (!is(bias_t, dtype) || tensor_buffer_rank(bias_t) != 1))) {
        set_error(error, capacity, f32
                  ? "LayerNorm requires compatible F32 tensors and nonnegative epsilon"
                  : "LayerNorm requires compatible F16 tensors and nonnegative epsilon");
        return 0;
    }
    const size_t width = last_dim(x);
    if (width == 0 || (scale != nullptr && tensor_buffer_shape(scale)[0] != width) ||
        (bias_t != nullptr && tensor_buffer_shape(bias_t)[0] != width)) {
        set_error(error, capacity, "LayerNorm affine parameter width does not match input");
        return 0;
    }
    bool host;
    if (!common_storage({x, scale, bias_t, y}, &host))
        return storage_error("LayerNorm", error, capacity);
    const size_t rows = tensor_buffer_element_count(x) / width;
    if (rows == 0) return 1;
    Staging st("LayerNorm", host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    const void *ps = src(st, scale);
    const void *pb = src(st, bias_t);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    const hipError_t status =
        f32 ? k::layer_norm_f32(as<float>(px), as<float>(ps), as<float>(pb), as<float>(py),
                                rows, width, eps, st.stream())
            : k::layer_norm_f16(as<uint16_t>(px), as<uint16_t>(ps), as<uint16_t>(pb),
                                as<uint16_t>(py), rows, width, eps, st.stream());
    return st.finish(status) ? 1 : 0;
}

int softmax(TensorDType dtype, Buf x, int causal, TensorBuffer *y, char *error,
            size_t capacity) {
    const size_t rank = tensor_buffer_rank(x);
    if (!is(x, dtype) || !is(y, dtype) || !same_shape(x, y) || rank == 0 ||
        (causal != 0 && causal != 1) || (causal && rank < 2)) {
        set_error(error, capacity,
                  "softmax requires same-shaped %s tensors of rank >= 1 (rank >= 2 and "
                  "causal 0 or 1 for the causal form)",
                  dtype == TENSOR_DTYPE_F32 ? "F32" : "F16");
        return 0;
    }
    bool host;
    if (!common_storage({x, y}, &host)) return storage_error("softmax", error, capacity);
    const size_t width = last_dim(x);
    if (width == 0 || tensor_buffer_element_count(x) == 0) return 1;
    const size_t rows = tensor_buffer_element_count(x) / width;
    const size_t q_len = causal ? (size_t)tensor_buffer_shape(x)[rank - 2] : 0;
    Staging st("softmax", host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    const hipError_t status =
        dtype == TENSOR_DTYPE_F32
            ? k::softmax_f32(as<float>(px), as<float>(py), rows, width, q_len, st.stream())
            : k::softmax_f16(as<uint16_t>(px), as<uint16_t>(py), rows, width, q_len,
                             st.stream());
    return st.finish(status) ? 1 : 0;
}

int row_reduce(const char *op, TensorDType dtype, bool max, Buf x, TensorBuffer *y,
               char *error, size_t capacity) {
    const size_t rank = tensor_buffer_rank(x);
    const size_t width = last_dim(x);
    const size_t rows = width == 0 ? 0 : tensor_buffer_element_count(x) / width;
    if (!is(x, dtype) || !is(y, TENSOR_DTYPE_F32) || rank == 0 || width == 0 ||
        tensor_buffer_element_count(y) != (rows == 0 ? 0 : rows)) {
        set_error(error, capacity,
                  "%s requires a %s input of rank >= 1 with a nonzero last dimension and an "
                  "F32 output with one element per row", op,
                  dtype == TENSOR_DTYPE_F32 ? "F32" : "F16");
        return 0;
    }
    bool host;
    if (!common_storage({x, y}, &host)) return storage_error(op, error, capacity);
    if (rows == 0) return 1;
    Staging st(op, host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    hipError_t status;
    if (dtype == TENSOR_DTYPE_F32)
        status = max ? k::row_max_f32(as<float>(px), as<float>(py), rows, width, st.stream())
                     : k::row_sum_f32(as<float>(px), as<float>(py), rows, width, st.stream());
    else
        status = max ? k::row_max_f16(as<uint16_t>(px), as<float>(py), rows, width, st.stream())
                     : k::row_sum_f16(as<uint16_t>(px), as<float>(py), rows, width, st.stream());
    return st.finish(status) ? 1 : 0;
}

int argmax(TensorDType dtype, Buf x, TensorBuffer *index, char *error, size_t capacity) {
    const size_t n = tensor_buffer_element_count(x);
    if (!is(x, dtype) || !is(index, TENSOR_DTYPE_U32) ||
        tensor_buffer_element_count(index) != 1 || n == 0 || n > 0xffffffffu) {
        set_error(error, capacity,
                  "argmax requires a non-empty %s input of at most 2^32-1 elements and a "
                  "one-element U32 output", dtype == TENSOR_DTYPE_F32 ? "F32" : "F16");
        return 0;
    }
    bool host;
    if (!common_storage({x, index}, &host)) return storage_error("argmax", error, capacity);
    Staging st("argmax", host, error, capacity);
    if (!st.begin()) return 0;
    void *partials = grid_reduce_partials(error, capacity);
    if (partials == nullptr) return 0;
    const void *px = src(st, x);
    void *pi = dst(st, index);
    if (st.failed()) return 0;
    hipError_t status;
    {
        std::lock_guard<std::mutex> lock(grid_reduce_mutex());
        status = dtype == TENSOR_DTYPE_F32
                     ? k::argmax_f32(as<float>(px), n, as<uint32_t>(pi), partials, st.stream())
                     : k::argmax_f16(as<uint16_t>(px), n, as<uint32_t>(pi), partials,
                                     st.stream());
    }
    return st.finish(status) ? 1 : 0;
}

int rope(TensorDType dtype, TensorBuffer *q, TensorBuffer *k, size_t qh, size_t kh,
         size_t dim, double theta, size_t offset, char *error, size_t capacity) {
    const size_t qn = tensor_buffer_element_count(q), kn = tensor_buffer_element_count(k);
    const bool shape_ok = qh > 0 && kh > 0 && dim > 0 && dim % 2 == 0 && dim <= 65536 &&
                          qh <= (1u << 20) && kh <= (1u << 20) && qn % (qh * dim) == 0 &&
                          kn == qn / (qh * dim) * kh * dim &&
                          qn / (qh * dim) * (dim / 2) <= 0xffffffffu;
    if (!is(q, dtype) || !is(k, dtype) || !shape_ok || !std::isfinite(theta) || theta <= 0.0) {
        set_error(error, capacity,
                  "RoPE requires %s query [seq, query_heads, head_dim] and key [seq, "
                  "key_heads, head_dim] with an even head_dim <= 65536 and a finite positive "
                  "theta", dtype == TENSOR_DTYPE_F32 ? "F32" : "F16");
        return 0;
    }
    bool host;
    if (!common_storage({q, k}, &host)) return storage_error("RoPE", error, capacity);
    const size_t seq = qn / (qh * dim);
    if (seq == 0) return 1;
    Staging st("RoPE", host, error, capacity);
    if (!st.begin()) return 0;
    void *pq = srcdst(st, q);
    void *pk = srcdst(st, k);
    if (st.failed()) return 0;
    const size_t table_bytes =
        k::rope_table_bytes(seq, qh, kh, dim, dtype == TENSOR_DTYPE_F32 ? 4 : 2, pq, pk);
    ScratchBlock table(table_bytes);
    if (table_bytes != 0 && table.get() == nullptr) {
        set_error(error, capacity, "RoPE: out of device memory for the angle table");
        return 0;
    }
    const hipError_t status =
        dtype == TENSOR_DTYPE_F32
            ? k::rope_f32(as<float>(pq), as<float>(pk), seq, qh, kh, dim, theta, offset,
                          table.get(), st.stream())
            : k::rope_f16(as<uint16_t>(pq), as<uint16_t>(pk), seq, qh, kh, dim, theta, offset,
                          table.get(), st.stream());
    return st.finish(status) ? 1 : 0;
}

// Broadcast operand of a view: same rank, every dim 1 or the view's.
bool broadcastable(Buf t, const TensorView *v, uint64_t *shape_out) {
    if (t == nullptr) {
        for (size_t d = 0; d < v->rank; ++d) shape_out[d] = 1;
        return true;
    }
    if (tensor_buffer_rank(t) != v->rank) return false;
    for (size_t d = 0; d < v->rank; ++d) {
        const uint64_t s = tensor_buffer_shape(t)[d];
        if (s != 1 && s != v->shape[d]) return false;
        shape_out[d] = s;
    }
    return true;
}

int view_add_mul(TensorDType dtype, Buf x, const TensorView *v, Buf addend, Buf mult,
                 TensorBuffer *y, char *error, size_t capacity) {
    const char *type = dtype == TENSOR_DTYPE_F32 ? "F32" : "F16";
    if (!is(x, dtype) || !is(y, dtype) || v == nullptr || v->rank == 0 ||
        v->rank > TENSOR_VIEW_MAX_RANK || (addend && !is(addend, dtype)) ||
        (mult && !is(mult, dtype))) {
        set_error(error, capacity, "view add/mul requires %s input, output and operands and a "
                  "view of rank 1..%d", type, TENSOR_VIEW_MAX_RANK);
        return 0;
    }
    // bounds of the view inside x, and the output shape
    const uint64_t numel = tensor_buffer_element_count(x);
    uint64_t count = 1, reach = v->offset;
    bool empty = false, ok = tensor_buffer_rank(y) == v->rank;
    for (size_t d = 0; d < v->rank && ok; ++d) {
        if (v->strides[d] < 0) ok = false;
        if (v->shape[d] == 0) empty = true;
        if (ok && tensor_buffer_shape(y)[d] != v->shape[d]) ok = false;
        if (v->shape[d] > 0 && v->shape[d] > 0xffffffffull) ok = false;
    }
    if (ok && !empty) {
        for (size_t d = 0; d < v->rank; ++d) {
            count *= v->shape[d];
            reach += (v->shape[d] - 1) * (uint64_t)v->strides[d];
        }
        ok = reach < numel;
    }
    if (!ok) {
        set_error(error, capacity, "view add/mul requires non-negative strides, a view that "
                  "lies inside the input, and an output of the view's shape");
        return 0;
    }
    k::ViewArgs args{};
    args.rank = (int)v->rank;
    args.offset = v->offset;
    for (size_t d = 0; d < v->rank; ++d) {
        args.shape[d] = v->shape[d];
        args.strides[d] = v->strides[d];
    }
    if (!broadcastable(addend, v, args.addend_shape) || !broadcastable(mult, v, args.mult_shape)) {
        set_error(error, capacity, "view add/mul operands must have the view's rank with each "
                  "dimension 1 or equal to the view's");
        return 0;
    }
    bool host;
    if (!common_storage({x, addend, mult, y}, &host))
        return storage_error("view add/mul", error, capacity);
    if (empty) return 1;
    (void)count;
    Staging st("view add/mul", host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    const void *pa = src(st, addend);
    const void *pm = src(st, mult);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    const hipError_t status =
        dtype == TENSOR_DTYPE_F32
            ? k::view_add_mul_f32(as<float>(px), args, as<float>(pa), as<float>(pm),
                                  as<float>(py), st.stream())
            : k::view_add_mul_f16(as<uint16_t>(px), args, as<uint16_t>(pa), as<uint16_t>(pm),
                                  as<uint16_t>(py), st.stream());
    return st.finish(status) ? 1 : 0;
}

int fill(bool normal, TensorBuffer *t, uint64_t seed, uint64_t stream, float a, float b,
         char *error, size_t capacity) {
    if (!is(t, TENSOR_DTYPE_F32) && !is(t, TENSOR_DTYPE_F16)) {
        set_error(error, capacity, "random fill requires an F32 or F16 tensor");
        return 0;
    }
    if (!std::isfinite(a) || !std::isfinite(b)) {
        set_error(error, capacity, "random fill parameters must be finite");
        return 0;
    }
    const size_t n = tensor_buffer_element_count(t);
    if (n == 0) return 1;
    Staging st("random fill", tensor_buffer_storage(t) == TENSOR_BUFFER_STORAGE_HOST, error,
               capacity);
    if (!st.begin()) return 0;
    void *p = dst(st, t);
    if (st.failed()) return 0;
    const hipError_t status =
        normal ? k::fill_normal(tensor_buffer_dtype(t), p, n, seed, stream, a, b, st.stream())
               : k::fill_uniform(tensor_buffer_dtype(t), p, n, seed, stream, a, b, st.stream());
    return st.finish(status) ? 1 : 0;
}

// ---- embedding lookup (reference src/common/tensor_ops.c:41-161) ----------

// Reads index `i` of a host index buffer as the reference does (:41-84):
// false for a non-index dtype or a negative signed value.
bool host_index(Buf indices, size_t i, uint64_t *id) {
    const unsigned char *p = static_cast<const unsigned char *>(tensor_buffer_data(indices));
    switch (tensor_buffer_dtype(indices)) {
        case TENSOR_DTYPE_I16: { int16_t v; std::memcpy(&v, p + i * 2, 2); *id = (uint64_t)v; return v >= 0; }
        case TENSOR_DTYPE_U16: { uint16_t v; std::memcpy(&v, p + i * 2, 2); *id = v; return true; }
        case TENSOR_DTYPE_I32: { int32_t v; std::memcpy(&v, p + i * 4, 4); *id = (uint64_t)v; return v >= 0; }
        case TENSOR_DTYPE_U32: { uint32_t v; std::memcpy(&v, p + i * 4, 4); *id = v; return true; }
        case TENSOR_DTYPE_I64: { int64_t v; std::memcpy(&v, p + i * 8, 8); *id = (uint64_t)v; return v >= 0; }
        case TENSOR_DTYPE_U64: std::memcpy(id, p + i * 8, 8); return true;
        default: return false;
    }
}

// An event of the calling host thread for waiting on one point of the SDK
// stream: created on first use and kept for the thread's lifetime (null if
// it cannot be created; callers then wait for the whole stream).
hipEvent_t thread_event() {
    thread_local hipEvent_t event = nullptr;
    thread_local bool tried = false;
    if (!tried) {
        tried = true;
        if (hipEventCreateWithFlags(&event, hipEventDisableTiming) != hipSuccess) event = nullptr;
    }
    return event;
}

int embedding_lookup(TensorDType dtype, Buf table, Buf indices, TensorBuffer *out, char *error,
                     size_t capacity) {
    const bool f32 = dtype == TENSOR_DTYPE_F32;
    // the F32 entry point also insists on an index dtype up front; the F16
    // one finds a non-index dtype when it reads the first index (:86-101,
    // :130-152)
    if (!is(table, dtype) || !is(out, dtype) || indices == nullptr ||
        tensor_buffer_rank(table) != 2 || tensor_buffer_rank(indices) != 1 ||
        tensor_buffer_rank(out) != 2 ||
        (f32 && !k::embedding_index_type(tensor_buffer_dtype(indices)))) {
        set_error(error, capacity, "embedding lookup requires a rank-2 %s table, integer rank-1 "
                  "indices, and rank-2 %s output", f32 ? "F32" : "F16", f32 ? "F32" : "F16");
        return 0;
    }
    const uint64_t *ts = tensor_buffer_shape(table), *os = tensor_buffer_shape(out);
    const size_t count = tensor_buffer_element_count(indices);
    if (ts[0] == 0 || ts[1] == 0 || os[0] != count || os[1] != ts[1]) {
        set_error(error, capacity, "embedding table and output dimensions do not match");
        return 0;
    }
    bool host;
    if (!common_storage({table, indices, out}, &host))
        return storage_error("embedding lookup", error, capacity);
    if (count == 0) return 1;
    const char *bad_index = "embedding index is negative or outside the table";
    const TensorDType index_dtype = tensor_buffer_dtype(indices);
    if (!k::embedding_index_type(index_dtype)) {
        set_error(error, capacity, "%s", bad_index);
        return 0;
    }
    // every index is checked before any row is written: on the host for host
    // buffers; for device buffers by a one-block kernel that also writes a
    // device word the gather (enqueued right behind it) reads, so a rejected
    // call writes no row, and the host waits for the check alone
    if (host) {
        for (size_t i = 0; i < count; ++i) {
            uint64_t id;
            if (!host_index(indices, i, &id) || id >= ts[0]) {
                set_error(error, capacity, "%s", bad_index);
                return 0;
            }
        }
    }
    Staging st("embedding lookup", host, error, capacity);
    if (!st.begin()) return 0;
    HostWord verdict;
    ScratchBlock skip(host ? 0 : sizeof(uint32_t));
    hipEvent_t checked = nullptr;
    if (!host) {
        if (verdict.get() == nullptr || skip.get() == nullptr) {
            set_error(error, capacity, "embedding lookup: cannot allocate the index verdict");
            return 0;
        }
        if (!hip_ok(k::embedding_check(index_dtype, tensor_buffer_device_handle_internal(indices),
                                       count, ts[0], verdict.get(),
                                       static_cast<uint32_t *>(skip.get()), st.stream()),
                    "embedding lookup: index check launch", error, capacity))
            return 0;
        checked = thread_event();
        if (checked != nullptr && hipEventRecord(checked, st.stream()) != hipSuccess)
            checked = nullptr;
    }
    const void *pt = src(st, table);
    const void *pi = src(st, indices);
    void *po = dst(st, out);
    if (st.failed()) return 0;
    const size_t elem = f32 ? 4 : 2;
    const hipError_t status =
        k::embedding_gather(index_dtype, pt, ts[0], (size_t)ts[1] * elem, elem, pi, count, po,
                            static_cast<const uint32_t *>(skip.get()), st.stream());
    if (!host) {
        // without the event, wait for the gather as well
        if (!hip_ok(checked != nullptr ? hipEventSynchronize(checked)
                                       : hipStreamSynchronize(st.stream()),
                    "embedding lookup: waiting for the index check", error, capacity))
            return 0;
        if (verdict.read() != 0) {
            set_error(error, capacity, "%s", bad_index);
            return 0;
        }
    }
    return st.finish(status) ? 1 : 0;
}

}  // namespace

extern "C" {

// ---- include/tensor_ops.h ------------------------------------------------

int tensor_embedding_lookup_f32(Buf table, Buf indices, TensorBuffer *output, char *error,
                                size_t capacity) {
    return embedding_lookup(TENSOR_DTYPE_F32, table, indices, output, error, capacity);
}
int tensor_embedding_lookup_f16(Buf table, Buf indices, TensorBuffer *output, char *error,
                                size_t capacity) {
    return embedding_lookup(TENSOR_DTYPE_F16, table, indices, output, error, capacity);
}

int tensor_rms_norm_f32(Buf input, Buf weight, float epsilon, TensorBuffer *output,
                        char *error, size_t capacity) {
    return rms(TENSOR_DTYPE_F32, input, weight, epsilon, output, error, capacity);
}
int tensor_rms_norm_f16(Buf input, Buf weight, float epsilon, TensorBuffer *output,
                        char *error, size_t capacity) {
    return rms(TENSOR_DTYPE_F16, input, weight, epsilon, output, error, capacity);
}
int tensor_layer_norm_f32(Buf input, Buf scale, Buf bias_t, float epsilon, TensorBuffer *output,
                          char *error, size_t capacity) {
    return layer(TENSOR_DTYPE_F32, input, scale, bias_t, epsilon, output, error, capacity);
}
int tensor_layer_norm_f16(Buf input, Buf scale, Buf bias_t, float epsilon, TensorBuffer *output,
                          char *error, size_t capacity) {
    return layer(TENSOR_DTYPE_F16, input, scale, bias_t, epsilon, output, error, capacity);
}
int tensor_silu_f32(Buf input, TensorBuffer *output, char *error, size_t capacity) {
    return unary("SiLU", "SiLU requires same-shaped F32 tensors", TENSOR_DTYPE_F32,
                 k::Unary::Silu, input, output, error, capacity);
}
int tensor_silu_f16(Buf input, TensorBuffer *output, char *error, size_t capacity) {
    return unary("SiLU", "SiLU requires same-shaped F16 tensors", TENSOR_DTYPE_F16,
                 k::Unary::Silu, input, output, error, capacity);
}

// reference src/common/tensor_ops.c:575-622: the device branch goes through the
// preferred backend's residual_add_f16_device slot, as in the reference.
int tensor_residual_add_f16(Buf left, Buf right, TensorBuffer *output, char *error,
                            size_t capacity) {
    if (left == nullptr || right == nullptr || output == nullptr ||
        tensor_buffer_dtype(left) != TENSOR_DTYPE_F16 ||
        tensor_buffer_dtype(right) != TENSOR_DTYPE_F16 ||
        tensor_buffer_dtype(output) != TENSOR_DTYPE_F16 || !same_shape(left, right) ||
        !same_shape(left, output)) {
        set_error(error, capacity, "F16 residual add requires same-shaped F16 tensors");
        return 0;
    }
    const size_t count = tensor_buffer_element_count(left);
    const TensorBufferStorage storage = tensor_buffer_storage(left);
    if (storage != tensor_buffer_storage(right) || storage != tensor_buffer_storage(output)) {
        set_error(error, capacity, "F16 residual add operands must use the same storage type");
        return 0;
    }
    if (count == 0) return 1;
    if (storage == TENSOR_BUFFER_STORAGE_DEVICE) {
        const TensorComputeBackend *backend = tensor_compute_preferred_backend();
        if (backend == nullptr || backend->residual_add_f16_device == nullptr ||
            !backend->residual_add_f16_device(tensor_buffer_device_handle_internal(left),
                                              tensor_buffer_device_handle_internal(right),
                                              tensor_buffer_device_handle_internal(output),
                                              count)) {
            set_error(error, capacity, "device F16 residual add backend operation failed");
            return 0;
        }
        return 1;
    }
    return binary("F16 residual add", "F16 residual add requires same-shaped F16 tensors",
                  TENSOR_DTYPE_F16, k::Binary::Add, left, right, output, error, capacity);
}

// ---- include/tensor_ops_ext.h --------------------------------------------

int tensor_add_f32(Buf a, Buf b, TensorBuffer *y, char *error, size_t capacity) {
    return binary("F32 add", "F32 add requires same-shaped F32 tensors", TENSOR_DTYPE_F32,
                  k::Binary::Add, a, b, y, error, capacity);
}
int tensor_mul_f32(Buf a, Buf b, TensorBuffer *y, char *error, size_t capacity) {
    return binary("F32 multiply", "F32 multiply requires same-shaped F32 tensors",
                  TENSOR_DTYPE_F32, k::Binary::Mul, a, b, y, error, capacity);
}
int tensor_mul_f16(Buf a, Buf b, TensorBuffer *y, char *error, size_t capacity) {
    return binary("F16 multiply", "F16 multiply requires same-shaped F16 tensors",
                  TENSOR_DTYPE_F16, k::Binary::Mul, a, b, y, error, capacity);
}
int tensor_gelu_f32(Buf x, TensorBuffer *y, char *error, size_t capacity) {
    return unary("GELU", "GELU requires same-shaped F32 tensors", TENSOR_DTYPE_F32,
                 k::Unary::Gelu, x, y, error, capacity);
}
int tensor_gelu_f16(Buf x, TensorBuffer *y, char *error, size_t capacity) {
    return unary("GELU", "GELU requires same-shaped F16 tensors", TENSOR_DTYPE_F16,
                 k::Unary::Gelu, x, y, error, capacity);
}
int tensor_gelu_multiply_f16(Buf x, Buf gate, TensorBuffer *y, char *error, size_t capacity) {
    return binary("GELU multiply", "GELU multiply requires same-shaped F16 tensors",
                  TENSOR_DTYPE_F16, k::Binary::GeluMul, x, gate, y, error, capacity);
}
int tensor_relu_f16(Buf x, TensorBuffer *y, char *error, size_t capacity) {
    return unary("ReLU", "ReLU requires same-shaped F16 tensors", TENSOR_DTYPE_F16,
                 k::Unary::Relu, x, y, error, capacity);
}
int tensor_silu_multiply_f32(Buf gate, Buf up, TensorBuffer *y, char *error, size_t capacity) {
    return binary("SiLU multiply", "SiLU multiply requires same-shaped F32 tensors",
                  TENSOR_DTYPE_F32, k::Binary::SiluMul, gate, up, y, error, capacity);
}
int tensor_silu_multiply_f16(Buf gate, Buf up, TensorBuffer *y, char *error, size_t capacity) {
    return binary("SiLU multiply", "SiLU multiply requires same-shaped F16 tensors",
                  TENSOR_DTYPE_F16, k::Binary::SiluMul, gate, up, y, error, capacity);
}
int tensor_bias_add_f32(Buf x, Buf b, TensorBuffer *y, char *error, size_t capacity) {
    return bias("bias add", TENSOR_DTYPE_F32, false, x, b, y, error, capacity);
}
int tensor_bias_add_f16(Buf x, Buf b, TensorBuffer *y, char *error, size_t capacity) {
    return bias("bias add", TENSOR_DTYPE_F16, false, x, b, y, error, capacity);
}
int tensor_bias_gelu_f32(Buf x, Buf b, TensorBuffer *y, char *error, size_t capacity) {
    return bias("bias GELU", TENSOR_DTYPE_F32, true, x, b, y, error, capacity);
}
int tensor_bias_gelu_f16(Buf x, Buf b, TensorBuffer *y, char *error, size_t capacity) {
    return bias("bias GELU", TENSOR_DTYPE_F16, true, x, b, y, error, capacity);
}
int tensor_view_add_mul_f16(Buf x, const TensorView *view, Buf addend, Buf mult,
                            TensorBuffer *y, char *error, size_t capacity) {
    return view_add_mul(TENSOR_DTYPE_F16, x, view, addend, mult, y, error, capacity);
}
int tensor_view_add_mul_f32(Buf x, const TensorView *view, Buf addend, Buf mult,
                            TensorBuffer *y, char *error, size_t capacity) {
    return view_add_mul(TENSOR_DTYPE_F32, x, view, addend, mult, y, error, capacity);
}
int tensor_softmax_f32(Buf x, int causal, TensorBuffer *y, char *error, size_t capacity) {
    return softmax(TENSOR_DTYPE_F32, x, causal, y, error, capacity);
}
int tensor_softmax_f16(Buf x, int causal, TensorBuffer *y, char *error, size_t capacity) {
    return softmax(TENSOR_DTYPE_F16, x, causal, y, error, capacity);
}
int tensor_row_sum_f32(Buf x, TensorBuffer *y, char *error, size_t capacity) {
    return row_reduce("row sum", TENSOR_DTYPE_F32, false, x, y, error, capacity);
}
int tensor_row_sum_f16(Buf x, TensorBuffer *y, char *error, size_t capacity) {
    return row_reduce("row sum", TENSOR_DTYPE_F16, false, x, y, error, capacity);
}
int tensor_row_max_f32(Buf x, TensorBuffer *y, char *error, size_t capacity) {
    return row_reduce("row max", TENSOR_DTYPE_F32, true, x, y, error, capacity);
}
int tensor_row_max_f16(Buf x, TensorBuffer *y, char *error, size_t capacity) {
    return row_reduce("row max", TENSOR_DTYPE_F16, true, x, y, error, capacity);
}

int tensor_residual_rms_norm_f16(Buf x, Buf residual, Buf weight, float epsilon,
                                 TensorBuffer *sum, TensorBuffer *y, char *error,
                                 size_t capacity) {
    if (!is(x, TENSOR_DTYPE_F16) || !is(residual, TENSOR_DTYPE_F16) ||
        !is(weight, TENSOR_DTYPE_F16) || !is(sum, TENSOR_DTYPE_F16) || !is(y, TENSOR_DTYPE_F16) ||
        tensor_buffer_rank(x) == 0 || tensor_buffer_rank(weight) != 1 ||
        !same_shape(x, residual) || !same_shape(x, sum) || !same_shape(x, y) ||
        !std::isfinite(epsilon) || epsilon < 0.0f || sum == y) {
        set_error(error, capacity,
                  "residual RMSNorm requires same-shaped F16 input, residual, sum and output "
                  "(sum distinct from output), an F16 rank-1 weight and nonnegative epsilon");
        return 0;
    }
    const size_t width = last_dim(x);
    if (width == 0 || tensor_buffer_shape(weight)[0] != width) {
        set_error(error, capacity, "RMSNorm weight width does not match input");
        return 0;
    }
    bool host;
    if (!common_storage({x, residual, weight, sum, y}, &host))
        return storage_error("residual RMSNorm", error, capacity);
    const size_t rows = tensor_buffer_element_count(x) / width;
    if (rows == 0) return 1;
    Staging st("residual RMSNorm", host, error, capacity);
    if (!st.begin()) return 0;
    const void *px = src(st, x);
    const void *pr = src(st, residual);
    const void *pw = src(st, weight);
    void *ps = dst(st, sum);
    void *py = dst(st, y);
    if (st.failed()) return 0;
    return st.finish(k::rms_norm_f16(as<uint16_t>(px), as<uint16_t>(pr), as<uint16_t>(ps),
                                     as<uint16_t>(pw), as<uint16_t>(py), rows, width, epsilon,
                                     st.stream()))
               ? 1
               : 0;
}

int tensor_sum_max_f32(Buf x, TensorBuffer *sum, TensorBuffer *max, char *error,
                       size_t capacity) {
    if (!is(x, TENSOR_DTYPE_F32) || tensor_buffer_element_count(x) == 0 ||
        (sum == nullptr && max == nullptr) ||
        (sum != nullptr && (!is(sum, TENSOR_DTYPE_F64) || tensor_buffer_element_count(sum) != 1)) ||
        (max != nullptr && (!is(max, TENSOR_DTYPE_F32) || tensor_buffer_element_count(max) != 1))) {
        set_error(error, capacity,
                  "sum/max requires a non-empty F32 input, a one-element F64 sum output "
                  "and/or a one-element F32 max output");
        return 0;
    }
    bool host;
    if (!common_storage({x, sum, max}, &host)) return storage_error("sum/max", error, capacity);
    Staging st("sum/max", host, error, capacity);
    if (!st.begin()) return 0;
    void *partials = grid_reduce_partials(error, capacity);
    if (partials == nullptr) return 0;
    const void *px = src(st, x);
    void *ps = dst(st, sum);
    void *pm = dst(st, max);
    if (st.failed()) return 0;
    hipError_t status;
    {
        std::lock_guard<std::mutex> lock(grid_reduce_mutex());
        status = k::sum_max_f32(as<float>(px), tensor_buffer_element_count(x), as<double>(ps),
                                as<float>(pm), partials, st.stream());
    }
    return st.finish(status) ? 1 : 0;
}

// tensor_sum_max_f32 for callers that cannot allocate (code under HIP graph
// capture, serving loops that forbid hipMalloc). Same validation, kernels and
// results; the operands must be device tensors (host operands would be staged
// through allocated memory), and the pass-1 partials live in the library's
// 128 KiB device array instead of the grid-reduction buffer. Nothing here
// allocates: the array's address is looked up once per device
// (hipGetSymbolAddress), launches go to the SDK stream. Pass 1 writes every
// partial pass 2 reads, so the array needs no clearing between calls; calls
// enqueued on one GPU from this library are ordered by the SDK stream and the
// mutex below, and any other use of the array that overlaps them races.
int tensor_sum_max_f32_no_alloc(Buf x, TensorBuffer *sum, TensorBuffer *max, char *error,
                                size_t capacity) {
    if (!is(x, TENSOR_DTYPE_F32) || tensor_buffer_element_count(x) == 0 ||
        (sum == nullptr && max == nullptr) ||
        (sum != nullptr && (!is(sum, TENSOR_DTYPE_F64) || tensor_buffer_element_count(sum) != 1)) ||
        (max != nullptr && (!is(max, TENSOR_DTYPE_F32) || tensor_buffer_element_count(max) != 1))) {
        set_error(error, capacity,
                  "sum/max requires a non-empty F32 input, a one-element F64 sum output "
                  "and/or a one-element F32 max output");
        return 0;
    }
    for (Buf t : {x, static_cast<Buf>(sum), static_cast<Buf>(max)}) {
        if (t != nullptr && tensor_buffer_storage(t) != TENSOR_BUFFER_STORAGE_DEVICE) {
            set_error(error, capacity,
                      "sum/max without allocation requires device-storage operands");
            return 0;
        }
    }
    const size_t n = tensor_buffer_element_count(x);
    const size_t need = k::sum_max_partials_bytes(n);
    if (need > k::no_alloc_scratch_bytes()) {
        set_error(error, capacity,
                  "sum/max without allocation needs %zu bytes of partials for %zu elements, "
                  "more than its %zu-byte scratch",
                  need, n, k::no_alloc_scratch_bytes());
        return 0;
    }
    if (!sdk_ready(error, capacity)) return 0;
    void *scratch = nullptr;
    if (!hip_ok(k::no_alloc_scratch(&scratch), "sum/max scratch address (hipGetSymbolAddress)",
                error, capacity))
        return 0;
    static std::mutex order;
    hipError_t status;
    {
        std::lock_guard<std::mutex> lock(order);
        status = k::sum_max_f32_no_alloc(
            as<float>(tensor_buffer_device_handle_internal(x)), n,
            sum == nullptr ? nullptr : as<double>(tensor_buffer_device_handle_internal(sum)),
            max == nullptr ? nullptr : as<float>(tensor_buffer_device_handle_internal(max)),
            scratch, k::no_alloc_scratch_bytes(), sdk_stream());
    }
    if (status != hipSuccess) {
        set_error(error, capacity, "sum/max: kernel launch failed: %s", hipGetErrorString(status));
        return 0;
    }
    return 1;
}

int tensor_argmax_f32(Buf x, TensorBuffer *index, char *error, size_t capacity) {
    return argmax(TENSOR_DTYPE_F32, x, index, error, capacity);
}
int tensor_argmax_f16(Buf x, TensorBuffer *index, char *error, size_t capacity) {
    return argmax(TENSOR_DTYPE_F16, x, index, error, capacity);
}

int tensor_rope_f32(TensorBuffer *q, TensorBuffer *k, size_t qh, size_t kh, size_t dim,
                    double theta, size_t offset, char *error, size_t capacity) {
    return rope(TENSOR_DTYPE_F32, q, k, qh, kh, dim, theta, offset, error, capacity);
}
int tensor_rope_f16(TensorBuffer *q, TensorBuffer *k, size_t qh, size_t kh, size_t dim,
                    double theta, size_t offset, char *error, size_t capacity) {
    return rope(TENSOR_DTYPE_F16, q, k, qh, kh, dim, theta, offset, error, capacity);
}

int tensor_fill_uniform(TensorBuffer *t, uint64_t seed, uint64_t stream, float low, float high,
                        char *error, size_t capacity) {
    return fill(false, t, seed, stream, low, high, error, capacity);
}
int tensor_fill_normal(TensorBuffer *t, uint64_t seed, uint64_t stream, float mean,
                       float std_dev, char *error, size_t capacity) {
    return fill(true, t, seed, stream, mean, std_dev, error, capacity);
}

void *tensor_device_hip_stream(void) {
    return sdk_ready(nullptr, 0) ? (void *)sdk_stream() : nullptr;
}

// ---- tensor_buffer_convert (reference src/common/tensor_buffer.c:274-298) ----

int tensor_buffer_convert(Buf source, TensorDType target, TensorBuffer **result, char *error,
                          size_t capacity) {
    if (result != nullptr) *result = nullptr;
    auto supported = [](TensorDType d) {
        return d == TENSOR_DTYPE_F32 || d == TENSOR_DTYPE_F16 || d == TENSOR_DTYPE_BF16;
    };
    if (source == nullptr || result == nullptr || !supported(tensor_buffer_dtype(source)) ||
        !supported(target)) {
        set_error(error, capacity, "conversion supports F32, F16, and BF16 tensors");
        return 0;
    }
    const bool host = tensor_buffer_storage(source) == TENSOR_BUFFER_STORAGE_HOST;
    TensorBuffer *out = nullptr;
    const int created =
        host ? tensor_buffer_create(target, tensor_buffer_shape(source),
                                    tensor_buffer_rank(source), &out, error, capacity)
             : tensor_buffer_create_device(target, tensor_buffer_shape(source),
                                           tensor_buffer_rank(source), &out, error, capacity);
    if (!created) return 0;
    const size_t n = tensor_buffer_element_count(source);
    if (n > 0) {
        Staging st("conversion", host, error, capacity);
        bool ok = st.begin();
        if (ok) {
            const void *px = src(st, source);
            void *py = dst(st, out);
            ok = !st.failed();
            if (ok) {
                hipError_t status;
                if (tensor_buffer_dtype(source) == target)
                    status = hipMemcpyAsync(py, px, tensor_buffer_byte_length(source),
                                            hipMemcpyDeviceToDevice, st.stream());
                else
                    status = k::convert(tensor_buffer_dtype(source), px, target, py, n,
                                        st.stream());
                ok = st.finish(status);
            }
        }
        if (!ok) {
            tensor_buffer_free(out);
            return 0;
        }
    }
    *result = out;
    return 1;
}

}  // extern "C"
