// Attention entry points of the HIP library.
//
// 1. The accelerator attention table (include/attention_backend.h; layout of
//    the reference's src/attention_backend.h:6-44), returned by
//    tensor_attention_cuda_backend() -- the slot src/common/attention.c
//    consults (attention.c:10-35, :196-209, :402-429) -- and by
//    tensor_attention_hip_backend(). `run` / `run_f16` take host pointers,
//    like the CUDA backend's (attention_cuda.cu:71-99, :1108-1110): operands
//    are staged through the device pool, the kernel runs on the SDK stream,
//    the output is copied back before the slot returns. Argument checks
//    mirror the CUDA wrapper's: non-null pointers, nonzero sizes, Hq a
//    multiple of Hkv, finite scale, no size_t overflow.
// 2. tensor_sdpa_device_f32 / _f16 (include/tensor_ops_ext.h): the same
//    attention on device-storage TensorBuffers, enqueued and returning.
#include "kernels.hpp"
#include "sdk.hpp"
#include "staging.hpp"

#include "attention_backend.h"
#include "tensor_buffer.h"
#include "tensor_ops_ext.h"

#include <cmath>
#include <cstring>

using namespace icsdk;

namespace {

bool mul_ok(size_t a, size_t b, size_t *out) {
    if (b != 0 && a > SIZE_MAX / b) return false;
    *out = a * b;
    return true;
}

// Element counts of q, k, v, out and the mask for a shape, or false on
// overflow or a shape the kernels do not take.
struct SdpaCounts {
    size_t q, k, v, out, mask;
};

bool sdpa_counts(const k::SdpaShape &s, size_t elem, SdpaCounts *c) {
    if (s.batch == 0 || s.q_heads == 0 || s.kv_heads == 0 || s.q_len == 0 || s.kv_len == 0 ||
        s.head_dim == 0 || s.value_dim == 0 || s.q_heads % s.kv_heads != 0)
        return false;
    size_t bq, bk;
    if (!mul_ok(s.batch, s.q_heads, &bq) || !mul_ok(bq, s.q_len, &bq) ||
        !mul_ok(s.batch, s.kv_heads, &bk) || !mul_ok(bk, s.kv_len, &bk) ||
        !mul_ok(bq, s.head_dim, &c->q) || !mul_ok(bk, s.head_dim, &c->k) ||
        !mul_ok(bk, s.value_dim, &c->v) || !mul_ok(bq, s.value_dim, &c->out) ||
        !mul_ok(s.q_len, s.kv_len, &c->mask))
        return false;
    for (size_t n : {c->q, c->k, c->v, c->out, c->mask})
        if (n > SIZE_MAX / elem) return false;
    return true;
}

template <typename T>
int host_run(const T *q, const T *k, const T *v, const T *mask, T *out, size_t batch,
             size_t qh, size_t kvh, size_t ql, size_t kl, size_t dim, size_t vdim, float scale,
             int causal) {
    const k::SdpaShape shape{batch, qh, kvh, ql, kl, dim, vdim};
    SdpaCounts c;
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr ||
        !std::isfinite(scale) || (causal != 0 && causal != 1) ||
        !sdpa_counts(shape, sizeof(T), &c))
        return 0;
    Staging st("hip attention", true, nullptr, 0);
    if (!st.begin()) return 0;
    const void *pq = st.in(q, c.q * sizeof(T));
    const void *pk = st.in(k, c.k * sizeof(T));
    const void *pv = st.in(v, c.v * sizeof(T));
    const void *pm = mask ? st.in(mask, c.mask * sizeof(T)) : nullptr;
    void *po = st.out(out, c.out * sizeof(T));
    if (st.failed()) return 0;
    const size_t ws_want = k::sdpa_workspace_bytes(shape, sizeof(T) == 4, causal != 0);
    ScratchBlock workspace(ws_want);
    const size_t ws_bytes = workspace.get() ? ws_want : 0;
    hipError_t status;
    if constexpr (sizeof(T) == 4)
        status = k::sdpa_f32(static_cast<const float *>(pq), static_cast<const float *>(pk),
                             static_cast<const float *>(pv), static_cast<const float *>(pm),
                             static_cast<float *>(po), shape, scale, causal != 0,
                             workspace.get(), ws_bytes, st.stream());
    else
        status = k::sdpa_f16(static_cast<const uint16_t *>(pq),
                             static_cast<const uint16_t *>(pk),
                             static_cast<const uint16_t *>(pv),
                             static_cast<const uint16_t *>(pm), static_cast<uint16_t *>(po),
                             shape, scale, causal != 0, workspace.get(), ws_bytes, st.stream());
    return st.finish(status) ? 1 : 0;
}

int run_f32(const float *q, const float *k, const float *v, const float *m, float *o, size_t b,
            size_t qh, size_t kh, size_t ql, size_t kl, size_t d, size_t vd, float s, int c) {
    return host_run(q, k, v, m, o, b, qh, kh, ql, kl, d, vd, s, c);
}

int run_f16(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *m,
            uint16_t *o, size_t b, size_t qh, size_t kh, size_t ql, size_t kl, size_t d,
            size_t vd, float s, int c) {
    return host_run(q, k, v, m, o, b, qh, kh, ql, kl, d, vd, s, c);
}

int attention_available(void) { return sdk_ready(nullptr, 0) ? 1 : 0; }

const TensorAttentionBackendOps &hip_table() {
    static const TensorAttentionBackendOps table = [] {
        TensorAttentionBackendOps t;
        std::memset(&t, 0, sizeof t);
        t.kind = TENSOR_ATTENTION_BACKEND_CUDA;
        t.name = "hip";
        t.is_available = attention_available;
        t.run = run_f32;
        t.run_f16 = run_f16;
        return t;
    }();
    return table;
}

// ---- device-storage SDPA ---------------------------------------------------

bool device_tensor(const TensorBuffer *t, TensorDType dtype, size_t rank) {
    return t != nullptr && tensor_buffer_dtype(t) == dtype && tensor_buffer_rank(t) == rank &&
           tensor_buffer_storage(t) == TENSOR_BUFFER_STORAGE_DEVICE;
}

// Validation and messages follow tensor_sdpa_f32/f16 (src/common/attention.c:
// 211-266, :402-427), with device storage in place of host storage and no
// workspace (the device path needs none).
int sdpa_device(TensorDType dtype, const TensorBuffer *q, const TensorBuffer *k,
                const TensorBuffer *v, const TensorBuffer *mask, float scale, int causal,
                TensorBuffer *out, char *error, size_t capacity) {
    const char *type = dtype == TENSOR_DTYPE_F32 ? "F32" : "F16";
    if (!device_tensor(q, dtype, 4) || !device_tensor(k, dtype, 4) ||
        !device_tensor(v, dtype, 4) || !device_tensor(out, dtype, 4) ||
        (mask != nullptr && !device_tensor(mask, dtype, 2)) || !std::isfinite(scale) ||
        (causal != 0 && causal != 1)) {
        set_error(error, capacity, "device SDPA requires rank-4 %s device tensors, finite "
                  "scale, and optional rank-2 %s device mask", type, type);
        return 0;
    }
    const uint64_t *qs = tensor_buffer_shape(q), *ks = tensor_buffer_shape(k);
    const uint64_t *vs = tensor_buffer_shape(v), *os = tensor_buffer_shape(out);
    const k::SdpaShape shape{(size_t)qs[0], (size_t)qs[1], (size_t)ks[1], (size_t)qs[2],
                             (size_t)ks[2], (size_t)qs[3], (size_t)vs[3]};
    if (shape.batch == 0 || shape.q_heads == 0 || shape.kv_heads == 0 || shape.q_len == 0 ||
        shape.kv_len == 0 || shape.head_dim == 0 || shape.value_dim == 0 ||
        qs[0] != ks[0] || qs[0] != vs[0] || ks[1] != vs[1] ||
        shape.q_heads % shape.kv_heads != 0 || ks[2] != vs[2] || ks[3] != qs[3] ||
        os[0] != qs[0] || os[1] != qs[1] || os[2] != qs[2] || os[3] != vs[3]) {
        set_error(error, capacity, "SDPA tensor dimensions do not match");
        return 0;
    }
    if (mask != nullptr) {
        const uint64_t *ms = tensor_buffer_shape(mask);
        if (ms[0] != shape.q_len || ms[1] != shape.kv_len) {
            set_error(error, capacity, "SDPA mask shape must be [query_length, key_length]");
            return 0;
        }
    }
    if (shape.head_dim > 512 || shape.value_dim > 512) {
        set_error(error, capacity, "device SDPA supports head and value dimensions up to 512");
        return 0;
    }
    if (!sdk_ready(error, capacity)) return 0;
    auto dev = [](const TensorBuffer *t) -> void * {
        return t ? tensor_buffer_device_handle_internal(t) : nullptr;
    };
    // split-key partials live in a pool block, returned right after the
    // launches (later users of the block enqueue behind them on the stream)
    const size_t ws_want = k::sdpa_workspace_bytes(shape, dtype == TENSOR_DTYPE_F32, causal != 0);
    ScratchBlock workspace(ws_want);
    const size_t ws_bytes = workspace.get() ? ws_want : 0;
    const hipError_t status =
        dtype == TENSOR_DTYPE_F32
            ? k::sdpa_f32(static_cast<const float *>(dev(q)), static_cast<const float *>(dev(k)),
                          static_cast<const float *>(dev(v)),
                          static_cast<const float *>(dev(mask)), static_cast<float *>(dev(out)),
                          shape, scale, causal != 0, workspace.get(), ws_bytes, sdk_stream())
            : k::sdpa_f16(static_cast<const uint16_t *>(dev(q)),
                          static_cast<const uint16_t *>(dev(k)),
                          static_cast<const uint16_t *>(dev(v)),
                          static_cast<const uint16_t *>(dev(mask)),
                          static_cast<uint16_t *>(dev(out)), shape, scale, causal != 0,
                          workspace.get(), ws_bytes, sdk_stream());
    return hip_ok(status, "device SDPA: kernel launch", error, capacity) ? 1 : 0;
}

}  // namespace

extern "C" {

const TensorAttentionBackendOps *tensor_attention_cuda_backend(void) { return &hip_table(); }
const TensorAttentionBackendOps *tensor_attention_hip_backend(void) { return &hip_table(); }

int tensor_sdpa_device_f32(const TensorBuffer *query, const TensorBuffer *key,
                           const TensorBuffer *value, const TensorBuffer *additive_mask,
                           float scale, int causal, TensorBuffer *output, char *error,
                           size_t error_capacity) {
    return sdpa_device(TENSOR_DTYPE_F32, query, key, value, additive_mask, scale, causal,
                       output, error, error_capacity);
}

int tensor_sdpa_device_f16(const TensorBuffer *query, const TensorBuffer *key,
                           const TensorBuffer *value, const TensorBuffer *additive_mask,
                           float scale, int causal, TensorBuffer *output, char *error,
                           size_t error_capacity) {
    return sdpa_device(TENSOR_DTYPE_F16, query, key, value, additive_mask, scale, causal,
                       output, error, error_capacity);
}

}  // extern "C"
