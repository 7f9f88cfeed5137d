/* Accelerator attention table.
 *
 * TensorAttentionBackendOps is the reference's src/attention_backend.h:6-44,
 * kept field for field: src/common/attention.c reaches an accelerator only
 * through tensor_attention_cuda_backend() / tensor_attention_metal_backend()
 * (attention.c:10-35, :196-209, :402-429), calling `run` / `run_f16` with
 * host pointers. In a HIP build this library provides
 * tensor_attention_cuda_backend() (the reference's accelerator slot, whose
 * stub src/platform/cuda/attention_cuda_stub.c it replaces): it returns the
 * HIP table. Its `kind` is TENSOR_ATTENTION_BACKEND_CUDA, the slot's value
 * in the reference's enum, which has no HIP member; `name` is "hip".
 *
 * Only `is_available`, `run` and `run_f16` are provided; every decode slot
 * is NULL, which attention.c treats as "not available". The decode slots'
 * pointer parameters are typed `const void *` here (the reference's decoder
 * layer and paged-request structs are only ever passed by pointer), which
 * leaves the layout unchanged.
 */
#ifndef ATTENTION_BACKEND_H
#define ATTENTION_BACKEND_H

#include "tensor_quant.h"

#include <stddef.h>
#include <stdint.h>

/* reference include/attention.h:12-17 */
typedef enum {
    TENSOR_ATTENTION_BACKEND_CPU,
    TENSOR_ATTENTION_BACKEND_METAL,
    TENSOR_ATTENTION_BACKEND_CUDA,
    TENSOR_ATTENTION_BACKEND_QNN_HTP
} TensorAttentionBackend;

/* reference src/attention_backend.h:6-44 */
typedef struct {
    TensorAttentionBackend kind;
    const char *name;
    int (*is_available)(void);
    /* q [B,Hq,Lq,D], k [B,Hkv,Lkv,D], v [B,Hkv,Lkv,Dv], additive_mask
       [Lq,Lkv] or NULL, output [B,Hq,Lq,Dv]; host pointers; synchronous */
    int (*run)(const float *query, const float *key, const float *value,
               const float *additive_mask, float *output,
               size_t batch, size_t query_heads, size_t kv_heads,
               size_t query_length, size_t kv_length, size_t head_dim,
               size_t value_dim, float scale, int causal);
    int (*run_f16)(const uint16_t *query, const uint16_t *key,
                   const uint16_t *value, const uint16_t *additive_mask,
                   uint16_t *output, size_t batch, size_t query_heads,
                   size_t kv_heads, size_t query_length, size_t kv_length,
                   size_t head_dim, size_t value_dim, float scale, int causal);
    int (*decode)(const float *, const float *, const float *, const float *,
                  const float *, float *, size_t, size_t, size_t, size_t, size_t);
    int (*decode_sequence_available)(void);
    int (*decode_sequence)(const void *, size_t, const float *, uint32_t, size_t, uint32_t *,
                           const float *const *, const float *const *, size_t, size_t,
                           size_t, size_t, size_t, size_t, size_t, float, double,
                           const float *, const float *, size_t);
    int (*decode_sequence_f16_available)(void);
    int (*decode_sequence_f16)(const void *, size_t, const uint16_t *, uint32_t, size_t,
                               uint32_t *, const uint16_t *const *,
                               const uint16_t *const *, size_t, size_t, size_t, size_t,
                               size_t, size_t, size_t, float, double, const uint16_t *,
                               const uint16_t *, size_t);
    int (*decode_sequence_quant_f16_available)(TensorWeightQuantization);
    int (*decode_sequence_quant_f16)(const void *, size_t, const uint16_t *, uint32_t,
                                     size_t, uint32_t *, const uint16_t *const *,
                                     const uint16_t *const *, size_t, size_t, size_t,
                                     size_t, size_t, size_t, size_t, float, double,
                                     const uint16_t *, const uint8_t *, size_t,
                                     TensorWeightQuantization);
    int (*decode_sequence_paged)(const void *);
    void (*decode_cache_clear)(void);
} TensorAttentionBackendOps;

#ifdef __cplusplus
extern "C" {
#endif

/* reference src/attention_backend.h:50 (stub: src/platform/cuda/
   attention_cuda_stub.c); here the HIP table */
const TensorAttentionBackendOps *tensor_attention_cuda_backend(void);
/* the same table under its own name (no reference counterpart) */
const TensorAttentionBackendOps *tensor_attention_hip_backend(void);

#ifdef __cplusplus
}
#endif

#endif
