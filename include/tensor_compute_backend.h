/* Compute backend vtable.
 *
 * The struct layouts below are ABI: member order and types are identical to
 * include/tensor_compute_backend.h:9-122 of the reference, so a caller built
 * against the reference header reads the same slots from this library.
 *
 * Slot conventions (reference tensor_compute_cuda.cu:399-504, 740-746):
 *   - plain slots take host pointers (float* or uint16_t* holding IEEE f16
 *     bits) and are synchronous: on return the host output is written;
 *   - *_device slots take raw device addresses and only enqueue work;
 *   - every slot returns 1 on success, 0 on failure;
 *   - a NULL slot means the backend does not offer that operation; callers
 *     in the reference test for NULL before calling.
 *
 * The HIP backend ("hip") fills the elementwise, broadcast, normalisation,
 * RoPE, argmax and embedding slots, and the GEMM-based linear*,
 * linear*_device, linear_q8_0_f16 / linear_q4_0_f16 (+ _device),
 * rms_norm_linear_f32, mlp_f16 and qkv_f16 slots (hipBLASLt GEMMs and the
 * library's quantized GEMV/MFMA kernels; host-pointer weights stay on the
 * device per host address until release_cache). The whole-layer slots
 * (vision_layer_*, vision_sequence_*, mlp_f32) stay NULL.
 */
#ifndef TENSOR_COMPUTE_BACKEND_H
#define TENSOR_COMPUTE_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#include "tensor_quant.h"

/* reference include/tensor_compute_backend.h:9-26 */
typedef struct {
    const uint16_t *norm1_scale;
    const uint16_t *norm1_bias;
    const uint16_t *q_weight;
    const uint16_t *q_bias;
    const uint16_t *k_weight;
    const uint16_t *k_bias;
    const uint16_t *v_weight;
    const uint16_t *v_bias;
    const uint16_t *out_weight;
    const uint16_t *out_bias;
    const uint16_t *norm2_scale;
    const uint16_t *norm2_bias;
    const uint16_t *fc1_weight;
    const uint16_t *fc1_bias;
    const uint16_t *fc2_weight;
    const uint16_t *fc2_bias;
} TensorVisionLayerF16;

/* reference :28-39 */
typedef struct {
    const uint16_t *norm1_scale, *norm1_bias;
    const uint8_t *q_weight, *k_weight, *v_weight;
    const uint16_t *q_bias, *k_bias, *v_bias;
    const uint8_t *out_weight;
    const uint16_t *out_bias;
    const uint16_t *norm2_scale, *norm2_bias;
    const uint8_t *fc1_weight;
    const uint16_t *fc1_bias;
    const uint8_t *fc2_weight;
    const uint16_t *fc2_bias;
} TensorVisionLayerQuantF16;

/* reference :41-47 */
typedef struct {
    const float *norm1_scale, *norm1_bias;
    const float *q_weight, *q_bias, *k_weight, *k_bias, *v_weight, *v_bias;
    const float *out_weight, *out_bias;
    const float *norm2_scale, *norm2_bias;
    const float *fc1_weight, *fc1_bias, *fc2_weight, *fc2_bias;
} TensorVisionLayerF32;

/* reference :49-122. Argument meaning per slot (rows/width/count are
   element counts):
     rms_norm(x, w, y, rows, width, eps); layer_norm(x, scale, bias, y, rows,
     width, eps); bias_add(x, bias, y, rows, width) with y[i] = x[i] +
     bias[i % width]; gelu(x, y, n); gelu_multiply(x, gate, y, n) =
     gelu(x)*gate; relu(x, y, n); rope(q, k, seq, q_heads, kv_heads, head_dim,
     theta[, offset]) in place on [seq, heads, head_dim]; silu_multiply(gate,
     up, y, n) = silu(gate)*up; residual_add(a, b, y, n); argmax(x, n, &index)
     = first index of the maximum. */
typedef struct {
    const char *name;
    int (*is_available)(void);
    int (*linear_f32)(const float *, const float *, float *, size_t, size_t, size_t);
    int (*linear_f16)(const uint16_t *, const uint16_t *, uint16_t *, size_t, size_t, size_t);
    int (*embedding_f16)(const uint16_t *, const uint32_t *, uint16_t *, size_t, size_t, size_t);
    int (*rms_norm_f16)(const uint16_t *, const uint16_t *, uint16_t *, size_t, size_t, float);
    int (*layer_norm_f16)(const uint16_t *, const uint16_t *, const uint16_t *, uint16_t *, size_t, size_t, float);
    int (*bias_add_f16)(const uint16_t *, const uint16_t *, uint16_t *, size_t, size_t);
    int (*gelu_f16)(const uint16_t *, uint16_t *, size_t);
    /* GELU(input) * gate, evaluated on the GPU. */
    int (*gelu_multiply_f16)(const uint16_t *, const uint16_t *, uint16_t *, size_t);
    int (*relu_f16)(const uint16_t *, uint16_t *, size_t);
    int (*rope_f16)(uint16_t *, uint16_t *, size_t, size_t, size_t, size_t, double, size_t);
    int (*silu_multiply_f16)(const uint16_t *, const uint16_t *, uint16_t *, size_t);
    int (*residual_add_f16)(const uint16_t *, const uint16_t *, uint16_t *, size_t);
    int (*argmax_f16)(const uint16_t *, size_t, uint32_t *);
    int (*embedding_f32)(const float *, const uint32_t *, float *, size_t, size_t, size_t);
    int (*rms_norm_f32)(const float *, const float *, float *, size_t, size_t, float);
    int (*rms_norm_linear_f32)(const float *, const float *, float *,
                               const float *, float *, size_t, size_t, size_t,
                               float);
    int (*layer_norm_f32)(const float *, const float *, const float *, float *, size_t, size_t, float);
    int (*bias_add_f32)(const float *, const float *, float *, size_t, size_t);
    int (*gelu_f32)(const float *, float *, size_t);
    int (*rope_f32)(float *, float *, size_t, size_t, size_t, size_t, double);
    int (*silu_multiply_f32)(const float *, const float *, float *, size_t);
    int (*residual_add_f32)(const float *, const float *, float *, size_t);
    int (*argmax_f32)(const float *, size_t, uint32_t *);
    void (*release_cache)(void);
    int (*mlp_f32)(const float *, const float *, const float *, const float *,
                   const float *, float *, size_t, size_t, size_t, size_t);
    int (*mlp_f16)(const uint16_t *, const uint16_t *, const uint16_t *,
                   const uint16_t *, const uint16_t *, uint16_t *,
                   size_t, size_t, size_t, size_t);
    int (*qkv_f16)(const uint16_t *, const uint16_t *, const uint16_t *,
                   const uint16_t *, const uint16_t *, const uint16_t *,
                   const uint16_t *, uint16_t *, uint16_t *,
                   uint16_t *, size_t, size_t, size_t);
    int (*vision_layer_f16)(uint16_t *, const TensorVisionLayerF16 *, size_t,
                            size_t, size_t, float);
    int (*vision_layer_f32)(float *, const TensorVisionLayerF32 *, size_t,
                            size_t, size_t, float);
    void *(*vision_sequence_begin_f16)(const uint16_t *, size_t, size_t);
    int (*vision_sequence_layer_f16)(void *, const TensorVisionLayerF16 *,
                                    size_t, size_t, size_t, float);
    int (*vision_sequence_finish_f16)(void *, uint16_t *);
    void (*vision_sequence_release_f16)(void *);
    int (*vision_sequence_layer_quant_f16)(void *,
        const TensorVisionLayerQuantF16 *, TensorWeightQuantization,
        size_t, size_t, size_t, float);
    void *(*vision_sequence_begin_f32)(const float *, size_t, size_t);
    int (*vision_sequence_layer_f32)(void *, const TensorVisionLayerF32 *,
                                    size_t, size_t, size_t, float);
    int (*vision_sequence_finish_f32)(void *, float *);
    void (*vision_sequence_release_f32)(void *);
    int (*linear_f32_device)(const void *, const void *, void *, size_t,
                             size_t, size_t);
    int (*linear_f16_device)(const void *, const void *, void *, size_t,
                             size_t, size_t);
    int (*linear_q8_0_f16_device)(const void *, const void *, void *, size_t,
                                  size_t, size_t);
    int (*linear_q4_0_f16_device)(const void *, const void *, void *, size_t,
                                  size_t, size_t);
    int (*linear_q8_0_f16)(const uint16_t *, const uint8_t *, uint16_t *,
                           size_t, size_t, size_t);
    int (*linear_q4_0_f16)(const uint16_t *, const uint8_t *, uint16_t *,
                           size_t, size_t, size_t);
    int (*bias_add_f32_device)(const void *, const void *, void *, size_t,
                               size_t);
    int (*bias_add_f16_device)(const void *, const void *, void *, size_t,
                               size_t);
    int (*residual_add_f16_device)(const void *, const void *, void *, size_t);
} TensorComputeBackend;

#ifdef __cplusplus
extern "C" {
#endif

/* reference :128-130. In this library the Metal and CUDA getters return
   tables whose is_available() is 0 (as the reference's stubs,
   src/platform/cuda/tensor_compute_cuda_stub.c:7-12), and the preferred
   backend follows TENSOR_BACKEND: unset, "", "auto" or "hip" select the HIP
   backend when a GPU is present; any other value yields NULL
   (reference dispatch: src/common/backend_dispatch.c:10-35). */
const TensorComputeBackend *tensor_compute_metal_backend(void);
const TensorComputeBackend *tensor_compute_cuda_backend(void);
const TensorComputeBackend *tensor_compute_preferred_backend(void);

/* The HIP table itself (name "hip"); no reference counterpart, it is the
   backend a HIP build adds beside the CUDA and Metal getters. */
const TensorComputeBackend *tensor_compute_hip_backend(void);

#ifdef __cplusplus
}
#endif

#endif
