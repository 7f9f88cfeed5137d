/* ABI layout probe -- TEST INFRASTRUCTURE ONLY.
 * Compiled twice by tests/test_library_host.py: once against the reference's
 * include/ and once against this repository's include/. Prints sizeof and
 * offsetof for the public structs and the enum values so the two can be
 * compared line for line. */
#include <stddef.h>
#include <stdio.h>

#include "tensor_buffer.h"
#include "tensor_compute_backend.h"
#include "tensor_device.h"

#define FIELD(s, f) printf(#s "." #f " %zu\n", offsetof(s, f))

int main(void) {
    printf("sizeof TensorComputeBackend %zu\n", sizeof(TensorComputeBackend));
    printf("sizeof TensorVisionLayerF16 %zu\n", sizeof(TensorVisionLayerF16));
    printf("sizeof TensorVisionLayerQuantF16 %zu\n", sizeof(TensorVisionLayerQuantF16));
    printf("sizeof TensorVisionLayerF32 %zu\n", sizeof(TensorVisionLayerF32));
    FIELD(TensorComputeBackend, name); FIELD(TensorComputeBackend, is_available);
    FIELD(TensorComputeBackend, linear_f32); FIELD(TensorComputeBackend, linear_f16);
    FIELD(TensorComputeBackend, embedding_f16); FIELD(TensorComputeBackend, rms_norm_f16);
    FIELD(TensorComputeBackend, layer_norm_f16); FIELD(TensorComputeBackend, bias_add_f16);
    FIELD(TensorComputeBackend, gelu_f16); FIELD(TensorComputeBackend, gelu_multiply_f16);
    FIELD(TensorComputeBackend, relu_f16); FIELD(TensorComputeBackend, rope_f16);
    FIELD(TensorComputeBackend, silu_multiply_f16); FIELD(TensorComputeBackend, residual_add_f16);
    FIELD(TensorComputeBackend, argmax_f16); FIELD(TensorComputeBackend, embedding_f32);
    FIELD(TensorComputeBackend, rms_norm_f32); FIELD(TensorComputeBackend, rms_norm_linear_f32);
    FIELD(TensorComputeBackend, layer_norm_f32); FIELD(TensorComputeBackend, bias_add_f32);
    FIELD(TensorComputeBackend, gelu_f32); FIELD(TensorComputeBackend, rope_f32);
    FIELD(TensorComputeBackend, silu_multiply_f32); FIELD(TensorComputeBackend, residual_add_f32);
    FIELD(TensorComputeBackend, argmax_f32); FIELD(TensorComputeBackend, release_cache);
    FIELD(TensorComputeBackend, mlp_f32); FIELD(TensorComputeBackend, mlp_f16);
    FIELD(TensorComputeBackend, qkv_f16); FIELD(TensorComputeBackend, vision_layer_f16);
    FIELD(TensorComputeBackend, vision_layer_f32);
    FIELD(TensorComputeBackend, vision_sequence_begin_f16);
    FIELD(TensorComputeBackend, vision_sequence_layer_f16);
    FIELD(TensorComputeBackend, vision_sequence_finish_f16);
    FIELD(TensorComputeBackend, vision_sequence_release_f16);
    FIELD(TensorComputeBackend, vision_sequence_layer_quant_f16);
    FIELD(TensorComputeBackend, vision_sequence_begin_f32);
    FIELD(TensorComputeBackend, vision_sequence_layer_f32);
    FIELD(TensorComputeBackend, vision_sequence_finish_f32);
    FIELD(TensorComputeBackend, vision_sequence_release_f32);
    FIELD(TensorComputeBackend, linear_f32_device); FIELD(TensorComputeBackend, linear_f16_device);
    FIELD(TensorComputeBackend, linear_q8_0_f16_device);
    FIELD(TensorComputeBackend, linear_q4_0_f16_device);
    FIELD(TensorComputeBackend, linear_q8_0_f16); FIELD(TensorComputeBackend, linear_q4_0_f16);
    FIELD(TensorComputeBackend, bias_add_f32_device);
    FIELD(TensorComputeBackend, bias_add_f16_device);
    FIELD(TensorComputeBackend, residual_add_f16_device);
    printf("F16 %d BF16 %d F32 %d F64 %d U32 %d UNKNOWN %d\n", TENSOR_DTYPE_F16, TENSOR_DTYPE_BF16,
           TENSOR_DTYPE_F32, TENSOR_DTYPE_F64, TENSOR_DTYPE_U32, TENSOR_DTYPE_UNKNOWN);
    printf("HOST %d DEVICE %d Q8 %d Q4 %d\n", TENSOR_BUFFER_STORAGE_HOST,
           TENSOR_BUFFER_STORAGE_DEVICE, TENSOR_WEIGHT_Q8_0, TENSOR_WEIGHT_Q4_0);
    return 0;
}
