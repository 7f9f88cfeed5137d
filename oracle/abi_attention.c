/* ABI layout probe for the accelerator attention table -- TEST
 * INFRASTRUCTURE ONLY. Compiled by tests/test_library_host.py against the
 * reference's src/attention_backend.h and against this repository's
 * include/attention_backend.h; prints sizeof, every offset and the backend
 * enum values so the two can be compared line for line. */
#include <stddef.h>
#include <stdio.h>

#include "attention_backend.h"

#define FIELD(f) printf("TensorAttentionBackendOps." #f " %zu\n", offsetof(TensorAttentionBackendOps, f))

int main(void) {
    printf("sizeof TensorAttentionBackendOps %zu\n", sizeof(TensorAttentionBackendOps));
    FIELD(kind); FIELD(name); FIELD(is_available); FIELD(run); FIELD(run_f16); FIELD(decode);
    FIELD(decode_sequence_available); FIELD(decode_sequence);
    FIELD(decode_sequence_f16_available); FIELD(decode_sequence_f16);
    FIELD(decode_sequence_quant_f16_available); FIELD(decode_sequence_quant_f16);
    FIELD(decode_sequence_paged); FIELD(decode_cache_clear);
    printf("CPU %d METAL %d CUDA %d QNN %d\n", TENSOR_ATTENTION_BACKEND_CPU,
           TENSOR_ATTENTION_BACKEND_METAL, TENSOR_ATTENTION_BACKEND_CUDA,
           TENSOR_ATTENTION_BACKEND_QNN_HTP);
    return 0;
}
