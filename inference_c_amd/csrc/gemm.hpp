// Library GEMMs (hipBLASLt) behind the linear and matmul entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "safetensors.h"

namespace icsdk {

// Row-major operands, f32 accumulation, F32 or F16 storage (dtype):
//   kLinear: y[rows][cols] = x[rows][inner] * w[cols][inner]^T (+ bias[cols])
//   kMatmul: y[rows][cols] = x[rows][inner] * w[inner][cols]   (+ bias[cols])
// The bias is added to the f32 accumulator before the single rounding to
// the output type. Requires rows, inner, cols >= 1. Enqueues on `stream`;
// on failure writes a message and returns false.
enum class GemmKind { kLinear, kMatmul };

bool gemm(GemmKind kind, TensorDType dtype, const void *x, const void *w, const void *bias,
          void *y, size_t rows, size_t inner, size_t cols, hipStream_t stream, char *error,
          size_t capacity);

// Frees the cached plans and the workspace (release_cache).
void gemm_release();

}  // namespace icsdk
