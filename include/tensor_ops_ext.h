/* Additional tensor operations of the HIP backend.
 *
 * These entry points are additive: include/tensor_ops.h and the other
 * reference headers keep their declarations. Each op here is one the
 * reference computes only inside its compute vtable, its CUDA kernels or its
 * model harnesses (cited per entry), or one it lacks and that is defined in
 * closed form.
 *
 * Conventions (as include/tensor_ops.h):
 *   - return 1 on success, 0 on failure with a message in (error, capacity);
 *   - outputs are preallocated by the caller with the documented shape;
 *   - all operands of a call share one storage kind; device-storage calls
 *     enqueue on the SDK stream and return, host-storage calls are staged
 *     through device memory and return when the host output is written;
 *   - f16 tensors hold IEEE binary16; all arithmetic is done in f32 and
 *     rounded to nearest even on store; reductions accumulate in f32 (f64 for
 *     the global sum).
 */
#ifndef TENSOR_OPS_EXT_H
#define TENSOR_OPS_EXT_H

#include "tensor_buffer.h"

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- same-shape elementwise ------------------------------------------- */

/* out = a + b, F32. Reference: the F32 GRAPH_ADD loop,
   src/common/tensor_graph.c:453-459; vtable residual_add_f32
   (tensor_compute_cuda.cu:361-364, op 0). Bit-exact (one IEEE add). */
int tensor_add_f32(const TensorBuffer *left, const TensorBuffer *right,
                   TensorBuffer *output, char *error, size_t error_capacity);
/* out = a * b. No reference op: one IEEE multiply (f16: in f32, then RNE). */
int tensor_mul_f32(const TensorBuffer *left, const TensorBuffer *right,
                   TensorBuffer *output, char *error, size_t error_capacity);
int tensor_mul_f16(const TensorBuffer *left, const TensorBuffer *right,
                   TensorBuffer *output, char *error, size_t error_capacity);

/* out[i] = gelu(x[i]) with the tanh approximation and the reference clamps:
   x >= 5 -> x, x <= -5 -> 0, else 0.5 x (1 + tanh(0.7978845608 (x +
   0.044715 x^3))). Reference: tests/smolvlm/src/app/vision_model.c:230-254,
   tensor_compute_cuda.cu:298-319 (vtable gelu_f32/gelu_f16). */
int tensor_gelu_f32(const TensorBuffer *input, TensorBuffer *output,
                    char *error, size_t error_capacity);
int tensor_gelu_f16(const TensorBuffer *input, TensorBuffer *output,
                    char *error, size_t error_capacity);
/* out = gelu(input) * gate. Reference: tensor_compute_cuda.cu:321-331. */
int tensor_gelu_multiply_f16(const TensorBuffer *input, const TensorBuffer *gate,
                             TensorBuffer *output, char *error,
                             size_t error_capacity);
/* out = max(x, 0). Reference: tensor_compute_cuda.cu:333-336. */
int tensor_relu_f16(const TensorBuffer *input, TensorBuffer *output,
                    char *error, size_t error_capacity);
/* SwiGLU: out = silu(gate) * up = gate / (1 + exp(-gate)) * up.
   Reference: tests/smolvlm/src/app/text_model.c:876-884,
   tensor_compute_cuda.cu:361-369 (op 1; the first operand is the one passed
   through SiLU). */
int tensor_silu_multiply_f32(const TensorBuffer *gate, const TensorBuffer *up,
                             TensorBuffer *output, char *error,
                             size_t error_capacity);
int tensor_silu_multiply_f16(const TensorBuffer *gate, const TensorBuffer *up,
                             TensorBuffer *output, char *error,
                             size_t error_capacity);

/* ---- row broadcast ------------------------------------------------------ */

/* out[r, c] = x[r, c] + bias[c] over the last dimension (bias rank 1, width
   = last dim). The _gelu variants apply gelu() above to the sum.
   Reference: tensor_compute_cuda.cu:338-359 (bias_f32/f16_kernel, i % width),
   vtable bias_add_f32/f16 and bias_add_*_device. */
int tensor_bias_add_f32(const TensorBuffer *input, const TensorBuffer *bias,
                        TensorBuffer *output, char *error,
                        size_t error_capacity);
int tensor_bias_add_f16(const TensorBuffer *input, const TensorBuffer *bias,
                        TensorBuffer *output, char *error,
                        size_t error_capacity);
int tensor_bias_gelu_f32(const TensorBuffer *input, const TensorBuffer *bias,
                         TensorBuffer *output, char *error,
                         size_t error_capacity);
int tensor_bias_gelu_f16(const TensorBuffer *input, const TensorBuffer *bias,
                         TensorBuffer *output, char *error,
                         size_t error_capacity);

/* ---- strided / permuted views with broadcast operands ------------------- */

#define TENSOR_VIEW_MAX_RANK 8

/* A strided view of a buffer, in elements: element (i0, .., i{rank-1}) of the
   view is buffer element offset + sum_k i_k * strides[k]. Strides may be any
   non-negative values (permutations, slices, broadcast via stride 0). */
typedef struct {
    size_t rank;
    uint64_t shape[TENSOR_VIEW_MAX_RANK];
    int64_t strides[TENSOR_VIEW_MAX_RANK];
    uint64_t offset;
} TensorView;

/* out = (view(x) + addend) * multiplier, written contiguous with the view's
   shape. addend and multiplier are contiguous tensors of the view's rank whose
   dimensions are 1 or equal to the view's (numpy broadcasting); either may be
   NULL (then 0 / 1 are used and that operation is skipped, so with both NULL
   this is a strided copy). Every view element must lie inside x.
   No reference op: TensorBuffer has no strides (tensor_buffer.c:12-22);
   defined in closed form. */
int tensor_view_add_mul_f16(const TensorBuffer *input, const TensorView *view,
                            const TensorBuffer *addend,
                            const TensorBuffer *multiplier,
                            TensorBuffer *output, char *error,
                            size_t error_capacity);
int tensor_view_add_mul_f32(const TensorBuffer *input, const TensorView *view,
                            const TensorBuffer *addend,
                            const TensorBuffer *multiplier,
                            TensorBuffer *output, char *error,
                            size_t error_capacity);

/* ---- row reductions over the last dimension ----------------------------- */

/* Row softmax with the reference's rules (src/common/attention.c:335-380):
   with causal != 0 the input is [..., q_len, k_len] and key k of query row q
   is masked to -inf when k > q + (k_len > q_len ? k_len - q_len : 0);
   max ignores NaN; a row whose max is -inf becomes all zeros; a row holding
   +inf puts 1/count on each +inf and 0 elsewhere; otherwise
   p = exp(s - max) / sum(exp(s - max)). */
int tensor_softmax_f32(const TensorBuffer *input, int causal,
                       TensorBuffer *output, char *error,
                       size_t error_capacity);
int tensor_softmax_f16(const TensorBuffer *input, int causal,
                       TensorBuffer *output, char *error,
                       size_t error_capacity);
/* out[r] = sum / max of row r (F32 output of shape input.shape[:-1], or [1]
   for rank-1 input). No reference op (closed form). max is NaN if the row
   holds a NaN. */
int tensor_row_sum_f32(const TensorBuffer *input, TensorBuffer *output,
                       char *error, size_t error_capacity);
int tensor_row_sum_f16(const TensorBuffer *input, TensorBuffer *output,
                       char *error, size_t error_capacity);
int tensor_row_max_f32(const TensorBuffer *input, TensorBuffer *output,
                       char *error, size_t error_capacity);
int tensor_row_max_f16(const TensorBuffer *input, TensorBuffer *output,
                       char *error, size_t error_capacity);
/* Fused residual add + RMSNorm, the first two steps of the reference's FP16
   decoder layer (tests/smolvlm/src/app/text_model.c:701,735):
   sum = f16(x + residual) is written, and normalized = rms_norm_f16(sum, weight,
   epsilon) exactly as tensor_rms_norm_f16 would compute it from the stored
   sum. */
int tensor_residual_rms_norm_f16(const TensorBuffer *input,
                                 const TensorBuffer *residual,
                                 const TensorBuffer *weight, float epsilon,
                                 TensorBuffer *sum_output,
                                 TensorBuffer *normalized_output, char *error,
                                 size_t error_capacity);

/* ---- whole-tensor reductions --------------------------------------------- */

/* Global sum (F64 [1] output, accumulated in f32 per lane and f64 across
   lanes and blocks) and max (F32 [1], NaN if any element is NaN) of an F32
   tensor, in one two-pass grid reduction. Either output may be NULL.
   No reference op (closed form). */
int tensor_sum_max_f32(const TensorBuffer *input, TensorBuffer *sum_output,
                       TensorBuffer *max_output, char *error,
                       size_t error_capacity);
/* tensor_sum_max_f32 without any allocation. No counterpart in the
   reference: it is for callers that cannot allocate device memory (code
   under HIP graph capture, serving loops that forbid hipMalloc). Same
   validation, kernels and results as tensor_sum_max_f32; every operand must
   be a device tensor (host operands are refused, since staging them would
   allocate). The pass-1 partials live in a 64 KiB device array of the
   library, one per GPU, held until the process ends; it covers every input
   size (the pass-1 grid is capped), and a launch whose partials would not fit
   is refused with a message. Pass 1 writes every partial pass 2 reads, so
   the array keeps the last call's contents harmlessly. Calls are ordered on
   the library's one stream; any other use of the array that overlaps a call
   on the same GPU races with it. */
int tensor_sum_max_f32_no_alloc(const TensorBuffer *input, TensorBuffer *sum_output,
                                TensorBuffer *max_output, char *error,
                                size_t error_capacity);
/* Index (U32 [1] output) of the first maximum, with the reference's scan
   semantics (tensor_compute_cuda.cu:386-397): NaN elements never win, and if
   element 0 is NaN the result is 0. At most 2^32-1 elements. */
int tensor_argmax_f32(const TensorBuffer *input, TensorBuffer *index_output,
                      char *error, size_t error_capacity);
int tensor_argmax_f16(const TensorBuffer *input, TensorBuffer *index_output,
                      char *error, size_t error_capacity);

/* ---- rotary position embedding ----------------------------------------- */

/* Split-half (NeoX) RoPE applied in place to query [seq, query_heads,
   head_dim] and key [seq, key_heads, head_dim] (any shape with that element
   count). Pair (d, d + head_dim/2) of position p is rotated by
   angle = (float)((double)(position_offset + p) / pow(theta, 2d/head_dim)).
   Reference: tests/smolvlm/src/app/text_model.c:463-497,
   tensor_compute_cuda.cu:371-384 (vtable rope_f16 / rope_f32). */
int tensor_rope_f32(TensorBuffer *query, TensorBuffer *key, size_t query_heads,
                    size_t key_heads, size_t head_dim, double theta,
                    size_t position_offset, char *error,
                    size_t error_capacity);
int tensor_rope_f16(TensorBuffer *query, TensorBuffer *key, size_t query_heads,
                    size_t key_heads, size_t head_dim, double theta,
                    size_t position_offset, char *error,
                    size_t error_capacity);

/* ---- synthetic inputs --------------------------------------------------- */

/* Fill an F32 or F16 tensor with a counter-based splitmix64 stream: element
   i of (seed, stream) is a pure function of (seed, stream, i), so any range
   of it can be regenerated on the host. Uniform: lo + (hi - lo) * u with a
   24-bit u in [0, 1). Normal: Box-Muller in double, rounded to f32 (then to
   f16 by RNE). No reference counterpart (the reference has no PRNG). */
int tensor_fill_uniform(TensorBuffer *buffer, uint64_t seed, uint64_t stream,
                        float low, float high, char *error,
                        size_t error_capacity);
int tensor_fill_normal(TensorBuffer *buffer, uint64_t seed, uint64_t stream,
                       float mean, float std_dev, char *error,
                       size_t error_capacity);

/* ---- stream ------------------------------------------------------------- */

/* ---- attention on device buffers ------------------------------------------ */

/* Scaled dot-product attention on device-storage TensorBuffers, enqueued on
   the SDK stream: q [B,Hq,Lq,D], k [B,Hkv,Lkv,D], v [B,Hkv,Lkv,Dv],
   additive_mask [Lq,Lkv] or NULL, output [B,Hq,Lq,Dv]; query head h reads kv
   head h / (Hq / Hkv); causal masks key j of query i when
   j > i + (Lkv > Lq ? Lkv - Lq : 0). The arithmetic is the accelerator
   attention table's (include/attention_backend.h; the reference's CUDA
   backend, src/platform/cuda/attention_cuda.cu:25-99): a row whose largest
   score is not finite is all zeros, otherwise softmax(scores) @ v with f32
   accumulation. Mask values are used as given. D and Dv up to 512.
   No reference op: the reference's tensor_sdpa_f32/f16
   (src/common/attention.c:211-431) take host buffers only; shape checks and
   their messages are the same. */
int tensor_sdpa_device_f32(const TensorBuffer *query, const TensorBuffer *key,
                           const TensorBuffer *value,
                           const TensorBuffer *additive_mask, float scale,
                           int causal, TensorBuffer *output, char *error,
                           size_t error_capacity);
int tensor_sdpa_device_f16(const TensorBuffer *query, const TensorBuffer *key,
                           const TensorBuffer *value,
                           const TensorBuffer *additive_mask, float scale,
                           int causal, TensorBuffer *output, char *error,
                           size_t error_capacity);

/* The hipStream_t every SDK operation is ordered on (created on first use on
   the current device). Callers may record HIP events on it or make other
   streams wait on it. No reference counterpart (the CUDA backend uses the
   legacy default stream). */
void *tensor_device_hip_stream(void);

#ifdef __cplusplus
}
#endif

#endif
