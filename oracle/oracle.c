/* CPU oracle for the tensor-ops hot path — TEST INFRASTRUCTURE ONLY.
 * See oracle.h for what each function follows and how it is pinned.
 * Compiled with -std=c11 -ffp-contract=off: every float expression below is
 * evaluated as written, with no fused multiply-add.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- conversions -------------------------------------------------------- */

static uint32_t bits_of(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    return bits;
}

static float float_of(uint32_t bits) {
    float value;
    memcpy(&value, &bits, sizeof value);
    return value;
}

/* Follows src/common/tensor_f16.c:17-42: exact widening; subnormal halves are
   m * 2^-24 (exact in f32); NaN payload bits move to the top of the f32
   fraction unchanged. */
float orc_f16_to_f32(uint16_t value) {
    const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    const uint32_t exponent = (value >> 10) & 0x1fu;
    const uint32_t mantissa = value & 0x3ffu;
    if (exponent == 0x1fu) return float_of(sign | 0x7f800000u | (mantissa << 13));
    if (exponent != 0) return float_of(sign | ((exponent + 112u) << 23) | (mantissa << 13));
    const float magnitude = (float)mantissa * 0x1p-24f;
    return sign ? -magnitude : magnitude;
}

/* Follows src/common/tensor_f16.c:48-85: round to nearest even; values at or
   above 65520 become infinity; results below 2^-14 are rounded on the 2^-24
   grid (subnormals kept, exact ties to even); NaN keeps its sign and top ten
   payload bits, with a zero payload forced to 1. */
uint16_t orc_f32_to_f16(float value) {
    const uint32_t bits = bits_of(value);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t magnitude = bits & 0x7fffffffu;
    if (magnitude > 0x7f800000u) {
        const uint16_t payload = (uint16_t)((magnitude >> 13) & 0x3ffu);
        return (uint16_t)(sign | 0x7c00u | (payload ? payload : 1u));
    }
    if (magnitude >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
    if (magnitude >= 0x38800000u) {                                   /* >= 2^-14 */
        const uint32_t rebased = magnitude - 0x38000000u;              /* exponent - 112 */
        const uint32_t rounded = rebased + 0x0fffu + ((rebased >> 13) & 1u);
        return (uint16_t)(sign | (rounded >> 13));
    }
    if (magnitude <= 0x33000000u) return sign;                        /* <= 2^-25 */
    const uint32_t exponent = magnitude >> 23;                         /* 102..112 */
    const uint32_t significand = (magnitude & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - exponent;                            /* 14..24 */
    uint32_t quotient = significand >> shift;
    const uint32_t remainder = significand & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (remainder > half || (remainder == half && (quotient & 1u))) quotient++;
    return (uint16_t)(sign | quotient);
}

/* src/common/tensor_f16.c:44-46 */
float orc_bf16_to_f32(uint16_t value) { return float_of((uint32_t)value << 16); }

/* src/common/tensor_buffer.c:44-51: NaN is quietened, otherwise RNE. */
uint16_t orc_f32_to_bf16(float value) {
    const uint32_t bits = bits_of(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

void orc_f32_to_bf16_array(const float *x, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_f32_to_bf16(x[i]);
}

void orc_f16_to_f32_array(const uint16_t *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_f16_to_f32(x[i]);
}

void orc_f32_to_f16_array(const float *x, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_f32_to_f16(x[i]);
}

/* ---- synthetic inputs --------------------------------------------------- */

#define GOLDEN_GAMMA 0x9e3779b97f4a7c15ull

/* splitmix64 output function (Steele, Lea, Flood, "Fast splittable
   pseudorandom number generators", OOPSLA 2014). */
static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t orc_rng_bits(uint64_t seed, uint64_t stream, uint64_t index) {
    const uint64_t key = mix64(seed + GOLDEN_GAMMA * (2u * stream + 1u));
    return mix64(key + GOLDEN_GAMMA * (index + 1u));
}

static float uniform_value(uint64_t bits, float low, float high) {
    const float unit = (float)(bits >> 40) * 0x1p-24f;
    return low + (high - low) * unit;
}

static float normal_value(uint64_t bits, float mean, float std_dev) {
    const uint64_t second = mix64(bits ^ 0xd1b54a32d192ed03ull);
    const double u1 = (double)((bits >> 11) + 1u) * 0x1p-53;   /* (0, 1] */
    const double u2 = (double)(second >> 11) * 0x1p-53;         /* [0, 1) */
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    return (float)((double)mean + (double)std_dev * z);
}

void orc_fill_uniform_f32(float *y, size_t n, uint64_t seed, uint64_t stream,
                          uint64_t first, float low, float high) {
    for (size_t i = 0; i < n; i++)
        y[i] = uniform_value(orc_rng_bits(seed, stream, first + i), low, high);
}

void orc_fill_uniform_f16(uint16_t *y, size_t n, uint64_t seed, uint64_t stream,
                          uint64_t first, float low, float high) {
    for (size_t i = 0; i < n; i++)
        y[i] = orc_f32_to_f16(uniform_value(orc_rng_bits(seed, stream, first + i), low, high));
}

void orc_fill_normal_f32(float *y, size_t n, uint64_t seed, uint64_t stream,
                         uint64_t first, float mean, float std_dev) {
    for (size_t i = 0; i < n; i++)
        y[i] = normal_value(orc_rng_bits(seed, stream, first + i), mean, std_dev);
}

void orc_fill_normal_f16(uint16_t *y, size_t n, uint64_t seed, uint64_t stream,
                         uint64_t first, float mean, float std_dev) {
    for (size_t i = 0; i < n; i++)
        y[i] = orc_f32_to_f16(normal_value(orc_rng_bits(seed, stream, first + i), mean, std_dev));
}

/* ---- elementwise -------------------------------------------------------- */

/* src/common/tensor_graph.c:453-459 */
void orc_add_f32(const float *a, const float *b, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}

/* closed form: one IEEE multiply */
void orc_mul_f32(const float *a, const float *b, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = a[i] * b[i];
}

/* src/common/tensor_ops.c:614-620 */
void orc_add_f16(const uint16_t *a, const uint16_t *b, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = orc_f32_to_f16(orc_f16_to_f32(a[i]) + orc_f16_to_f32(b[i]));
}

/* closed form, same widening/rounding as the f16 add */
void orc_mul_f16(const uint16_t *a, const uint16_t *b, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = orc_f32_to_f16(orc_f16_to_f32(a[i]) * orc_f16_to_f32(b[i]));
}

/* src/common/tensor_ops.c:554-557 */
void orc_silu_f32(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        y[i] = v / (1.0f + expf(-v));
    }
}

/* src/common/tensor_ops.c:568-571 */
void orc_silu_f16(const uint16_t *x, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float v = orc_f16_to_f32(x[i]);
        y[i] = orc_f32_to_f16(v / (1.0f + expf(-v)));
    }
}

/* tests/smolvlm/src/app/vision_model.c:242-253; the same expression as
   tensor_compute_cuda.cu:302-305. Evaluated left to right in float:
   ((0.5*v) * (1 + tanhf(c1 * (v + ((c2*v)*v)*v)))). */
float orc_gelu_scalar(float v) {
    if (v >= 5.0f) return v;
    if (v <= -5.0f) return 0.0f;
    return 0.5f * v * (1.0f + tanhf(0.7978845608f * (v + 0.044715f * v * v * v)));
}

/* The same formula, constants and clamps evaluated in double: the arbiter
   for the cancellation of 1 + tanh(u) near v = -5. */
double orc_gelu_scalar_f64(double v) {
    const double c1 = (double)0.7978845608f, c2 = (double)0.044715f;
    if (v >= 5.0) return v;
    if (v <= -5.0) return 0.0;
    return 0.5 * v * (1.0 + tanh(c1 * (v + c2 * v * v * v)));
}

void orc_gelu_f32(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_gelu_scalar(x[i]);
}

/* tensor_compute_cuda.cu:310-319 (x >= 5 keeps the input half, which equals
   rounding the f32 value back) */
void orc_gelu_f16(const uint16_t *x, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_f32_to_f16(orc_gelu_scalar(orc_f16_to_f32(x[i])));
}

void orc_gelu_f64(const double *x, double *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_gelu_scalar_f64(x[i]);
}

/* tensor_compute_cuda.cu:321-331 */
void orc_gelu_multiply_f16(const uint16_t *x, const uint16_t *gate, uint16_t *y,
                           size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = orc_f32_to_f16(orc_gelu_scalar(orc_f16_to_f32(x[i])) * orc_f16_to_f32(gate[i]));
}

/* tensor_compute_cuda.cu:333-336: fmaxf(v, 0) rounded back; NaN and -0
   give +0. */
void orc_relu_f16(const uint16_t *x, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float v = orc_f16_to_f32(x[i]);
        y[i] = orc_f32_to_f16(v > 0.0f ? v : 0.0f);
    }
}

/* tests/smolvlm/src/app/text_model.c:880-883 and tensor_compute_cuda.cu:363 */
void orc_silu_multiply_f32(const float *gate, const float *up, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float v = gate[i];
        y[i] = v / (1.0f + expf(-v)) * up[i];
    }
}

/* tensor_compute_cuda.cu:366-369 (op 1) */
void orc_silu_multiply_f16(const uint16_t *gate, const uint16_t *up, uint16_t *y,
                           size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float v = orc_f16_to_f32(gate[i]);
        y[i] = orc_f32_to_f16(v / (1.0f + expf(-v)) * orc_f16_to_f32(up[i]));
    }
}

/* tensor_compute_cuda.cu:338-347 (i % width broadcast, optional GELU) */
void orc_bias_add_f32(const float *x, const float *bias, float *y, size_t rows,
                      size_t width, int gelu) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < width; c++) {
            const float v = x[r * width + c] + bias[c];
            y[r * width + c] = gelu ? orc_gelu_scalar(v) : v;
        }
}

/* tensor_compute_cuda.cu:349-359 */
void orc_bias_add_f16(const uint16_t *x, const uint16_t *bias, uint16_t *y,
                      size_t rows, size_t width, int gelu) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < width; c++) {
            const float v = orc_f16_to_f32(x[r * width + c]) + orc_f16_to_f32(bias[c]);
            y[r * width + c] = orc_f32_to_f16(gelu ? orc_gelu_scalar(v) : v);
        }
}

/* ---- row reductions ----------------------------------------------------- */

/* src/common/tensor_ops.c:418-428: sequential float sum of squares,
   scale = 1/sqrtf(sum/width + eps), y = (x * scale) * w */
void orc_rms_norm_f32(const float *x, const float *w, float *y, size_t rows,
                      size_t width, float eps) {
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * width;
        float squares = 0.0f;
        for (size_t c = 0; c < width; c++) squares += row[c] * row[c];
        const float scale = 1.0f / sqrtf(squares / (float)width + eps);
        for (size_t c = 0; c < width; c++) y[r * width + c] = row[c] * scale * w[c];
    }
}

/* src/common/tensor_ops.c:447-457 */
void orc_rms_norm_f16(const uint16_t *x, const uint16_t *w, uint16_t *y,
                      size_t rows, size_t width, float eps) {
    for (size_t r = 0; r < rows; r++) {
        const uint16_t *row = x + r * width;
        float squares = 0.0f;
        for (size_t c = 0; c < width; c++) {
            const float v = orc_f16_to_f32(row[c]);
            squares += v * v;
        }
        const float scale = 1.0f / sqrtf(squares / (float)width + eps);
        for (size_t c = 0; c < width; c++)
            y[r * width + c] = orc_f32_to_f16(orc_f16_to_f32(row[c]) * scale * orc_f16_to_f32(w[c]));
    }
}

/* src/common/tensor_ops.c:485-503: mean, then sum of squared deviations,
   inverse_std = 1/sqrtf(var/width + eps), optional scale then bias */
void orc_layer_norm_f32(const float *x, const float *scale, const float *bias,
                        float *y, size_t rows, size_t width, float eps) {
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * width;
        float mean = 0.0f;
        for (size_t c = 0; c < width; c++) mean += row[c];
        mean /= (float)width;
        float variance = 0.0f;
        for (size_t c = 0; c < width; c++) {
            const float d = row[c] - mean;
            variance += d * d;
        }
        const float inverse_std = 1.0f / sqrtf(variance / (float)width + eps);
        for (size_t c = 0; c < width; c++) {
            float v = (row[c] - mean) * inverse_std;
            if (scale) v *= scale[c];
            if (bias) v += bias[c];
            y[r * width + c] = v;
        }
    }
}

/* src/common/tensor_ops.c:525-541 */
void orc_layer_norm_f16(const uint16_t *x, const uint16_t *scale,
                        const uint16_t *bias, uint16_t *y, size_t rows,
                        size_t width, float eps) {
    for (size_t r = 0; r < rows; r++) {
        const uint16_t *row = x + r * width;
        float mean = 0.0f;
        for (size_t c = 0; c < width; c++) mean += orc_f16_to_f32(row[c]);
        mean /= (float)width;
        float variance = 0.0f;
        for (size_t c = 0; c < width; c++) {
            const float d = orc_f16_to_f32(row[c]) - mean;
            variance += d * d;
        }
        const float inverse_std = 1.0f / sqrtf(variance / (float)width + eps);
        for (size_t c = 0; c < width; c++) {
            float v = (orc_f16_to_f32(row[c]) - mean) * inverse_std;
            if (scale) v *= orc_f16_to_f32(scale[c]);
            if (bias) v += orc_f16_to_f32(bias[c]);
            y[r * width + c] = orc_f32_to_f16(v);
        }
    }
}

/* residual add (tensor_ops.c:614-620) followed by RMSNorm of the stored sum
   (tensor_ops.c:447-457), as tests/smolvlm/src/app/text_model.c:735 then :701 */
void orc_residual_rms_norm_f16(const uint16_t *x, const uint16_t *r,
                               const uint16_t *w, uint16_t *sum, uint16_t *y,
                               size_t rows, size_t width, float eps) {
    orc_add_f16(x, r, sum, rows * width);
    orc_rms_norm_f16(sum, w, y, rows, width, eps);
}

/* src/common/attention.c:335-380 applied to one row of scores already in
   `row` (f32). q_len == 0 means no causal mask. */
static void softmax_row(float *row, size_t width, size_t q_len, size_t q) {
    const size_t offset = q_len && width > q_len ? width - q_len : 0;
    float maximum = -INFINITY;
    size_t positive_infinities = 0;
    for (size_t k = 0; k < width; k++) {
        if (q_len && k > q + offset) row[k] = -INFINITY;
        if (row[k] == INFINITY) positive_infinities++;
        if (row[k] > maximum) maximum = row[k];
    }
    if (maximum == -INFINITY) {
        for (size_t k = 0; k < width; k++) row[k] = 0.0f;
        return;
    }
    float denominator = 0.0f;
    if (positive_infinities == 0) {
        for (size_t k = 0; k < width; k++) {
            row[k] = expf(row[k] - maximum);
            denominator += row[k];
        }
    } else {
        denominator = (float)positive_infinities;
        for (size_t k = 0; k < width; k++) row[k] = row[k] == INFINITY ? 1.0f : 0.0f;
    }
    for (size_t k = 0; k < width; k++) row[k] /= denominator;
}

void orc_softmax_f32(const float *x, float *y, size_t rows, size_t width,
                     size_t q_len) {
    for (size_t r = 0; r < rows; r++) {
        memcpy(y + r * width, x + r * width, width * sizeof(float));
        softmax_row(y + r * width, width, q_len, q_len ? r % q_len : 0);
    }
}

void orc_softmax_f16(const uint16_t *x, uint16_t *y, size_t rows, size_t width,
                     size_t q_len) {
    float *row = malloc(width * sizeof(float));
    if (row == NULL) return;
    for (size_t r = 0; r < rows; r++) {
        for (size_t k = 0; k < width; k++) row[k] = orc_f16_to_f32(x[r * width + k]);
        softmax_row(row, width, q_len, q_len ? r % q_len : 0);
        for (size_t k = 0; k < width; k++) y[r * width + k] = orc_f32_to_f16(row[k]);
    }
    free(row);
}

/* closed form: float64 accumulation, plus sum |x| for error bounds */
void orc_row_sum_f32(const float *x, double *sum, double *abs_sum, size_t rows,
                     size_t width) {
    for (size_t r = 0; r < rows; r++) {
        double s = 0.0, a = 0.0;
        for (size_t c = 0; c < width; c++) {
            s += (double)x[r * width + c];
            a += fabs((double)x[r * width + c]);
        }
        sum[r] = s;
        if (abs_sum) abs_sum[r] = a;
    }
}

void orc_row_sum_f16(const uint16_t *x, double *sum, double *abs_sum,
                     size_t rows, size_t width) {
    for (size_t r = 0; r < rows; r++) {
        double s = 0.0, a = 0.0;
        for (size_t c = 0; c < width; c++) {
            const double v = (double)orc_f16_to_f32(x[r * width + c]);
            s += v;
            a += fabs(v);
        }
        sum[r] = s;
        if (abs_sum) abs_sum[r] = a;
    }
}

static float max_with_nan(const float *values, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (isnan(values[i])) return NAN;
        if (values[i] > m) m = values[i];
    }
    return m;
}

/* closed form: exact max, NaN if the row holds a NaN */
void orc_row_max_f32(const float *x, float *y, size_t rows, size_t width) {
    for (size_t r = 0; r < rows; r++) y[r] = max_with_nan(x + r * width, width);
}

void orc_row_max_f16(const uint16_t *x, float *y, size_t rows, size_t width) {
    for (size_t r = 0; r < rows; r++) {
        float m = -INFINITY;
        for (size_t c = 0; c < width; c++) {
            const float v = orc_f16_to_f32(x[r * width + c]);
            if (isnan(v)) { m = NAN; break; }
            if (v > m) m = v;
        }
        y[r] = m;
    }
}

/* ---- whole-tensor reductions ------------------------------------------- */

/* closed form: float64 sum and sum |x|, exact max (NaN propagates) */
void orc_sum_max_f32(const float *x, size_t n, double *sum, double *abs_sum,
                     float *max) {
    double s = 0.0, a = 0.0;
    for (size_t i = 0; i < n; i++) {
        s += (double)x[i];
        a += fabs((double)x[i]);
    }
    if (sum) *sum = s;
    if (abs_sum) *abs_sum = a;
    if (max) *max = max_with_nan(x, n);
}

/* tensor_compute_cuda.cu:386-397: linear scan from element 0, strict > */
uint32_t orc_argmax_f32(const float *x, size_t n) {
    size_t best = 0;
    float maximum = x[0];
    for (size_t i = 1; i < n; i++)
        if (x[i] > maximum) { maximum = x[i]; best = i; }
    return (uint32_t)best;
}

uint32_t orc_argmax_f16(const uint16_t *x, size_t n) {
    size_t best = 0;
    float maximum = orc_f16_to_f32(x[0]);
    for (size_t i = 1; i < n; i++) {
        const float v = orc_f16_to_f32(x[i]);
        if (v > maximum) { maximum = v; best = i; }
    }
    return (uint32_t)best;
}

/* ---- rope --------------------------------------------------------------- */

/* tests/smolvlm/src/app/text_model.c:477-496 (f32, in place) with the
   position offset of tensor_compute_cuda.cu:376-383 */
void orc_rope_f32(float *q, float *k, size_t seq, size_t qh, size_t kh,
                  size_t dim, double theta, size_t offset) {
    const size_t half = dim / 2;
    for (size_t p = 0; p < seq; p++)
        for (size_t d = 0; d < half; d++) {
            const float angle = (float)((double)(offset + p) /
                                        pow(theta, (2.0 * (double)d) / (double)dim));
            const float c = cosf(angle), s = sinf(angle);
            for (size_t h = 0; h < qh; h++) {
                float *base = q + (p * qh + h) * dim;
                const float left = base[d], right = base[d + half];
                base[d] = left * c - right * s;
                base[d + half] = right * c + left * s;
            }
            for (size_t h = 0; h < kh; h++) {
                float *base = k + (p * kh + h) * dim;
                const float left = base[d], right = base[d + half];
                base[d] = left * c - right * s;
                base[d + half] = right * c + left * s;
            }
        }
}

/* tensor_compute_cuda.cu:371-384 with f16 storage */
void orc_rope_f16(uint16_t *q, uint16_t *k, size_t seq, size_t qh, size_t kh,
                  size_t dim, double theta, size_t offset) {
    const size_t half = dim / 2;
    for (size_t p = 0; p < seq; p++)
        for (size_t d = 0; d < half; d++) {
            const float angle = (float)((double)(offset + p) /
                                        pow(theta, (2.0 * (double)d) / (double)dim));
            const float c = cosf(angle), s = sinf(angle);
            for (size_t pass = 0; pass < 2; pass++) {
                uint16_t *data = pass ? k : q;
                const size_t heads = pass ? kh : qh;
                for (size_t h = 0; h < heads; h++) {
                    uint16_t *base = data + (p * heads + h) * dim;
                    const float left = orc_f16_to_f32(base[d]);
                    const float right = orc_f16_to_f32(base[d + half]);
                    base[d] = orc_f32_to_f16(left * c - right * s);
                    base[d + half] = orc_f32_to_f16(right * c + left * s);
                }
            }
        }
}

/* ---- strided views ------------------------------------------------------ */

static size_t broadcast_offset(const uint64_t *shape, size_t rank,
                               const uint64_t *index) {
    size_t offset = 0;
    for (size_t d = 0; d < rank; d++)
        offset = offset * (size_t)shape[d] + (shape[d] == 1 ? 0 : (size_t)index[d]);
    return offset;
}

/* closed form: y[i] = (x[view(i)] + addend[bcast(i)]) * mult[bcast(i)] in f32,
   rounded to f16 */
void orc_view_add_mul_f16(const uint16_t *x, size_t rank, const uint64_t *shape,
                          const int64_t *strides, uint64_t offset,
                          const uint16_t *addend, const uint64_t *addend_shape,
                          const uint16_t *mult, const uint64_t *mult_shape,
                          uint16_t *y) {
    size_t total = 1;
    for (size_t d = 0; d < rank; d++) total *= (size_t)shape[d];
    uint64_t index[16] = {0};
    for (size_t i = 0; i < total; i++) {
        size_t rest = i;
        int64_t source = (int64_t)offset;
        for (size_t d = rank; d-- > 0;) {
            index[d] = rest % shape[d];
            rest /= shape[d];
            source += (int64_t)index[d] * strides[d];
        }
        float v = orc_f16_to_f32(x[source]);
        if (addend) v = v + orc_f16_to_f32(addend[broadcast_offset(addend_shape, rank, index)]);
        if (mult) v = v * orc_f16_to_f32(mult[broadcast_offset(mult_shape, rank, index)]);
        y[i] = orc_f32_to_f16(v);
    }
}

void orc_view_add_mul_f32(const float *x, size_t rank, const uint64_t *shape,
                          const int64_t *strides, uint64_t offset,
                          const float *addend, const uint64_t *addend_shape,
                          const float *mult, const uint64_t *mult_shape,
                          float *y) {
    size_t total = 1;
    for (size_t d = 0; d < rank; d++) total *= (size_t)shape[d];
    uint64_t index[16] = {0};
    for (size_t i = 0; i < total; i++) {
        size_t rest = i;
        int64_t source = (int64_t)offset;
        for (size_t d = rank; d-- > 0;) {
            index[d] = rest % shape[d];
            rest /= shape[d];
            source += (int64_t)index[d] * strides[d];
        }
        float v = x[source];
        if (addend) v = v + addend[broadcast_offset(addend_shape, rank, index)];
        if (mult) v = v * mult[broadcast_offset(mult_shape, rank, index)];
        y[i] = v;
    }
}

/* ---- embedding lookup ---------------------------------------------------- */

/* Index reading follows src/common/tensor_ops.c:41-84: I16/U16/I32/U32/I64/
   U64 only (TensorDType numbering 4..9), signed values below zero rejected. */
static int read_index(const void *indices, int dtype, size_t position, uint64_t *out) {
    const unsigned char *p = (const unsigned char *)indices;
    switch (dtype) {
        case 4: { int16_t v; memcpy(&v, p + position * 2, 2); if (v < 0) return 0; *out = (uint64_t)v; return 1; }
        case 5: { uint16_t v; memcpy(&v, p + position * 2, 2); *out = v; return 1; }
        case 6: { int32_t v; memcpy(&v, p + position * 4, 4); if (v < 0) return 0; *out = (uint64_t)v; return 1; }
        case 7: { uint32_t v; memcpy(&v, p + position * 4, 4); *out = v; return 1; }
        case 8: { int64_t v; memcpy(&v, p + position * 8, 8); if (v < 0) return 0; *out = (uint64_t)v; return 1; }
        case 9: { uint64_t v; memcpy(&v, p + position * 8, 8); *out = v; return 1; }
        default: return 0;
    }
}

/* Follows src/common/tensor_ops.c:86-161: every index is checked (readable,
   not negative, below table_rows) before any row is written; then row i of
   the output is a byte copy of table row indices[i]. */
int orc_embedding_lookup(const void *table, size_t table_rows, size_t row_bytes,
                         const void *indices, int index_dtype, size_t count, void *out) {
    for (size_t i = 0; i < count; i++) {
        uint64_t id;
        if (!read_index(indices, index_dtype, i, &id) || id >= table_rows) return 0;
    }
    for (size_t i = 0; i < count; i++) {
        uint64_t id = 0;
        read_index(indices, index_dtype, i, &id);
        memcpy((unsigned char *)out + i * row_bytes,
               (const unsigned char *)table + (size_t)id * row_bytes, row_bytes);
    }
    return 1;
}

/* Follows the compute-table slot semantics of
   src/platform/cuda/tensor_compute_cuda.cu:53-67: uint32 ids, an id at or
   past table_rows yields a zero row. */
void orc_embedding_gather_u32(const void *table, size_t table_rows, size_t row_bytes,
                              const uint32_t *ids, size_t count, void *out) {
    for (size_t i = 0; i < count; i++) {
        unsigned char *dst = (unsigned char *)out + i * row_bytes;
        if (ids[i] < table_rows)
            memcpy(dst, (const unsigned char *)table + (size_t)ids[i] * row_bytes, row_bytes);
        else
            memset(dst, 0, row_bytes);
    }
}

/* ---- scaled dot-product attention (accelerator semantics) ---------------- */

/* Follows the accelerator path that tensor_sdpa_f32/f16 take
   (src/common/attention.c:196-209, :402-429) as the CUDA backend computes it,
   src/platform/cuda/attention_cuda.cu:25-99:
     score = (sum_d q[d] k[d], in d order) * scale, + mask[q][k] if a mask is
             given, and -inf where causal and key > query + (kv_len - q_len);
     row max over the non-NaN scores; a row whose max is not finite becomes
             all zeros; otherwise p = expf(s - max), sum in key order,
             p *= (sum == 0 ? 0 : 1 / sum);
     out[dv] = sum over keys (in order) of p * v[key][dv].
   Layouts: q [B, Hq, Lq, D], k [B, Hkv, Lkv, D], v [B, Hkv, Lkv, Dv],
   mask [Lq, Lkv], out [B, Hq, Lq, Dv]; query head h reads kv head
   h / (Hq / Hkv). `scores` is caller scratch of Lkv floats. Inputs are read
   through `load` (f32 or f16 bits), outputs written through `store`. */
typedef float (*orc_load_fn)(const void *, size_t);
static float load_f32(const void *p, size_t i) { return ((const float *)p)[i]; }
static float load_f16(const void *p, size_t i) { return orc_f16_to_f32(((const uint16_t *)p)[i]); }

static void sdpa_generic(const void *q, const void *k, const void *v, const void *mask,
                         void *out, int f16, size_t batch, size_t qh, size_t kvh, size_t ql,
                         size_t kl, size_t dim, size_t vdim, float scale, int causal,
                         float *scores) {
    const orc_load_fn load = f16 ? load_f16 : load_f32;
    const size_t group = qh / kvh;
    const size_t offset = kl > ql ? kl - ql : 0;
    for (size_t b = 0; b < batch; b++)
        for (size_t h = 0; h < qh; h++) {
            const size_t kv = h / group;
            for (size_t i = 0; i < ql; i++) {
                const size_t qo = ((b * qh + h) * ql + i) * dim;
                float maximum = -INFINITY;
                for (size_t j = 0; j < kl; j++) {
                    const size_t ko = ((b * kvh + kv) * kl + j) * dim;
                    float sum = 0.0f;
                    for (size_t d = 0; d < dim; d++) sum += load(q, qo + d) * load(k, ko + d);
                    sum *= scale;
                    if (mask != NULL) sum += load(mask, i * kl + j);
                    if (causal && j > i + offset) sum = -INFINITY;
                    scores[j] = sum;
                    if (sum > maximum) maximum = sum;
                }
                const size_t oo = ((b * qh + h) * ql + i) * vdim;
                if (!isfinite(maximum)) {
                    for (size_t j = 0; j < kl; j++) scores[j] = 0.0f;
                } else {
                    float total = 0.0f;
                    for (size_t j = 0; j < kl; j++) {
                        scores[j] = expf(scores[j] - maximum);
                        total += scores[j];
                    }
                    const float inverse = total == 0.0f ? 0.0f : 1.0f / total;
                    for (size_t j = 0; j < kl; j++) scores[j] *= inverse;
                }
                for (size_t e = 0; e < vdim; e++) {
                    float acc = 0.0f;
                    for (size_t j = 0; j < kl; j++)
                        acc += scores[j] * load(v, ((b * kvh + kv) * kl + j) * vdim + e);
                    if (f16) ((uint16_t *)out)[oo + e] = orc_f32_to_f16(acc);
                    else ((float *)out)[oo + e] = acc;
                }
            }
        }
}

void orc_sdpa_f32(const float *q, const float *k, const float *v, const float *mask, float *out,
                  size_t batch, size_t qh, size_t kvh, size_t ql, size_t kl, size_t dim,
                  size_t vdim, float scale, int causal, float *scores) {
    sdpa_generic(q, k, v, mask, out, 0, batch, qh, kvh, ql, kl, dim, vdim, scale, causal, scores);
}

void orc_sdpa_f16(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *mask,
                  uint16_t *out, size_t batch, size_t qh, size_t kvh, size_t ql, size_t kl,
                  size_t dim, size_t vdim, float scale, int causal, float *scores) {
    sdpa_generic(q, k, v, mask, out, 1, batch, qh, kvh, ql, kl, dim, vdim, scale, causal, scores);
}

/* Per output element, sum over keys of p * |v| (same p as above), the scale
   against which a reordered accumulation's error is bounded. Written as f64. */
void orc_sdpa_abs_weight(const void *q, const void *k, const void *v, const void *mask,
                         double *out, int f16, size_t batch, size_t qh, size_t kvh, size_t ql,
                         size_t kl, size_t dim, size_t vdim, float scale, int causal,
                         float *scores) {
    const orc_load_fn load = f16 ? load_f16 : load_f32;
    const size_t group = qh / kvh;
    const size_t offset = kl > ql ? kl - ql : 0;
    for (size_t b = 0; b < batch; b++)
        for (size_t h = 0; h < qh; h++) {
            const size_t kv = h / group;
            for (size_t i = 0; i < ql; i++) {
                const size_t qo = ((b * qh + h) * ql + i) * dim;
                float maximum = -INFINITY;
                for (size_t j = 0; j < kl; j++) {
                    const size_t ko = ((b * kvh + kv) * kl + j) * dim;
                    float sum = 0.0f;
                    for (size_t d = 0; d < dim; d++) sum += load(q, qo + d) * load(k, ko + d);
                    sum *= scale;
                    if (mask != NULL) sum += load(mask, i * kl + j);
                    if (causal && j > i + offset) sum = -INFINITY;
                    scores[j] = sum;
                    if (sum > maximum) maximum = sum;
                }
                double total = 0.0;
                if (isfinite(maximum))
                    for (size_t j = 0; j < kl; j++) total += exp((double)scores[j] - maximum);
                const size_t oo = ((b * qh + h) * ql + i) * vdim;
                for (size_t e = 0; e < vdim; e++) {
                    double acc = 0.0;
                    if (isfinite(maximum) && total > 0.0)
                        for (size_t j = 0; j < kl; j++)
                            acc += exp((double)scores[j] - maximum) / total *
                                   fabs((double)load(v, ((b * kvh + kv) * kl + j) * vdim + e));
                    out[oo + e] = acc;
                }
            }
        }
}

/* ---- matmul / linear (src/common/tensor_ops.c:163-398) ------------------ */

/* tensor_ops.c:163-193 (f32) and :195-215 (f16 through f32): one float sum
   per output, started at 0, over the inner index in order. */
void orc_matmul_f32(const float *a, const float *b, float *y, size_t rows, size_t inner,
                    size_t cols) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) {
            float sum = 0.0f;
            for (size_t k = 0; k < inner; k++) sum += a[r * inner + k] * b[k * cols + c];
            y[r * cols + c] = sum;
        }
}

void orc_matmul_f16(const uint16_t *a, const uint16_t *b, uint16_t *y, size_t rows,
                    size_t inner, size_t cols) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) {
            float sum = 0.0f;
            for (size_t k = 0; k < inner; k++)
                sum += orc_f16_to_f32(a[r * inner + k]) * orc_f16_to_f32(b[k * cols + c]);
            y[r * cols + c] = orc_f32_to_f16(sum);
        }
}

/* Host path of tensor_linear_f32 (tensor_ops.c:290-307) and _f16 (:389-396):
   y[r][o] = bias[o] (or 0) + sum_i x[r][i] * w[o][i], one float sum in input
   order; f16 rounds once at the end. */
void orc_linear_f32(const float *x, const float *w, const float *bias, float *y, size_t rows,
                    size_t in, size_t out) {
    for (size_t r = 0; r < rows; r++)
        for (size_t o = 0; o < out; o++) {
            float sum = bias == NULL ? 0.0f : bias[o];
            for (size_t i = 0; i < in; i++) sum += x[r * in + i] * w[o * in + i];
            y[r * out + o] = sum;
        }
}

void orc_linear_f16(const uint16_t *x, const uint16_t *w, const uint16_t *bias, uint16_t *y,
                    size_t rows, size_t in, size_t out) {
    for (size_t r = 0; r < rows; r++)
        for (size_t o = 0; o < out; o++) {
            float sum = bias == NULL ? 0.0f : orc_f16_to_f32(bias[o]);
            for (size_t i = 0; i < in; i++)
                sum += orc_f16_to_f32(x[r * in + i]) * orc_f16_to_f32(w[o * in + i]);
            y[r * out + o] = orc_f32_to_f16(sum);
        }
}

/* ---- Q8_0 / Q4_0 weights (src/common/tensor_quant.c) --------------------- */

/* The quantizer's own scale rounding (tensor_quant.c:28-46): round to nearest
   even for normal halves. Below 2^-14 the reference adds half of the dropped
   range and shifts by 13 - e instead of 14 - e, so the stored bits are
   round-half-up(v * 2^25): twice the subnormal value v would round to.
   Magnitudes under 2^-25 become signed zero. Kept as the reference has it:
   the packed bytes are its format. */
static uint16_t quant_scale_to_f16(float value) {
    const uint32_t bits = bits_of(value);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const int exponent = (int)((bits >> 23) & 255u) - 127 + 15;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent <= 0) {
        if (exponent < -10) return sign;
        mantissa |= 0x800000u;
        const int shift = 13 + -exponent;
        return (uint16_t)(sign | ((mantissa + (1u << (shift - 1))) >> shift));
    }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    mantissa += 0xfffu + ((mantissa >> 13) & 1u);
    if (mantissa & 0x800000u) return (uint16_t)(sign | (uint16_t)((exponent + 1) << 10));
    return (uint16_t)(sign | (uint16_t)(exponent << 10) | (uint16_t)(mantissa >> 13));
}

uint16_t orc_quant_scale_to_f16(float value) { return quant_scale_to_f16(value); }

/* tensor_quantize_linear_weight_f16 (tensor_quant.c:48-100) into `dst`
   ([out, in/32, 34 or 18] bytes). Per 32-weight block: Q8_0 stores
   scale = max|x| / 127 and q = clamp(lrintf(x / scale), -127, 127) as int8;
   Q4_0 stores scale = x* / -8 (x* the first element of largest magnitude)
   and q = clamp((int)(x / scale + 8.5), 0, 15) packed two per byte (element
   j low nibble, j + 16 high nibble). Returns 0 (dst partly written) on a
   non-finite weight or unsupported arguments. */
int orc_quantize_f16(const uint16_t *weight, size_t out, size_t in, int format, uint8_t *dst) {
    const size_t block_bytes = format == 1 ? 34 : format == 2 ? 18 : 0;
    if (weight == NULL || out == 0 || in == 0 || in % 32 || block_bytes == 0) return 0;
    const size_t blocks = in / 32;
    for (size_t row = 0; row < out; row++)
        for (size_t b = 0; b < blocks; b++) {
            float x[32], max_abs = 0.0f, max_signed = 0.0f;
            for (size_t j = 0; j < 32; j++) {
                x[j] = orc_f16_to_f32(weight[row * in + b * 32 + j]);
                if (!isfinite(x[j])) return 0;
                if (fabsf(x[j]) > max_abs) max_abs = fabsf(x[j]);
                if (fabsf(x[j]) > fabsf(max_signed)) max_signed = x[j];
            }
            uint8_t *block = dst + (row * blocks + b) * block_bytes;
            const float scale = format == 1 ? max_abs / 127.0f : max_signed / -8.0f;
            const uint16_t half = quant_scale_to_f16(scale);
            block[0] = (uint8_t)half;
            block[1] = (uint8_t)(half >> 8);
            const float inverse = scale == 0.0f ? 0.0f : 1.0f / scale;
            if (format == 1) {
                for (size_t j = 0; j < 32; j++) {
                    long q = lrintf(x[j] * inverse);
                    if (q < -127) q = -127;
                    if (q > 127) q = 127;
                    block[2 + j] = (uint8_t)(int8_t)q;
                }
            } else {
                for (size_t j = 0; j < 16; j++) {
                    int lo = (int)(x[j] * inverse + 8.5f);
                    int hi = (int)(x[j + 16] * inverse + 8.5f);
                    lo = lo < 0 ? 0 : lo > 15 ? 15 : lo;
                    hi = hi < 0 ? 0 : hi > 15 ? 15 : hi;
                    block[2 + j] = (uint8_t)(lo | (hi << 4));
                }
            }
        }
    return 1;
}

/* Weight k (0..31) of a packed block: int8 for Q8_0, nibble - 8 for Q4_0
   (src/platform/cuda/tensor_compute_cuda.cu:230-233). */
static int quant_value(const uint8_t *block, int q8, size_t k) {
    if (q8) return (int)(int8_t)block[2 + k];
    const uint8_t packed = block[2 + (k & 15)];
    return (int)(k < 16 ? packed & 15 : packed >> 4) - 8;
}

static float quant_scale(const uint8_t *block) {
    return orc_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
}

/* The CUDA backend's quantized linear (tensor_compute_cuda.cu:216-238):
   y[r][o] = f16(sum over blocks b, then k of fmaf(x[r][32b+k], scale_b * q,
   sum)), one float sum per output started at 0. */
void orc_linear_quant_f16(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                          size_t in, size_t out, int q8) {
    const size_t blocks = in / 32, block_bytes = q8 ? 34 : 18;
    for (size_t r = 0; r < rows; r++)
        for (size_t o = 0; o < out; o++) {
            const uint8_t *base = w + o * blocks * block_bytes;
            float sum = 0.0f;
            for (size_t b = 0; b < blocks; b++) {
                const uint8_t *block = base + b * block_bytes;
                const float scale = quant_scale(block);
                for (size_t k = 0; k < 32; k++)
                    sum = fmaf(orc_f16_to_f32(x[r * in + b * 32 + k]),
                               scale * (float)quant_value(block, q8, k), sum);
            }
            y[r * out + o] = orc_f32_to_f16(sum);
        }
}

/* sum over k of |x[r][k] * scale * q| in double: the error scale of any
   reordered accumulation of the products above. */
void orc_linear_quant_abs_weight(const uint16_t *x, const uint8_t *w, double *y, size_t rows,
                                 size_t in, size_t out, int q8) {
    const size_t blocks = in / 32, block_bytes = q8 ? 34 : 18;
    for (size_t r = 0; r < rows; r++)
        for (size_t o = 0; o < out; o++) {
            const uint8_t *base = w + o * blocks * block_bytes;
            double sum = 0.0;
            for (size_t b = 0; b < blocks; b++) {
                const uint8_t *block = base + b * block_bytes;
                const double scale = quant_scale(block);
                for (size_t k = 0; k < 32; k++)
                    sum += fabs((double)orc_f16_to_f32(x[r * in + b * 32 + k]) * scale *
                                (double)quant_value(block, q8, k));
            }
            y[r * out + o] = sum;
        }
}
