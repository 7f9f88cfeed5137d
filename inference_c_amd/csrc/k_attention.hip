// Scaled dot-product attention for gfx950, with the accelerator semantics of
// the reference's attention backends (src/platform/cuda/attention_cuda.cu:
// 25-99):
//     s[j]   = (sum over d, in order, of q[d] k[j][d]) * scale (+ mask[i][j]),
//              -inf where causal and j > i + (kv_len - q_len);
//     a row whose maximum score (NaN ignored) is not finite is all zeros;
//     p[j]   = exp(s[j] - max) / sum_j exp(s[j] - max);
//     out[e] = sum_j p[j] v[j][e].
// q [B, Hq, Lq, D], k [B, Hkv, Lkv, D], v [B, Hkv, Lkv, Dv], mask [Lq, Lkv],
// out [B, Hq, Lq, Dv]; query head h reads kv head h / (Hq / Hkv).
//
// Row kernel (any D, Dv up to 512; f32 and f16): one wave per query row,
// keys in chunks of 64 with the running max and sum of an online softmax.
// Within a chunk, lane j owns key j: it forms the score as a sequential f32
// dot product (the same order and roundings as the reference, so scores are
// bit-identical), the wave folds the chunk into the running max and sum, and
// then lane e owns output element e (+64, +128, ...) and accumulates
// p[j] * v[j][e] over the chunk, reading p[j] and q[d] from the owning lane
// with v_readlane. No LDS and no barriers. The weights are normalised once at
// the end (acc / sum) rather than per weight, and the online rescaling
// reorders the roundings of p; outputs therefore agree with the reference to
// a few roundings of sum_j p_j |v_j|.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

constexpr int kMaxRowRegs = 8;  // D, Dv <= 8 * 64

struct SdpaArgs {
    uint32_t batch, qh, kvh, group;   // group = qh / kvh
    uint32_t ql, kl, dim, vdim;
    uint32_t causal_offset;           // kl > ql ? kl - ql : 0
    float scale;
    int causal;
};

__device__ inline float broadcast_lane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// exp for the softmax weights: libm-accurate for f32 outputs, the hardware
// exp2 path for f16 outputs (its error is far below half an f16 ulp).
template <typename S>
__device__ inline float attn_exp(float x) {
    if constexpr (sizeof(S) == 2) return fast_exp(x);
    else return expf(x);
}

// Score of the lane's key row: q . k in d order (sequential f32 sums, no
// contraction), q[d] taken from lane d % 64 of register d / 64. kVec: rows
// are whole, aligned 16-byte vectors.
template <typename S, bool kVec>
__device__ inline float row_dot(const float (&qreg)[kMaxRowRegs], const S *krow, uint32_t dim) {
    constexpr uint32_t E = Vec16<S>::N;
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) {
        const uint32_t d0 = (uint32_t)t * kWave;
        if (d0 >= dim) break;
        const uint32_t dn = min(dim - d0, (uint32_t)kWave);
        if constexpr (kVec) {
            for (uint32_t dd = 0; dd < dn; dd += E) {
                const Vec16<S> kv = load16(krow + d0 + dd);
#pragma unroll
                for (uint32_t e = 0; e < E; ++e)
                    sum = sum + broadcast_lane(qreg[t], (int)(dd + e)) * Elem<S>::load(kv.v[e]);
            }
        } else {
            for (uint32_t dd = 0; dd < dn; ++dd)
                sum = sum + broadcast_lane(qreg[t], (int)dd) * Elem<S>::load(krow[d0 + dd]);
        }
    }
    return sum;
}

template <typename S, bool kVec>
__global__ __launch_bounds__(kBlock) void sdpa_row_kernel(const S *__restrict__ q,
                                                          const S *__restrict__ k,
                                                          const S *__restrict__ v,
                                                          const S *__restrict__ mask,
                                                          S *__restrict__ out, SdpaArgs a) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const size_t row = (size_t)blockIdx.x * (kBlock / kWave) +
                       (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const size_t rows = (size_t)a.batch * a.qh * a.ql;
    if (row >= rows) return;
    const uint32_t i = (uint32_t)(row % a.ql);          // query position
    const size_t bh = row / a.ql;                        // batch * qh + head
    const uint32_t head = (uint32_t)(bh % a.qh);
    const size_t b = bh / a.qh;
    const size_t kv = b * a.kvh + head / a.group;
    const S *qrow = q + row * a.dim;
    const S *kbase = k + kv * a.kl * a.dim;
    const S *vbase = v + kv * a.kl * a.vdim;

    // q[d] lives in lane d % 64, register d / 64
    float qreg[kMaxRowRegs];
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) {
        const uint32_t d = lane + t * kWave;
        qreg[t] = d < a.dim ? Elem<S>::load(qrow[d]) : 0.0f;
    }
    float acc[kMaxRowRegs];
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) acc[t] = 0.0f;
    const float neg_inf = -__builtin_inff();
    float m = neg_inf, l = 0.0f;
    bool nan_seen = false;
    // keys past `last` are masked by the causal rule for this row
    const uint64_t last = a.causal ? (uint64_t)i + a.causal_offset : (uint64_t)a.kl - 1;
    for (uint32_t c0 = 0; c0 < a.kl && (uint64_t)c0 <= last; c0 += kWave) {
        const uint32_t j = c0 + lane;
        const bool live = j < a.kl;
        float s = neg_inf;
        if (live) {
            s = row_dot<S, kVec>(qreg, kbase + (size_t)j * a.dim, a.dim) * a.scale;
            if (mask) s = s + Elem<S>::load(mask[(size_t)i * a.kl + j]);
            if (a.causal && (uint64_t)j > last) s = neg_inf;
        }
        // a NaN score never becomes the max, but a row with a finite max and
        // a NaN score is NaN (its sum is)
        nan_seen = nan_seen || wave_any(s != s);
        const float m_new = fmaxf(m, wave_max(s));
        if (m_new == neg_inf) continue;                  // nothing visible yet
        const float alpha = attn_exp<S>(m - m_new);      // 0 when m was -inf
        const float p = live ? attn_exp<S>(s - m_new) : 0.0f;
        l = l * alpha + wave_sum(p);
        m = m_new;
        const uint32_t n = min(a.kl - c0, (uint32_t)kWave);
#pragma unroll
        for (int t = 0; t < kMaxRowRegs; ++t) acc[t] = acc[t] * alpha;
        for (uint32_t jj = 0; jj < n; ++jj) {
            const float pj = broadcast_lane(p, (int)jj);
            const S *vrow = vbase + (size_t)(c0 + jj) * a.vdim;
#pragma unroll
            for (int t = 0; t < kMaxRowRegs; ++t) {
                const uint32_t e = lane + t * kWave;
                if (e < a.vdim) acc[t] = acc[t] + pj * Elem<S>::load(vrow[e]);
            }
        }
    }
    const bool zero = !__builtin_isfinite(m);
    const float inverse = l == 0.0f ? 0.0f : 1.0f / l;
    const float nan = __builtin_nanf("");
    S *orow = out + row * a.vdim;
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) {
        const uint32_t e = lane + t * kWave;
        if (e < a.vdim)
            orow[e] = Elem<S>::store(zero ? 0.0f : nan_seen ? nan : acc[t] * inverse);
    }
}

template <typename S>
hipError_t launch_sdpa(const S *q, const S *k, const S *v, const S *mask, S *out,
                       const k::SdpaShape &sh, float scale, bool causal, hipStream_t s) {
    if (sh.batch == 0 || sh.q_heads == 0 || sh.kv_heads == 0 || sh.q_len == 0 ||
        sh.kv_len == 0 || sh.head_dim == 0 || sh.value_dim == 0 ||
        sh.q_heads % sh.kv_heads != 0)
        return hipErrorInvalidValue;
    if (sh.head_dim > (size_t)kMaxRowRegs * kWave || sh.value_dim > (size_t)kMaxRowRegs * kWave)
        return hipErrorInvalidValue;
    const uint64_t lim = 0xffffffffull;
    if (sh.batch > lim || sh.q_heads > lim || sh.kv_heads > lim || sh.q_len > lim ||
        sh.kv_len > lim)
        return hipErrorInvalidValue;
    SdpaArgs a{};
    a.batch = (uint32_t)sh.batch;
    a.qh = (uint32_t)sh.q_heads;
    a.kvh = (uint32_t)sh.kv_heads;
    a.group = (uint32_t)(sh.q_heads / sh.kv_heads);
    a.ql = (uint32_t)sh.q_len;
    a.kl = (uint32_t)sh.kv_len;
    a.dim = (uint32_t)sh.head_dim;
    a.vdim = (uint32_t)sh.value_dim;
    a.causal_offset = a.kl > a.ql ? a.kl - a.ql : 0;
    a.scale = scale;
    a.causal = causal ? 1 : 0;
    const size_t rows = sh.batch * sh.q_heads * sh.q_len;
    const size_t waves_per_block = kBlock / kWave;
    const size_t blocks = (rows + waves_per_block - 1) / waves_per_block;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    constexpr size_t E = Vec16<S>::N;
    if (sh.head_dim % E == 0 && ((uintptr_t)k & 15u) == 0)
        hipLaunchKernelGGL((sdpa_row_kernel<S, true>), dim3((unsigned)blocks), dim3(kBlock), 0, s,
                           q, k, v, mask, out, a);
    else
        hipLaunchKernelGGL((sdpa_row_kernel<S, false>), dim3((unsigned)blocks), dim3(kBlock), 0,
                           s, q, k, v, mask, out, a);
    return hipGetLastError();
}

}  // namespace

namespace k {

hipError_t sdpa_f32(const float *q, const float *k, const float *v, const float *mask,
                    float *out, const SdpaShape &shape, float scale, bool causal,
                    hipStream_t s) {
    return launch_sdpa<float>(q, k, v, mask, out, shape, scale, causal, s);
}

hipError_t sdpa_f16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                    const uint16_t *mask, uint16_t *out, const SdpaShape &shape, float scale,
                    bool causal, hipStream_t s) {
    auto h = [](const uint16_t *p) { return reinterpret_cast<const _Float16 *>(p); };
    return launch_sdpa<_Float16>(h(q), h(k), h(v), h(mask), reinterpret_cast<_Float16 *>(out),
                                 shape, scale, causal, s);
}

}  // namespace k
}  // namespace icsdk
