// Split-half (NeoX) rotary position embedding for gfx950, in place on
// q [seq, q_heads, dim] and k [seq, k_heads, dim].
//
// Two kernels on the SDK stream:
//   1. table: one lane per (position, pair d < dim/2) computes the rotation
//      exactly as the reference does -- angle = (float)((double)(offset + p) /
//      pow(theta, 2d/dim)) in double, then cosf/sinf in f32 -- into a
//      (cos, sin) table of seq * dim/2 float pairs (1 MiB for 4096 x 32);
//   2. rotate: one lane per 16-byte vector of q then k (rows of dim elements
//      read and written contiguously, non-temporal hint); each lane also
//      reads the vector holding the other half of its pairs (same cache
//      lines) and the pairs' cos/sin from the table (L2-resident), and
//      rotates in f32 (left*c - right*s, right*c + left*s, no contraction).
//      A pure streaming pass over q and k.
// The table lives in device scratch supplied by the caller.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

// A block covers kBlock consecutive table entries (positions x pairs). The
// pair denominators pow(theta, 2d/dim) depend on the pair only: the block
// computes each needed one once into LDS, then every lane forms its angle.
constexpr int kMaxDenoms = kBlock;

__global__ __launch_bounds__(kBlock) void rope_table_kernel(float2 *__restrict__ table,
                                                            uint32_t seq, uint32_t half,
                                                            uint32_t dim, double theta,
                                                            uint64_t offset) {
    __shared__ double denom[kMaxDenoms];
    const size_t first = (size_t)blockIdx.x * kBlock;
    const size_t entries = (size_t)seq * half;
    // pairs touched by this block: a contiguous (wrapping) run starting at first % half
    const uint32_t d_first = (uint32_t)(first % half);
    const uint32_t needed = half < (uint32_t)kBlock ? half : (uint32_t)kBlock;
    if (threadIdx.x < needed) {
        const uint32_t d = (d_first + threadIdx.x) % half;
        denom[threadIdx.x] = pow(theta, (2.0 * (double)d) / (double)dim);
    }
    __syncthreads();
    const size_t i = first + threadIdx.x;
    if (i >= entries) return;
    const uint32_t p = (uint32_t)(i / half);
    const uint32_t d = (uint32_t)(i - (size_t)p * half);
    const uint32_t slot = (d + half - d_first) % half;  // < needed
    const float angle = (float)((double)(offset + p) / denom[slot]);
    float c, sn;
    sincosf(angle, &sn, &c);
    table[i] = make_float2(c, sn);
}

template <typename S>
__device__ inline void rotate_pair(float l, float r, float c, float s, S &lo, S &ro) {
    lo = Elem<S>::store(l * c - r * s);
    ro = Elem<S>::store(r * c + l * s);
}

// One 16-byte vector per lane over the rows of q then the rows of k (each
// row = one head at one position, dim elements): a wave reads and writes
// whole rows contiguously. The vector holding the left chunk c of a pair
// block and the one holding the right chunk c are `half / E` vectors apart (a
// power of two, so the partner is index ^ (half/E)); each lane also loads its
// partner's vector (same cache lines, so no extra HBM traffic) and writes its
// own half of the rotation.
template <typename S, int kPartnerXor>
__global__ __launch_bounds__(kBlock) void rope_vec_kernel(S *__restrict__ q, S *__restrict__ k,
                                                          const float2 *__restrict__ table,
                                                          uint64_t q_vectors, uint64_t vectors,
                                                          FastDiv q_heads, FastDiv k_heads,
                                                          uint32_t dim) {
    constexpr int E = Vec16<S>::N;
    constexpr int kRowShift = __builtin_ctz(2 * kPartnerXor);  // vectors per head row = 2 * half/E
    const uint64_t v = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    const bool active = v < vectors;
    const bool in_q = v < q_vectors;
    const uint64_t local = in_q ? v : v - q_vectors;   // vector index inside q or k
    S *data = in_q ? q : k;
    const uint64_t row = local >> kRowShift;
    const uint32_t j = (uint32_t)(local & (2 * kPartnerXor - 1));
    const uint32_t p = fast_div((uint32_t)row, in_q ? q_heads : k_heads);
    const uint32_t half = dim / 2;
    const bool left = j < (uint32_t)kPartnerXor;
    const uint32_t d0 = (left ? j : j - kPartnerXor) * E;   // first pair of this vector
    if (!active) return;
    // the lane's own vector, its partner's vector (same head row, so the same
    // cache lines) and its pairs' cos/sin (L1/L2-resident) are all requested
    // before any is used
    const Vec16<S> mine = load16_stream(data + local * E);
    const Vec16<S> partner = load16(data + (local ^ (uint64_t)kPartnerXor) * E);
    float2 cs[E];
    const float2 *tp = table + (size_t)p * half + d0;
#pragma unroll
    for (int e = 0; e < E; ++e) cs[e] = tp[e];
    Vec16<S> out;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float2 t = cs[e];
        const float a = Elem<S>::load(mine.v[e]), b = Elem<S>::load(partner.v[e]);
        // left lane: l*c - r*s with l = a, r = b; right lane: r*c + l*s with r = a, l = b
        out.v[e] = Elem<S>::store(left ? a * t.x - b * t.y : a * t.x + b * t.y);
    }
    store16_stream(data + local * E, out);
}

// one pair per lane (head_dim/2 not a multiple of the vector, or unaligned)
template <typename S>
__global__ __launch_bounds__(kBlock) void rope_scalar_kernel(S *__restrict__ q, S *__restrict__ k,
                                                             const float2 *__restrict__ table,
                                                             size_t items, size_t per_pos,
                                                             uint32_t half, uint32_t qh,
                                                             uint32_t kh, uint32_t dim) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t item = (size_t)blockIdx.x * kBlock + threadIdx.x; item < items; item += stride) {
        const size_t p = item / per_pos;
        const size_t rest = item - p * per_pos;
        const uint32_t head = (uint32_t)(rest / half);
        const uint32_t d = (uint32_t)(rest - (size_t)head * half);
        S *base = head < qh ? q + (p * qh + head) * dim : k + (p * kh + (head - qh)) * dim;
        const float2 t = table[p * half + d];
        rotate_pair<S>(Elem<S>::load(base[d]), Elem<S>::load(base[d + half]), t.x, t.y, base[d],
                       base[d + half]);
    }
}

template <typename S>
hipError_t launch_rope(S *q, S *k, size_t seq, size_t qh, size_t kh, size_t dim, double theta,
                       size_t offset, void *table_scratch, hipStream_t s) {
    if (seq == 0) return hipSuccess;
    const size_t half = dim / 2;
    if (dim == 0 || dim % 2 || seq * half > 0xffffffffu || qh + kh > 0xffffffu)
        return hipErrorInvalidValue;
    auto *table = static_cast<float2 *>(table_scratch);
    const size_t entries = seq * half;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((entries + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, s, table, (uint32_t)seq, (uint32_t)half, (uint32_t)dim,
                       theta, (uint64_t)offset);
    constexpr size_t E = Vec16<S>::N;
    const size_t heads = qh + kh;
    const size_t chunks = half / E;  // vectors per half row
    const bool vector = half % E == 0 && chunks >= 1 && chunks <= 32 &&
                        (chunks & (chunks - 1)) == 0 && ((uintptr_t)q & 15u) == 0 &&
                        ((uintptr_t)k & 15u) == 0 && seq * heads < (size_t{1} << 32);
    if (vector) {
        const uint64_t q_vectors = (uint64_t)seq * qh * (dim / E);
        const uint64_t vectors = q_vectors + (uint64_t)seq * kh * (dim / E);
        const dim3 grid((unsigned)((vectors + kBlock - 1) / kBlock)), block(kBlock);
        const FastDiv qd = make_fast_div((uint32_t)qh), kd = make_fast_div((uint32_t)kh);
        switch (chunks) {
            case 1: hipLaunchKernelGGL((rope_vec_kernel<S, 1>), grid, block, 0, s, q, k, table, q_vectors, vectors, qd, kd, (uint32_t)dim); break;
            case 2: hipLaunchKernelGGL((rope_vec_kernel<S, 2>), grid, block, 0, s, q, k, table, q_vectors, vectors, qd, kd, (uint32_t)dim); break;
            case 4: hipLaunchKernelGGL((rope_vec_kernel<S, 4>), grid, block, 0, s, q, k, table, q_vectors, vectors, qd, kd, (uint32_t)dim); break;
            case 8: hipLaunchKernelGGL((rope_vec_kernel<S, 8>), grid, block, 0, s, q, k, table, q_vectors, vectors, qd, kd, (uint32_t)dim); break;
            case 16: hipLaunchKernelGGL((rope_vec_kernel<S, 16>), grid, block, 0, s, q, k, table, q_vectors, vectors, qd, kd, (uint32_t)dim); break;
            default: hipLaunchKernelGGL((rope_vec_kernel<S, 32>), grid, block, 0, s, q, k, table, q_vectors, vectors, qd, kd, (uint32_t)dim); break;
        }
    } else {
        const size_t per_pos = heads * half;
        const size_t items = seq * per_pos;
        size_t grid = (items + kBlock - 1) / kBlock;
        if (grid > (size_t{1} << 20)) grid = size_t{1} << 20;
        hipLaunchKernelGGL((rope_scalar_kernel<S>), dim3((unsigned)grid), dim3(kBlock), 0, s, q, k,
                           table, items, per_pos, (uint32_t)half, (uint32_t)qh, (uint32_t)kh,
                           (uint32_t)dim);
    }
    return hipGetLastError();
}

}  // namespace

namespace k {

size_t rope_table_bytes(size_t seq, size_t dim) { return seq * (dim / 2) * sizeof(float2); }

hipError_t rope_f32(float *q, float *k, size_t seq, size_t qh, size_t kh, size_t dim,
                    double theta, size_t offset, void *table, hipStream_t s) {
    return launch_rope<float>(q, k, seq, qh, kh, dim, theta, offset, table, s);
}

hipError_t rope_f16(uint16_t *q, uint16_t *k, size_t seq, size_t qh, size_t kh, size_t dim,
                    double theta, size_t offset, void *table, hipStream_t s) {
    return launch_rope<_Float16>(reinterpret_cast<_Float16 *>(q), reinterpret_cast<_Float16 *>(k),
                                 seq, qh, kh, dim, theta, offset, table, s);
}

}  // namespace k
}  // namespace icsdk
