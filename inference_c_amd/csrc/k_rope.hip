// Split-half (NeoX) rotary position embedding for gfx950, in place on
// q [seq, q_heads, dim] and k [seq, k_heads, dim].
//
// One 256-thread block per position (grid-stride over positions). The block
// first computes the position's dim/2 rotation angles exactly as the
// reference does -- angle = (float)((double)(offset + p) / pow(theta, 2d/dim))
// in double, then cosf/sinf in f32 -- into LDS, then every (head, 8-pair
// chunk) work item loads the 16-byte left and right halves, rotates them in
// f32 (left*c - right*s, right*c + left*s, no contraction) and stores them
// back. q and k of a position are handled by the same block, so the angles
// are computed once per position.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

constexpr int kMaxHalf = 2048;

template <typename S>
__device__ inline void rotate_vec(S *base, uint32_t d0, uint32_t half, const float *cs,
                                  const float *sn) {
    constexpr int E = Vec16<S>::N;
    Vec16<S> left = load16(base + d0);
    Vec16<S> right = load16(base + d0 + half);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float l = Elem<S>::load(left.v[e]);
        const float r = Elem<S>::load(right.v[e]);
        const float c = cs[d0 + e], s = sn[d0 + e];
        left.v[e] = Elem<S>::store(l * c - r * s);
        right.v[e] = Elem<S>::store(r * c + l * s);
    }
    store16(base + d0, left);
    store16(base + d0 + half, right);
}

template <typename S>
__device__ inline void rotate_one(S *base, uint32_t d, uint32_t half, const float *cs,
                                  const float *sn) {
    const float l = Elem<S>::load(base[d]);
    const float r = Elem<S>::load(base[d + half]);
    const float c = cs[d], s = sn[d];
    base[d] = Elem<S>::store(l * c - r * s);
    base[d + half] = Elem<S>::store(r * c + l * s);
}

template <typename S, bool kVector>
__global__ __launch_bounds__(kBlock) void rope_kernel(S *__restrict__ q, S *__restrict__ k,
                                                      size_t seq, uint32_t qh, uint32_t kh,
                                                      uint32_t dim, double theta,
                                                      size_t offset) {
    __shared__ float cs[kMaxHalf];
    __shared__ float sn[kMaxHalf];
    constexpr uint32_t E = kVector ? Vec16<S>::N : 1;
    const uint32_t half = dim / 2;
    const uint32_t chunks = half / E;
    const uint32_t items = (qh + kh) * chunks;
    for (size_t p = blockIdx.x; p < seq; p += gridDim.x) {
        __syncthreads();  // previous position's readers are done with cs/sn
        for (uint32_t d = threadIdx.x; d < half; d += kBlock) {
            const double denom = pow(theta, (2.0 * (double)d) / (double)dim);
            const float angle = (float)((double)(offset + p) / denom);
            cs[d] = cosf(angle);
            sn[d] = sinf(angle);
        }
        __syncthreads();
        for (uint32_t item = threadIdx.x; item < items; item += kBlock) {
            const uint32_t head = item / chunks;
            const uint32_t d0 = (item - head * chunks) * E;
            S *base = head < qh ? q + (p * qh + head) * dim
                                : k + (p * kh + (head - qh)) * dim;
            if constexpr (kVector) rotate_vec(base, d0, half, cs, sn);
            else rotate_one(base, d0, half, cs, sn);
        }
    }
}

template <typename S>
hipError_t launch_rope(S *q, S *k, size_t seq, size_t qh, size_t kh, size_t dim,
                       double theta, size_t offset, hipStream_t s) {
    if (seq == 0) return hipSuccess;
    if (dim == 0 || dim % 2 || dim / 2 > kMaxHalf || qh > 0xffffffu || kh > 0xffffffu)
        return hipErrorInvalidValue;
    constexpr size_t E = Vec16<S>::N;
    const size_t half = dim / 2;
    const bool vector = half % E == 0 && ((uintptr_t)q & 15u) == 0 &&
                        ((uintptr_t)k & 15u) == 0;
    const unsigned grid = (unsigned)(seq < 65536 ? seq : 65536);
    if (vector)
        hipLaunchKernelGGL((rope_kernel<S, true>), dim3(grid), dim3(kBlock), 0, s, q, k, seq,
                           (uint32_t)qh, (uint32_t)kh, (uint32_t)dim, theta, offset);
    else
        hipLaunchKernelGGL((rope_kernel<S, false>), dim3(grid), dim3(kBlock), 0, s, q, k, seq,
                           (uint32_t)qh, (uint32_t)kh, (uint32_t)dim, theta, offset);
    return hipGetLastError();
}

}  // namespace

namespace k {

hipError_t rope_f32(float *q, float *k, size_t seq, size_t qh, size_t kh, size_t dim,
                    double theta, size_t offset, hipStream_t s) {
    return launch_rope<float>(q, k, seq, qh, kh, dim, theta, offset, s);
}

hipError_t rope_f16(uint16_t *q, uint16_t *k, size_t seq, size_t qh, size_t kh,
                    size_t dim, double theta, size_t offset, hipStream_t s) {
    return launch_rope<_Float16>(reinterpret_cast<_Float16 *>(q),
                                 reinterpret_cast<_Float16 *>(k), seq, qh, kh, dim, theta,
                                 offset, s);
}

}  // namespace k
}  // namespace icsdk
