// Whole-tensor reductions for gfx950: sum+max of an f32 tensor and argmax.
//
// Two passes. Pass 1: a fixed grid (kPartials blocks) streams the tensor with
// 16-byte loads, kUnroll vectors in flight per lane; each lane folds every
// group of 16 values in f32 and adds the group total to an f64 accumulator,
// so the rounding error stays near 16 f32 ulps of the group magnitude
// regardless of the tensor size. Lanes combine through DPP/shuffles, waves
// through LDS, and each block writes one partial. Pass 2: one block folds the
// partials in f64 and writes the result. No atomics and no counters, so the
// partial buffer needs no clearing between calls.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

constexpr int kPartials = 2048;
constexpr int kUnroll = 4;

struct Partial {
    double sum;
    float max;      // NaN when any element was NaN
    uint32_t index; // argmax: index of the block's best value (kNone if none)
};
constexpr uint32_t kNone = 0xffffffffu;

// ---- sum + max -------------------------------------------------------------

__device__ inline void fold(const f32x4 &v, float &group, float &m, bool &nan) {
    group += (v.x + v.y) + (v.z + v.w);
    m = fmaxf(fmaxf(m, fmaxf(v.x, v.y)), fmaxf(v.z, v.w));
    nan |= (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
}

__global__ __launch_bounds__(kBlock) void sum_max_pass1(const float *__restrict__ x,
                                                        size_t nvec, size_t n,
                                                        Partial *__restrict__ partials) {
    __shared__ double lds_sum[kBlock / kWave];
    __shared__ float lds_max[kBlock / kWave];
    __shared__ int lds_nan[kBlock / kWave];
    const f32x4 *xv = reinterpret_cast<const f32x4 *>(x);
    const size_t stride = (size_t)gridDim.x * kBlock;
    size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
    double total = 0.0;
    float m = -__builtin_inff();
    bool nan = false;
    for (; i + (kUnroll - 1) * stride < nvec; i += kUnroll * stride) {
        f32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(xv + i + u * stride);
        float group = 0.0f;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) fold(v[u], group, m, nan);
        total += (double)group;
    }
    for (; i < nvec; i += stride) {
        const f32x4 v = __builtin_nontemporal_load(xv + i);
        float group = 0.0f;
        fold(v, group, m, nan);
        total += (double)group;
    }
    if (blockIdx.x == 0 && threadIdx.x < n - nvec * 4) {
        const float v = x[nvec * 4 + threadIdx.x];
        total += (double)v;
        m = fmaxf(m, v);
        nan |= v != v;
    }
    total = wave_sum_f64(total);
    m = wave_max(m);
    const bool wave_nan = wave_any(nan);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        lds_sum[wave] = total;
        lds_max[wave] = m;
        lds_nan[wave] = wave_nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = 0.0;
        float bm = -__builtin_inff();
        int any_nan = 0;
        for (int w = 0; w < kBlock / kWave; ++w) {
            s += lds_sum[w];
            bm = fmaxf(bm, lds_max[w]);
            any_nan |= lds_nan[w];
        }
        partials[blockIdx.x] = Partial{s, any_nan ? __builtin_nanf("") : bm, 0};
    }
}

__global__ __launch_bounds__(kBlock) void sum_max_pass2(const Partial *__restrict__ partials,
                                                        int count, double *sum_out,
                                                        float *max_out) {
    __shared__ double lds_sum[kBlock / kWave];
    __shared__ float lds_max[kBlock / kWave];
    __shared__ int lds_nan[kBlock / kWave];
    double s = 0.0;
    float m = -__builtin_inff();
    bool nan = false;
    for (int i = threadIdx.x; i < count; i += kBlock) {
        s += partials[i].sum;
        m = fmaxf(m, partials[i].max);
        nan |= partials[i].max != partials[i].max;
    }
    s = wave_sum_f64(s);
    m = wave_max(m);
    const bool wave_nan = wave_any(nan);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        lds_sum[wave] = s;
        lds_max[wave] = m;
        lds_nan[wave] = wave_nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double total = 0.0;
        float bm = -__builtin_inff();
        int any_nan = 0;
        for (int w = 0; w < kBlock / kWave; ++w) {
            total += lds_sum[w];
            bm = fmaxf(bm, lds_max[w]);
            any_nan |= lds_nan[w];
        }
        if (sum_out) *sum_out = total;
        if (max_out) *max_out = any_nan ? __builtin_nanf("") : bm;
    }
}

// ---- argmax ------------------------------------------------------------------

// (value, index) with "greater value wins, equal value -> lower index wins";
// NaN never compares greater, so it never wins. kNone marks "nothing yet".
__device__ inline void better(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ inline void wave_argmax(float &bv, uint32_t &bi) {
    for (int offset = 32; offset > 0; offset >>= 1) {
        const float ov = __shfl_xor(bv, offset, kWave);
        const uint32_t oi = __shfl_xor(bi, offset, kWave);
        better(bv, bi, ov, oi);
    }
}

template <typename S>
__global__ __launch_bounds__(kBlock) void argmax_pass1(const S *__restrict__ x, size_t n,
                                                       Partial *__restrict__ partials) {
    __shared__ float lds_v[kBlock / kWave];
    __shared__ uint32_t lds_i[kBlock / kWave];
    constexpr int E = Vec16<S>::N;
    const size_t nvec = n / E;
    const size_t stride = (size_t)gridDim.x * kBlock;
    float bv = -__builtin_inff();
    uint32_t bi = kNone;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < nvec; i += stride) {
        const Vec16<S> v = load16_stream(x + i * E);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float f = Elem<S>::load(v.v[e]);
            if (f > bv) {  // strict: within one lane indices ascend
                bv = f;
                bi = (uint32_t)(i * E + e);
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < n - nvec * E) {
        const uint32_t t = (uint32_t)(nvec * E + threadIdx.x);
        better(bv, bi, Elem<S>::load(x[t]), t);
    }
    wave_argmax(bv, bi);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        lds_v[wave] = bv;
        lds_i[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / kWave; ++w) better(bv, bi, lds_v[w], lds_i[w]);
        partials[blockIdx.x] = Partial{0.0, bv, bi};
    }
}

template <typename S>
__global__ __launch_bounds__(kBlock) void argmax_pass2(const S *__restrict__ x,
                                                       const Partial *__restrict__ partials,
                                                       int count, uint32_t *index_out) {
    __shared__ float lds_v[kBlock / kWave];
    __shared__ uint32_t lds_i[kBlock / kWave];
    float bv = -__builtin_inff();
    uint32_t bi = kNone;
    for (int i = threadIdx.x; i < count; i += kBlock) better(bv, bi, partials[i].max, partials[i].index);
    wave_argmax(bv, bi);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        lds_v[wave] = bv;
        lds_i[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / kWave; ++w) better(bv, bi, lds_v[w], lds_i[w]);
        const float first = Elem<S>::load(x[0]);
        // The reference scans from element 0 with a strict '>': a NaN first
        // element is never replaced, and when the largest non-NaN value is
        // -inf (or there is none) element 0 is never beaten either.
        *index_out = (first != first || bi == kNone || bv == -__builtin_inff()) ? 0u : bi;
    }
}

inline int pass1_grid(size_t work) {
    const size_t blocks = (work + (size_t)kBlock * kUnroll - 1) / ((size_t)kBlock * kUnroll);
    return blocks < 1 ? 1 : (blocks > (size_t)kPartials ? kPartials : (int)blocks);
}

}  // namespace

namespace k {

size_t grid_reduce_scratch_bytes() { return sizeof(Partial) * kPartials; }

hipError_t sum_max_f32(const float *x, size_t n, double *sum_out, float *max_out,
                       void *partials, hipStream_t s) {
    if (n == 0) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15u) != 0) return hipErrorInvalidValue;
    const size_t nvec = n / 4;
    const int grid = pass1_grid(nvec);
    auto *p = static_cast<Partial *>(partials);
    hipLaunchKernelGGL(sum_max_pass1, dim3(grid), dim3(kBlock), 0, s, x, nvec, n, p);
    hipLaunchKernelGGL(sum_max_pass2, dim3(1), dim3(kBlock), 0, s, p, grid, sum_out, max_out);
    return hipGetLastError();
}

template <typename S>
hipError_t argmax_launch(const S *x, size_t n, uint32_t *index_out, void *partials,
                         hipStream_t s) {
    if (n == 0 || n > 0xffffffffu || ((uintptr_t)x & 15u) != 0) return hipErrorInvalidValue;
    const int grid = pass1_grid(n / Vec16<S>::N);
    auto *p = static_cast<Partial *>(partials);
    hipLaunchKernelGGL((argmax_pass1<S>), dim3(grid), dim3(kBlock), 0, s, x, n, p);
    hipLaunchKernelGGL((argmax_pass2<S>), dim3(1), dim3(kBlock), 0, s, x, p, grid, index_out);
    return hipGetLastError();
}

hipError_t argmax_f32(const float *x, size_t n, uint32_t *index_out, void *partials,
                      hipStream_t s) {
    return argmax_launch<float>(x, n, index_out, partials, s);
}

hipError_t argmax_f16(const uint16_t *x, size_t n, uint32_t *index_out, void *partials,
                      hipStream_t s) {
    return argmax_launch<_Float16>(reinterpret_cast<const _Float16 *>(x), n, index_out,
                                   partials, s);
}

}  // namespace k
}  // namespace icsdk
