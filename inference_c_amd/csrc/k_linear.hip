// Linear layers with few input rows (decode): y[r][o] = sum_i x[r][i] w[o][i]
// (+ bias[o]) for f16 or f32 weights stored [out, in] row-major, the layout
// of the reference's tensor_linear_* (src/common/tensor_ops.c:318-398;
// the CUDA backend's cuBLAS call, tensor_compute_cuda.cu:174-265).
//
// At one to four input rows the product is a stream over the weights
// (2 or 4 bytes each, read once) with a few flops per byte, so it is written
// as a GEMV rather than handed to a GEMM library: a wave owns O output rows
// (O = 1 measured fastest) and walks them, each lane reading 16-byte vectors
// at a 64-vector (1 KiB) stride, so every load instruction reads 1 KiB of
// one weight row contiguously, kUnroll of them in flight. Lane l's slice of
// x (R rows) is loaded once per vector position and reused for the O rows.
// f16: v_dot2_f32_f16 (exact products, f32 sums); f32: fma. The lanes'
// partial sums are folded with DPP; the bias is added in f32 before the
// result is rounded to the output type. Bound: HBM bytes of the weights.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace k {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kUnroll = 4;   // vector positions in flight per lane

// sum of the products of one 16-byte vector of weights and of x
template <typename T>
__device__ inline float vec_dot(const u32x4 &w, const u32x4 &x, float acc) {
    if constexpr (sizeof(T) == 2) {
        // elements copied into scalars before the bit casts (a bit cast of a
        // vector element compiles to one of element 0)
        const uint32_t wa[4] = {w.x, w.y, w.z, w.w}, xa[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, wa[i]), __builtin_bit_cast(half2_t, xa[i]),
                                         acc, false);
    } else {
        const f32x4 wf = __builtin_bit_cast(f32x4, w), xf = __builtin_bit_cast(f32x4, x);
        acc = __builtin_fmaf(wf.x, xf.x, acc);
        acc = __builtin_fmaf(wf.y, xf.y, acc);
        acc = __builtin_fmaf(wf.z, xf.z, acc);
        acc = __builtin_fmaf(wf.w, xf.w, acc);
    }
    return acc;
}

// Grid: x = waves of O output rows (4 waves per block), y = groups of R
// input rows. Requires x, w 16-byte aligned and in a multiple of the
// elements per 16 bytes (every row then starts 16-byte aligned).
template <typename T, int R, int O>
__global__ __launch_bounds__(kBlock) void gemv_kernel(const T *__restrict__ x, const T *__restrict__ w,
                                                      const T *__restrict__ bias, T *__restrict__ y,
                                                      uint32_t rows, uint32_t in, uint32_t out) {
    constexpr uint32_t E = 16 / sizeof(T);
    const uint32_t lane = threadIdx.x & (kWave - 1);
    // the wave's index in the grid, formed without the work-item number
    // (blockIdx.x * kBlock), which would wrap in 32 bits for a large grid
    const uint32_t wave =
        __builtin_amdgcn_readfirstlane(blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave);
    const uint32_t o0 = wave * O;
    if (o0 >= out) return;
    const uint32_t r0 = blockIdx.y * R;
    const uint32_t nvec = in / E;
    // rows past the end are clamped onto the last one (computed, not stored)
    const u32x4 *wrow[O];
    const u32x4 *xrow[R];
#pragma unroll
    for (int o = 0; o < O; ++o)
        wrow[o] = reinterpret_cast<const u32x4 *>(w + (size_t)min(o0 + o, out - 1) * in);
#pragma unroll
    for (int r = 0; r < R; ++r)
        xrow[r] = reinterpret_cast<const u32x4 *>(x + (size_t)min(r0 + r, rows - 1) * in);
    float acc[O][R];
#pragma unroll
    for (int o = 0; o < O; ++o)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[o][r] = 0.0f;

    constexpr uint32_t kStep = kWave * kUnroll;
    uint32_t v0 = 0;
    // whole steps: every lane's kUnroll vectors exist
    for (; v0 + kStep <= nvec; v0 += kStep) {
        u32x4 wv[kUnroll][O], xv[kUnroll][R];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint32_t v = v0 + kWave * u + lane;
#pragma unroll
            for (int o = 0; o < O; ++o) wv[u][o] = __builtin_nontemporal_load(wrow[o] + v);
#pragma unroll
            for (int r = 0; r < R; ++r) xv[u][r] = xrow[r][v];
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
#pragma unroll
            for (int o = 0; o < O; ++o)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[o][r] = vec_dot<T>(wv[u][o], xv[u][r], acc[o][r]);
    }
    // the rest, one vector position at a time
    for (uint32_t v = v0 + lane; v < nvec; v += kWave) {
#pragma unroll
        for (int o = 0; o < O; ++o) {
            const u32x4 wv = __builtin_nontemporal_load(wrow[o] + v);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[o][r] = vec_dot<T>(wv, xrow[r][v], acc[o][r]);
        }
    }
#pragma unroll
    for (int o = 0; o < O; ++o) {
        const float b = bias != nullptr ? (float)bias[min(o0 + o, out - 1)] : 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float total = wave_sum(acc[o][r]) + b;
            if (lane == 0 && o0 + o < out && r0 + r < rows) y[(size_t)(r0 + r) * out + o0 + o] = (T)total;
        }
    }
}

template <typename T, int R, int O>
hipError_t launch(const T *x, const T *w, const T *bias, T *y, size_t rows, size_t in, size_t out,
                  hipStream_t s) {
    constexpr size_t kWavesPerBlock = kBlock / kWave;
    const size_t waves = (out + O - 1) / O;
    const dim3 grid((unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock), (unsigned)((rows + R - 1) / R));
    gemv_kernel<T, R, O><<<grid, kBlock, 0, s>>>(x, w, bias, y, (uint32_t)rows, (uint32_t)in, (uint32_t)out);
    return hipGetLastError();
}

template <typename T>
hipError_t gemv(const T *x, const T *w, const T *bias, T *y, size_t rows, size_t in, size_t out,
                hipStream_t s) {
    // one output row per wave (1 x 8192 -> 8192 f16: 21.9 us; 2 rows 22.5,
    // 4 rows 30.6; hipBLASLt 26.0)
    constexpr int O = 1;
    switch (rows) {
    case 1: return launch<T, 1, O>(x, w, bias, y, rows, in, out, s);
    case 2: return launch<T, 2, O>(x, w, bias, y, rows, in, out, s);
    case 3: return launch<T, 3, O>(x, w, bias, y, rows, in, out, s);
    default: return launch<T, 4, O>(x, w, bias, y, rows, in, out, s);
    }
}

}  // namespace

hipError_t linear_gemv(bool f32, const void *x, const void *w, const void *bias, void *y,
                       size_t rows, size_t in, size_t out, hipStream_t s) {
    const size_t elem = f32 ? 4 : 2;
    // The launch is one wave (64 work-items) per output row: out * 64 must
    // stay below 2^32, the dispatch packet's work-item count. Larger `out`
    // is declined here (hipErrorNotSupported), and the caller takes the
    // library GEMM.
    if (rows == 0 || rows > kGemvMaxRows || in == 0 || out == 0 || in % (16 / elem) != 0 ||
        in > 0xffffffffu || out > 0xffffffffu / kWave ||
        (((uintptr_t)x | (uintptr_t)w) & 15u) != 0)
        return hipErrorNotSupported;
    if (f32)
        return gemv(static_cast<const float *>(x), static_cast<const float *>(w),
                    static_cast<const float *>(bias), static_cast<float *>(y), rows, in, out, s);
    return gemv(static_cast<const _Float16 *>(x), static_cast<const _Float16 *>(w),
                static_cast<const _Float16 *>(bias), static_cast<_Float16 *>(y), rows, in, out, s);
}

}  // namespace k
}  // namespace icsdk
