// Synthetic-input generation and dtype conversion for gfx950.
//
// fill: element i of (seed, stream) is a pure function of (seed, stream, i):
// a counter-based splitmix64 hash (Steele, Lea & Flood, OOPSLA 2014). Uniform
// values use the top 24 bits; normal values use Box-Muller in double on two
// 53-bit uniforms. The same definitions run on the host in the test oracle,
// so any slice of a device-generated tensor can be regenerated on the CPU.
//
// convert: F32 <-> F16 <-> BF16 with the reference's bit rules for every
// input, NaNs included: f16 NaN payloads move unchanged into the top of the
// f32 fraction; f32 -> f16 keeps the sign and top ten payload bits of a NaN
// (a zero payload becomes 1); f32 -> bf16 quietens NaN and otherwise rounds
// to nearest even. Non-NaN values go through the hardware conversions, which
// are exact (widening) or round to nearest even with subnormals.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

constexpr uint64_t kGamma = 0x9e3779b97f4a7c15ull;

__device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__device__ inline float uniform_value(uint64_t bits, float low, float high) {
    const float unit = (float)(bits >> 40) * 0x1p-24f;
    return low + (high - low) * unit;
}

__device__ inline float normal_value(uint64_t bits, float mean, float std_dev) {
    const uint64_t second = mix64(bits ^ 0xd1b54a32d192ed03ull);
    const double u1 = (double)((bits >> 11) + 1u) * 0x1p-53;
    const double u2 = (double)(second >> 11) * 0x1p-53;
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    return (float)((double)mean + (double)std_dev * z);
}

template <typename S, bool kNormal>
__global__ __launch_bounds__(kBlock) void fill_kernel(S *__restrict__ y, size_t n,
                                                      uint64_t key, float a, float b) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        const uint64_t bits = mix64(key + kGamma * (i + 1u));
        const float v = kNormal ? normal_value(bits, a, b) : uniform_value(bits, a, b);
        y[i] = Elem<S>::store(v);
    }
}

template <bool kNormal>
hipError_t launch_fill(TensorDType dtype, void *y, size_t n, uint64_t seed, uint64_t stream,
                       float a, float b, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint64_t key_host = [&] {
        uint64_t z = seed + kGamma * (2u * stream + 1u);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }();
    size_t grid = (n + kBlock * 8 - 1) / (kBlock * 8);
    if (grid > (size_t{1} << 20)) grid = size_t{1} << 20;
    if (dtype == TENSOR_DTYPE_F32)
        hipLaunchKernelGGL((fill_kernel<float, kNormal>), dim3((unsigned)grid), dim3(kBlock), 0,
                           s, static_cast<float *>(y), n, key_host, a, b);
    else if (dtype == TENSOR_DTYPE_F16)
        hipLaunchKernelGGL((fill_kernel<_Float16, kNormal>), dim3((unsigned)grid), dim3(kBlock),
                           0, s, static_cast<_Float16 *>(y), n, key_host, a, b);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// ---- conversion --------------------------------------------------------------

__device__ inline float f16_bits_to_f32(uint16_t h) {
    if ((h & 0x7c00u) == 0x7c00u && (h & 0x3ffu) != 0)
        return __builtin_bit_cast(float, ((uint32_t)(h & 0x8000u) << 16) | 0x7f800000u |
                                              ((uint32_t)(h & 0x3ffu) << 13));
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ inline uint16_t f32_to_f16_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        const uint32_t payload = (u >> 13) & 0x3ffu;
        return (uint16_t)(((u >> 16) & 0x8000u) | 0x7c00u | (payload ? payload : 1u));
    }
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ inline uint16_t f32_to_bf16_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ inline float bf16_bits_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

template <TensorDType kFrom>
__device__ inline float read_as_f32(const void *x, size_t i) {
    if constexpr (kFrom == TENSOR_DTYPE_F32) return static_cast<const float *>(x)[i];
    else if constexpr (kFrom == TENSOR_DTYPE_F16) return f16_bits_to_f32(static_cast<const uint16_t *>(x)[i]);
    else return bf16_bits_to_f32(static_cast<const uint16_t *>(x)[i]);
}

template <TensorDType kTo>
__device__ inline void write_from_f32(void *y, size_t i, float v) {
    if constexpr (kTo == TENSOR_DTYPE_F32) static_cast<float *>(y)[i] = v;
    else if constexpr (kTo == TENSOR_DTYPE_F16) static_cast<uint16_t *>(y)[i] = f32_to_f16_bits(v);
    else static_cast<uint16_t *>(y)[i] = f32_to_bf16_bits(v);
}

template <TensorDType kFrom, TensorDType kTo>
__global__ __launch_bounds__(kBlock) void convert_kernel(const void *__restrict__ x,
                                                         void *__restrict__ y, size_t n) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        write_from_f32<kTo>(y, i, read_as_f32<kFrom>(x, i));
}

template <TensorDType kFrom>
hipError_t convert_from(const void *x, TensorDType to, void *y, size_t n, dim3 grid,
                        hipStream_t s) {
    switch (to) {
        case TENSOR_DTYPE_F32:
            hipLaunchKernelGGL((convert_kernel<kFrom, TENSOR_DTYPE_F32>), grid, dim3(kBlock), 0, s, x, y, n);
            break;
        case TENSOR_DTYPE_F16:
            hipLaunchKernelGGL((convert_kernel<kFrom, TENSOR_DTYPE_F16>), grid, dim3(kBlock), 0, s, x, y, n);
            break;
        case TENSOR_DTYPE_BF16:
            hipLaunchKernelGGL((convert_kernel<kFrom, TENSOR_DTYPE_BF16>), grid, dim3(kBlock), 0, s, x, y, n);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

namespace k {

hipError_t fill_uniform(TensorDType dtype, void *y, size_t n, uint64_t seed, uint64_t stream,
                        float low, float high, hipStream_t s) {
    return launch_fill<false>(dtype, y, n, seed, stream, low, high, s);
}

hipError_t fill_normal(TensorDType dtype, void *y, size_t n, uint64_t seed, uint64_t stream,
                       float mean, float std_dev, hipStream_t s) {
    return launch_fill<true>(dtype, y, n, seed, stream, mean, std_dev, s);
}

hipError_t convert(TensorDType from, const void *x, TensorDType to, void *y, size_t n,
                   hipStream_t s) {
    if (n == 0) return hipSuccess;
    size_t g = (n + kBlock * 8 - 1) / (kBlock * 8);
    if (g > (size_t{1} << 20)) g = size_t{1} << 20;
    const dim3 grid((unsigned)g);
    switch (from) {
        case TENSOR_DTYPE_F32: return convert_from<TENSOR_DTYPE_F32>(x, to, y, n, grid, s);
        case TENSOR_DTYPE_F16: return convert_from<TENSOR_DTYPE_F16>(x, to, y, n, grid, s);
        case TENSOR_DTYPE_BF16: return convert_from<TENSOR_DTYPE_BF16>(x, to, y, n, grid, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace k
}  // namespace icsdk
