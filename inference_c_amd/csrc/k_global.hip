// Whole-tensor reductions for gfx950: sum+max of an f32 tensor and argmax.
//
// Two passes. Pass 1 (sum+max): block b streams the contiguous chunk of
// kChunk 16-byte vectors starting at b * kChunk, kVpl vectors in flight per
// lane per step (one-shot chunks measured ~15% faster on MI355X than a
// persistent grid-stride loop: 88% vs 76% of HBM peak reading 4 GiB). 32
// vectors x 8 steps per lane (1 MiB chunks, 150 VGPRs, 3 waves per SIMD)
// ran 2^30 f32 in 606.2-606.8 us, 32 x 4 in 607.7-609.7 and 8 x 16 (8 waves
// per SIMD) in 612.1-613.5; 32 x 16 and 32 x 32 slower again. Past
// kMaxPartials chunks the grid strides over chunks. Each lane folds every
// 32 values (8 vectors) in f32 and adds that total to an f64 accumulator, so
// the rounding error stays near 32 f32 ulps of the group magnitude regardless
// of the tensor size. Lanes combine through shuffles, waves through LDS, and
// each block writes one partial. Pass 2: one 1024-lane block loads all
// partials at once, folds them in f64 and writes the result. No atomics and
// no counters, so the partial buffer needs no clearing between calls.
#include "kern_common.hpp"
#include "kernels.hpp"

#include <mutex>

namespace icsdk {
namespace {

constexpr int kPartials = 2048;     // argmax pass-1 grid
constexpr int kUnroll = 4;          // argmax vectors in flight per lane
constexpr int kVpl = 32;            // sum+max vectors in flight per lane (a multiple of 8)
constexpr int kSteps = 8;           // sum+max steps per chunk
constexpr size_t kChunk = (size_t)kBlock * kVpl * kSteps;  // 1 MiB of f32
static_assert(kVpl % 8 == 0, "whole f32 groups of 8 vectors");
constexpr int kMaxPartials = 4096;  // sum+max pass-1 grid cap (4 GiB per sweep: 2^30 f32 one-shot)
constexpr int kFoldBlock = 1024;    // pass-2 lanes

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

// One chunk: kSteps steps of kVpl coalesced vectors per lane. kGuard: the
// chunk runs past nvec (the last one), so vectors past the end are skipped.
template <bool kGuard>
__device__ inline void sum_max_chunk(const f32x4 *__restrict__ xv, size_t first, size_t nvec,
                                     double &total, float &m, bool &nan) {
#pragma unroll 1
    for (int step = 0; step < kSteps; ++step) {
        const size_t base = first + (size_t)step * kVpl * kBlock + threadIdx.x;
        f32x4 v[kVpl];
#pragma unroll
        for (int u = 0; u < kVpl; ++u) {
            const size_t i = base + (size_t)u * kBlock;
            if constexpr (kGuard) {
                v[u] = __builtin_nontemporal_load(xv + (i < nvec ? i : 0));
            } else {
                v[u] = __builtin_nontemporal_load(xv + i);
            }
        }
        // groups of 8 vectors (32 values) fold in f32, each into the f64 total
#pragma unroll
        for (int g = 0; g < kVpl / 8; ++g) {
            float group = 0.0f;
#pragma unroll
            for (int u = 8 * g; u < 8 * g + 8; ++u) {
                if constexpr (kGuard) {
                    if (base + (size_t)u * kBlock >= nvec) continue;
                }
                fold(v[u], group, m, nan);
            }
            total += (double)group;
        }
    }
}

__global__ __launch_bounds__(kBlock) void sum_max_pass1(const float *__restrict__ x,
                                                        size_t nvec, size_t n,
                                                        Partial *__restrict__ partials) {
    __shared__ double lds_sum[kBlock / kWave];
    __shared__ float lds_max[kBlock / kWave];
    __shared__ int lds_nan[kBlock / kWave];
    const f32x4 *xv = reinterpret_cast<const f32x4 *>(x);
    double total = 0.0;
    float m = -__builtin_inff();
    bool nan = false;
    for (size_t chunk = blockIdx.x; chunk * kChunk < nvec; chunk += gridDim.x) {
        const size_t first = chunk * kChunk;
        if (first + kChunk <= nvec) sum_max_chunk<false>(xv, first, nvec, total, m, nan);
        else sum_max_chunk<true>(xv, first, nvec, total, m, nan);
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

// count <= kMaxPartials = 4 * kFoldBlock: every lane's partials are
// requested before any is folded.
__global__ __launch_bounds__(kFoldBlock) void sum_max_pass2(const Partial *__restrict__ partials,
                                                            int count, double *sum_out,
                                                            float *max_out) {
    constexpr int kPer = kMaxPartials / kFoldBlock;
    __shared__ double lds_sum[kFoldBlock / kWave];
    __shared__ float lds_max[kFoldBlock / kWave];
    __shared__ int lds_nan[kFoldBlock / kWave];
    Partial p[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = (int)threadIdx.x + j * kFoldBlock;
        p[j] = partials[i < count ? i : 0];
    }
    double s = 0.0;
    float m = -__builtin_inff();
    bool nan = false;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        if ((int)threadIdx.x + j * kFoldBlock >= count) continue;
        s += p[j].sum;
        m = fmaxf(m, p[j].max);
        nan |= p[j].max != p[j].max;
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
        for (int w = 0; w < kFoldBlock / kWave; ++w) {
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
}  // namespace icsdk

// Partials of the allocation-free sum+max (tensor_sum_max_f32_no_alloc): one
// Partial per pass-1 block, and the pass-1 grid never exceeds kMaxPartials
// blocks (past that the blocks stride over chunks), so 64 KiB covers every
// input size. Each device the library runs on holds its own copy until the
// process ends. Host code never passes this name to a kernel: its device
// address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char
    scratch[sizeof(icsdk::Partial) * icsdk::kMaxPartials];

namespace icsdk {
namespace k {

size_t no_alloc_scratch_bytes() { return sizeof(scratch); }

hipError_t no_alloc_scratch(void **ptr) {
    constexpr int kMaxDevices = 64;
    static std::mutex lookup;
    static void *address[kMaxDevices] = {};
    *ptr = nullptr;
    int device = -1;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return status;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(lookup);
    if (address[device] == nullptr) {
        void *found = nullptr;
        status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
        if (status != hipSuccess) return status;
        address[device] = found;
    }
    *ptr = address[device];
    return hipSuccess;
}

size_t sum_max_partials_bytes(size_t n) {
    const size_t chunks = (n / 4 + kChunk - 1) / kChunk;
    const size_t grid = chunks < 1 ? 1 : (chunks > (size_t)kMaxPartials ? kMaxPartials : chunks);
    return grid * sizeof(Partial);
}

hipError_t sum_max_f32_no_alloc(const float *x, size_t n, double *sum_out, float *max_out,
                                void *scratch_ptr, size_t scratch_bytes, hipStream_t s) {
    if (n == 0 || ((uintptr_t)x & 15u) != 0 || scratch_ptr == nullptr ||
        sum_max_partials_bytes(n) > scratch_bytes)
        return hipErrorInvalidValue;
    return sum_max_f32(x, n, sum_out, max_out, scratch_ptr, s);
}


size_t grid_reduce_scratch_bytes() {
    return sizeof(Partial) * (kMaxPartials > kPartials ? kMaxPartials : kPartials);
}

hipError_t sum_max_f32(const float *x, size_t n, double *sum_out, float *max_out,
                       void *partials, hipStream_t s) {
    if (n == 0) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15u) != 0) return hipErrorInvalidValue;
    const size_t nvec = n / 4;
    const int grid = (int)(sum_max_partials_bytes(n) / sizeof(Partial));
    auto *p = static_cast<Partial *>(partials);
    hipLaunchKernelGGL(sum_max_pass1, dim3(grid), dim3(kBlock), 0, s, x, nvec, n, p);
    hipLaunchKernelGGL(sum_max_pass2, dim3(1), dim3(kFoldBlock), 0, s, p, grid, sum_out,
                       max_out);
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
