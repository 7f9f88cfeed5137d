// Strided view with broadcast operands for gfx950:
//     y[i] = (x[view(i)] + addend[bcast(i)]) * mult[bcast(i)]
// with y contiguous in the view's shape.
//
// Three paths, chosen on the host from the strides:
//   vector  - the view's last dimension is contiguous in x (stride 1) and all
//             offsets are multiples of the 16-byte vector: every lane
//             decomposes its output-vector index with multiply-high
//             divisions, gathers one 16-byte vector of x (each a run of the
//             innermost dimension), applies the broadcast operands (a vector
//             when the operand spans the last dimension, a scalar when it is
//             broadcast along it) and stores 16 bytes;
//   tile    - x's contiguous dimension is another view dimension p (a
//             transpose of p with the last dimension): 64x64 tiles are read
//             along p, staged through LDS (padded against bank conflicts) and
//             written along the last dimension, so both sides stay coalesced;
//   scalar  - anything else: one element per lane.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

constexpr int kMaxRank = 8;

struct ViewPlan {
    int rank;
    FastDiv dims[kMaxRank];        // output extents (last one in vectors for the vector path)
    int64_t x_stride[kMaxRank];    // x element strides
    uint64_t a_stride[kMaxRank];   // addend element strides (0 where broadcast)
    uint64_t m_stride[kMaxRank];   // multiplier element strides (0 where broadcast)
    uint64_t x_offset;
    int a_vec;                     // addend varies along the last dim
    int m_vec;                     // multiplier varies along the last dim
};

template <typename S>
__device__ inline float opt_load(const S *p, uint64_t i) {
    return Elem<S>::load(p[i]);
}

// ---- vector path -------------------------------------------------------------

template <typename S>
__global__ __launch_bounds__(kBlock) void view_vec_kernel(const S *__restrict__ x,
                                                          const S *__restrict__ addend,
                                                          const S *__restrict__ mult,
                                                          S *__restrict__ y, uint32_t nvec,
                                                          ViewPlan plan) {
    constexpr int E = Vec16<S>::N;
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nvec; v += stride) {
        uint32_t rest = v;
        int64_t xo = (int64_t)plan.x_offset;
        uint64_t ao = 0, mo = 0;
#pragma unroll
        for (int d = kMaxRank - 1; d >= 0; --d) {
            if (d < plan.rank) {
                const uint32_t q = fast_div(rest, plan.dims[d]);
                uint32_t idx = rest - q * plan.dims[d].divisor;
                rest = q;
                if (d == plan.rank - 1) idx *= E;  // last dim counted in vectors
                xo += (int64_t)idx * plan.x_stride[d];
                ao += (uint64_t)idx * plan.a_stride[d];
                mo += (uint64_t)idx * plan.m_stride[d];
            }
        }
        const Vec16<S> xv = load16(x + xo);
        Vec16<S> av{}, mv{};
        float as = 0.0f, ms = 1.0f;
        if (addend) {
            if (plan.a_vec) av = load16(addend + ao);
            else as = Elem<S>::load(addend[ao]);
        }
        if (mult) {
            if (plan.m_vec) mv = load16(mult + mo);
            else ms = Elem<S>::load(mult[mo]);
        }
        Vec16<S> out;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float r = Elem<S>::load(xv.v[e]);
            if (addend) r = r + (plan.a_vec ? Elem<S>::load(av.v[e]) : as);
            if (mult) r = r * (plan.m_vec ? Elem<S>::load(mv.v[e]) : ms);
            out.v[e] = Elem<S>::store(r);
        }
        store16_stream(y + (size_t)v * E, out);
    }
}

// ---- scalar path -------------------------------------------------------------

struct ScalarPlan {
    int rank;
    uint64_t shape[kMaxRank];
    int64_t x_stride[kMaxRank];
    uint64_t a_stride[kMaxRank];
    uint64_t m_stride[kMaxRank];
    uint64_t x_offset;
};

template <typename S>
__global__ __launch_bounds__(kBlock) void view_scalar_kernel(const S *__restrict__ x,
                                                             const S *__restrict__ addend,
                                                             const S *__restrict__ mult,
                                                             S *__restrict__ y, size_t n,
                                                             ScalarPlan plan) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        size_t rest = i;
        int64_t xo = (int64_t)plan.x_offset;
        uint64_t ao = 0, mo = 0;
        for (int d = plan.rank - 1; d >= 0; --d) {
            const uint64_t idx = rest % plan.shape[d];
            rest /= plan.shape[d];
            xo += (int64_t)idx * plan.x_stride[d];
            ao += idx * plan.a_stride[d];
            mo += idx * plan.m_stride[d];
        }
        float r = Elem<S>::load(x[xo]);
        if (addend) r = r + Elem<S>::load(addend[ao]);
        if (mult) r = r * Elem<S>::load(mult[mo]);
        y[i] = Elem<S>::store(r);
    }
}

// ---- LDS-tiled transpose path ------------------------------------------------

// Output dims are viewed as [outer..., P, inner..., L] where dimension p has
// x stride 1 and L is the last view dimension. A block moves one 64x64 tile
// of (p, last) for one combination of the remaining indices ("batch").
constexpr int kTile = 64;

struct TilePlan {
    int rank;
    int p;                          // view dim with x stride 1
    uint64_t shape[kMaxRank];
    int64_t x_stride[kMaxRank];
    uint64_t a_stride[kMaxRank];
    uint64_t m_stride[kMaxRank];
    uint64_t y_stride[kMaxRank];    // contiguous output strides
    uint64_t x_offset;
    uint64_t batches;               // product of the dims other than p and last
    uint32_t tiles_p, tiles_l;
};

template <typename S>
__global__ __launch_bounds__(kBlock) void view_tile_kernel(const S *__restrict__ x,
                                                           const S *__restrict__ addend,
                                                           const S *__restrict__ mult,
                                                           S *__restrict__ y, TilePlan plan) {
    __shared__ float tile[kTile][kTile + 1];
    const int last = plan.rank - 1;
    const uint64_t block = blockIdx.x;
    const uint32_t tl = (uint32_t)(block % plan.tiles_l);
    const uint32_t tp = (uint32_t)((block / plan.tiles_l) % plan.tiles_p);
    uint64_t batch = block / ((uint64_t)plan.tiles_l * plan.tiles_p);
    // base offsets from the batch index (dims other than p and last)
    int64_t xb = (int64_t)plan.x_offset;
    uint64_t ab = 0, mb = 0, yb = 0;
    for (int d = last - 1; d >= 0; --d) {
        if (d == plan.p) continue;
        const uint64_t idx = batch % plan.shape[d];
        batch /= plan.shape[d];
        xb += (int64_t)idx * plan.x_stride[d];
        ab += idx * plan.a_stride[d];
        mb += idx * plan.m_stride[d];
        yb += idx * plan.y_stride[d];
    }
    const uint64_t p0 = (uint64_t)tp * kTile, l0 = (uint64_t)tl * kTile;
    const uint64_t np = plan.shape[plan.p], nl = plan.shape[last];
    // read: consecutive threads walk p (contiguous in x)
    const uint32_t tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
    for (uint32_t r = ty; r < kTile; r += kBlock / kTile) {
        const uint64_t pi = p0 + tx, li = l0 + r;
        if (pi < np && li < nl)
            tile[r][tx] = Elem<S>::load(x[xb + (int64_t)pi * plan.x_stride[plan.p] +
                                          (int64_t)li * plan.x_stride[last]]);
    }
    __syncthreads();
    // write: consecutive threads walk the last dim (contiguous in y)
    for (uint32_t r = ty; r < kTile; r += kBlock / kTile) {
        const uint64_t pi = p0 + r, li = l0 + tx;
        if (pi < np && li < nl) {
            float v = tile[tx][r];
            if (addend) v = v + Elem<S>::load(addend[ab + pi * plan.a_stride[plan.p] +
                                                      li * plan.a_stride[last]]);
            if (mult) v = v * Elem<S>::load(mult[mb + pi * plan.m_stride[plan.p] +
                                                  li * plan.m_stride[last]]);
            y[yb + pi * plan.y_stride[plan.p] + li] = Elem<S>::store(v);
        }
    }
}

inline bool aligned16(const void *p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Contiguous strides of a broadcast operand, zeroed where its dim is 1.
inline void broadcast_strides(const uint64_t *shape, int rank, uint64_t *out) {
    uint64_t s = 1;
    for (int d = rank - 1; d >= 0; --d) {
        out[d] = shape[d] == 1 ? 0 : s;
        s *= shape[d];
    }
}

template <typename S>
hipError_t launch_view(const S *x, const k::ViewArgs &v, const S *addend, const S *mult,
                       S *y, hipStream_t s) {
    constexpr int E = Vec16<S>::N;
    const int rank = v.rank;
    if (rank < 1 || rank > kMaxRank) return hipErrorInvalidValue;
    uint64_t n = 1;
    for (int d = 0; d < rank; ++d) n *= v.shape[d];
    if (n == 0) return hipSuccess;
    uint64_t a_stride[kMaxRank] = {}, m_stride[kMaxRank] = {};
    broadcast_strides(v.addend_shape, rank, a_stride);
    broadcast_strides(v.mult_shape, rank, m_stride);
    const int last = rank - 1;

    // vector path
    bool vec = v.strides[last] == 1 && v.shape[last] % E == 0 && v.offset % E == 0 &&
               aligned16(x) && aligned16(y) && aligned16(addend) && aligned16(mult) &&
               n / E < (uint64_t{1} << 32);
    for (int d = 0; d < last && vec; ++d) vec = v.strides[d] % E == 0 && v.shape[d] < (uint64_t{1} << 32);
    const bool a_vec = addend && v.addend_shape[last] != 1;
    const bool m_vec = mult && v.mult_shape[last] != 1;
    for (int d = 0; d < last && vec; ++d) {
        if (a_vec) vec = a_stride[d] % E == 0;
        if (vec && m_vec) vec = m_stride[d] % E == 0;
    }
    if (vec) {
        ViewPlan plan{};
        plan.rank = rank;
        for (int d = 0; d < rank; ++d) {
            const uint64_t extent = d == last ? v.shape[d] / E : v.shape[d];
            plan.dims[d] = make_fast_div((uint32_t)extent);
            plan.x_stride[d] = v.strides[d];
            plan.a_stride[d] = a_stride[d];
            plan.m_stride[d] = m_stride[d];
        }
        plan.x_offset = v.offset;
        plan.a_vec = a_vec;
        plan.m_vec = m_vec;
        const uint64_t nvec = n / E;
        uint64_t grid = (nvec + kBlock * 4 - 1) / (kBlock * 4);
        if (grid > (1u << 20)) grid = 1u << 20;
        hipLaunchKernelGGL((view_vec_kernel<S>), dim3((unsigned)grid), dim3(kBlock), 0, s, x,
                           addend, mult, y, (uint32_t)nvec, plan);
        return hipGetLastError();
    }

    // tile path: exactly one view dim p != last has x stride 1
    int p = -1;
    for (int d = 0; d < last; ++d)
        if (v.strides[d] == 1 && v.shape[d] > 1) p = p < 0 ? d : -2;
    if (p >= 0 && v.strides[last] != 1 && v.shape[last] > 1) {
        TilePlan plan{};
        plan.rank = rank;
        plan.p = p;
        uint64_t ys = 1;
        for (int d = last; d >= 0; --d) {
            plan.shape[d] = v.shape[d];
            plan.x_stride[d] = v.strides[d];
            plan.a_stride[d] = a_stride[d];
            plan.m_stride[d] = m_stride[d];
            plan.y_stride[d] = ys;
            ys *= v.shape[d];
        }
        plan.x_offset = v.offset;
        plan.batches = n / (v.shape[p] * v.shape[last]);
        plan.tiles_p = (uint32_t)((v.shape[p] + kTile - 1) / kTile);
        plan.tiles_l = (uint32_t)((v.shape[last] + kTile - 1) / kTile);
        const uint64_t blocks = plan.batches * plan.tiles_p * plan.tiles_l;
        if (blocks < (uint64_t{1} << 31)) {
            hipLaunchKernelGGL((view_tile_kernel<S>), dim3((unsigned)blocks), dim3(kBlock), 0,
                               s, x, addend, mult, y, plan);
            return hipGetLastError();
        }
    }

    ScalarPlan plan{};
    plan.rank = rank;
    for (int d = 0; d < rank; ++d) {
        plan.shape[d] = v.shape[d];
        plan.x_stride[d] = v.strides[d];
        plan.a_stride[d] = a_stride[d];
        plan.m_stride[d] = m_stride[d];
    }
    plan.x_offset = v.offset;
    uint64_t grid = (n + kBlock * 4 - 1) / (kBlock * 4);
    if (grid > (1u << 20)) grid = 1u << 20;
    hipLaunchKernelGGL((view_scalar_kernel<S>), dim3((unsigned)grid), dim3(kBlock), 0, s, x,
                       addend, mult, y, (size_t)n, plan);
    return hipGetLastError();
}

}  // namespace

namespace k {

hipError_t view_add_mul_f32(const float *x, const ViewArgs &v, const float *addend,
                            const float *mult, float *y, hipStream_t s) {
    return launch_view<float>(x, v, addend, mult, y, s);
}

hipError_t view_add_mul_f16(const uint16_t *x, const ViewArgs &v, const uint16_t *addend,
                            const uint16_t *mult, uint16_t *y, hipStream_t s) {
    return launch_view<_Float16>(reinterpret_cast<const _Float16 *>(x), v,
                                 reinterpret_cast<const _Float16 *>(addend),
                                 reinterpret_cast<const _Float16 *>(mult),
                                 reinterpret_cast<_Float16 *>(y), s);
}

}  // namespace k
}  // namespace icsdk
