// Strided view with broadcast operands for gfx950:
//     y[i] = (x[view(i)] + addend[bcast(i)]) * mult[bcast(i)]
// with y contiguous in the view's shape.
//
// Four paths, chosen on the host from the strides:
//   vector  - the view's last dimension is contiguous in x (stride 1) and all
//             offsets are multiples of the 16-byte vector: every lane
//             decomposes its output-vector index with multiply-high
//             divisions, gathers one 16-byte vector of x (each a run of the
//             innermost dimension), applies the broadcast operands (a vector
//             when the operand spans the last dimension, a scalar when it is
//             broadcast along it) and stores 16 bytes;
//   vector tile - as vector, but the output dim next to the last one is not
//             adjacent to it in x while another dim is (a permutation such as
//             (0,2,1,3)): 8x8 tiles of contiguous runs are transposed through
//             LDS so that reads and writes are both contiguous 8-run rows;
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

// ---- LDS-staged vector tile path ----------------------------------------------

// For views whose last dimension L is contiguous in x and in the output but
// whose next-outer output dimension o is not adjacent to L in x, while some
// other dimension t is (x stride of t == L): e.g. a (0,2,1,3) permutation.
// A block moves an 8 x 8 tile of (o, t) "units" (one unit = the L contiguous
// elements, kVpu 16-byte vectors): it reads the tile as 8 rows of 8
// x-contiguous units, stages them in LDS, and writes 8 rows of 8
// output-contiguous units, so both HBM streams are contiguous runs of
// 8 * L elements. LDS rows are padded by 128 bytes so that the 16-lane
// phases of ds_read_b128 fall on disjoint banks when kVpu = 8.
constexpr int kTileUnits = 8;

struct TileVecPlan {
    int rank;
    int o, t;                       // tiled dims (o = rank - 2)
    uint64_t shape[kMaxRank];
    int64_t x_stride[kMaxRank];
    uint64_t a_stride[kMaxRank];
    uint64_t m_stride[kMaxRank];
    uint64_t y_stride[kMaxRank];
    uint64_t x_offset;
    uint32_t tiles_o, tiles_t;
    int a_vec, m_vec;
};

template <typename S, int kVpu>
__global__ __launch_bounds__(kBlock) void view_tile_vec_kernel(const S *__restrict__ x,
                                                               const S *__restrict__ addend,
                                                               const S *__restrict__ mult,
                                                               S *__restrict__ y,
                                                               TileVecPlan plan) {
    constexpr int E = Vec16<S>::N;
    constexpr int kRow = kTileUnits * kVpu + 8;  // vectors per LDS row (padded)
    constexpr int kVecs = kTileUnits * kTileUnits * kVpu;
    __shared__ Vec16<S> lds[kTileUnits * kRow];
    const int last = plan.rank - 1;
    const uint64_t block = blockIdx.x;
    const uint32_t bt = (uint32_t)(block % plan.tiles_t);
    const uint32_t bo = (uint32_t)((block / plan.tiles_t) % plan.tiles_o);
    uint64_t batch = block / ((uint64_t)plan.tiles_t * plan.tiles_o);
    int64_t xb = (int64_t)plan.x_offset;
    uint64_t ab = 0, mb = 0, yb = 0;
    for (int d = last - 1; d >= 0; --d) {
        if (d == plan.o || d == plan.t) continue;
        const uint64_t idx = batch % plan.shape[d];
        batch /= plan.shape[d];
        xb += (int64_t)idx * plan.x_stride[d];
        ab += idx * plan.a_stride[d];
        mb += idx * plan.m_stride[d];
        yb += idx * plan.y_stride[d];
    }
    const uint64_t o0 = (uint64_t)bo * kTileUnits, t0 = (uint64_t)bt * kTileUnits;
    const uint64_t no = plan.shape[plan.o], nt = plan.shape[plan.t];
    constexpr int kPer = (kVecs + kBlock - 1) / kBlock;  // vectors per thread per phase
    // read: o-rows of t-contiguous units (all of this thread's loads in flight)
    Vec16<S> xin[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int v = threadIdx.x + u * kBlock;
        const int oi = v / (kTileUnits * kVpu);
        const int rem = v - oi * (kTileUnits * kVpu);
        const int ti = rem / kVpu, c = rem - ti * kVpu;
        const bool ok = v < kVecs && o0 + oi < no && t0 + ti < nt;
        xin[u] = load16_stream(x + (ok ? xb + (int64_t)(o0 + oi) * plan.x_stride[plan.o] +
                                              (int64_t)(t0 + ti) * plan.x_stride[plan.t] + c * E
                                         : xb));
    }
    // the write phase's broadcast operands are fetched before the barrier
    Vec16<S> av[kPer], mv[kPer];
    float as[kPer], ms[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int v = threadIdx.x + u * kBlock;
        const int ti = v / (kTileUnits * kVpu);
        const int rem = v - ti * (kTileUnits * kVpu);
        const int oi = rem / kVpu, c = rem - oi * kVpu;
        const bool ok = v < kVecs && o0 + oi < no && t0 + ti < nt;
        as[u] = 0.0f;
        ms[u] = 1.0f;
        if (addend) {
            const uint64_t ao = ok ? ab + (t0 + ti) * plan.a_stride[plan.t] +
                                         (o0 + oi) * plan.a_stride[plan.o] : 0;
            if (plan.a_vec) av[u] = load16(addend + ao + (ok ? (uint64_t)c * E : 0));
            else as[u] = Elem<S>::load(addend[ao]);
        }
        if (mult) {
            const uint64_t mo = ok ? mb + (t0 + ti) * plan.m_stride[plan.t] +
                                         (o0 + oi) * plan.m_stride[plan.o] : 0;
            if (plan.m_vec) mv[u] = load16(mult + mo + (ok ? (uint64_t)c * E : 0));
            else ms[u] = Elem<S>::load(mult[mo]);
        }
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int v = threadIdx.x + u * kBlock;
        const int oi = v / (kTileUnits * kVpu);
        const int rem = v - oi * (kTileUnits * kVpu);
        const int ti = rem / kVpu, c = rem - ti * kVpu;
        if (v < kVecs) lds[oi * kRow + ti * kVpu + c] = xin[u];
    }
    __syncthreads();
    // write: t-rows of o-contiguous units
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int v = threadIdx.x + u * kBlock;
        const int ti = v / (kTileUnits * kVpu);
        const int rem = v - ti * (kTileUnits * kVpu);
        const int oi = rem / kVpu, c = rem - oi * kVpu;
        if (v >= kVecs || o0 + oi >= no || t0 + ti >= nt) continue;
        const Vec16<S> xv = lds[oi * kRow + ti * kVpu + c];
        Vec16<S> out;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float r = Elem<S>::load(xv.v[e]);
            if (addend) r = r + (plan.a_vec ? Elem<S>::load(av[u].v[e]) : as[u]);
            if (mult) r = r * (plan.m_vec ? Elem<S>::load(mv[u].v[e]) : ms[u]);
            out.v[e] = Elem<S>::store(r);
        }
        store16_stream(y + yb + (t0 + ti) * plan.y_stride[plan.t] +
                           (o0 + oi) * plan.y_stride[plan.o] + (uint64_t)c * E,
                       out);
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
    // LDS tile path: o = rank-2 is not next to the last dim in x but some
    // other dim t is (x stride == L); both streams become contiguous runs.
    if (vec && rank >= 3) {
        const int o = rank - 2;
        const int64_t L = (int64_t)v.shape[last];
        int t = -1;
        for (int d = 0; d < last; ++d)
            if (d != o && v.strides[d] == L && v.shape[d] > 1) t = d;
        const uint64_t vpu = v.shape[last] / E;
        if (t >= 0 && v.strides[o] != L && v.shape[o] > 1 &&
            (vpu == 1 || vpu == 2 || vpu == 4 || vpu == 8 || vpu == 16)) {
            TileVecPlan plan{};
            plan.rank = rank;
            plan.o = o;
            plan.t = t;
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
            plan.tiles_o = (uint32_t)((v.shape[o] + kTileUnits - 1) / kTileUnits);
            plan.tiles_t = (uint32_t)((v.shape[t] + kTileUnits - 1) / kTileUnits);
            plan.a_vec = a_vec;
            plan.m_vec = m_vec;
            const uint64_t batches = n / (v.shape[o] * v.shape[t] * v.shape[last]);
            const uint64_t blocks = batches * plan.tiles_o * plan.tiles_t;
            if (blocks < (uint64_t{1} << 31)) {
                const dim3 grid((unsigned)blocks), block(kBlock);
                switch (vpu) {
                    case 1: hipLaunchKernelGGL((view_tile_vec_kernel<S, 1>), grid, block, 0, s, x, addend, mult, y, plan); break;
                    case 2: hipLaunchKernelGGL((view_tile_vec_kernel<S, 2>), grid, block, 0, s, x, addend, mult, y, plan); break;
                    case 4: hipLaunchKernelGGL((view_tile_vec_kernel<S, 4>), grid, block, 0, s, x, addend, mult, y, plan); break;
                    case 8: hipLaunchKernelGGL((view_tile_vec_kernel<S, 8>), grid, block, 0, s, x, addend, mult, y, plan); break;
                    default: hipLaunchKernelGGL((view_tile_vec_kernel<S, 16>), grid, block, 0, s, x, addend, mult, y, plan); break;
                }
                return hipGetLastError();
            }
        }
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
