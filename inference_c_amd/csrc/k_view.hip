// Strided view with broadcast operands for gfx950:
//     y[i] = (x[view(i)] + addend[bcast(i)]) * mult[bcast(i)]
// with y contiguous in the view's shape.
//
// The host first coalesces the view: dimensions of extent 1 are dropped and a
// dimension is merged into its inner neighbour when x, the addend and the
// multiplier all step through both as through one (a contiguous tensor
// becomes rank 1, a (0,2,1,3) permutation stays rank 4). Then one of three
// paths runs, chosen from the coalesced strides:
//   gather  - the innermost dimension is contiguous in x and every offset is
//             a multiple of the 16-byte vector. One output vector per lane on
//             a one-shot grid: the block's outer coordinates are decomposed
//             once per block, the lane adds its (row, vector) offsets, loads
//             one 16-byte run of x, applies the broadcast operands (a vector
//             where the operand varies along the innermost dimension, a
//             scalar where it is broadcast along it) and stores 16 bytes
//             through L2. Each run is a whole contiguous vector, so no loaded
//             byte is wasted and no staging is needed; measured on MI355X
//             this beats staging the same permutation through LDS tiles at
//             every run length from 16 to 256 bytes;
//   tile    - x's contiguous dimension is another view dimension p (a
//             transpose of p with the innermost dimension): 64x64 tiles are
//             read along p, staged through LDS (padded against bank
//             conflicts) and written along the innermost dimension, so both
//             HBM streams stay coalesced;
//   scalar  - anything else: one element per lane.
#include "kern_common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <type_traits>

namespace icsdk {
namespace {

constexpr int kMaxRank = 8;

// The view after coalescing (element strides; 0 where an operand broadcasts).
struct Coalesced {
    int rank;
    uint64_t shape[kMaxRank];
    int64_t x_stride[kMaxRank];
    uint64_t a_stride[kMaxRank];
    uint64_t m_stride[kMaxRank];
};

// Contiguous strides of a broadcast operand, zeroed where its dim is 1.
inline void broadcast_strides(const uint64_t *shape, int rank, uint64_t *out) {
    uint64_t s = 1;
    for (int d = rank - 1; d >= 0; --d) {
        out[d] = shape[d] == 1 ? 0 : s;
        s *= shape[d];
    }
}

Coalesced coalesce(const k::ViewArgs &v, const uint64_t *a_stride, const uint64_t *m_stride) {
    Coalesced c{};
    // walk from the innermost dimension outwards, building c back to front
    int r = 0;
    uint64_t shape[kMaxRank];
    int64_t xs[kMaxRank];
    uint64_t as[kMaxRank], ms[kMaxRank];
    for (int d = v.rank - 1; d >= 0; --d) {
        if (v.shape[d] == 1) continue;
        if (r > 0) {
            const int in = r - 1;
            const bool merge = v.strides[d] == xs[in] * (int64_t)shape[in] &&
                               a_stride[d] == as[in] * shape[in] &&
                               m_stride[d] == ms[in] * shape[in];
            if (merge) {
                shape[in] *= v.shape[d];
                continue;
            }
        }
        shape[r] = v.shape[d];
        xs[r] = v.strides[d];
        as[r] = a_stride[d];
        ms[r] = m_stride[d];
        ++r;
    }
    if (r == 0) {  // every extent is 1
        shape[0] = 1;
        xs[0] = 1;
        as[0] = ms[0] = 0;
        r = 1;
    }
    c.rank = r;
    for (int i = 0; i < r; ++i) {
        c.shape[i] = shape[r - 1 - i];
        c.x_stride[i] = xs[r - 1 - i];
        c.a_stride[i] = as[r - 1 - i];
        c.m_stride[i] = ms[r - 1 - i];
    }
    return c;
}

// ---- gather path -------------------------------------------------------------

// The coalesced view is split into outer dims 0..R-3 and an inner plane of
// dims R-2 (rows) and R-1 (runs, counted in 16-byte vectors). A block covers
// kBlock consecutive vectors of one inner plane: its outer coordinates and
// their offsets are decomposed once per block from blockIdx (block-uniform,
// so the compiler keeps them in scalar registers and off the vector ALU),
// and each lane only splits its plane index into (row, vector) and adds two
// products per operand, in 32 bits. The quarter-rate 32-bit multiplies of a
// full per-lane decomposition otherwise sit between every lane and its load.
struct GatherPlan {
    int outer_rank;                // dims 0..outer_rank-1 (R - 2, or 0)
    FastDiv outer[kMaxRank];       // their extents
    uint64_t ox[kMaxRank], oa[kMaxRank], om[kMaxRank];  // their element strides
    FastDiv plane_blocks;          // blocks per inner plane
    FastDiv vecs;                  // vectors per row (innermost extent / E)
    int vecs_log2;                 // log2(vecs) when vecs is a power of two, else -1
    uint32_t plane;                // vectors per inner plane (rows * vecs)
    uint32_t row_x, row_a, row_m;  // element strides of the row dim
    uint64_t x_offset;
};

// How a broadcast operand enters: absent, one 16-byte vector per output
// vector (it varies along the innermost dimension) or one element per output
// vector (broadcast along it). A compile-time choice, so that every load of
// the kernel is unconditional: a load behind a run-time branch is followed by
// a wait for all outstanding loads, which would serialise the three streams.
enum OperandKind { kNone = 0, kVector = 1, kScalar = 2 };

template <typename S, int kA, int kM>
__global__ __launch_bounds__(kBlock) void view_gather_kernel(const S *__restrict__ x,
                                                             const S *__restrict__ addend,
                                                             const S *__restrict__ mult,
                                                             S *__restrict__ y,
                                                             GatherPlan plan) {
    constexpr int E = Vec16<S>::N;
    // block-uniform part
    const uint32_t b = blockIdx.x;
    uint32_t outer = fast_div(b, plan.plane_blocks);
    const uint32_t in_block = b - outer * plan.plane_blocks.divisor;
    const uint64_t out_vec0 = (uint64_t)outer * plan.plane + (uint64_t)in_block * kBlock;
    uint64_t xb = plan.x_offset, ab = 0, mb = 0;
    for (int d = plan.outer_rank - 1; d >= 0; --d) {
        uint32_t idx = outer;
        if (d > 0) {
            const uint32_t q = fast_div(outer, plan.outer[d]);
            idx = outer - q * plan.outer[d].divisor;
            outer = q;
        }
        xb += idx * plan.ox[d];
        ab += idx * plan.oa[d];
        mb += idx * plan.om[d];
    }
    // lane part
    const uint32_t t = in_block * kBlock + threadIdx.x;  // vector index inside the plane
    if (t >= plan.plane) return;
    const uint32_t row = plan.vecs_log2 >= 0 ? t >> plan.vecs_log2 : fast_div(t, plan.vecs);
    const uint32_t vec = t - row * plan.vecs.divisor;
    const Vec16<S> xv = load16_stream(x + xb + (row * plan.row_x + vec * E));
    Vec16<S> av, mv;
    float a_scalar = 0.0f, m_scalar = 1.0f;
    if constexpr (kA == kVector) av = load16(addend + ab + (row * plan.row_a + vec * E));
    if constexpr (kA == kScalar) a_scalar = Elem<S>::load(addend[ab + row * plan.row_a]);
    if constexpr (kM == kVector) mv = load16(mult + mb + (row * plan.row_m + vec * E));
    if constexpr (kM == kScalar) m_scalar = Elem<S>::load(mult[mb + row * plan.row_m]);
    Vec16<S> out;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        float r = Elem<S>::load(xv.v[e]);
        if constexpr (kA != kNone) r = r + (kA == kVector ? Elem<S>::load(av.v[e]) : a_scalar);
        if constexpr (kM != kNone) r = r * (kM == kVector ? Elem<S>::load(mv.v[e]) : m_scalar);
        out.v[e] = Elem<S>::store(r);
    }
    const OutWindow window(y + out_vec0 * E, kBlock * 16u);
    window.store16(threadIdx.x * 16u, out);
}

// Short gather: the common views -- at most two outer dims, whole blocks of
// kBlock vectors per inner plane, a power-of-two number of vectors per row,
// and every element offset below 2^32. The outer coordinates are blockIdx.z
// and blockIdx.y (a 3-D grid), strides are 32-bit, the row split is a shift
// and there is no bounds test: a wave reaches its loads after a few
// independent scalar loads instead of the general plan's chain of dependent
// ones (config-4 shape, measured in isolation: 23.6 -> 22.7 us).
struct ShortPlan {
    uint32_t ox[2], oa[2], om[2];  // element strides of the outer dims (grid z, y)
    uint32_t x_offset;
    uint32_t vecs_log2;            // log2(vectors per row)
    uint32_t row_x, row_a, row_m;  // element strides of the row dim
};

template <typename S, int kA, int kM>
__global__ __launch_bounds__(kBlock) void view_gather_short_kernel(const S *__restrict__ x,
                                                                   const S *__restrict__ addend,
                                                                   const S *__restrict__ mult,
                                                                   S *__restrict__ y,
                                                                   ShortPlan plan) {
    constexpr int E = Vec16<S>::N;
    const uint32_t xb = plan.x_offset + blockIdx.z * plan.ox[0] + blockIdx.y * plan.ox[1];
    const uint32_t ab = blockIdx.z * plan.oa[0] + blockIdx.y * plan.oa[1];
    const uint32_t mb = blockIdx.z * plan.om[0] + blockIdx.y * plan.om[1];
    const uint32_t plane_vec0 = blockIdx.x * kBlock;
    const size_t out_vec0 = ((size_t)blockIdx.z * gridDim.y + blockIdx.y) * (gridDim.x * kBlock) +
                            plane_vec0;
    const uint32_t t = plane_vec0 + threadIdx.x;
    const uint32_t row = t >> plan.vecs_log2;
    const uint32_t vec = t - (row << plan.vecs_log2);
    const Vec16<S> xv = load16_stream(x + (xb + row * plan.row_x + vec * E));
    Vec16<S> av, mv;
    float a_scalar = 0.0f, m_scalar = 1.0f;
    if constexpr (kA == kVector) av = load16(addend + (ab + row * plan.row_a + vec * E));
    if constexpr (kA == kScalar) a_scalar = Elem<S>::load(addend[ab + row * plan.row_a]);
    if constexpr (kM == kVector) mv = load16(mult + (mb + row * plan.row_m + vec * E));
    if constexpr (kM == kScalar) m_scalar = Elem<S>::load(mult[mb + row * plan.row_m]);
    Vec16<S> out;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        float r = Elem<S>::load(xv.v[e]);
        if constexpr (kA != kNone) r = r + (kA == kVector ? Elem<S>::load(av.v[e]) : a_scalar);
        if constexpr (kM != kNone) r = r * (kM == kVector ? Elem<S>::load(mv.v[e]) : m_scalar);
        out.v[e] = Elem<S>::store(r);
    }
    const OutWindow window(y + out_vec0 * E, kBlock * 16u);
    window.store16(threadIdx.x * 16u, out);
}

// The short plan of a view the gather path takes, or false when the view
// needs the general kernel.
template <typename S>
bool short_plan(const Coalesced &c, uint64_t x_offset, uint64_t n, ShortPlan *plan, dim3 *grid) {
    constexpr uint64_t E = Vec16<S>::N;
    const int last = c.rank - 1;
    const int outer_rank = c.rank >= 2 ? c.rank - 2 : 0;
    if (outer_rank > 2 || n > 0xffffffffull) return false;
    // offsets are unsigned 32-bit sums: a negative stride would make the
    // reach below wrap (and the base offset be truncated) undetected
    for (int d = 0; d < c.rank; ++d)
        if (c.x_stride[d] < 0) return false;
    const uint64_t vecs = c.shape[last] / E;
    const uint64_t rows = c.rank >= 2 ? c.shape[last - 1] : 1;
    const uint64_t plane = rows * vecs;
    if ((vecs & (vecs - 1)) != 0 || plane % kBlock != 0 || plane / kBlock > 0x7fffffffull)
        return false;
    uint64_t ext[2] = {1, 1}, ox[2] = {0, 0}, oa[2] = {0, 0}, om[2] = {0, 0};
    for (int d = 0; d < outer_rank; ++d) {
        const int slot = 2 - outer_rank + d;
        ext[slot] = c.shape[d];
        ox[slot] = (uint64_t)c.x_stride[d];
        oa[slot] = c.a_stride[d];
        om[slot] = c.m_stride[d];
    }
    if (ext[0] > 65535 || ext[1] > 65535) return false;
    const uint64_t row_x = c.rank >= 2 ? (uint64_t)c.x_stride[last - 1] : 0;
    const uint64_t row_a = c.rank >= 2 ? c.a_stride[last - 1] : 0;
    const uint64_t row_m = c.rank >= 2 ? c.m_stride[last - 1] : 0;
    // the largest element offset each operand is addressed at, in 32 bits
    auto reach = [&](uint64_t base, const uint64_t (&o)[2], uint64_t row, uint64_t inner) {
        return base + (ext[0] - 1) * o[0] + (ext[1] - 1) * o[1] + (rows - 1) * row + inner;
    };
    if (reach(x_offset, ox, row_x, vecs * E) > 0xffffffffull ||
        reach(0, oa, row_a, vecs * E) > 0xffffffffull || reach(0, om, row_m, vecs * E) > 0xffffffffull)
        return false;
    *plan = ShortPlan{{(uint32_t)ox[0], (uint32_t)ox[1]}, {(uint32_t)oa[0], (uint32_t)oa[1]},
                      {(uint32_t)om[0], (uint32_t)om[1]}, (uint32_t)x_offset,
                      (uint32_t)__builtin_ctzll(vecs), (uint32_t)row_x, (uint32_t)row_a,
                      (uint32_t)row_m};
    *grid = dim3((unsigned)(plane / kBlock), (unsigned)ext[1], (unsigned)ext[0]);
    return true;
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

// Transposes without operands in whole 16-byte vectors of E elements (8 for
// f16, 4 for f32; the tile's dims and every row start a multiple of E
// elements and 16-byte aligned; the launcher checks): a tile's 64 x rows (64
// elements along p, contiguous in x) are read as 64 / E vectors each into LDS
// rows [l], vector c of row l at slot c ^ (l / E); each output row (64
// elements along the last dim, contiguous in y) is gathered from one LDS
// column, E reads per vector, and written as 64 / E vectors. With the slot
// swizzle the 64 lanes of a gather read distinct banks (f16: 32, lanes 2m
// and 2m + 1 sharing a dword; f32: 64). A block takes
// kVecTiles tiles along the last dim, all of a lane's loads issued first
// ([4096, 4096]: one tile per block 15.0 us, two 13.1, four 12.7-12.8). The
// scalar kernel below moves one element per lane per access.
//
// Everything a wave needs before its first load arrives as a plain scalar
// argument (preloaded in SGPRs; the tile grid split by multiply-high
// divisions); the plan is read only by blocks past the first batch.
// 64 x 64 tiles per block along the last dim: 4 for 2-byte elements (32 KB
// of LDS), 1 for f32 (16 KB; f32 [4096, 4096]: 29.7 us with 2, 27.7 with 1)
template <typename S> constexpr uint32_t kVecTiles = sizeof(S) == 2 ? 4 : 1;
template <typename S>
__global__ __launch_bounds__(kBlock) void view_tile_vec_kernel(
    const S *__restrict__ x, S *__restrict__ y, uint32_t tiles_l, uint32_t tl_mul,
    uint32_t tl_shift, uint32_t tiles_p, uint32_t tp_mul, uint32_t tp_shift, uint32_t np,
    uint32_t nl, uint32_t xs_last, uint32_t x_offset, uint32_t ys, TilePlan plan) {
    static_assert(sizeof(S) == 2 || sizeof(S) == 4, "2- or 4-byte elements");
    constexpr uint32_t E = Vec16<S>::N;              // elements per 16-byte vector
    constexpr uint32_t kSlots = kTile / E;           // vectors per 64-element row
    constexpr uint32_t kRowsPerPass = kBlock / kSlots;
    constexpr uint32_t kTiles = kVecTiles<S>;
    using U = std::conditional_t<sizeof(S) == 2, uint16_t, uint32_t>;
    __shared__ u32x4 tile[kTiles][kTile][kSlots];
    const uint32_t block = blockIdx.x;
    const uint32_t rest = fast_div(block, FastDiv{tiles_l, tl_mul, tl_shift});
    const uint32_t tl = block - rest * tiles_l;
    uint32_t batch = fast_div(rest, FastDiv{tiles_p, tp_mul, tp_shift});
    const uint32_t tp = rest - batch * tiles_p;
    int64_t xb = (int64_t)x_offset;
    uint64_t yb = 0;
    if (batch != 0) {   // block-uniform; batch 0 has every batch index 0
        const int last = plan.rank - 1;
        uint64_t b = batch;
        for (int d = last - 1; d >= 0; --d) {
            if (d == plan.p) continue;
            const uint64_t idx = b % plan.shape[d];
            b /= plan.shape[d];
            xb += (int64_t)idx * plan.x_stride[d];
            yb += idx * plan.y_stride[d];
        }
    }
    const uint32_t p0 = tp * kTile, l0 = tl * (kTiles * kTile);
    const uint32_t c = threadIdx.x % kSlots;
#pragma unroll
    for (uint32_t tt = 0; tt < kTiles; ++tt)
#pragma unroll
    for (uint32_t pass = 0; pass < kTile / kRowsPerPass; ++pass) {
        const uint32_t l = threadIdx.x / kSlots + kRowsPerPass * pass;
        const uint32_t li = l0 + kTile * tt + l, pi = p0 + E * c;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (li < nl && pi < np)
            v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(
                x + xb + (int64_t)li * xs_last + pi));
        tile[tt][l][c ^ (l / E % kSlots)] = v;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t tt = 0; tt < kTiles; ++tt)
#pragma unroll
    for (uint32_t pass = 0; pass < kTile / kRowsPerPass; ++pass) {
        const uint32_t pr = threadIdx.x / kSlots + kRowsPerPass * pass;
        const uint32_t pi = p0 + pr, li = l0 + kTile * tt + E * c;
        if (pi < np && li < nl) {
            // element (l = E c + k, p = pr): row l, slot (pr / E) ^ c, element pr % E
            uint32_t h[E];
#pragma unroll
            for (uint32_t k = 0; k < E; ++k) {
                const U *row = reinterpret_cast<const U *>(&tile[tt][E * c + k][0]);
                h[k] = row[(((pr / E) ^ c) * E) + pr % E];
            }
            u32x4 o;
            if constexpr (sizeof(S) == 2)
                o = u32x4{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16};
            else
                o = u32x4{h[0], h[1], h[2], h[3]};
            *reinterpret_cast<u32x4 *>(y + yb + (uint64_t)pi * ys + li) = o;
        }
    }
}

inline bool aligned16(const void *p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Gather-path plan for a coalesced view, or false when the view does not fit
// it: innermost dim not contiguous or not whole vectors, offsets not
// vector-aligned, or a plane whose lane offsets or a grid that exceeds 32 bits.
template <typename S>
bool gather_plan(const Coalesced &c, uint64_t x_offset, uint64_t n, bool have_a, bool have_m,
                 GatherPlan *plan, uint32_t *blocks) {
    constexpr uint64_t E = Vec16<S>::N;
    const int last = c.rank - 1;
    if (c.x_stride[last] != 1 || c.shape[last] % E != 0 || x_offset % E != 0) return false;
    for (int d = 0; d < last; ++d)
        if (c.x_stride[d] < 0) return false;  // offsets are unsigned sums
    const bool a_vec = have_a && c.a_stride[last] != 0;
    const bool m_vec = have_m && c.m_stride[last] != 0;
    for (int d = 0; d < last; ++d) {
        if (c.x_stride[d] % E != 0) return false;
        if (a_vec && c.a_stride[d] % E != 0) return false;
        if (m_vec && c.m_stride[d] % E != 0) return false;
    }
    const uint64_t vecs = c.shape[last] / E;
    const uint64_t rows = c.rank >= 2 ? c.shape[last - 1] : 1;
    const uint64_t row_x = c.rank >= 2 ? (uint64_t)c.x_stride[last - 1] : 0;
    const uint64_t row_a = c.rank >= 2 ? c.a_stride[last - 1] : 0;
    const uint64_t row_m = c.rank >= 2 ? c.m_stride[last - 1] : 0;
    const uint64_t plane = rows * vecs;
    const uint64_t plane_blocks = (plane + kBlock - 1) / kBlock;
    const uint64_t outer = n / (plane * E);
    const uint64_t lim = 0xffffffffull;
    if (plane > lim / 2 || plane_blocks * outer > 0x7fffffffull || outer > lim ||
        (rows - 1) * row_x + vecs * E > lim || (rows - 1) * row_a + vecs * E > lim ||
        (rows - 1) * row_m + vecs * E > lim)
        return false;
    *plan = GatherPlan{};
    plan->outer_rank = c.rank >= 2 ? c.rank - 2 : 0;
    for (int d = 0; d < plan->outer_rank; ++d) {
        plan->outer[d] = make_fast_div((uint32_t)c.shape[d]);
        plan->ox[d] = (uint64_t)c.x_stride[d];
        plan->oa[d] = c.a_stride[d];
        plan->om[d] = c.m_stride[d];
    }
    plan->plane_blocks = make_fast_div((uint32_t)plane_blocks);
    plan->vecs = make_fast_div((uint32_t)vecs);
    plan->vecs_log2 = (vecs & (vecs - 1)) == 0 ? __builtin_ctzll(vecs) : -1;
    plan->plane = (uint32_t)plane;
    plan->row_x = (uint32_t)row_x;
    plan->row_a = (uint32_t)row_a;
    plan->row_m = (uint32_t)row_m;
    plan->x_offset = x_offset;
    *blocks = (uint32_t)(plane_blocks * outer);
    return true;
}

// ---- copy path ---------------------------------------------------------------

// A view that coalesces to one contiguous run, with neither operand, is a
// copy of that run: one 16-byte vector per lane over a 1-D grid, the
// arguments plain scalars (preloaded in SGPRs), nothing in front of the load
// but the lane's offset. kWhole: the run is a whole number of blocks, so no
// lane needs the bounds select; otherwise lanes past the end re-read vector
// 0 and the last block's output window ends at the run's end (their stores
// are dropped by the range check). Measured on MI355X against the gather
// kernels' copy of the same run: 0.7-0.8 us less per launch at 67-268 MB
// (the gather kernels form outer coordinates and 64-bit addresses first).
template <typename S, bool kWhole>
__global__ __launch_bounds__(kBlock) void view_copy_kernel(const S *__restrict__ x,
                                                           S *__restrict__ y, uint32_t vecs) {
    constexpr uint32_t E = Vec16<S>::N;
    const uint32_t v0 = blockIdx.x * kBlock;
    const uint32_t v = v0 + threadIdx.x;
    const Vec16<S> xv = load16_stream(x + (size_t)(kWhole || v < vecs ? v : 0u) * E);
    const uint32_t left = vecs - v0;
    const OutWindow w(y + (size_t)v0 * E, (kWhole || left >= kBlock ? kBlock : left) * 16u);
    w.store16(threadIdx.x * 16u, xv);
}

template <typename S>
hipError_t launch_view(const S *x, const k::ViewArgs &v, const S *addend,
                       const S *mult, S *y, hipStream_t s) {
    const int rank = v.rank;
    if (rank < 1 || rank > kMaxRank) return hipErrorInvalidValue;
    uint64_t n = 1;
    for (int d = 0; d < rank; ++d) n *= v.shape[d];
    if (n == 0) return hipSuccess;
    uint64_t a_stride[kMaxRank] = {}, m_stride[kMaxRank] = {};
    broadcast_strides(v.addend_shape, rank, a_stride);
    broadcast_strides(v.mult_shape, rank, m_stride);
    if (!addend) std::fill(a_stride, a_stride + rank, 0);
    if (!mult) std::fill(m_stride, m_stride + rank, 0);
    const Coalesced c = coalesce(v, a_stride, m_stride);
    const int last = c.rank - 1;

    if (!addend && !mult && c.rank == 1 && c.x_stride[0] == 1 && aligned16(x + v.offset) &&
        aligned16(y) && n % Vec16<S>::N == 0 && n / Vec16<S>::N <= 0xffffffffull - kBlock) {
        const uint32_t vecs = (uint32_t)(n / Vec16<S>::N);
        const dim3 grid((vecs + kBlock - 1) / kBlock), block(kBlock);
        if (vecs % kBlock == 0)
            hipLaunchKernelGGL((view_copy_kernel<S, true>), grid, block, 0, s, x + v.offset, y, vecs);
        else
            hipLaunchKernelGGL((view_copy_kernel<S, false>), grid, block, 0, s, x + v.offset, y, vecs);
        return hipGetLastError();
    }

    GatherPlan gp;
    uint32_t blocks = 0;
    if (aligned16(x) && aligned16(y) && aligned16(addend) && aligned16(mult) &&
        gather_plan<S>(c, v.offset, n, addend != nullptr, mult != nullptr, &gp, &blocks)) {
        const int ka = !addend ? kNone : c.a_stride[last] != 0 ? kVector : kScalar;
        const int km = !mult ? kNone : c.m_stride[last] != 0 ? kVector : kScalar;
        ShortPlan sp;
        dim3 short_grid;
        const bool use_short = short_plan<S>(c, v.offset, n, &sp, &short_grid);
        const dim3 grid(blocks), block(kBlock);
#define ICSDK_GATHER(A, M)                                                                      \
    do {                                                                                        \
        if (use_short)                                                                          \
            hipLaunchKernelGGL((view_gather_short_kernel<S, A, M>), short_grid, block, 0, s, x,  \
                               addend, mult, y, sp);                                            \
        else                                                                                    \
            hipLaunchKernelGGL((view_gather_kernel<S, A, M>), grid, block, 0, s, x, addend,     \
                               mult, y, gp);                                                    \
    } while (0)
        switch (ka * 3 + km) {
            case 0: ICSDK_GATHER(kNone, kNone); break;
            case 1: ICSDK_GATHER(kNone, kVector); break;
            case 2: ICSDK_GATHER(kNone, kScalar); break;
            case 3: ICSDK_GATHER(kVector, kNone); break;
            case 4: ICSDK_GATHER(kVector, kVector); break;
            case 5: ICSDK_GATHER(kVector, kScalar); break;
            case 6: ICSDK_GATHER(kScalar, kNone); break;
            case 7: ICSDK_GATHER(kScalar, kVector); break;
            default: ICSDK_GATHER(kScalar, kScalar); break;
        }
#undef ICSDK_GATHER
        return hipGetLastError();
    }

    // tile path: exactly one coalesced dim p != last has x stride 1
    int p = -1;
    for (int d = 0; d < last; ++d)
        if (c.x_stride[d] == 1) p = p < 0 ? d : -2;
    if (p >= 0 && c.x_stride[last] != 1) {
        TilePlan plan{};
        plan.rank = c.rank;
        plan.p = p;
        uint64_t ys = 1;
        for (int d = last; d >= 0; --d) {
            plan.shape[d] = c.shape[d];
            plan.x_stride[d] = c.x_stride[d];
            plan.a_stride[d] = c.a_stride[d];
            plan.m_stride[d] = c.m_stride[d];
            plan.y_stride[d] = ys;
            ys *= c.shape[d];
        }
        plan.x_offset = v.offset;
        plan.batches = n / (c.shape[p] * c.shape[last]);
        plan.tiles_p = (uint32_t)((c.shape[p] + kTile - 1) / kTile);
        plan.tiles_l = (uint32_t)((c.shape[last] + kTile - 1) / kTile);
        const uint64_t blocks = plan.batches * plan.tiles_p * plan.tiles_l;
        if (blocks < (uint64_t{1} << 31)) {
            {
                // whole 16-byte vectors: p and last a multiple of E elements,
                // every x row and batch offset too, both tensors 16-byte aligned
                // (the scalar arguments hold dims, the x row stride, the
                // offset and the output row stride in 32 bits)
                const uint64_t lim = 0xffffffffull;
                constexpr uint64_t E = Vec16<S>::N;
                bool vec = addend == nullptr && mult == nullptr && c.shape[p] % E == 0 &&
                           c.shape[last] % E == 0 && v.offset % E == 0 &&
                           ((uintptr_t)x & 15u) == 0 && ((uintptr_t)y & 15u) == 0 &&
                           c.shape[p] + kTile <= lim && c.shape[last] + kTile <= lim &&
                           c.x_stride[last] > 0 && (uint64_t)c.x_stride[last] <= lim &&
                           v.offset <= lim && plan.y_stride[p] <= lim;
                for (int d = 0; d <= last; ++d)
                    if (d != p && c.x_stride[d] % (int64_t)E != 0) vec = false;
                if (vec) {
                    const uint32_t pairs_l = (plan.tiles_l + kVecTiles<S> - 1) / kVecTiles<S>;
                    const uint64_t vblocks = plan.batches * plan.tiles_p * pairs_l;
                    const FastDiv dl = make_fast_div(pairs_l), dp = make_fast_div(plan.tiles_p);
                    hipLaunchKernelGGL((view_tile_vec_kernel<S>), dim3((unsigned)vblocks),
                                       dim3(kBlock), 0, s, x, y, pairs_l, dl.multiplier,
                                       dl.shift, plan.tiles_p, dp.multiplier, dp.shift,
                                       (uint32_t)c.shape[p], (uint32_t)c.shape[last],
                                       (uint32_t)c.x_stride[last], (uint32_t)v.offset,
                                       (uint32_t)plan.y_stride[p], plan);
                    return hipGetLastError();
                }
            }
            hipLaunchKernelGGL((view_tile_kernel<S>), dim3((unsigned)blocks), dim3(kBlock), 0,
                               s, x, addend, mult, y, plan);
            return hipGetLastError();
        }
    }

    ScalarPlan plan{};
    plan.rank = c.rank;
    for (int d = 0; d < c.rank; ++d) {
        plan.shape[d] = c.shape[d];
        plan.x_stride[d] = c.x_stride[d];
        plan.a_stride[d] = c.a_stride[d];
        plan.m_stride[d] = c.m_stride[d];
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
