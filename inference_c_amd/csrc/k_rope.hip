// Split-half (NeoX) rotary position embedding for gfx950, in place on
// q [seq, q_heads, dim] and k [seq, k_heads, dim].
//
// Fused path (half = dim/2 a multiple of the 16-byte vector, half <= 128,
// 16-byte aligned tensors): one kernel. The host computes the pair
// denominators pow(theta, 2d/dim) in double with the C library's pow, as the
// reference does, and passes them as kernel arguments. A block covers whole
// positions: each lane pair first issues the loads of its (head row, chunk)
// items -- one lane the left vector (pairs d..d+E-1), its partner 32 lanes
// away the right vector (pairs d+half..), both streamed, so a wave's load
// covers whole contiguous rows -- then a few lanes compute the block's
// rotations, angle = (float)((double)(offset + p) / denom[d]) and sincosf,
// into LDS, and after one barrier the pair exchanges its vectors across the
// wave halves, every lane rotates its side's pairs in f32 (left*c - right*s,
// right*c + left*s, no contraction) and stores its vector, written through
// L2 into the bytes it came from. Every q/k byte is read once and written
// once; the angles cost `half` sincos per position, shared by all heads of
// the position.
//
// Table path (other shapes): a table kernel computes the same (cos, sin) per
// (position, pair) into device scratch, then one lane per pair rotates.
#include "kern_common.hpp"
#include "kernels.hpp"

#include <cmath>

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

// table path: one pair per lane
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


// ---- fused path ------------------------------------------------------------

constexpr int kMaxHalf = 128;       // pairs per head row on the fused path (<= kBlock)
constexpr int kLdsPairs = 2048;     // (position, pair) rotations per block

struct RopeDenoms {
    double d[kMaxHalf];
};

// Item = (position, row, chunk): row < qh is a q head, else a k head; chunk
// c covers pairs c*E .. c*E+E-1. Items are numbered position-major; block
// (x, y) owns items y*kIt*128 .. +kIt*128 of positions x*ppb ..
// x*ppb+ppb-1 and computes those positions' rotations. Wave w of the block
// takes the item groups w*kIt .. w*kIt+kIt-1 (32 items each), so its kIt
// groups are consecutive: when a position has a multiple of 32*kIt items
// (config 5: 256), all of a wave's items share one position and each lane
// one chunk, and the lane reads its E rotations from LDS once instead of
// once per item (a read is skipped whenever no lane of the wave needs a
// different slot than for the previous group).
//
// Lanes l and l + 32 of a wave share an item: lane l < 32 moves the item's
// left vector, lane l + 32 its right vector (half elements further on). A
// wave's 32 items are consecutive, so each of its load and store
// instructions covers whole rows -- 32 / kChunks rows of 2 * half elements,
// one contiguous run -- instead of the left (or right) halves of twice as
// many rows. One v_permlane32_swap per dword then gives every lane both
// vectors (lanes 0-31 keep theirs in the first result and receive lane + 32's
// in the second; lanes 32-63 receive lane - 32's in the first and keep theirs
// in the second, so in every lane the first result is the left vector and the
// second the right one), and each lane writes its own side:
// left' = l*c + r*(-s) (== l*c - r*s exactly), right' = r*c + l*s.
// A lane handles kIt items; its loads are issued unconditionally (a lane
// past the end re-reads item 0, which lane 0 loads anyway) so that no branch
// makes it wait for one item before requesting the next, and there is no
// loop, so nothing waits for the loads before the rotations are computed.
constexpr uint32_t kPairItems = kBlock / 2;   // items per block and per kIt

// Items per lane pair the host aims for (1, 2, 4 or 8).
#ifndef ICSDK_ROPE_ITEMS
#define ICSDK_ROPE_ITEMS 8
#endif

template <typename S, int kChunks, int kIt>
__global__ __launch_bounds__(kBlock) void rope_fused_kernel(S *__restrict__ q, S *__restrict__ k,
                                                            uint32_t seq, uint32_t qh,
                                                            uint32_t kh, uint32_t ppb,
                                                            FastDiv per_pos_div, uint64_t offset,
                                                            RopeDenoms denom) {
    constexpr int E = Vec16<S>::N;
    constexpr uint32_t half = kChunks * E;
    extern __shared__ float2 rot[];  // ppb * half rotations
    const uint32_t per_pos = per_pos_div.divisor;   // (qh + kh) * kChunks
    const uint32_t p0 = blockIdx.x * ppb;
    const uint32_t npos = min(ppb, seq - p0);
    const uint32_t items = npos * per_pos;
    const uint32_t rot_entries = npos * half;
    const uint32_t it0 = blockIdx.y * (uint32_t)(kIt * kPairItems);
    const uint32_t lane = threadIdx.x & (kWave - 1), side = lane >> 5;
    const uint32_t wave = threadIdx.x / kWave;
    Vec16<S> v[kIt];
    uint32_t off[kIt];   // element offset of the lane's vector in its q / k window
    bool in_q[kIt];
    uint32_t slot[kIt];  // index of the item's first rotation in `rot`
    bool ok[kIt];
    // block-uniform windows over this block's positions of q and of k
    S *const q0 = q + (size_t)p0 * qh * (2 * half);
    S *const k0 = k + (size_t)p0 * kh * (2 * half);
#pragma unroll
    for (int u = 0; u < kIt; ++u) {
        const uint32_t raw = it0 + (wave * kIt + u) * 32 + (lane & 31);
        ok[u] = raw < items;
        const uint32_t item = ok[u] ? raw : 0u;
        // multiply-high division: a 32-bit divide by the run-time per_pos was
        // ~40 instructions in front of each of the lane's loads
        const uint32_t pp = fast_div(item, per_pos_div);
        const uint32_t rest = item - pp * per_pos;
        const uint32_t row = rest / kChunks;
        const uint32_t c = rest - row * kChunks;
        in_q[u] = row < qh;
        off[u] = (in_q[u] ? pp * qh + row : pp * kh + (row - qh)) * (2 * half) + c * E +
                 side * half;
        slot[u] = pp * half + c * E;
        v[u] = load16_stream((in_q[u] ? q0 : k0) + off[u]);
    }
    // The denominators go to LDS through scalar loads (uniform addresses,
    // counted by lgkmcnt), so computing the rotations never waits for the
    // data loads above, which are counted by vmcnt.
    __shared__ double den[half];
    if (threadIdx.x == 0) {
#pragma unroll
        for (uint32_t d = 0; d < half; ++d) den[d] = denom.d[d];
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < rot_entries; e += kBlock) {
        const uint32_t pp = e / half;
        const float angle = (float)((double)(offset + p0 + pp) / den[e & (half - 1)]);
        float c, sn;
        sincosf(angle, &sn, &c);
        rot[e] = make_float2(c, sn);
    }
    __syncthreads();
    // results go back through L2 (write-through stores) into the same bytes
    const OutWindow q_out(q0, npos * qh * (2 * half) * (uint32_t)sizeof(S));
    const OutWindow k_out(k0, npos * kh * (2 * half) * (uint32_t)sizeof(S));
    float2 t[E];   // the rotations of the lane's current slot
#pragma unroll
    for (int u = 0; u < kIt; ++u) {
        // wave-uniform: read the rotations unless every lane keeps its slot
        if (u == 0 || __builtin_amdgcn_ballot_w64(slot[u] != slot[u - 1]) != 0) {
#pragma unroll
            for (int e = 0; e < E; ++e) t[e] = rot[slot[u] + e];
        }
        // every lane takes part in the swap (a lane past the end holds item 0)
        const uint4 words = __builtin_bit_cast(uint4, v[u]);
        const uint32_t w[4] = {words.x, words.y, words.z, words.w};
        uint32_t lw[4], rw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const auto r = __builtin_amdgcn_permlane32_swap(w[j], w[j], false, false);
            lw[j] = r[0];
            rw[j] = r[1];
        }
        if (!ok[u]) continue;
        const Vec16<S> lv = __builtin_bit_cast(Vec16<S>, uint4{lw[0], lw[1], lw[2], lw[3]});
        const Vec16<S> rv = __builtin_bit_cast(Vec16<S>, uint4{rw[0], rw[1], rw[2], rw[3]});
        Vec16<S> out;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float l = Elem<S>::load(lv.v[e]), r = Elem<S>::load(rv.v[e]);
            const float a = side ? r : l, b = side ? l : r, sb = side ? t[e].y : -t[e].y;
            out.v[e] = Elem<S>::store(a * t[e].x + b * sb);
        }
        // The window is chosen per wave (a descriptor must be wave-uniform):
        // a wave whose items all lie in q, or all in k, writes through its
        // window; a wave that straddles the two uses ordinary stores.
        const uint32_t bytes = off[u] * (uint32_t)sizeof(S);
        const uint64_t active = __builtin_amdgcn_ballot_w64(true);
        const uint64_t q_lanes = __builtin_amdgcn_ballot_w64(in_q[u]);
        if (q_lanes == active) {
            q_out.store16(bytes, out);
        } else if (q_lanes == 0) {
            k_out.store16(bytes, out);
        } else {
            store16_stream((in_q[u] ? q0 : k0) + off[u], out);
        }
    }
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Vectors per half row on the fused path, or 0 when the shape takes the
// table path.
template <typename S>
uint32_t fused_chunks(size_t seq, size_t qh, size_t kh, size_t dim, const void *q,
                      const void *k) {
    constexpr size_t E = Vec16<S>::N;
    const size_t half = dim / 2;
    if (half % E != 0 || half > (size_t)kMaxHalf || !aligned16(q) || !aligned16(k)) return 0;
    const size_t chunks = half / E;
    if (chunks != 1 && chunks != 2 && chunks != 4 && chunks != 8 && chunks != 16 && chunks != 32)
        return 0;
    // grid.x * kBlock work-items must stay below 2^32; grid.y <= 16384
    if (seq > (size_t{1} << 24) || (qh + kh) * chunks > 0xffffffu) return 0;
    return (uint32_t)chunks;
}

template <typename S>
hipError_t launch_rope(S *q, S *k, size_t seq, size_t qh, size_t kh, size_t dim, double theta,
                       size_t offset, void *table_scratch, hipStream_t s) {
    if (seq == 0) return hipSuccess;
    const size_t half = dim / 2;
    if (dim == 0 || dim % 2 || seq * half > 0xffffffffu || qh + kh > 0xffffffu)
        return hipErrorInvalidValue;
    const size_t heads = qh + kh;
    if (const uint32_t chunks = fused_chunks<S>(seq, qh, kh, dim, q, k)) {
        RopeDenoms denom{};
        for (size_t d = 0; d < half; ++d)
            denom.d[d] = std::pow(theta, (2.0 * (double)d) / (double)dim);
        // whole positions per block: up to kTargetIt items per lane pair
        // (the loads of 8 items in flight per lane measured fastest at the
        // BASELINE shape: 4 positions of 64 rows x 4 chunks, 14.4 -> 13.0 us),
        // and at most kLdsPairs rotations
        constexpr size_t kTargetIt = ICSDK_ROPE_ITEMS;
        const size_t per_pos = heads * chunks;
        size_t ppb = per_pos >= kTargetIt * kPairItems ? 1 : kTargetIt * kPairItems / per_pos;
        if (ppb * half > (size_t)kLdsPairs) ppb = (size_t)kLdsPairs / half;
        if (ppb > seq) ppb = seq;
        if (ppb < 1) ppb = 1;
        const uint32_t a = (uint32_t)seq, b = (uint32_t)qh, c = (uint32_t)kh, d = (uint32_t)ppb;
        // items per lane: 1, 2, 4 or 8; positions with more items than 8 per
        // lane are split over blockIdx.y
        const size_t pairs_needed = (ppb * per_pos + kPairItems - 1) / kPairItems;
        const int it = pairs_needed <= 1 ? 1 : pairs_needed <= 2 ? 2 : pairs_needed <= 4 ? 4 : 8;
        const size_t splits = (ppb * per_pos + (size_t)it * kPairItems - 1) / ((size_t)it * kPairItems);
        const FastDiv per_pos_div = make_fast_div((uint32_t)per_pos);
        const dim3 grid((unsigned)((seq + ppb - 1) / ppb), (unsigned)splits), block(kBlock);
        const size_t lds = ppb * half * sizeof(float2);
#define ICSDK_ROPE(CH, IT)                                                                      \
    hipLaunchKernelGGL((rope_fused_kernel<S, CH, IT>), grid, block, lds, s, q, k, a, b, c, d,    \
                       per_pos_div, (uint64_t)offset, denom)
#define ICSDK_ROPE_IT(CH)                                                                       \
    do {                                                                                        \
        if (it == 1) ICSDK_ROPE(CH, 1);                                                         \
        else if (it == 2) ICSDK_ROPE(CH, 2);                                                    \
        else if (it == 4) ICSDK_ROPE(CH, 4);                                                    \
        else ICSDK_ROPE(CH, 8);                                                                 \
    } while (0)
        switch (chunks) {
            case 1: ICSDK_ROPE_IT(1); break;
            case 2: ICSDK_ROPE_IT(2); break;
            case 4: ICSDK_ROPE_IT(4); break;
            case 8: ICSDK_ROPE_IT(8); break;
            case 16: ICSDK_ROPE_IT(16); break;
            default: ICSDK_ROPE_IT(32); break;
        }
#undef ICSDK_ROPE_IT
#undef ICSDK_ROPE
        return hipGetLastError();
    }
    if (table_scratch == nullptr) return hipErrorInvalidValue;
    auto *table = static_cast<float2 *>(table_scratch);
    const size_t entries = seq * half;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((entries + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, s, table, (uint32_t)seq, (uint32_t)half, (uint32_t)dim,
                       theta, (uint64_t)offset);
    const size_t per_pos = heads * half;
    const size_t items = seq * per_pos;
    size_t grid = (items + kBlock - 1) / kBlock;
    if (grid > (size_t{1} << 20)) grid = size_t{1} << 20;
    hipLaunchKernelGGL((rope_scalar_kernel<S>), dim3((unsigned)grid), dim3(kBlock), 0, s, q, k,
                       table, items, per_pos, (uint32_t)half, (uint32_t)qh, (uint32_t)kh,
                       (uint32_t)dim);
    return hipGetLastError();
}

}  // namespace

namespace k {

size_t rope_table_bytes(size_t seq, size_t qh, size_t kh, size_t dim, size_t elem,
                        const void *q, const void *k) {
    const bool fused = elem == 4 ? fused_chunks<float>(seq, qh, kh, dim, q, k) != 0
                                 : fused_chunks<_Float16>(seq, qh, kh, dim, q, k) != 0;
    return fused ? 0 : seq * (dim / 2) * sizeof(float2);
}

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
