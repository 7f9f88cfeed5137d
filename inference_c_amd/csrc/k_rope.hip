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

// ---- group path ------------------------------------------------------------

// Shapes whose q rows and k rows each fill whole groups of 32 (row, chunk)
// items (qh * kChunks and kh * kChunks multiples of 32). A group is then a
// contiguous 1 KB run of one tensor at one position (32 / kChunks rows of
// 2 * half elements), and group n of a tensor is simply its bytes
// n * 1024 .. n * 1024 + 1023. Lane l < 32 of a wave holds the left vector
// of row (l % 32) / kChunks, chunk l % kChunks of a group, lane l + 32 the
// right vector of the same pairs, so a lane's offset inside a group is a
// constant of its lane number.
//
// Blocks alternate between the tensors (even blocks q, odd blocks k, while
// both have blocks left; then the larger one's), so at any time the grid
// streams q and k of neighbouring positions. Wave w of a tensor's blocks
// owns that tensor's groups w * kIt .. w * kIt + kIt - 1: its offsets are
// linear in the group number and need no per-group scalar work; a group
// past the tensor's end gets an offset beyond the tensor's buffer range (its
// loads return zeros, the hardware drops its stores). Each wave computes the
// rotations of the positions its groups touch into its own slice of LDS (no
// block barrier, no serial set-up); each lane turns its chunk's (cos, sin)
// into the coefficients of its side -- left lanes l' = l*c + r*(-s), right
// lanes r' = l*s + r*c, the same two products and one sum as l*c - r*s and
// r*c + l*s -- and per group it does one 16-byte load, four
// v_permlane32_swap and E pairs of products.
//
// Why this layout (measured on MI355X at configs[4]'s shape, q and k
// [4096, 32, 64] f16, back to back over rotated sets): all waves of the
// launch start together, and scalar instructions in front of a wave's first
// load delay it while the CU's one scalar unit serves 16 waves. The fused
// kernel below (generic item math) ran 145 scalar and 907 vector
// instructions per wave, 13.1 us; the same work numbered position-major
// (a position's q groups then its k groups) needed ~130 scalar instructions
// before the first load, 12.5 us; this layout 25, 11.9 us, against 11.5 us
// for an in-place copy of the same bytes.
constexpr uint32_t kGroupBytes = 1024;        // 32 items x 2 vectors x 16 bytes
constexpr uint32_t kDeadOffset = 0xfffff000u;  // beyond any buffer range the host allows

// Arguments: everything a wave needs before its first load comes first, as
// plain scalars, so that it arrives preloaded in SGPRs (an aggregate argument
// ends the preloaded run); q_mul/q_shift and k_mul/k_shift are the
// multiply-high divisions by qg and kg (FastDiv).
template <typename S, int kChunks, int kIt>
__global__ __launch_bounds__(kBlock) void rope_group_kernel(
    S *__restrict__ q, S *__restrict__ k, uint32_t q_bytes, uint32_t k_bytes, uint32_t nbq,
    uint32_t nbk, uint32_t qg, uint32_t q_mul, uint32_t q_shift, uint32_t kg, uint32_t k_mul,
    uint32_t k_shift, uint32_t npos_w, uint64_t offset, RopeDenoms denom) {
    constexpr uint32_t E = Vec16<S>::N;
    constexpr uint32_t half = kChunks * E;
    extern __shared__ float2 rot[];   // per wave: npos_w * half rotations
    const uint32_t lane = threadIdx.x & (kWave - 1), side = lane >> 5, c = lane % kChunks;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    float2 *const mine = rot + wave * npos_w * half;
    const uint32_t lane_off =
        (((lane & 31) / kChunks) * 2 * half + c * E + side * half) * (uint32_t)sizeof(S);
    // this block's tensor and its block index in that tensor
    const uint32_t both = min(nbq, nbk);
    const bool in_q = blockIdx.x < 2 * both ? (blockIdx.x & 1u) == 0 : nbq > nbk;
    const uint32_t bt = blockIdx.x < 2 * both ? blockIdx.x >> 1 : blockIdx.x - both;
    const uint32_t g0 = (bt * (kBlock / kWave) + wave) * kIt;
    // groups per position of this tensor
    const FastDiv div = in_q ? FastDiv{qg, q_mul, q_shift} : FastDiv{kg, k_mul, k_shift};
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        in_q ? q : k, 0, (int)(in_q ? q_bytes : k_bytes), kRawBufferWord3);
    // groups of this wave inside the tensor; the others get an offset
    // beyond every buffer range (<= 2^31 bytes), so the hardware returns
    // zeros for their loads and drops their stores
    const uint32_t bytes = in_q ? q_bytes : k_bytes;
    const uint32_t live = bytes / kGroupBytes > g0 ? bytes / kGroupBytes - g0 : 0u;
    uint32_t off[kIt];
#pragma unroll
    for (int u = 0; u < kIt; ++u) off[u] = (g0 + u) * kGroupBytes + lane_off;
    if (live < (uint32_t)kIt) {   // wave-uniform: only a tensor's last waves
#pragma unroll
        for (int u = 0; u < kIt; ++u)
            if ((uint32_t)u >= live) off[u] = kDeadOffset;
    }
    Vec16<S> v[kIt];
#pragma unroll
    for (int u = 0; u < kIt; ++u)
        v[u] = __builtin_bit_cast(Vec16<S>, __builtin_amdgcn_raw_buffer_load_b128(
                                                rs, (int)off[u], 0, kPolicyStream));
    // the groups' positions, relative to the wave's first (scalar)
    const uint32_t p_first = fast_div(g0, div);
    uint32_t rel[kIt];
    {
        uint32_t j = g0 - p_first * div.divisor, r = 0;
#pragma unroll
        for (int u = 0; u < kIt; ++u) {
            rel[u] = r;
            const bool wrap = ++j == div.divisor;
            j = wrap ? 0u : j;
            r += wrap ? 1u : 0u;
        }
    }
    const uint32_t entries = (rel[kIt - 1] + 1) * half;
    for (uint32_t e = lane; e < entries; e += kWave) {
        const uint32_t d = e % half;
        const float angle = (float)((double)(offset + p_first + e / half) / denom.d[d]);
        float cs, sn;
        sincosf(angle, &sn, &cs);
        mine[e] = make_float2(cs, sn);
    }
    // the slice is this wave's alone: its writes before the other lanes' reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // -0 as an addend the compiler cannot fold: fma(a, b, -0) rounds a * b
    // once, the same value as the product, so the f16 paths below multiply
    // with v_fma_mix_f32 (the f16 operand widened inside the instruction)
    float nz;
    asm("v_mov_b32 %0, 0x80000000" : "=v"(nz));
    float ca[E], cb[E];   // this side's coefficients of the left and right values
#pragma unroll
    for (int u = 0; u < kIt; ++u) {
        if (u == 0 || rel[u] != rel[u - 1]) {   // wave-uniform
            const float2 *t = mine + rel[u] * half + c * E;
#pragma unroll
            for (uint32_t e = 0; e < E; ++e) {
                const float2 cs = t[e];
                ca[e] = side ? cs.y : cs.x;
                cb[e] = side ? cs.x : -cs.y;
            }
        }
        const uint4 words = __builtin_bit_cast(uint4, v[u]);
        const uint32_t w[4] = {words.x, words.y, words.z, words.w};
        uint32_t lw[4], rw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // lanes 0-31 keep their word in the first result and receive lane
            // + 32's in the second; lanes 32-63 the reverse: in every lane the
            // first result is the left vector, the second the right one
            const auto r = __builtin_amdgcn_permlane32_swap(w[i], w[i], false, false);
            lw[i] = r[0];
            rw[i] = r[1];
        }
        const Vec16<S> lv = __builtin_bit_cast(Vec16<S>, uint4{lw[0], lw[1], lw[2], lw[3]});
        const Vec16<S> rv = __builtin_bit_cast(Vec16<S>, uint4{rw[0], rw[1], rw[2], rw[3]});
        Vec16<S> out;
        if constexpr (std::is_same_v<S, _Float16>) {
#pragma unroll
            for (uint32_t e = 0; e < E; ++e)
                out.v[e] = (_Float16)(__builtin_fmaf((float)lv.v[e], ca[e], nz) +
                                      __builtin_fmaf((float)rv.v[e], cb[e], nz));
        } else {
#pragma unroll
            for (uint32_t e = 0; e < E; ++e)
                out.v[e] = Elem<S>::store(Elem<S>::load(lv.v[e]) * ca[e] +
                                          Elem<S>::load(rv.v[e]) * cb[e]);
        }
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, out), rs, (int)off[u], 0,
                                               kPolicyDeviceScope);
    }
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Vectors per half row on the group path, or 0 when the shape does not fit it.
template <typename S>
uint32_t group_chunks(size_t seq, size_t qh, size_t kh, size_t dim, const void *q,
                      const void *k) {
    constexpr size_t E = Vec16<S>::N;
    const size_t half = dim / 2;
    if (half % E != 0 || half > (size_t)kMaxHalf || !aligned16(q) || !aligned16(k)) return 0;
    const size_t chunks = half / E;
    if (chunks != 1 && chunks != 2 && chunks != 4 && chunks != 8 && chunks != 16 && chunks != 32)
        return 0;
    if ((qh * chunks) % 32 != 0 || (kh * chunks) % 32 != 0) return 0;
    // byte offsets in 32 bits, with kDeadOffset beyond every tensor
    const size_t q_bytes = seq * qh * dim * sizeof(S), k_bytes = seq * kh * dim * sizeof(S);
    if (q_bytes > (size_t{1} << 31) || k_bytes > (size_t{1} << 31) || seq > (size_t{1} << 24))
        return 0;
    return (uint32_t)chunks;
}

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
    if (const uint32_t chunks = group_chunks<S>(seq, qh, kh, dim, q, k)) {
        RopeDenoms denom{};
        for (size_t d = 0; d < half; ++d)
            denom.d[d] = std::pow(theta, (2.0 * (double)d) / (double)dim);
        // groups per position of each tensor, and in all
        const uint32_t qg = (uint32_t)(qh * chunks / 32), kg = (uint32_t)(kh * chunks / 32);
        const size_t groups = seq * (size_t)(qg + kg);
        // groups per wave: 8 loads in flight per lane while that leaves at
        // least 1024 blocks (configs[4]: 32768 groups, 1024 blocks of 4 waves)
        const int it = groups >= 32768 ? 8 : groups >= 16384 ? 4 : groups >= 8192 ? 2 : 1;
        const size_t per_block = (size_t)it * (kBlock / kWave);
        const uint32_t nbq = (uint32_t)((seq * qg + per_block - 1) / per_block);
        const uint32_t nbk = (uint32_t)((seq * kg + per_block - 1) / per_block);
        const dim3 grid(nbq + nbk), block(kBlock);
        // positions one wave's groups can touch (its first group anywhere in a position)
        const uint32_t gmin = qg < kg ? qg : kg;
        const uint32_t npos_w = (uint32_t)((it + gmin - 2) / gmin + 1);
        const size_t lds = (size_t)(kBlock / kWave) * npos_w * half * sizeof(float2);
        const uint32_t qb = (uint32_t)(seq * qh * dim * sizeof(S)),
                       kb = (uint32_t)(seq * kh * dim * sizeof(S));
        const FastDiv q_div = make_fast_div(qg), k_div = make_fast_div(kg);
#define ICSDK_ROPE_G(CH, IT)                                                                    \
    hipLaunchKernelGGL((rope_group_kernel<S, CH, IT>), grid, block, lds, s, q, k, qb, kb, nbq,  \
                       nbk, qg, q_div.multiplier, q_div.shift, kg, k_div.multiplier,            \
                       k_div.shift, npos_w, (uint64_t)offset, denom)
#define ICSDK_ROPE_G_IT(CH)                                                                     \
    do {                                                                                        \
        if (it == 1) ICSDK_ROPE_G(CH, 1);                                                       \
        else if (it == 2) ICSDK_ROPE_G(CH, 2);                                                  \
        else if (it == 4) ICSDK_ROPE_G(CH, 4);                                                  \
        else ICSDK_ROPE_G(CH, 8);                                                               \
    } while (0)
        switch (chunks) {
            case 1: ICSDK_ROPE_G_IT(1); break;
            case 2: ICSDK_ROPE_G_IT(2); break;
            case 4: ICSDK_ROPE_G_IT(4); break;
            case 8: ICSDK_ROPE_G_IT(8); break;
            case 16: ICSDK_ROPE_G_IT(16); break;
            default: ICSDK_ROPE_G_IT(32); break;
        }
#undef ICSDK_ROPE_G_IT
#undef ICSDK_ROPE_G
        return hipGetLastError();
    }
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
    const bool fused = elem == 4 ? group_chunks<float>(seq, qh, kh, dim, q, k) != 0 ||
                                       fused_chunks<float>(seq, qh, kh, dim, q, k) != 0
                                 : group_chunks<_Float16>(seq, qh, kh, dim, q, k) != 0 ||
                                       fused_chunks<_Float16>(seq, qh, kh, dim, q, k) != 0;
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
