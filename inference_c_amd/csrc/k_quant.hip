// Q8_0 / Q4_0 weights: the quantizer and the quantized linear (GEMV) kernels.
//
// Packed layout (reference src/common/tensor_quant.c:48-100): an [out, in]
// f16 matrix becomes [out, in/32, block] bytes; each 32-weight block is a
// little-endian f16 scale followed by 32 int8 values (Q8_0, 34 bytes) or by
// 16 bytes holding weight j in the low nibble and weight j+16 in the high
// nibble of byte j, stored as value + 8 (Q4_0, 18 bytes).
//
// quant_gemv_kernel (one or two input rows) and quant_mma_kernel (three or more):
// y[r][o] = f16(sum_b scale_b * sum_k x[r][32b+k] * q_bk).
//
// GEMV: a wave works on O output rows in chunks of 64 blocks -- with one
// input row (and with two for Q4_0) the block's 4 waves share O rows and
// take every 4th chunk (their sums meet in LDS: four short waves per block
// instead of one long one, so a launch has no long last round); with two
// Q8_0 rows each wave owns O rows and walks all their chunks.
// Each chunk of each row is a contiguous byte range; the wave reads it with
// coalesced 16-byte loads (the aligned 16-byte segments covering the range)
// into its own LDS region, then lane l takes block l of the chunk from LDS:
// blocks start on 2-byte boundaries, so the lane reads the 4-byte words
// covering its block. (Loading each lane's block straight from memory -- 34
// bytes at a 34-byte lane stride -- spreads every load instruction over ~17
// cache lines and ran at half the rate.) One v_perm_b32 per value-byte pair
// both re-aligns it and turns it into two exact f16 subnormals, multiplied
// with the x pairs by v_dot2_f32_f16 in f32 (gemv_block below); x for the
// lane's block is loaded once per chunk and reused for all O rows. The
// wave's partial sums (kept as 2^-24 times the dot products, the value
// offset's share starting each block's sum) are folded with DPP at the end.
// Bound: HBM bytes of the packed weights (1.0625 or 0.5625 bytes per weight).
#include "kern_common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace icsdk {
namespace k {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

template <bool kQ8> struct Fmt {
    static constexpr uint32_t kBytes = kQ8 ? 34 : 18;
};

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled.
template <int N, int I = 0, typename F> __device__ inline void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

__device__ inline half2_t as_half2(uint32_t bits) { return __builtin_bit_cast(half2_t, bits); }

// GEMV block arithmetic. Lane l of a chunk owns block l; the block starts at
// an even byte offset `off` of the staged row, so the kWin 4-byte words read
// from off & ~3 hold it (with at most 2 bytes either side): its value byte k
// sits at window byte 2 + k + sh, sh = off & 2, and its scale at bytes sh,
// sh + 1. Value-byte pair j (bytes 2j, 2j + 1) lies in one word -- word
// pair (w_m, w_m+1) holds pair 2m at bytes 2 + sh, 3 + sh and pair 2m + 1 at
// 4 + sh, 5 + sh -- so one v_perm_b32 with a per-lane selector re-aligns it
// and spreads it into the low bytes of two halves at once: 0x00bb00aa, two
// f16 subnormals a * 2^-24, b * 2^-24. Their products with x are exact in
// f32 (v_dot2_f32_f16); the constant part of the value encoding is removed
// once per block through the block's x sum X (shared by the wave's rows):
//   Q8: byte ^ 0x80 = q + 128      sum x q = 2^24 S - 128 X
//   Q4: nibble n = w + 8 (low nibbles masked in place, high nibbles as 16 n)
//                                  sum x w = 2^24 (S + H / 16) - 8 X
template <bool kQ8> struct GemvFmt {
    static constexpr int kWin = kQ8 ? 9 : 5;
};

struct GemvSel {
    uint32_t a, b, s;   // value pairs 2m and 2m + 1 of (w_m, w_m+1); the scale of w_0
    GemvSel() = default;
    __device__ explicit GemvSel(uint32_t sh)
        : a(sh ? 0x0c050c04u : 0x0c030c02u), b(sh ? 0x0c070c06u : 0x0c050c04u),
          s(sh ? 0x0c0c0302u : 0x0c0c0100u) {}
};

// v_dot2_f32_f16 d = a.lo * b.lo + a.hi * b.hi + c with c in its own
// register (the compiler's accumulate-in-place form needs a copy of c per
// chain when c is shared)
__device__ inline float dot2_from(half2_t a, half2_t b, float c) {
    float d;
    asm volatile("v_dot2_f32_f16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// 2^-24 * sum_k x_k w_k of one block (f32) for each of R input rows, and
// the block's scale (f16 bits in the low half); x[r] holds row r's 32 f16
// of the block as 16 pairs, base[r] = -offset * 2^-24 * (their sum), the
// value offset's share. The weights are decoded once for the R rows.
template <bool kQ8, int R>
__device__ inline void gemv_block(const uint8_t *chunk, uint32_t off, const GemvSel &sel,
                                  const uint32_t (&x)[R][16], const float (&base)[R], uint32_t &scale,
                                  float (&dot)[R]) {
    constexpr int W = GemvFmt<kQ8>::kWin;
    const uint32_t *words = reinterpret_cast<const uint32_t *>(chunk + (off & ~3u));
    uint32_t e[W];
#pragma unroll
    for (int i = 0; i < W; ++i) e[i] = words[i];
    scale = __builtin_amdgcn_perm(e[0], e[0], sel.s);
    float s0[R], s1[R];
    if constexpr (kQ8) {
#pragma unroll
        for (int i = 0; i < W; ++i) e[i] ^= 0x80808080u;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const half2_t pa = as_half2(__builtin_amdgcn_perm(e[m + 1], e[m], sel.a));
            const half2_t pb = as_half2(__builtin_amdgcn_perm(e[m + 1], e[m], sel.b));
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (m == 0) {
                    s0[r] = dot2_from(pa, as_half2(x[r][0]), base[r]);
                    s1[r] = dot2_from(pb, as_half2(x[r][1]), 0.0f);
                } else {
                    s0[r] = __builtin_amdgcn_fdot2(pa, as_half2(x[r][2 * m]), s0[r], false);
                    s1[r] = __builtin_amdgcn_fdot2(pb, as_half2(x[r][2 * m + 1]), s1[r], false);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) dot[r] = s0[r] + s1[r];
    } else {
        // s: low nibbles (weight k at k), h: high nibbles (weight k at 16 k)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t pa = __builtin_amdgcn_perm(e[m + 1], e[m], sel.a);
            const uint32_t pb = __builtin_amdgcn_perm(e[m + 1], e[m], sel.b);
            const half2_t la = as_half2(pa & 0x000f000fu), lb = as_half2(pb & 0x000f000fu);
            const half2_t ha = as_half2(pa & 0x00f000f0u), hb = as_half2(pb & 0x00f000f0u);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (m == 0) {
                    s0[r] = dot2_from(la, as_half2(x[r][0]), base[r]);
                    s1[r] = dot2_from(ha, as_half2(x[r][8]), 0.0f);
                } else {
                    s0[r] = __builtin_amdgcn_fdot2(la, as_half2(x[r][2 * m]), s0[r], false);
                    s1[r] = __builtin_amdgcn_fdot2(ha, as_half2(x[r][8 + 2 * m]), s1[r], false);
                }
                s0[r] = __builtin_amdgcn_fdot2(lb, as_half2(x[r][2 * m + 1]), s0[r], false);
                s1[r] = __builtin_amdgcn_fdot2(hb, as_half2(x[r][8 + 2 * m + 1]), s1[r], false);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) dot[r] = __builtin_fmaf(s1[r], 0.0625f, s0[r]);
    }
}

// One output by the reference's own chain (tensor_compute_cuda.cu:216-238):
// sum = fmaf(x_k, scale_b * q_k, sum) over the blocks b of the row, then the
// 32 values k of each, from 0. The fix-up for an output whose fast sum is
// not finite. Finite x and finite scales keep every partial sum of the fast
// kernels finite (at most ~2^30 for f16 operands), and a non-finite x makes
// the reference's sum non-finite too, but the offset decode forms
// x (q + offset) - offset x, so x = +-Inf gives Inf - Inf = NaN where the
// reference's x * (scale q) gives +-Inf (NaN only for q = 0, a zero scale
// or infinities of both signs). Running the reference's chain for those
// outputs makes them equal to the reference's bit for bit. `xrow` is the
// input row (16-byte aligned), `wrow` the packed weight row (2-byte
// aligned). Rare: only rows with an infinity or NaN take it.
template <bool kQ8>
__device__ inline float reference_chain(const uint16_t *xrow, const uint8_t *wrow,
                                        uint32_t blocks) {
    constexpr uint32_t kBytes = Fmt<kQ8>::kBytes;
    float sum = 0.0f;
#pragma unroll 1
    for (uint32_t b = 0; b < blocks; ++b) {
        const uint16_t *blk = reinterpret_cast<const uint16_t *>(wrow + (uint64_t)b * kBytes);
        uint16_t half_words[kBytes / 2];
#pragma unroll
        for (uint32_t i = 0; i < kBytes / 2; ++i) half_words[i] = blk[i];
        const u32x4 *xp = reinterpret_cast<const u32x4 *>(xrow + (uint64_t)b * 32);
        uint32_t xw[16];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const u32x4 t = xp[v];
            xw[4 * v] = t.x;
            xw[4 * v + 1] = t.y;
            xw[4 * v + 2] = t.z;
            xw[4 * v + 3] = t.w;
        }
        const float scale = (float)__builtin_bit_cast(_Float16, half_words[0]);
#pragma unroll
        for (uint32_t k = 0; k < 32; ++k) {
            int q;
            if constexpr (kQ8) {
                const uint32_t byte = k;   // value byte k sits at block byte 2 + k
                q = (int)(int8_t)(uint8_t)(half_words[1 + byte / 2] >> (8 * (byte & 1)));
            } else {
                const uint32_t byte = k & 15;
                const uint8_t packed = (uint8_t)(half_words[1 + byte / 2] >> (8 * (byte & 1)));
                q = (int)(k < 16 ? packed & 15 : packed >> 4) - 8;
            }
            const uint16_t xb = (uint16_t)(xw[k / 2] >> (16 * (k & 1)));
            sum = __builtin_fmaf((float)__builtin_bit_cast(_Float16, xb), scale * (float)q, sum);
        }
    }
    return sum;
}

// Grid: x = waves of O output rows (4 waves per block), y = groups of R
// input rows. Requires x rows 16-byte aligned, w 4-byte aligned, in % 32 == 0.
template <bool kQ8, int R, int O, bool kSplit>
__global__ __launch_bounds__(kBlock) void quant_gemv_kernel(const uint16_t *__restrict__ x,
                                                            const uint8_t *__restrict__ w,
                                                            uint16_t *__restrict__ y,
                                                            uint32_t rows, uint32_t in,
                                                            uint32_t out) {
    constexpr uint32_t kBytes = Fmt<kQ8>::kBytes;
    constexpr uint32_t kChunk = kWave * kBytes;        // bytes of 64 blocks
    constexpr uint32_t kVecs = kChunk / 16 + 2;        // 16-byte segments covering a chunk
    __shared__ __attribute__((aligned(16))) uint8_t stage[kBlock / kWave][O][kVecs * 16];
    const uint32_t lane = threadIdx.x & (kWave - 1);
    uint8_t (*region)[kVecs * 16] = stage[threadIdx.x / kWave];
    // kSplit: the block's 4 waves share its O output rows and take every
    // 4th chunk of 64 blocks (wave k: chunks k, k + 4, ...), their sums
    // meeting in LDS; else each wave owns O rows and walks all their chunks
    constexpr uint32_t kWaves = kBlock / kWave;
    constexpr uint32_t kParts = kSplit ? kWaves : 1;
    const uint32_t wib = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t kpart = kSplit ? wib : 0;
    const uint32_t o0 = (kSplit ? blockIdx.x : blockIdx.x * kWaves + wib) * O;
    if (o0 >= out) return;   // with kSplit the whole block
    const uint32_t r0 = blockIdx.y * R;
    const uint32_t blocks = in / 32;
    const uint64_t row_bytes = (uint64_t)blocks * kBytes;
    // input rows past the end are clamped onto the last one (computed, not stored)
    const uint16_t *xrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) xrow[r] = x + (uint64_t)min(r0 + r, rows - 1) * in;
    // rows past the end are clamped onto the last one (computed, not stored).
    // A chunk of 64 blocks is a whole number of 16-byte segments, so every
    // chunk of a row starts `lead` bytes into its first segment, and lane
    // l's block starts at lead + kBytes * l: its alignment (and selectors)
    // are the same in every chunk.
    auto row_of = [&](uint32_t o) -> uint64_t { return (uint64_t)min(o0 + o, out - 1); };
    auto lead_of = [&](uint64_t row) -> uint32_t {
        return (uint32_t)((reinterpret_cast<uintptr_t>(w) + row * row_bytes) & 15u);
    };
    uint32_t lead[O];
#pragma unroll
    for (int o = 0; o < O; ++o) lead[o] = lead_of(row_of(o));
    const uint8_t *tile = w + row_of(0) * row_bytes;
    // lane l's selectors: its block's alignment is the row's lead parity
    // flipped on odd lanes (kBytes is 2 mod 4), so two sets serve every row.
    // (A lane past a partial chunk's end reads its own block's place in the
    // region with them: stale words, decoded to finite values, discarded.)
    const GemvSel sel_lead0((kBytes * lane) & 2u), sel_lead2((2 + kBytes * lane) & 2u);

    float acc[O][R];
#pragma unroll
    for (int o = 0; o < O; ++o)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[o][r] = 0.0f;

    for (uint32_t c0 = kpart * kWave; c0 < blocks; c0 += kParts * kWave) {
        const uint32_t nb = min((uint32_t)kWave, blocks - c0);
        // the aligned 16-byte segments holding this chunk of each row; a
        // segment never crosses a page, so the bytes around the chunk that
        // share its first and last segment are safe to read. Lanes past the
        // chunk's last segment load nothing (inactive lanes cost the address
        // unit nothing; loading the last segment again in them measured
        // 8% slower for Q8).
        constexpr uint32_t kRowPasses = (kVecs + kWave - 1) / kWave;
        u32x4 segr[O][kRowPasses];
#pragma unroll
        for (int o = 0; o < O; ++o) {
            const uint8_t *src = tile + (row_of(o) - row_of(0)) * row_bytes + (uint64_t)c0 * kBytes - lead[o];
            const uint32_t nvec = (lead[o] + nb * kBytes + 15) / 16;
#pragma unroll
            for (int i = 0; i < (int)kRowPasses; ++i) {
                const uint32_t v = lane + kWave * i;
                segr[o][i] = v < nvec ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src) + v)
                                      : u32x4{0, 0, 0, 0};
            }
        }
        const uint32_t b = c0 + min(lane, nb - 1);
        uint32_t xv[R][16];
        float base[R];   // -offset * 2^-24 * (the x sum of the lane's block)
        const half2_t one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32x4 *xp = reinterpret_cast<const u32x4 *>(xrow[r] + (uint64_t)b * 32);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const u32x4 t = xp[v];
                xv[r][4 * v] = t.x;
                xv[r][4 * v + 1] = t.y;
                xv[r][4 * v + 2] = t.z;
                xv[r][4 * v + 3] = t.w;
            }
            float xs0 = 0.0f, xs1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                xs0 = __builtin_amdgcn_fdot2(as_half2(xv[r][i]), one2, xs0, false);
                xs1 = __builtin_amdgcn_fdot2(as_half2(xv[r][i + 1]), one2, xs1, false);
            }
            // -offset * 2^-24 * sum (exact: a power of two times the sum)
            base[r] = (xs0 + xs1) * (kQ8 ? -0x1p-17f : -0x1p-21f);
        }
#pragma unroll
        for (int o = 0; o < O; ++o)
#pragma unroll
            for (int i = 0; i < (int)kRowPasses; ++i)
                if (lane + kWave * i < kVecs)
                    *reinterpret_cast<u32x4 *>(&region[o][(lane + kWave * i) * 16]) = segr[o][i];
        // the region is this wave's alone: order its LDS writes before the
        // reads of other lanes, and the reads before the next chunk's writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const bool live = lane < nb;
#pragma unroll
        for (int o = 0; o < O; ++o) {
            // lane l's block, also past a partial chunk's end (inside the
            // region: its words are stale, decoded to finite values)
            const uint32_t off = lead[o] + lane * kBytes;
            uint32_t scale;
            float dot[R];
            gemv_block<kQ8, R>(region[o], off, (lead[o] & 2u) ? sel_lead2 : sel_lead0, xv, base, scale,
                               dot);
            // a lane past the chunk's end adds 0 * (its dot: finite unless
            // the chunk's last block of x holds an infinity or NaN, and then
            // the row's output is redone below)
            const _Float16 sc = __builtin_bit_cast(_Float16, (uint16_t)(live ? scale : 0u));
#pragma unroll
            for (int r = 0; r < R; ++r) acc[o][r] = __builtin_fmaf((float)sc, dot[r], acc[o][r]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    // sums are kept as 2^-24 times the dot products until here (exact). An
    // output whose sum is not finite is redone by the reference's chain.
    if constexpr (kSplit) {
        __shared__ float part[kWaves][O * R];
#pragma unroll
        for (int o = 0; o < O; ++o)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float t = wave_sum(acc[o][r]);
                if (lane == 0) part[kpart][o * R + r] = t;
            }
        __syncthreads();
        if (threadIdx.x < O * R) {
            const uint32_t o = threadIdx.x / R, r = threadIdx.x % R;
            float total = 0.0f;
#pragma unroll
            for (uint32_t k = 0; k < kWaves; ++k) total += part[k][threadIdx.x];
            total *= 0x1p24f;
            if (o0 + o < out && r0 + r < rows) {
                if (!__builtin_isfinite(total))
                    total = reference_chain<kQ8>(x + (uint64_t)(r0 + r) * in,
                                                 w + (uint64_t)(o0 + o) * row_bytes, blocks);
                y[(uint64_t)(r0 + r) * out + o0 + o] = __builtin_bit_cast(uint16_t, (_Float16)total);
            }
        }
    } else {
        uint32_t bad = 0;   // wave-uniform: outputs (bit o * R + r) whose sum is not finite
#pragma unroll
        for (int o = 0; o < O; ++o)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float total = wave_sum(acc[o][r]) * 0x1p24f;
                if (!__builtin_isfinite(total)) bad |= 1u << (o * R + r);
                if (lane == 0 && o0 + o < out && r0 + r < rows)
                    y[(uint64_t)(r0 + r) * out + o0 + o] = __builtin_bit_cast(uint16_t, (_Float16)total);
            }
        // rare; one output at a time so the chain is inlined once
#pragma unroll 1
        while (bad != 0) {
            const uint32_t j = (uint32_t)__builtin_ctz(bad);
            bad &= bad - 1;
            const uint32_t o = j / R, r = j % R;
            if (lane == 0 && o0 + o < out && r0 + r < rows) {
                const float total = reference_chain<kQ8>(x + (uint64_t)(r0 + r) * in,
                                                         w + (uint64_t)(o0 + o) * row_bytes, blocks);
                y[(uint64_t)(r0 + r) * out + o0 + o] = __builtin_bit_cast(uint16_t, (_Float16)total);
            }
        }
    }
}

// quant_mma_kernel (kXRows = 16 input rows per block row, or 4): each 32-weight block of 16
// output rows o is one v_mfma_f32_16x16x32_f16 against the same block of 16
// x rows r: B = the 16 x 32 weight tile, lane l holding o = l % 16 and 8 of
// its k, decoded exactly to f16; A = the x rows at the same k; D[r][o] lands
// in lane l as r = 4 (l / 16) + i, o = l % 16, so one scale per lane and
// block. Each weight is decoded once for all 16 rows.
//
// Decode. A value byte u (Q8: the int8 XOR 0x80, i.e. q + 128; Q4: a nibble
// shifted up by 4, i.e. 16 n) becomes the f16 bit pattern 0x00uu, the
// subnormal u * 2^-24 -- one v_perm_b32 per two weights, no subtraction. The
// products x * u * 2^-24 are exact in f32. The offset (Q8: 128; Q4: 16 * 8)
// is removed by a second MFMA of the same x against a constant B of
// -128 * 2^-24, accumulated onto the first, so
//   D = 2^-24 * sum_k x_k q_k        (Q8)    D = 2^-20 * sum_k x_k (n_k - 8)   (Q4)
// and acc = fma(scale, D, acc) with the f16 scale read straight into
// v_fma_mix_f32. The result is multiplied by 2^24 (2^20) before rounding to
// f16 (exact: a power of two). Per 32-weight block and lane: 8 (Q8) or 7
// (Q4) VALU operations of decode, 4 FMAs, 2 MFMAs.
//
// k order. The MFMA sums over its 32 k in any order, so x and the weights
// only have to agree: Q8 lane group g = lane / 16 takes weights 8g .. 8g+7
// (value bytes 8g .. 8g+7); Q4 lane group g takes weights 4g .. 4g+3 (low
// nibbles of value bytes 4g .. 4g+3) and 16+4g .. 16+4g+3 (their high
// nibbles), so a Q4 lane reads one 4-byte word per block.
//
// Data movement. A block's kWaves = 4 waves own 4 tiles of 16 output rows
// and walk the same weight blocks (k) in chunks of 16, so the x rows of a
// chunk (up to 16 rows x 1 KB) are loaded once per block -- contiguous 16-byte loads
// into a double-buffered LDS chunk -- and every wave reads its MFMA operand
// from there. (Each wave loading x in the MFMA layout itself moved 1 KB per
// 512 weights through the address unit and bound the kernel.) Each wave
// stages its 16 rows' next chunk of weights in registers with coalesced
// 16-byte loads while it computes the current one from its LDS region.
// Measured limits ([28672, 8192] Q8_0, 4 and 16 rows): the loads, staging
// and barriers alone take 44-50 us, the decode and MFMAs alone ~40 us
// (about 2 waves per SIMD: 448 blocks, and a k split per block does not fit
// in LDS); prefetching 2 or 3 chunks ahead, or issuing the offset MFMA
// first, measured no faster. One-wave blocks (kWaves = 1, kXRows = 4: each
// wave stages its own x) serve Q4_0 with up to 4 input rows. kLines (Q8_0
// with rows at one phase to the 128-byte lines) loads each line of the
// weights once, carrying a chunk's first bytes over from the chunk before.
template <bool kQ8, uint32_t kWaves, uint32_t kXRows, uint32_t kChunk, bool kLines>
__global__ __launch_bounds__(kWave * kWaves) void quant_mma_kernel(const uint16_t *__restrict__ x,
                                                                   const uint8_t *__restrict__ w,
                                                                   uint16_t *__restrict__ y,
                                                                   uint32_t rows, uint32_t in,
                                                                   uint32_t out) {
    constexpr uint32_t kBytes = Fmt<kQ8>::kBytes;
    constexpr uint32_t kThreads = kWave * kWaves;
    constexpr uint32_t kTiles = kWaves;                       // output tiles per block
    // kChunk weight blocks per chunk; at 16 a row's chunk is 544 (Q8) or
    // 288 bytes contiguous. 8 blocks ran ~45% slower (shorter runs per row at the
    // memory); 32 do not fit twice per CU in LDS with 4-wave blocks. The
    // one-wave blocks (Q4_0, up to 4 rows) take 32: half the chunk
    // boundaries, whose 128-byte lines are read twice (4 rows: 1.20 -> 1.07
    // x the packed bytes, the same time).
    constexpr uint32_t kChunkBytes = kChunk * kBytes;         // a multiple of 16
    // kLines: most bytes a chunk takes over from the chunk before, and a
    // row's LDS window
    constexpr uint32_t kCarry = kLines ? 96 : 0;
    constexpr uint32_t kSpan = kChunkBytes + kCarry;
    // segments a row's chunk is loaded from (kLines: its window; else the
    // segments covering the chunk, one spare either side)
    constexpr uint32_t kVecs = kLines ? kSpan / 16 : kChunkBytes / 16 + 2;
    constexpr uint32_t kRowStride = (kVecs + 1) * 16;         // one spare segment per row: banks
    constexpr uint32_t kSegs = 16 * kVecs;
    constexpr uint32_t kPasses = (kSegs + kWave - 1) / kWave;
    constexpr uint32_t kStage = 16 * kRowStride;              // weight bytes per wave
    constexpr uint32_t kXSegs = kChunk * 4;                   // 16-byte segments of an x row's chunk
    constexpr uint32_t kXRow = kXSegs * 16 + 16;              // (+ bank pad)
    constexpr uint32_t kXBuf = kXRows * kXRow;
    constexpr uint32_t kXPasses = kXRows * kXSegs / kThreads; // x segments per thread
    static_assert(kChunkBytes % 16 == 0, "chunks start at one offset in their first segment");
    static_assert(!kLines || (kChunkBytes % 128 == 32 && kSegs % kWave == 0 && kWaves > 1),
                  "line windows: chunks 32 bytes past a line multiple, whole passes, shared x");
    static_assert(kXRows * kXSegs % kThreads == 0, "x chunks split evenly over the threads");
    static_assert(kXRows % 4 == 0 && kXRows <= 16, "whole row groups of the MFMA's D");
    __shared__ __attribute__((aligned(16))) uint8_t wstage[kTiles * kStage];
    // x double-buffered when waves share it; a lone wave reuses one buffer
    // (its reads of a chunk come before its stores of the next)
    constexpr uint32_t kXBufs = kWaves > 1 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) uint8_t xstage[kXBufs][kXBuf];
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t tile_i = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t pt = threadIdx.x;
    uint8_t *region = wstage + tile_i * kStage;
    // this wave's tile: rows o0 .. o0+15 (a tile past the end stages the
    // last row and stores nothing; it still loads its share of x)
    const uint32_t o0 = blockIdx.x * (16 * kTiles) + 16 * tile_i;
    const uint32_t t0 = min(o0, out - 1);
    const uint32_t last_row = min(15u, out - 1 - t0);
    const uint32_t r0 = blockIdx.y * kXRows;
    const uint32_t xrows = min(kXRows, rows - r0);
    const uint32_t blocks = in / 32;
    const uint64_t row_bytes = (uint64_t)blocks * kBytes;
    const uint32_t col = lane % 16, grp = lane / 16;
    const uint32_t kb0 = 0, kb1 = blocks;
    const uint32_t steps = (blocks + kChunk - 1) / kChunk;

    // ---- weights: pass i, lane l loads segment v = l + 64 i of the tile's
    // 16 row covers (row v / kVecs, segment v % kVecs); rows past the end
    // are clamped onto the last one. Every chunk starts a whole multiple of
    // 16 bytes into its row, so a row's chunks all start `lead` bytes into
    // their first segment; offsets are from
    // tile + c0 * kBytes - 16 (none negative) and fit 32 bits (the launcher
    // checks 16 rows do).
    const uint8_t *tile = w + (uint64_t)t0 * row_bytes;
    auto lead_of = [&](uint32_t row) -> uint32_t {
        return (uint32_t)((reinterpret_cast<uintptr_t>(tile) + (uint64_t)row * row_bytes) & 15u);
    };
    // the offset of segment v of a chunk of nb blocks, clamped onto the
    // chunk's last segment (kLines: not clamped; the line windows bound it)
    auto seg_off = [&](uint32_t v, uint32_t nb) -> uint32_t {
        const uint32_t row = min(min(v / kVecs, 15u), last_row), sidx = v % kVecs;
        const uint32_t lead = lead_of(row);
        const uint32_t last = kLines ? kVecs - 1 : (lead + nb * kBytes + 15) / 16 - 1;
        return (uint32_t)(row * row_bytes) - lead + 16 + 16 * min(sidx, last);
    };
    uint32_t off_full[kPasses], lds_dst[kPasses];
#pragma unroll
    for (int i = 0; i < (int)kPasses; ++i) {
        const uint32_t v = lane + kWave * i;
        off_full[i] = seg_off(v, kChunk);
        lds_dst[i] = min(v / kVecs, 15u) * kRowStride + (v % kVecs) * 16;
    }
    // kLines (every row at one phase to the 128-byte lines: row_bytes a
    // multiple of 128): each line is loaded by one chunk only. Chunk c loads
    // the segments from where chunk c - 1 stopped to the end of the line
    // holding its own last byte (at most F + kSpan, F = the chunk's start
    // rounded down to 16; the row's last chunk stops at its last segment);
    // the bytes [F, that start) -- at most kCarry, chunk c - 1 loaded them --
    // move within each LDS row from kChunkBytes to 0. With g = F mod 128
    // (one for all rows, repeating every 4 chunks) the window is
    // [min(roundup128(g + lead) - g, kCarry) (0 for the first chunk),
    //  min(roundup128(g + lead + kChunkBytes) - g, kSpan)) bytes past F, the
    // last chunk's end ceil16(lead + nb * kBytes); packed ws | we << 16.
    const uint32_t lead_u = lead_of(0);
    const uint32_t g_base = (uint32_t)((reinterpret_cast<uintptr_t>(tile) - lead_u) & 127u);
    const uint32_t last_c = steps - 1;
    auto window = [&](uint32_t c) -> uint32_t {
        const uint32_t g = (g_base + (c & 3u) * kChunkBytes) & 127u;
        const uint32_t ws = c == 0 ? 0u : min(((g + lead_u + 127u) & ~127u) - g, kCarry);
        const uint32_t we = c == last_c ? (lead_u + (kb1 - kChunk * c) * kBytes + 15u) & ~15u
                                        : min(((g + lead_u + kChunkBytes + 127u) & ~127u) - g, kSpan);
        return ws | max(we, ws) << 16;
    };
    auto in_window = [&](int i, uint32_t win) -> bool {
        const uint32_t ws = win & 0xffffu, we = win >> 16;
        return 16u * ((lane + kWave * (uint32_t)i) % kVecs) - ws < we - ws;
    };
    u32x4 seg[kPasses];
    auto fetch_w = [&](uint32_t c0) {
        const uint32_t nb = min((uint32_t)kChunk, kb1 - c0);
        const uint8_t *base = tile + (uint64_t)c0 * kBytes - 16;
        if constexpr (kLines) {
            const uint32_t win = window(c0 / kChunk);
#pragma unroll
            for (int i = 0; i < (int)kPasses; ++i)
                if (in_window(i, win))
                    seg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + off_full[i]));
            return;
        }
        // Non-temporal loads. Without kLines a row's chunks are not
        // line-aligned, so the line holding a chunk boundary is read by two
        // consecutive chunks and, not kept in L2 in between, comes from HBM
        // twice (Q8_0: 1.13 x the packed bytes at 4 rows). L2-allocating loads
        // read it once, but after other traffic has left the last-level cache
        // dirty (a 600 MB write just before) the launch took 95 us instead of
        // 48: the weights then evict that data.
        if (nb == kChunk) {
#pragma unroll
            for (int i = 0; i < (int)kPasses; ++i)
                seg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + off_full[i]));
        } else {
#pragma unroll
            for (int i = 0; i < (int)kPasses; ++i)
                seg[i] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(base + seg_off(lane + kWave * i, nb)));
        }
    };

    // ---- x: the block's threads stage the chunk of the x rows (thread t,
    // pass i: row (t + 256 i) / kXSegs, segment (t + 256 i) % kXSegs; past a
    // partial chunk's end the last segment again)
    const uint16_t *x_tile = x + (uint64_t)r0 * in;
    u32x4 xseg[kXPasses];
    auto fetch_x = [&](uint32_t c0) {
        const uint32_t nb = min((uint32_t)kChunk, kb1 - c0);
#pragma unroll
        for (int i = 0; i < (int)kXPasses; ++i) {
            const uint32_t flat = pt + kThreads * i, xr = flat / kXSegs;
            const uint32_t sg = min(flat % kXSegs, nb * 4 - 1);
            if (xr < xrows)
                xseg[i] = *reinterpret_cast<const u32x4 *>(x_tile + (uint64_t)xr * in +
                                                           (uint64_t)c0 * 32 + sg * 8);
        }
    };

    // ---- this lane's reads: weights of row `col` -- value bytes of block b
    // start at a0 + kBytes * b; a block's word-aligned cover starts at
    // f_even + kBytes * b for even b, f_odd + kBytes * (b - 1) for odd b
    // (kBytes is 2 mod 4, so the alignment alternates, and the re-aligning
    // selector with it); x of row min(col, xrows - 1)
    const uint32_t my_lead = lead_of(min(col, last_row));
    const uint32_t koff = kQ8 ? 8 * grp : 4 * grp;
    const uint32_t row_base = col * kRowStride;
    const uint32_t a0 = row_base + my_lead + 2 + koff;
    const uint32_t f_even = a0 & ~3u;
    const uint32_t f_odd = (a0 & 2u) ? f_even + 2 + kBytes : f_even - 2 + kBytes;
    const uint32_t sel_even = (a0 & 2u) ? 0x05040302u : 0x03020100u;
    const uint32_t sel_odd = (a0 & 2u) ? 0x03020100u : 0x05040302u;
    const uint32_t scale_base = row_base + my_lead;
    const uint32_t x_base = min(col, xrows - 1) * kXRow + 2 * koff;

    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const half8 offset_b = __builtin_bit_cast(half8, u32x4{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u});
    if (kb0 < kb1) {
        fetch_w(kb0);
        fetch_x(kb0);
    }
    for (uint32_t step = 0; step < steps; ++step) {
        const uint32_t c0 = kb0 + step * kChunk;
        const uint32_t nb = min((uint32_t)kChunk, kb1 - c0);
        uint8_t *xbuf = xstage[step % kXBufs];
        if constexpr (kLines) {
            if (step > 0) {
                // the bytes chunk c - 1 loaded for this chunk: kCarry bytes
                // of each row move from kChunkBytes to 0 (what lies past the
                // carried part is overwritten next)
                constexpr uint32_t kMoves = kCarry / 16;
                u32x4 moved[2];
#pragma unroll
                for (uint32_t m = 0; m < 2; ++m) {
                    const uint32_t u = lane + kWave * m;
                    if (u < 16 * kMoves)
                        moved[m] = *reinterpret_cast<const u32x4 *>(region + (u / kMoves) * kRowStride +
                                                                    kChunkBytes + (u % kMoves) * 16);
                }
#pragma unroll
                for (uint32_t m = 0; m < 2; ++m) {
                    const uint32_t u = lane + kWave * m;
                    if (u < 16 * kMoves)
                        *reinterpret_cast<u32x4 *>(region + (u / kMoves) * kRowStride + (u % kMoves) * 16) =
                            moved[m];
                }
            }
            const uint32_t win = window(step);
#pragma unroll
            for (int i = 0; i < (int)kPasses; ++i)
                if (in_window(i, win)) *reinterpret_cast<u32x4 *>(region + lds_dst[i]) = seg[i];
        } else {
#pragma unroll
            for (int i = 0; i < (int)kPasses; ++i)
                if (lane + kWave * i < kSegs) *reinterpret_cast<u32x4 *>(region + lds_dst[i]) = seg[i];
        }
#pragma unroll
        for (int i = 0; i < (int)kXPasses; ++i) {
            const uint32_t flat = pt + kThreads * i, xr = flat / kXSegs;
            if (xr < xrows) *reinterpret_cast<u32x4 *>(xbuf + xr * kXRow + (flat % kXSegs) * 16) = xseg[i];
        }
        // every wave's x rows and this wave's weights are in LDS; every wave
        // is past the step before the last, which read the other x buffer
        __syncthreads();
        if (c0 + kChunk < kb1) {
            fetch_w(c0 + kChunk);
            fetch_x(c0 + kChunk);
        }
        auto block = [&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const uint32_t cover = (j % 2 == 0 ? f_even : f_odd) + kBytes * (j & ~1);
            const uint32_t sel = j % 2 == 0 ? sel_even : sel_odd;
            const uint32_t *pw = reinterpret_cast<const uint32_t *>(region + cover);
            const uint16_t sbits = *reinterpret_cast<const uint16_t *>(region + scale_base + kBytes * j);
            const uint8_t *xa = xbuf + x_base + 64 * j;
            u32x4 bw, aw;
            if constexpr (kQ8) {
                const uint32_t e0 = pw[0], e1 = pw[1], e2 = pw[2];
                const uint32_t u0 = __builtin_amdgcn_perm(e1, e0, sel) ^ 0x80808080u;
                const uint32_t u1 = __builtin_amdgcn_perm(e2, e1, sel) ^ 0x80808080u;
                bw = u32x4{__builtin_amdgcn_perm(0u, u0, 0x0c010c00u), __builtin_amdgcn_perm(0u, u0, 0x0c030c02u),
                           __builtin_amdgcn_perm(0u, u1, 0x0c010c00u), __builtin_amdgcn_perm(0u, u1, 0x0c030c02u)};
                aw = *reinterpret_cast<const u32x4 *>(xa);
            } else {
                const uint32_t e0 = pw[0], e1 = pw[1];
                const uint32_t q = __builtin_amdgcn_perm(e1, e0, sel);
                const uint32_t hi = q & 0xf0f0f0f0u;
                const uint32_t lo = (q << 4) & 0xf0f0f0f0u;
                bw = u32x4{__builtin_amdgcn_perm(hi, lo, 0x0c010c00u), __builtin_amdgcn_perm(hi, lo, 0x0c030c02u),
                           __builtin_amdgcn_perm(hi, lo, 0x0c050c04u), __builtin_amdgcn_perm(hi, lo, 0x0c070c06u)};
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 lo_x = *reinterpret_cast<const u32x2 *>(xa);
                const u32x2 hi_x = *reinterpret_cast<const u32x2 *>(xa + 32);
                aw = u32x4{lo_x.x, lo_x.y, hi_x.x, hi_x.y};
            }
            const float scale = (float)__builtin_bit_cast(_Float16, sbits);
            const half8 ax = __builtin_bit_cast(half8, aw);
            f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, __builtin_bit_cast(half8, bw),
                                                            f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, offset_b, d, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(scale, d[i], acc[i]);
        };
        if (nb == kChunk) {
            // groups of kGroup blocks: every LDS read of the group first,
            // then the decodes, the MFMAs and the scale FMAs (in block
            // order, as block() does, so the sums are the same), so the
            // group's dependency chains overlap instead of running one block
            // at a time ([28672, 8192], two rounds on one box: Q4_0 3, 4, 8,
            // 16 rows 32.4 / 33.7 / 34.4 / 39.8 us against 33.2 / 34.4 /
            // 37.0 / 42.1 one block at a time, Q8_0 0.3-0.7% faster; groups
            // of 8 slower than either, of 16 past the register file)
            constexpr int kGroup = 4;
            static_for<kChunk / kGroup>([&](auto gc) {
                constexpr int g0 = decltype(gc)::value * kGroup;
                uint32_t e[kGroup][3];
                uint16_t sb[kGroup];
                u32x4 aw[kGroup], bw[kGroup];
                static_for<kGroup>([&](auto ic) {
                    constexpr int i = decltype(ic)::value, j = g0 + i;
                    const uint32_t cover = (j % 2 == 0 ? f_even : f_odd) + kBytes * (j & ~1);
                    const uint32_t *pw = reinterpret_cast<const uint32_t *>(region + cover);
                    sb[i] = *reinterpret_cast<const uint16_t *>(region + scale_base + kBytes * j);
                    const uint8_t *xa = xbuf + x_base + 64 * j;
                    e[i][0] = pw[0];
                    e[i][1] = pw[1];
                    if constexpr (kQ8) {
                        e[i][2] = pw[2];
                        aw[i] = *reinterpret_cast<const u32x4 *>(xa);
                    } else {
                        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                        const u32x2 lo_x = *reinterpret_cast<const u32x2 *>(xa);
                        const u32x2 hi_x = *reinterpret_cast<const u32x2 *>(xa + 32);
                        aw[i] = u32x4{lo_x.x, lo_x.y, hi_x.x, hi_x.y};
                    }
                });
                static_for<kGroup>([&](auto ic) {
                    constexpr int i = decltype(ic)::value, j = g0 + i;
                    const uint32_t sel = j % 2 == 0 ? sel_even : sel_odd;
                    if constexpr (kQ8) {
                        const uint32_t u0 = __builtin_amdgcn_perm(e[i][1], e[i][0], sel) ^ 0x80808080u;
                        const uint32_t u1 = __builtin_amdgcn_perm(e[i][2], e[i][1], sel) ^ 0x80808080u;
                        bw[i] = u32x4{__builtin_amdgcn_perm(0u, u0, 0x0c010c00u), __builtin_amdgcn_perm(0u, u0, 0x0c030c02u),
                                      __builtin_amdgcn_perm(0u, u1, 0x0c010c00u), __builtin_amdgcn_perm(0u, u1, 0x0c030c02u)};
                    } else {
                        const uint32_t q = __builtin_amdgcn_perm(e[i][1], e[i][0], sel);
                        const uint32_t hi = q & 0xf0f0f0f0u;
                        const uint32_t lo = (q << 4) & 0xf0f0f0f0u;
                        bw[i] = u32x4{__builtin_amdgcn_perm(hi, lo, 0x0c010c00u), __builtin_amdgcn_perm(hi, lo, 0x0c030c02u),
                                      __builtin_amdgcn_perm(hi, lo, 0x0c050c04u), __builtin_amdgcn_perm(hi, lo, 0x0c070c06u)};
                    }
                });
                f32x4 d[kGroup];
                static_for<kGroup>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    d[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, aw[i]),
                                                                  __builtin_bit_cast(half8, bw[i]),
                                                                  f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                });
                static_for<kGroup>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    d[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, aw[i]), offset_b,
                                                                  d[i], 0, 0, 0);
                });
                static_for<kGroup>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    const float scale = (float)__builtin_bit_cast(_Float16, sb[i]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(scale, d[i][r], acc[r]);
                });
            });
        } else {
            static_for<kChunk>([&](auto jc) {
                if ((uint32_t)decltype(jc)::value < nb) block(jc);
            });
        }
        // this wave's region is rewritten next: its reads come first
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    if (o0 >= out) return;
    const uint32_t o = o0 + col;
    const float unit = kQ8 ? 16777216.0f : 1048576.0f;   // 2^24, 2^20
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] *= unit;
    // an output whose sum is not finite (its x row holds an infinity or NaN)
    // is redone by the reference's chain, one (row, output) at a time so the
    // chain is inlined once
#pragma unroll 1
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = r0 + 4 * grp + i;
        if (4 * grp + i >= kXRows || r >= rows || o >= out) continue;
        float v = acc[0];
        v = i == 1 ? acc[1] : v;
        v = i == 2 ? acc[2] : v;
        v = i == 3 ? acc[3] : v;
        if (!__builtin_isfinite(v))
            v = reference_chain<kQ8>(x + (uint64_t)r * in, w + (uint64_t)o * row_bytes, blocks);
        y[(uint64_t)r * out + o] = __builtin_bit_cast(uint16_t, (_Float16)v);
    }
}

// Any alignment: one thread per output, bytes read one at a time, the
// reference's chain (tensor_compute_cuda.cu:216-238) operation for operation.
template <bool kQ8>
__global__ __launch_bounds__(kBlock) void quant_linear_scalar_kernel(const uint16_t *__restrict__ x,
                                                                     const uint8_t *__restrict__ w,
                                                                     uint16_t *__restrict__ y,
                                                                     uint64_t rows, uint32_t in,
                                                                     uint32_t out) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= rows * out) return;
    const uint64_t r = i / out, o = i % out;
    const uint32_t blocks = in / 32;
    const uint8_t *base = w + o * blocks * Fmt<kQ8>::kBytes;
    float sum = 0.0f;
    for (uint32_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = base + (uint64_t)b * Fmt<kQ8>::kBytes;
        const float scale = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[0] | (blk[1] << 8)));
        for (uint32_t k = 0; k < 32; ++k) {
            int v;
            if constexpr (kQ8) {
                v = (int)(int8_t)blk[2 + k];
            } else {
                const uint8_t packed = blk[2 + (k & 15)];
                v = (int)(k < 16 ? packed & 15 : packed >> 4) - 8;
            }
            const float xv = (float)__builtin_bit_cast(_Float16, x[r * in + b * 32 + k]);
            sum = __builtin_fmaf(xv, scale * (float)v, sum);
        }
    }
    y[i] = __builtin_bit_cast(uint16_t, (_Float16)sum);
}

// The quantizer's scale rounding (src/common/tensor_quant.c:28-46): round to
// nearest even in the normal range. Below 2^-14 the reference shifts one
// place short of binary16, storing round-half-up(v * 2^25) -- twice the
// subnormal value -- and that is the packed format, so it is kept; magnitudes
// under 2^-25 become signed zero.
__device__ inline uint16_t quant_scale_bits(float value) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int exponent = (int)((bits >> 23) & 255u) - 127 + 15;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        mantissa |= 0x800000u;
        const int shift = 13 - exponent;
        return (uint16_t)(sign | ((mantissa + (1u << (shift - 1))) >> shift));
    }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    mantissa += 0xfffu + ((mantissa >> 13) & 1u);
    if (mantissa & 0x800000u) return (uint16_t)(sign | (uint32_t)(exponent + 1) << 10);
    return (uint16_t)(sign | (uint32_t)exponent << 10 | (mantissa >> 13));
}

// One thread per 32-weight block; the arithmetic is the reference's, with
// every product, sum and quotient rounded on its own (no contraction).
// A non-finite weight sets *bad.
template <bool kQ8>
__global__ __launch_bounds__(kBlock) void quantize_kernel(const uint16_t *__restrict__ weight,
                                                          uint8_t *__restrict__ packed,
                                                          uint32_t *__restrict__ bad,
                                                          uint64_t total_blocks) {
    const uint64_t t = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= total_blocks) return;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(weight + t * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const Vec16<_Float16> h = __builtin_bit_cast(Vec16<_Float16>, src[i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[8 * i + j] = (float)h.v[j];
    }
    float max_abs = 0.0f, max_signed = 0.0f;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        finite = finite && __builtin_isfinite(v[j]);
        if (__builtin_fabsf(v[j]) > max_abs) max_abs = __builtin_fabsf(v[j]);
        if (__builtin_fabsf(v[j]) > __builtin_fabsf(max_signed)) max_signed = v[j];
    }
    if (!finite) __hip_atomic_store(bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float scale = kQ8 ? __fdiv_rn(max_abs, 127.0f) : __fdiv_rn(max_signed, -8.0f);
    const float inverse = scale == 0.0f ? 0.0f : __fdiv_rn(1.0f, scale);
    uint16_t *dst = reinterpret_cast<uint16_t *>(packed + t * Fmt<kQ8>::kBytes);
    dst[0] = quant_scale_bits(scale);
    if constexpr (kQ8) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int lo = (int)__builtin_rintf(__fmul_rn(v[2 * j], inverse));
            int hi = (int)__builtin_rintf(__fmul_rn(v[2 * j + 1], inverse));
            lo = min(max(lo, -127), 127);
            hi = min(max(hi, -127), 127);
            dst[1 + j] = (uint16_t)((uint32_t)(uint8_t)(int8_t)lo | (uint32_t)(uint8_t)(int8_t)hi << 8);
        }
    } else {
        uint32_t bytes[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int lo = (int)__fadd_rn(__fmul_rn(v[j], inverse), 8.5f);
            int hi = (int)__fadd_rn(__fmul_rn(v[j + 16], inverse), 8.5f);
            lo = min(max(lo, 0), 15);
            hi = min(max(hi, 0), 15);
            bytes[j] = (uint32_t)(lo | (hi << 4));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[1 + j] = (uint16_t)(bytes[2 * j] | bytes[2 * j + 1] << 8);
    }
}

template <bool kQ8, int R, int O, bool kSplit>
hipError_t launch_gemv(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                       size_t in, size_t out, hipStream_t s) {
    const size_t rows_per_block = kSplit ? O : O * (kBlock / kWave);
    const dim3 grid((unsigned)((out + rows_per_block - 1) / rows_per_block),
                    (unsigned)((rows + R - 1) / R));
    quant_gemv_kernel<kQ8, R, O, kSplit><<<grid, kBlock, 0, s>>>(x, w, y, (uint32_t)rows,
                                                                 (uint32_t)in, (uint32_t)out);
    return hipGetLastError();
}

template <bool kQ8>
hipError_t launch_mma(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows, size_t in,
                      size_t out, hipStream_t s) {
    if constexpr (!kQ8) {
        if (rows <= 4) {
            // Q4_0, up to 4 rows: one wave per block staging its own x rows,
            // so the tiles spread evenly over the CUs and no wave waits on
            // another ([28672, 8192], two boxes: 3 rows 31.8-33.5 us against
            // 36.2-37.3 for 4-wave blocks, 4 rows 33.3-37.2 against
            // 36.7-37.6). Q8_0 runs slower that way (4 rows 50.5 against
            // 47.2-47.8 us): its per-wave rate, not the spread, bounds it.
            const dim3 grid((unsigned)((out + 15) / 16), 1);
            quant_mma_kernel<kQ8, 1, 4, 32, false><<<grid, kWave, 0, s>>>(x, w, y, (uint32_t)rows,
                                                                  (uint32_t)in, (uint32_t)out);
            return hipGetLastError();
        }
    }
    constexpr size_t kRowsPerBlock = 16 * (kBlock / kWave);
    const dim3 grid((unsigned)((out + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)((rows + 15) / 16));
    // Q8_0 from 7 rows, rows at one phase to the 128-byte lines (in a
    // multiple of 2048): each line of the weights loaded once (16 rows:
    // 1.008 x the packed bytes with x read once per XCD, against 1.134 x at
    // 4 rows without). [28672, 8192] over three boxes: 7, 8 and 16 rows
    // 1-3% faster that way, 3-6 rows 0.4-5% slower (the carry move and the
    // masked extra load pass sit on each step's critical path), so fewer
    // rows keep the per-chunk loads. Q4_0's 4-wave launches ran 12-14%
    // slower that way (8 and 16 rows) and keep them too.
    if constexpr (kQ8) {
        if (rows >= 7 && in / 32 * Fmt<kQ8>::kBytes % 128 == 0) {
            quant_mma_kernel<kQ8, kBlock / kWave, 16, 16, true><<<grid, kBlock, 0, s>>>(
                x, w, y, (uint32_t)rows, (uint32_t)in, (uint32_t)out);
            return hipGetLastError();
        }
    }
    quant_mma_kernel<kQ8, kBlock / kWave, 16, 16, false><<<grid, kBlock, 0, s>>>(
        x, w, y, (uint32_t)rows, (uint32_t)in, (uint32_t)out);
    return hipGetLastError();
}

template <bool kQ8>
hipError_t linear_quant(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                        size_t in, size_t out, hipStream_t s) {
    // The vector kernels launch up to 64 work-items per output row (the
    // one-row GEMV: a 4-wave block per 4 rows); out * 64 must stay below
    // 2^32, the dispatch packet's work-item count. Past that (2^26 output
    // rows) the scalar kernel takes the call.
    const bool vector_path = reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                             reinterpret_cast<uintptr_t>(w) % 4 == 0 && in <= 0xffffffffu &&
                             out <= 0xffffffffu / kWave;
    if (!vector_path) {
        const size_t n = rows * out;
        const size_t blocks = (n + kBlock - 1) / kBlock;
        if (blocks > 0x7fffffffu || in > 0xffffffffu || out > 0xffffffffu) return hipErrorInvalidValue;
        quant_linear_scalar_kernel<kQ8><<<(unsigned)blocks, kBlock, 0, s>>>(x, w, y, rows,
                                                                              (uint32_t)in,
                                                                              (uint32_t)out);
        return hipGetLastError();
    }
    // One or two input rows: the GEMV, 4 output rows per wave, or per block
    // of 4 waves splitting the chunks (one row; two Q4_0 rows) (2, 6 and 8 measured
    // slower for both formats and both forms), decoding each weight once for the
    // rows. From three rows quant_mma_kernel, which decodes each weight once
    // for up to 16 ([28672, 8192] Q8_0: 2 rows 51 us GEMV vs 56 MFMA; 4 rows
    // 64 vs 52; Q4_0 2 rows 39 vs 44, 4 rows 52 vs 40). Its 32-bit offsets
    // bound `in`; past that every row takes the 1-row GEMV. Row groups per
    // launch stay within the grid's y limit.
    constexpr size_t kMaxGroups = 65535;
    const bool mma = rows > 2 && in <= (size_t{1} << 25);
    for (size_t r0 = 0; r0 < rows;) {
        const size_t left = rows - r0;
        hipError_t status;
        size_t done;
        if (mma) {
            done = left < kMaxGroups * 16 ? left : kMaxGroups * 16;
            status = launch_mma<kQ8>(x + r0 * in, w, y + r0 * out, done, in, out, s);
        } else if (left == 2) {
            // Two rows: Q4_0 splits the chunks over the block's 4 waves as
            // one row does (106 VGPRs, 4 waves per SIMD: [28672, 8192]
            // 32.4-32.7 us against 33.2-33.4 unsplit); Q8_0 does not (130
            // VGPRs leave 3 waves per SIMD: 48.5 against 45.5 us)
            done = 2;
            status = kQ8 ? launch_gemv<kQ8, 2, 4, false>(x + r0 * in, w, y + r0 * out, done, in, out, s)
                         : launch_gemv<kQ8, 2, 4, true>(x + r0 * in, w, y + r0 * out, done, in, out, s);
        } else {
            done = left < kMaxGroups ? left : kMaxGroups;
            status = launch_gemv<kQ8, 1, 4, true>(x + r0 * in, w, y + r0 * out, done, in, out, s);
        }
        if (status != hipSuccess) return status;
        r0 += done;
    }
    return hipSuccess;
}

}  // namespace

hipError_t linear_q8_0_f16(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                           size_t in, size_t out, hipStream_t s) {
    return linear_quant<true>(x, w, y, rows, in, out, s);
}

hipError_t linear_q4_0_f16(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                           size_t in, size_t out, hipStream_t s) {
    return linear_quant<false>(x, w, y, rows, in, out, s);
}

hipError_t quantize_f16(bool q8, const uint16_t *weight, uint8_t *packed, uint32_t *bad,
                        size_t total_blocks, hipStream_t s) {
    const size_t blocks = (total_blocks + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffffu) return hipErrorInvalidValue;
    if (q8)
        quantize_kernel<true><<<(unsigned)blocks, kBlock, 0, s>>>(weight, packed, bad, total_blocks);
    else
        quantize_kernel<false><<<(unsigned)blocks, kBlock, 0, s>>>(weight, packed, bad, total_blocks);
    return hipGetLastError();
}

}  // namespace k
}  // namespace icsdk
