// Q8_0 / Q4_0 weights: the quantizer and the quantized linear (GEMV) kernels.
//
// Packed layout (reference src/common/tensor_quant.c:48-100): an [out, in]
// f16 matrix becomes [out, in/32, block] bytes; each 32-weight block is a
// little-endian f16 scale followed by 32 int8 values (Q8_0, 34 bytes) or by
// 16 bytes holding weight j in the low nibble and weight j+16 in the high
// nibble of byte j, stored as value + 8 (Q4_0, 18 bytes).
//
// quant_gemv_kernel (1-4 input rows) and quant_mfma_kernel (5 or more):
// y[r][o] = f16(sum_b scale_b * sum_k x[r][32b+k] * q_bk).
// A wave owns O output rows and walks them in chunks of 64 blocks. Each
// chunk of each row is a contiguous byte range; the wave reads it with
// coalesced 16-byte loads (the aligned 16-byte segments covering the range)
// into its own LDS region, then lane l takes block l of the chunk from LDS:
// blocks start on 2-byte boundaries, so the lane reads the 4-byte words
// covering its block and re-aligns them with v_perm_b32. (Loading each
// lane's block straight from memory -- 34 bytes at a 34-byte lane stride --
// spreads every load instruction over ~17 cache lines and ran at half the
// rate.) The int8 / nibble values are turned into exact f16 pairs
// (0x6400 | byte is 1024 + byte; one packed f16 subtract removes the offset)
// and multiplied with the x pairs by v_dot2_f32_f16, f32 accumulation; x for
// the lane's block is loaded once per chunk and reused for all O rows. The
// wave's partial sums are folded with DPP at the end. Bound: HBM bytes of
// the packed weights (1.0625 or 0.5625 bytes per weight) at small row
// counts.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace k {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

template <bool kQ8> struct Fmt {
    static constexpr uint32_t kBytes = kQ8 ? 34 : 18;
    static constexpr int kWords = kQ8 ? 8 : 4;  // 4-byte words of packed values
};

__device__ inline half2_t as_half2(uint32_t bits) { return __builtin_bit_cast(half2_t, bits); }

// Reads the block at byte offset `off` (even) of an LDS chunk: its scale
// and its packed values re-aligned to 4-byte words. The reads cover the
// block and at most the 2 bytes before it; both tail reads are
// unconditional (an aligned block reads its last half-word twice and uses
// only the low half).
template <bool kQ8>
__device__ inline float read_block(const uint8_t *chunk, uint32_t off,
                                   uint32_t (&q)[Fmt<kQ8>::kWords]) {
    constexpr int W = Fmt<kQ8>::kWords;
    const uint32_t shift = off & 2u;
    const uint8_t *base = chunk + (off - shift);
    const uint32_t *words = reinterpret_cast<const uint32_t *>(base);
    uint32_t e[W + 1];
#pragma unroll
    for (int i = 0; i < W; ++i) e[i] = words[i];
    const uint16_t *tail = reinterpret_cast<const uint16_t *>(base + 4 * W);
    e[W] = (uint32_t)tail[0] | (uint32_t)tail[shift >> 1] << 16;
    const uint32_t sel = shift ? 0x07060504u : 0x05040302u;
#pragma unroll
    for (int i = 0; i < W; ++i) q[i] = __builtin_amdgcn_perm(e[i + 1], e[i], sel);
    const uint32_t scale_bits = shift ? (e[0] >> 16) : (e[0] & 0xffffu);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)scale_bits);
}

// sum_k x_k q_k of one block in f32; x holds the block's 32 f16 as 16 pairs.
template <bool kQ8>
__device__ inline float block_dot(const uint32_t (&q)[Fmt<kQ8>::kWords], const uint32_t (&x)[16]) {
    const half2_t bias8 = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + 128
    const half2_t bias4 = {(_Float16)1032.0f, (_Float16)1032.0f};  // 1024 + 8
    float s0 = 0.0f, s1 = 0.0f;
    if constexpr (kQ8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // int8 -> offset binary, two bytes per f16 pair
            const uint32_t u = q[j] ^ 0x80808080u;
            const half2_t lo = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias8;
            const half2_t hi = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias8;
            s0 = __builtin_amdgcn_fdot2(lo, as_half2(x[2 * j]), s0, false);
            s1 = __builtin_amdgcn_fdot2(hi, as_half2(x[2 * j + 1]), s1, false);
        }
    } else {
        // byte b of the word into the low byte of a half with 0x64 above it:
        // 0x64bb = 1024 + lo + 16 hi. Masking keeps 1024 + lo (0x640n) or
        // 1024 + 16 hi (0x64n0); the packed subtract leaves lo - 8 and
        // 16 (hi - 8), both exact in f16. The high-nibble products go to
        // their own sums, scaled by 1/16 (exact) at the end.
        const half2_t bias16 = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + 16 * 8
        float h0 = 0.0f, h1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, q[j], 0x04010400u);
            const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, q[j], 0x04030402u);
            const half2_t w01 = as_half2(p01 & 0xff0fff0fu) - bias4;
            const half2_t w23 = as_half2(p23 & 0xff0fff0fu) - bias4;
            const half2_t w1617 = as_half2(p01 & 0xfff0fff0u) - bias16;
            const half2_t w1819 = as_half2(p23 & 0xfff0fff0u) - bias16;
            s0 = __builtin_amdgcn_fdot2(w01, as_half2(x[2 * j]), s0, false);
            s1 = __builtin_amdgcn_fdot2(w23, as_half2(x[2 * j + 1]), s1, false);
            h0 = __builtin_amdgcn_fdot2(w1617, as_half2(x[8 + 2 * j]), h0, false);
            h1 = __builtin_amdgcn_fdot2(w1819, as_half2(x[8 + 2 * j + 1]), h1, false);
        }
        return (s0 + s1) + (h0 + h1) * 0.0625f;
    }
    return s0 + s1;
}

// Grid: x = waves of O output rows (4 waves per block), y = groups of R input
// rows. Requires x rows 16-byte aligned, w 4-byte aligned, in % 32 == 0.
template <bool kQ8, int R, int O>
__global__ __launch_bounds__(kBlock) void quant_gemv_kernel(const uint16_t *__restrict__ x,
                                                            const uint8_t *__restrict__ w,
                                                            uint16_t *__restrict__ y,
                                                            uint32_t rows, uint32_t in,
                                                            uint32_t out) {
    constexpr uint32_t kBytes = Fmt<kQ8>::kBytes;
    constexpr uint32_t kChunk = kWave * kBytes;        // bytes of 64 blocks
    constexpr uint32_t kVecs = kChunk / 16 + 2;        // 16-byte segments covering a chunk
    constexpr uint32_t kPasses = (kVecs + kWave - 1) / kWave;
    __shared__ __attribute__((aligned(16))) uint8_t stage[kBlock / kWave][O][kVecs * 16];
    const uint32_t lane = threadIdx.x & (kWave - 1);
    uint8_t (*region)[kVecs * 16] = stage[threadIdx.x / kWave];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(
        (blockIdx.x * kBlock + threadIdx.x) / kWave);
    const uint32_t o0 = wave * O;
    if (o0 >= out) return;
    const uint32_t r0 = blockIdx.y * R;
    const uint32_t blocks = in / 32;
    const uint64_t row_bytes = (uint64_t)blocks * kBytes;
    // rows past the end are clamped onto the last one (computed, not stored)
    const uint8_t *wrow[O];
    const uint16_t *xrow[R];
#pragma unroll
    for (int o = 0; o < O; ++o) wrow[o] = w + (uint64_t)min(o0 + o, out - 1) * row_bytes;
#pragma unroll
    for (int r = 0; r < R; ++r) xrow[r] = x + (uint64_t)min(r0 + r, rows - 1) * in;

    float acc[O][R];
#pragma unroll
    for (int o = 0; o < O; ++o)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[o][r] = 0.0f;

    for (uint32_t c0 = 0; c0 < blocks; c0 += kWave) {
        const uint32_t nb = min((uint32_t)kWave, blocks - c0);
        // the aligned 16-byte segments holding this chunk of each row; a
        // segment never crosses a page, so the bytes around the chunk that
        // share its first and last segment are safe to read
        uint32_t lead[O];
        u32x4 seg[O][kPasses];
#pragma unroll
        for (int o = 0; o < O; ++o) {
            const uint8_t *start = wrow[o] + (uint64_t)c0 * kBytes;
            lead[o] = (uint32_t)(reinterpret_cast<uintptr_t>(start) & 15u);
            const u32x4 *src = reinterpret_cast<const u32x4 *>(start - lead[o]);
            const uint32_t nvec = (lead[o] + nb * kBytes + 15) / 16;
#pragma unroll
            for (int i = 0; i < (int)kPasses; ++i) {
                const uint32_t v = lane + kWave * i;
                seg[o][i] = v < nvec ? __builtin_nontemporal_load(src + v) : u32x4{0, 0, 0, 0};
            }
        }
        const uint32_t b = c0 + min(lane, nb - 1);
        uint32_t xv[R][16];
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
        }
#pragma unroll
        for (int o = 0; o < O; ++o)
#pragma unroll
            for (int i = 0; i < (int)kPasses; ++i) {
                const uint32_t v = lane + kWave * i;
                if (v < kVecs) *reinterpret_cast<u32x4 *>(&region[o][v * 16]) = seg[o][i];
            }
        // the region is this wave's alone: order its LDS writes before the
        // reads of other lanes, and the reads before the next chunk's writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const bool live = lane < nb;
#pragma unroll
        for (int o = 0; o < O; ++o) {
            uint32_t q[Fmt<kQ8>::kWords];
            const float scale = read_block<kQ8>(region[o], lead[o] + (b - c0) * kBytes, q);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float part = scale * block_dot<kQ8>(q, xv[r]);
                acc[o][r] += live ? part : 0.0f;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int o = 0; o < O; ++o)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float total = wave_sum(acc[o][r]);
            if (lane == 0 && o0 + o < out && r0 + r < rows)
                y[(uint64_t)(r0 + r) * out + o0 + o] =
                    __builtin_bit_cast(uint16_t, (_Float16)total);
        }
}

// quant_mfma_kernel (several input rows): a block owns 16 output rows o and
// 16 * NR input rows r; its 4 waves split the weight blocks (k) in four and
// fold their sums through LDS at the end. For each 32-weight block: B = the
// 16 x 32 weight tile, transposed (lane l holds o = l % 16, k = 8 (l / 16)
// .. +7), decoded exactly to f16; A_n = x rows 16 n + l % 16 at the same k;
// one v_mfma_f32_16x16x32_f16 per n gives the block's dot products D[r][o]
// (lane l holds r = 4 (l / 16) + i, o = l % 16), accumulated as acc =
// fma(scale_o, D, acc) in f32 -- all of a lane's values share its o, so one
// scale per lane and block. Each weight is decoded once for all 16 NR rows
// (the GEMV decodes it once per row). W rows are staged through LDS in
// chunks of 16 blocks, coalesced 16-byte loads as in the GEMV.
template <bool kQ8, int NR>
__global__ __launch_bounds__(kBlock) void quant_mfma_kernel(const uint16_t *__restrict__ x,
                                                            const uint8_t *__restrict__ w,
                                                            uint16_t *__restrict__ y,
                                                            uint32_t rows, uint32_t in,
                                                            uint32_t out) {
    constexpr uint32_t kBytes = Fmt<kQ8>::kBytes;
    constexpr uint32_t kWaves = kBlock / kWave;
    constexpr uint32_t kChunkBlocks = 16;
    constexpr uint32_t kVecs = kChunkBlocks * kBytes / 16 + 2;   // segments covering a row's chunk
    constexpr uint32_t kSegs = 16 * kVecs;                       // per wave: 16 rows
    constexpr uint32_t kPasses = (kSegs + kWave - 1) / kWave;
    constexpr uint32_t kStage = 16 * kVecs * 16;                 // bytes per wave
    static_assert((size_t)kWaves * NR * kWave * 16 <= (size_t)kWaves * kStage, "fold fits the stage");
    __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves * kStage];
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wv = threadIdx.x / kWave;
    uint8_t *region = stage + wv * kStage;
    const uint32_t o0 = blockIdx.x * 16;   // < out (the grid covers out exactly)
    const uint32_t r0 = blockIdx.y * 16 * NR;
    const uint32_t blocks = in / 32;
    const uint64_t row_bytes = (uint64_t)blocks * kBytes;
    const uint32_t col = lane % 16, grp = lane / 16;
    // this wave's quarter of the weight blocks
    const uint32_t per = (blocks + kWaves - 1) / kWaves;
    const uint32_t kb0 = min(wv * per, blocks), kb1 = min(kb0 + per, blocks);
    // rows past the end are clamped onto the last one (computed, not stored)
    const uint8_t *my_row = w + (uint64_t)min(o0 + col, out - 1) * row_bytes;
    const uint16_t *xrow[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) xrow[n] = x + (uint64_t)min(r0 + 16 * n + col, rows - 1) * in + 8 * grp;
    f32x4 acc[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const half2_t bias8 = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + 128
    const half2_t bias4 = {(_Float16)1032.0f, (_Float16)1032.0f};  // 1024 + 8
    // Q4: lanes with k >= 16 take the high nibbles of bytes 8 (grp % 2) ..
    const uint32_t nibble_shift = kQ8 ? 0u : (grp >= 2 ? 4u : 0u);
    const uint32_t byte0 = 2 + 8 * (kQ8 ? grp : grp % 2);   // the lane's first value byte in a block

    for (uint32_t c0 = kb0; c0 < kb1; c0 += kChunkBlocks) {
        const uint32_t nb = min(kChunkBlocks, kb1 - c0);
        // stage: wave segment v is segment v % kVecs of row v / kVecs's
        // aligned cover; every lane loads (clamped), so no load sits behind
        // a per-lane branch
        u32x4 seg[kPasses];
#pragma unroll
        for (int i = 0; i < (int)kPasses; ++i) {
            const uint32_t v = lane + kWave * i;
            const uint32_t row = min(v / kVecs, 15u), sidx = v % kVecs;
            const uint8_t *start = w + (uint64_t)min(o0 + row, out - 1) * row_bytes + (uint64_t)c0 * kBytes;
            const uint32_t lead = (uint32_t)(reinterpret_cast<uintptr_t>(start) & 15u);
            const uint32_t last = (lead + nb * kBytes + 15) / 16 - 1;
            seg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(start - lead) + min(sidx, last));
        }
#pragma unroll
        for (int i = 0; i < (int)kPasses; ++i) {
            const uint32_t v = lane + kWave * i;
            if (v < kSegs) *reinterpret_cast<u32x4 *>(region + (v / kVecs) * (kVecs * 16) + (v % kVecs) * 16) = seg[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint32_t my_lead =
            (uint32_t)(reinterpret_cast<uintptr_t>(my_row + (uint64_t)c0 * kBytes) & 15u);
        const uint8_t *mine = region + col * (kVecs * 16);
        auto block = [&](uint32_t b) {
            const uint32_t off = my_lead + b * kBytes;   // even: the block's scale
            const uint32_t sword = *reinterpret_cast<const uint32_t *>(mine + (off & ~3u));
            const float scale = (float)__builtin_bit_cast(
                _Float16, (uint16_t)((off & 2u) ? sword >> 16 : sword & 0xffffu));
            // the lane's 8 value bytes, re-aligned from the 3 words covering them
            const uint32_t p = off + byte0;
            const uint32_t *pw = reinterpret_cast<const uint32_t *>(mine + (p & ~3u));
            const uint32_t e0 = pw[0], e1 = pw[1], e2 = pw[2];
            const uint32_t sel = (p & 2u) ? 0x05040302u : 0x03020100u;
            const uint32_t q[2] = {__builtin_amdgcn_perm(e1, e0, sel), __builtin_amdgcn_perm(e2, e1, sel)};
            half8 bq;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                half2_t lo, hi;
                if constexpr (kQ8) {
                    const uint32_t u = q[j] ^ 0x80808080u;
                    lo = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias8;
                    hi = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias8;
                } else {
                    const uint32_t u = q[j] >> nibble_shift;
                    lo = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u) & 0xff0fff0fu) - bias4;
                    hi = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u) & 0xff0fff0fu) - bias4;
                }
                bq[4 * j] = lo[0];
                bq[4 * j + 1] = lo[1];
                bq[4 * j + 2] = hi[0];
                bq[4 * j + 3] = hi[1];
            }
#pragma unroll
            for (int n = 0; n < NR; ++n) {
                const half8 ax = *reinterpret_cast<const half8 *>(xrow[n] + (uint64_t)(c0 + b) * 32);
                const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bq, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[n][i] = __builtin_fmaf(scale, d[i], acc[n][i]);
            }
        };
        if (nb == kChunkBlocks) {
#pragma unroll
            for (uint32_t b = 0; b < kChunkBlocks; ++b) block(b);
        } else {
            for (uint32_t b = 0; b < nb; ++b) block(b);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    // fold the 4 waves' sums: every wave reaches both barriers
    __syncthreads();
    f32x4 *fold = reinterpret_cast<f32x4 *>(stage);
#pragma unroll
    for (int n = 0; n < NR; ++n) fold[(wv * NR + n) * kWave + lane] = acc[n];
    __syncthreads();
    if (wv != 0) return;
    const uint32_t o = o0 + col;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
        f32x4 t = fold[n * kWave + lane];
#pragma unroll
        for (uint32_t u = 1; u < kWaves; ++u) t += fold[(u * NR + n) * kWave + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = r0 + 16 * n + 4 * grp + i;
            if (r < rows && o < out)
                y[(uint64_t)r * out + o] = __builtin_bit_cast(uint16_t, (_Float16)t[i]);
        }
    }
}

// Any alignment: one thread per output, bytes read one at a time.
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
        float part = 0.0f;
        for (uint32_t k = 0; k < 32; ++k) {
            int v;
            if constexpr (kQ8) {
                v = (int)(int8_t)blk[2 + k];
            } else {
                const uint8_t packed = blk[2 + (k & 15)];
                v = (int)(k < 16 ? packed & 15 : packed >> 4) - 8;
            }
            const float xv = (float)__builtin_bit_cast(_Float16, x[r * in + b * 32 + k]);
            part = __builtin_fmaf(xv, (float)v, part);
        }
        sum = __builtin_fmaf(scale, part, sum);
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

template <bool kQ8, int R, int O>
hipError_t launch_gemv(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                       size_t in, size_t out, hipStream_t s) {
    constexpr uint32_t kWavesPerBlock = kBlock / kWave;
    const size_t waves = (out + O - 1) / O;
    const dim3 grid((unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock),
                    (unsigned)((rows + R - 1) / R));
    quant_gemv_kernel<kQ8, R, O><<<grid, kBlock, 0, s>>>(x, w, y, (uint32_t)rows, (uint32_t)in,
                                                         (uint32_t)out);
    return hipGetLastError();
}

template <bool kQ8, int NR>
hipError_t launch_mfma(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows, size_t in,
                       size_t out, hipStream_t s) {
    if ((out + 15) / 16 > 0x7fffffffu) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((out + 15) / 16), (unsigned)((rows + 16 * NR - 1) / (16 * NR)));
    quant_mfma_kernel<kQ8, NR><<<grid, kBlock, 0, s>>>(x, w, y, (uint32_t)rows, (uint32_t)in,
                                                       (uint32_t)out);
    return hipGetLastError();
}

template <bool kQ8>
hipError_t linear_quant(const uint16_t *x, const uint8_t *w, uint16_t *y, size_t rows,
                        size_t in, size_t out, hipStream_t s) {
    const bool vector_path = reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                             reinterpret_cast<uintptr_t>(w) % 4 == 0 && in <= 0xffffffffu &&
                             out <= 0xffffffffu;
    if (!vector_path) {
        const size_t n = rows * out;
        const size_t blocks = (n + kBlock - 1) / kBlock;
        if (blocks > 0x7fffffffu || in > 0xffffffffu || out > 0xffffffffu) return hipErrorInvalidValue;
        quant_linear_scalar_kernel<kQ8><<<(unsigned)blocks, kBlock, 0, s>>>(x, w, y, rows,
                                                                              (uint32_t)in,
                                                                              (uint32_t)out);
        return hipGetLastError();
    }
    // row groups per launch stay within the grid's y limit
    constexpr size_t kMaxGroups = 65535;
    for (size_t r0 = 0; r0 < rows;) {
        const size_t left = rows - r0;
        const uint16_t *xr = x + r0 * in;
        uint16_t *yr = y + r0 * out;
        hipError_t status;
        size_t done;
        // up to 4 rows the GEMV (one dot per weight and row) is faster; from
        // 5 rows the MFMA kernel, which decodes each weight once for 16 or
        // 32 rows (8 rows of 8192 -> 28672: 98 -> 71 us for Q8, 16 rows 188
        // -> 84 us)
        if (left <= 1) {
            status = launch_gemv<kQ8, 1, kQ8 ? 4 : 2>(xr, w, yr, left, in, out, s);
            done = left;
        } else if (left <= 2) {
            status = launch_gemv<kQ8, 2, 4>(xr, w, yr, left, in, out, s);
            done = left;
        } else if (left <= 4) {
            status = launch_gemv<kQ8, 4, 4>(xr, w, yr, left, in, out, s);
            done = left;
        } else if (left <= 16) {
            status = launch_mfma<kQ8, 1>(xr, w, yr, left, in, out, s);
            done = left;
        } else {
            done = left < kMaxGroups * 32 ? left : kMaxGroups * 32;
            status = launch_mfma<kQ8, 2>(xr, w, yr, done, in, out, s);
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
