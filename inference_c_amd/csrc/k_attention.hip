// Scaled dot-product attention for gfx950, with the accelerator semantics of
// the reference's attention backends (src/platform/cuda/attention_cuda.cu:
// 25-99):
//     s[j]   = (sum over d, in order, of q[d] k[j][d]) * scale (+ mask[i][j]),
//              -inf where causal and j > i + (kv_len - q_len);
//     a row whose maximum score (NaN ignored) is not finite is all zeros;
//     p[j]   = exp(s[j] - max) / sum_j exp(s[j] - max);
//     out[e] = sum_j p[j] v[j][e].
// q [B, Hq, Lq, D], k [B, Hkv, Lkv, D], v [B, Hkv, Lkv, Dv], mask [Lq, Lkv],
// out [B, Hq, Lq, Dv]; query head h reads kv head h / (Hq / Hkv).
//
// Row kernel (any D, Dv up to 512; f32 and f16): one wave per query row,
// keys in chunks of 64 with the running max and sum of an online softmax.
// Within a chunk, lane j owns key j: it forms the score as a sequential f32
// dot product (the same order and roundings as the reference, so scores are
// bit-identical), the wave folds the chunk into the running max and sum, and
// then lane e owns output element e (+64, +128, ...) and accumulates
// p[j] * v[j][e] over the chunk, reading p[j] and q[d] from the owning lane
// with v_readlane. No LDS and no barriers. The weights are normalised once at
// the end (acc / sum) rather than per weight, and the online rescaling
// reorders the roundings of p; outputs therefore agree with the reference to
// a few roundings of sum_j p_j |v_j|.
#include "kern_common.hpp"
#include <algorithm>
#include "kernels.hpp"

namespace icsdk {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kMaxRowRegs = 8;  // D, Dv <= 8 * 64

struct SdpaArgs {
    uint32_t batch, qh, kvh, group;   // group = qh / kvh
    uint32_t ql, kl, dim, vdim;
    uint32_t causal_offset;           // kl > ql ? kl - ql : 0
    float scale;
    int causal;
    // Flash work schedule. Every (batch, head) has `items` work items; item r
    // is key-tile part `part` of `parts` of query block `qblock`, packed as
    // qblock | part << 16 | parts << 24 in item[r] when `table` is set (else
    // item r is query block qblocks - 1 - r, whole). A query block of n key
    // tiles has split_parts(n, split_tiles) parts; a part's block writes its
    // unnormalised output rows to part_o[part][row][D] and {running max, sum,
    // NaN flag, 0} to part_ml[part][row], merged by sdpa_combine_kernel.
    uint32_t items, qblocks;
    uint32_t split_tiles;   // 0: no query block is split
    uint32_t table;
    uint32_t xcd_heads;     // keep the q-heads of one kv head on one XCD
    float *part_o;
    f32x4 *part_ml;
    uint32_t item[128];
};
constexpr uint32_t kMaxFlashItems = 128;
constexpr uint32_t kMaxKeyParts = 8;
constexpr uint32_t kMinPartTiles = 4;   // a part amortises its set-up and the merge

// Key tiles (of tk keys) that the queries of query block j (bm queries) may
// see: all kl keys, or when causal those up to its last query + offset.
__host__ __device__ inline uint32_t flash_tiles(uint32_t ql, uint32_t kl, bool causal,
                                                uint32_t offset, uint32_t bm, uint32_t tk,
                                                uint32_t j) {
    const uint32_t last = j * bm + bm - 1 < ql - 1 ? j * bm + bm - 1 : ql - 1;
    const uint64_t seen = (uint64_t)last + offset + 1;
    const uint64_t key_end = causal && seen < kl ? seen : kl;
    return (uint32_t)((key_end + tk - 1) / tk);
}

// Parts of a query block of `tiles` key tiles: about tiles / split_tiles,
// each of at least kMinPartTiles tiles, at most kMaxKeyParts.
__host__ __device__ inline uint32_t split_parts(uint32_t tiles, uint32_t split_tiles) {
    if (split_tiles == 0) return 1;
    uint32_t n = (tiles + split_tiles - 1) / split_tiles;
    const uint32_t most = tiles / kMinPartTiles;
    n = n < most ? n : most;
    n = n < kMaxKeyParts ? n : kMaxKeyParts;
    return n < 1 ? 1 : n;
}

__device__ inline float broadcast_lane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// exp for the softmax weights: libm-accurate for f32 outputs, the hardware
// exp2 path for f16 outputs (its error is far below half an f16 ulp).
template <typename S>
__device__ inline float attn_exp(float x) {
    if constexpr (sizeof(S) == 2) return fast_exp(x);
    else return expf(x);
}

// Score of the lane's key row: q . k in d order (sequential f32 sums, no
// contraction), q[d] taken from lane d % 64 of register d / 64. kVec: rows
// are whole, aligned 16-byte vectors.
template <typename S, bool kVec>
__device__ inline float row_dot(const float (&qreg)[kMaxRowRegs], const S *krow, uint32_t dim) {
    constexpr uint32_t E = Vec16<S>::N;
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) {
        const uint32_t d0 = (uint32_t)t * kWave;
        if (d0 >= dim) break;
        const uint32_t dn = min(dim - d0, (uint32_t)kWave);
        if constexpr (kVec) {
            for (uint32_t dd = 0; dd < dn; dd += E) {
                const Vec16<S> kv = load16(krow + d0 + dd);
#pragma unroll
                for (uint32_t e = 0; e < E; ++e)
                    sum = sum + broadcast_lane(qreg[t], (int)(dd + e)) * Elem<S>::load(kv.v[e]);
            }
        } else {
            for (uint32_t dd = 0; dd < dn; ++dd)
                sum = sum + broadcast_lane(qreg[t], (int)dd) * Elem<S>::load(krow[d0 + dd]);
        }
    }
    return sum;
}

template <typename S, bool kVec>
__global__ __launch_bounds__(kBlock) void sdpa_row_kernel(const S *__restrict__ q,
                                                          const S *__restrict__ k,
                                                          const S *__restrict__ v,
                                                          const S *__restrict__ mask,
                                                          S *__restrict__ out, SdpaArgs a) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const size_t row = (size_t)blockIdx.x * (kBlock / kWave) +
                       (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const size_t rows = (size_t)a.batch * a.qh * a.ql;
    if (row >= rows) return;
    const uint32_t i = (uint32_t)(row % a.ql);          // query position
    const size_t bh = row / a.ql;                        // batch * qh + head
    const uint32_t head = (uint32_t)(bh % a.qh);
    const size_t b = bh / a.qh;
    const size_t kv = b * a.kvh + head / a.group;
    const S *qrow = q + row * a.dim;
    const S *kbase = k + kv * a.kl * a.dim;
    const S *vbase = v + kv * a.kl * a.vdim;

    // q[d] lives in lane d % 64, register d / 64
    float qreg[kMaxRowRegs];
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) {
        const uint32_t d = lane + t * kWave;
        qreg[t] = d < a.dim ? Elem<S>::load(qrow[d]) : 0.0f;
    }
    float acc[kMaxRowRegs];
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) acc[t] = 0.0f;
    const float neg_inf = -__builtin_inff();
    float m = neg_inf, l = 0.0f;
    bool nan_seen = false;
    // keys past `last` are masked by the causal rule for this row
    const uint64_t last = a.causal ? (uint64_t)i + a.causal_offset : (uint64_t)a.kl - 1;
    for (uint32_t c0 = 0; c0 < a.kl && (uint64_t)c0 <= last; c0 += kWave) {
        const uint32_t j = c0 + lane;
        const bool live = j < a.kl;
        float s = neg_inf;
        if (live) {
            s = row_dot<S, kVec>(qreg, kbase + (size_t)j * a.dim, a.dim) * a.scale;
            if (mask) s = s + Elem<S>::load(mask[(size_t)i * a.kl + j]);
            if (a.causal && (uint64_t)j > last) s = neg_inf;
        }
        // a NaN score never becomes the max, but a row with a finite max and
        // a NaN score is NaN (its sum is)
        nan_seen = nan_seen || wave_any(s != s);
        const float m_new = fmaxf(m, wave_max(s));
        if (m_new == neg_inf) continue;                  // nothing visible yet
        const float alpha = attn_exp<S>(m - m_new);      // 0 when m was -inf
        const float p = live ? attn_exp<S>(s - m_new) : 0.0f;
        l = l * alpha + wave_sum(p);
        m = m_new;
        const uint32_t n = min(a.kl - c0, (uint32_t)kWave);
#pragma unroll
        for (int t = 0; t < kMaxRowRegs; ++t) acc[t] = acc[t] * alpha;
        for (uint32_t jj = 0; jj < n; ++jj) {
            const float pj = broadcast_lane(p, (int)jj);
            const S *vrow = vbase + (size_t)(c0 + jj) * a.vdim;
#pragma unroll
            for (int t = 0; t < kMaxRowRegs; ++t) {
                const uint32_t e = lane + t * kWave;
                if (e < a.vdim) acc[t] = acc[t] + pj * Elem<S>::load(vrow[e]);
            }
        }
    }
    const bool zero = !__builtin_isfinite(m);
    const float inverse = l == 0.0f ? 0.0f : 1.0f / l;
    const float nan = __builtin_nanf("");
    S *orow = out + row * a.vdim;
#pragma unroll
    for (int t = 0; t < kMaxRowRegs; ++t) {
        const uint32_t e = lane + t * kWave;
        if (e < a.vdim)
            orow[e] = Elem<S>::store(zero ? 0.0f : nan_seen ? nan : acc[t] * inverse);
    }
}

// ---- MFMA flash kernel (f16, D = Dv in {64, 128}) ----------------------------

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

// A block owns BM queries of one (batch, head): 32 per wave (KS waves per
// 32 queries when the key tiles are split between them). Keys come in tiles
// of 64, staged in LDS by the whole block, double-buffered: the next step's
// global loads are issued before the current step is computed and land in
// the other buffer afterwards, so one barrier per step separates the
// writers of a buffer from its readers. K and V are both stored as
// [key][dim] rows, as they are in memory (16-byte loads and stores, 256
// contiguous bytes per row at D 128).
//
// v_mfma_f32_32x32x16_f16 lane layout (checked on the device): A[m][k] in
// lane l at m = l % 32, k = 8 (l / 32) + i; B[k][n] at n = l % 32,
// k = 8 (l / 32) + i; D[m][n] at n = l % 32, m = 8 (r / 4) + 4 (l / 32) + r % 4.
//
// Scores: S^T = K Q^T per 32-key half tile (A = K rows from LDS, B = the
// wave's Q rows, loaded once), so lane l holds query l % 32 and, of each
// half tile, keys 8 (r / 4) + 4 (l / 32) + r % 4; lane l ^ 32 holds the rest.
// The online softmax runs per lane pair (one swizzle for the max, one for
// the sum). P^T is then already the B operand of out^T = V^T P^T: chunk c of
// its k dimension is p[8c .. 8c + 7], keys 16c + 8 (i / 4) + 4 (l / 32) + i % 4.
// The matching A fragment (V^T: lane l needs V[16c + 4h + k][d] and
// V[16c + 8 + 4h + k][d], k = 0..3, d = l % 32, h = l / 32) comes from the
// [key][dim] V rows through two ds_read_b64_tr_b16: within each 16-lane
// group that instruction hands lane j element j % 4 of the 4-element vectors
// addressed by lanes j / 4 + 4k, k = 0..3 (checked on the device), so lane
// i of group g addresses row 16c + 4 (g / 2) + i / 4 (+ 8), columns
// 16 (g % 2) + 4 (i % 4) .. + 3.
constexpr int kFlashN = 64;    // keys per tile
constexpr float kLazyLog2 = 8.0f;   // rescale when a row maximum grows by more than 2^8
// s_waitcnt vmcnt(0) (GFX9 encoding: expcnt and lgkmcnt at their no-wait maxima)
constexpr int kWaitVmcnt0 = 0x0F70;

// Block -> work item. Blocks are numbered item-rank-major (all (batch, head)
// pairs of the largest item first), so the blocks dispatched first are the
// longest and the short ones fill in behind them. MI355X dispatches a
// launch's workgroups to its 8 XCDs round-robin (block b on XCD b % 8) and
// each XCD has its own 4 MB L2: with xcd_heads (batch * kv heads divisible
// by 8, so b % 8 == p % 8), XCD x takes the q-heads of kv units x, x + 8, ...
// and a kv head's K/V tiles are fetched into one L2 instead of all eight.
struct FlashItem {
    uint32_t bh, qblock, part, parts;
};
__device__ inline FlashItem flash_item(const SdpaArgs &a, uint32_t block) {
    const uint32_t bhs = a.batch * a.qh;
    const uint32_t r = block / bhs, p = block % bhs;
    FlashItem it;
    if (a.xcd_heads) {
        const uint32_t x = p % 8, i = p / 8;
        it.bh = (x + 8 * (i / a.group)) * a.group + i % a.group;
    } else {
        it.bh = p;
    }
    if (a.table) {
        const uint32_t e = a.item[r];
        it.qblock = e & 0xffffu;
        it.part = (e >> 16) & 0xffu;
        it.parts = e >> 24;
    } else {
        it.qblock = a.qblocks - 1 - r;
        it.part = 0;
        it.parts = 1;
    }
    return it;
}

// Max and sum of a value over the lane pair (l, l ^ 32). v_permlane32_swap
// with both operands v leaves every lane holding its own value in one result
// and its partner's in the other (lanes 0-31 keep r0 and receive lane + 32 in
// r1; lanes 32-63 receive lane - 32 in r0 and keep r1), so one cross-lane
// VALU op replaces a round trip through LDS (ds_bpermute).
// The two halves of the wave swap values with v_permlane32_swap: each lane
// gets back its own value and the one of lane +-32. The vector's elements
// are copied into scalars before the bit cast (a bit cast of an element of
// the returned vector reads element 0).
__device__ inline float pair_value(float v, float &partner) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const unsigned lo = r[0], hi = r[1];
    partner = __builtin_bit_cast(float, hi);
    return __builtin_bit_cast(float, lo);
}
__device__ inline float pair_max(float v) {
    float b;
    const float a = pair_value(v, b);
    return fmaxf(a, b);
}
__device__ inline float pair_sum(float v) {
    float b;
    const float a = pair_value(v, b);
    return a + b;
}

// Scheduling of an unrolled chain of N (LDS read, MFMA) pairs: the first
// kAhead reads, then one MFMA and one read alternately, then the last MFMAs.
// Each MFMA then consumes a fragment read kAhead MFMAs earlier (~128
// cycles), which covers the LDS latency; left to itself the scheduler reads
// one fragment ahead and every MFMA waits for its read.
// (R LDS reads per MFMA.)
template <int N, int R = 1>
__device__ inline void lds_read_ahead() {
    constexpr int kAhead = 4;
    constexpr int kMfma = 0x008, kDsRead = 0x100;
    __builtin_amdgcn_sched_group_barrier(kDsRead, kAhead * R, 0);
#pragma unroll
    for (int i = 0; i < N - kAhead; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kDsRead, R, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kMfma, kAhead, 0);
}

// A wave issuing a chain of MFMAs runs at raised priority, so that the
// other waves of its SIMD (in their softmax) take the issue cycles between
// its MFMAs instead of both waves reaching the same phase together.
__device__ inline void mfma_phase_begin() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_sched_barrier(0);
}
__device__ inline void mfma_phase_end() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
}

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));

// Four halves through the LDS transpose read (lane layout above).
__device__ inline half4 lds_read_tr(const _Float16 *p) {
    const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v *)(p));
    return __builtin_bit_cast(half4, r);
}

// A split block's result for one query: its lane pair holds the query's
// unnormalised output rows (out^T accumulator layout), the running max and
// sum, and the NaN flag.
template <int D, int VT>
__device__ inline void write_partial(const SdpaArgs &a, uint32_t split, size_t row, uint32_t half,
                                     const float16v (&o)[VT], float m, float l, bool nan_seen) {
    const size_t rows = (size_t)a.batch * a.qh * a.ql;
    float *prow = a.part_o + ((size_t)split * rows + row) * D;
#pragma unroll
    for (int tt = 0; tt < VT; ++tt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 quad = {o[tt][4 * g], o[tt][4 * g + 1], o[tt][4 * g + 2], o[tt][4 * g + 3]};
            *reinterpret_cast<f32x4 *>(prow + 32 * tt + 8 * g + 4 * half) = quad;
        }
    if (half == 0) a.part_ml[(size_t)split * rows + row] = f32x4{m, l, nan_seen ? 1.0f : 0.0f, 0.0f};
}

// Merges the parts of each split query row (rows first_row .. ql - 1 of
// every (batch, head): split query blocks are a suffix, since a later query
// block never sees fewer keys): M = max of the parts' maxima; a row whose M
// is not finite is zero; a NaN flag with a finite M makes the row NaN;
// otherwise out = (sum_s w_s o_s) * (1 / sum_s w_s l_s) with w_s =
// exp(m_s - M) (exp2 when the maxima are in log2 units). One thread per 8
// output elements (dim % 8 == 0 on the flash path).
//
// kParts >= the launch's largest part count: every part's (m, l) and output
// vectors are requested up front, unconditionally (a part index past the
// row's own count reads its last part again, which stays in bounds, and is
// left out of the sums), so a row costs one memory round trip; walking the
// parts in a run-time loop waited for each part's loads in turn.
template <typename S, bool kLog2, int kParts>
__global__ __launch_bounds__(kBlock) void sdpa_combine_kernel(SdpaArgs a, S *__restrict__ out,
                                                              uint32_t bm, uint32_t tk,
                                                              uint32_t first_row) {
    const size_t rows = (size_t)a.batch * a.qh * a.ql;
    const uint32_t suffix = a.ql - first_row;
    const uint32_t groups = a.dim / 8;
    const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= (size_t)a.batch * a.qh * suffix * groups) return;
    const size_t srow = i / groups;
    const uint32_t g = (uint32_t)(i % groups);
    const uint32_t qi = first_row + (uint32_t)(srow % suffix);
    const size_t row = srow / suffix * a.ql + qi;
    const uint32_t splits = split_parts(
        flash_tiles(a.ql, a.kl, a.causal != 0, a.causal_offset, bm, tk, qi / bm), a.split_tiles);
    f32x4 ml[kParts], po_lo[kParts], po_hi[kParts];
#pragma unroll
    for (int s = 0; s < kParts; ++s) {
        const size_t part = (size_t)min((uint32_t)s, splits - 1) * rows + row;
        ml[s] = a.part_ml[part];
        const f32x4 *po = reinterpret_cast<const f32x4 *>(a.part_o + part * a.dim + 8 * g);
        po_lo[s] = po[0];
        po_hi[s] = po[1];
    }
    float big = -__builtin_inff();
    bool nan_flag = false;
#pragma unroll
    for (int s = 0; s < kParts; ++s) {
        if ((uint32_t)s < splits) {
            big = fmaxf(big, ml[s].x);
            nan_flag = nan_flag || ml[s].z != 0.0f;
        }
    }
    f32x4 lo = {0.0f, 0.0f, 0.0f, 0.0f}, hi = lo;
    float total = 0.0f;
    if (__builtin_isfinite(big)) {
#pragma unroll
        for (int s = 0; s < kParts; ++s) {
            if ((uint32_t)s >= splits) continue;
            // a part that saw no visible key has sum 0 and output 0; every
            // other part is added even at weight 0, so a NaN it holds stays
            const float w = ml[s].x == -__builtin_inff() ? 0.0f
                            : kLog2 ? __builtin_amdgcn_exp2f(ml[s].x - big) : expf(ml[s].x - big);
            total += w * ml[s].y;
            lo += w * po_lo[s];
            hi += w * po_hi[s];
        }
    }
    const bool zero = !__builtin_isfinite(big);
    const float inverse = total == 0.0f ? 0.0f : 1.0f / total;
    const float nan = __builtin_nanf("");
    S res[8] __attribute__((aligned(16)));
#pragma unroll
    for (int j = 0; j < 8; ++j)
        res[j] = (S)(zero ? 0.0f : nan_flag ? nan : (j < 4 ? lo[j] : hi[j - 4]) * inverse);
    S *orow = out + row * a.dim + 8 * g;
    if constexpr (sizeof(S) == 2) {
        *reinterpret_cast<u32x4 *>(orow) = *reinterpret_cast<const u32x4 *>(res);
    } else {
        reinterpret_cast<u32x4 *>(orow)[0] = reinterpret_cast<const u32x4 *>(res)[0];
        reinterpret_cast<u32x4 *>(orow)[1] = reinterpret_cast<const u32x4 *>(res)[1];
    }
}

template <int D, int BM, bool kMask, bool kSplit, int KS>
__global__ __launch_bounds__(BM * 2 * KS) void sdpa_flash_kernel(const _Float16 *__restrict__ q,
                                                            const _Float16 *__restrict__ k,
                                                            const _Float16 *__restrict__ v,
                                                            const _Float16 *__restrict__ mask,
                                                            _Float16 *__restrict__ out,
                                                            SdpaArgs a) {
    constexpr int QW = BM / 32;              // query groups of 32: one wave each per key part
    constexpr int THREADS = BM * 2 * KS;
    constexpr int KC = D / 16;               // 16-dim chunks of Q K^T
    constexpr int VT = D / 32;               // 32-row tiles of out^T
    constexpr int KROW = D + 8;              // LDS row of K (halves)
    // LDS row of V (halves): 16 (D 128) or 48 (D 64) dwords past a multiple
    // of 64, so the 4 rows a transpose read takes per half wave start 16
    // banks apart (conflict-free)
    constexpr int VROW = D + 32;
    constexpr int KTILE = kFlashN * KROW;    // LDS halves of one K tile
    constexpr int VTILE = kFlashN * VROW;    // LDS halves of one V tile
    constexpr int TV = kFlashN * D / 8;      // 16-byte vectors per K or V tile
    constexpr int VECS = KS * TV;            // per operand and step (KS tiles)
    constexpr int PER = VECS / THREADS;      // per thread, per step, per operand
    static_assert(VECS % THREADS == 0, "tile load split");
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][KS * KTILE];
    __shared__ __attribute__((aligned(16))) _Float16 vs[2][KS * VTILE];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(tid / kWave);
    // wave w takes query group w % QW and key tile kpart of every step
    const uint32_t qgroup = wave % QW, kpart = wave / QW;
    const uint32_t col = lane & 31, half = lane >> 5;
    // the lane's transpose-read address in a V tile (chunk 0, d tile 0)
    const uint32_t v_lane =
        (4 * (lane / 32) + (lane % 16) / 4) * VROW + 16 * ((lane / 16) % 2) + 4 * (lane % 4);
    const FlashItem item = flash_item(a, blockIdx.x);
    const uint32_t qblock = item.qblock, bh = item.bh;
    const uint32_t head = bh % a.qh, b = bh / a.qh;
    const size_t kv_base = ((size_t)b * a.kvh + head / a.group) * a.kl;
    const uint32_t qw = qblock * BM + qgroup * 32;      // the wave's first query
    const uint32_t qi = qw + col;                       // the lane's query
    const bool q_live = qi < a.ql;
    const float neg_inf = -__builtin_inff();

    half8 qf[KC];
    {
        const _Float16 *qrow = q + ((size_t)bh * a.ql + (q_live ? qi : 0)) * D + 8 * half;
#pragma unroll
        for (int c = 0; c < KC; ++c) qf[c] = *reinterpret_cast<const half8 *>(qrow + 16 * c);
    }
    // wait for Q here: otherwise the wait analysis of the tile loop cannot
    // tell these loads from the next tile's prefetch and makes every S^T MFMA
    // wait for one more of the prefetch loads
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __builtin_amdgcn_sched_barrier(0);
    float16v o[VT];
#pragma unroll
    for (int t = 0; t < VT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
    float m = neg_inf, l = 0.0f;   // running max (log2 units) and sum
    bool nan_seen = false;
    constexpr float kLog2e = 1.4426950408889634f;
    const float scale2 = a.scale * kLog2e;

    // key tiles any query of the block can see; this block's part of them
    const uint32_t all_tiles = flash_tiles(a.ql, a.kl, a.causal != 0, a.causal_offset, BM,
                                           kFlashN, qblock);
    const uint32_t share = (all_tiles + item.parts - 1) / item.parts;
    const uint32_t t_begin = min(item.part * share, all_tiles);
    const uint32_t tiles = min(t_begin + share, all_tiles);
    const bool wave_live = qw < a.ql;
    const uint64_t wave_last_key = (uint64_t)min(qw + 31, a.ql - 1) + a.causal_offset;
    const uint64_t lane_last_key = (uint64_t)qi + a.causal_offset;

    // tile loads of a step (KS tiles from key k0): thread `tid` moves vectors
    // tid, tid + THREADS, ... of K and of V (per tile row-major: key, 8-dim
    // group). The loads take no branch:
    // rows past the end are clamped onto the last key and zeroed when
    // stashed. (A fetch with a bounds-tested branch per load let the
    // compiler merge the whole-tile loads into that path, behind a wait for
    // every load just issued: the prefetch no longer overlapped the tile's
    // MFMAs, 15-20% slower.)
    half8 kreg[PER], vreg[PER];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const uint32_t e = tid + u * THREADS, tk = k0 + e / TV * kFlashN, r = e % TV;
            const size_t row = (kv_base + min(tk + r / (D / 8), a.kl - 1)) * D + r % (D / 8) * 8;
            kreg[u] = *reinterpret_cast<const half8 *>(k + row);
            vreg[u] = *reinterpret_cast<const half8 *>(v + row);
        }
    };
    auto stash = [&](int buf, uint32_t k0) {
        if (k0 + KS * kFlashN > a.kl) {   // a ragged last step: zero the rows past the end
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const uint32_t e = tid + u * THREADS, tk = k0 + e / TV * kFlashN, r = e % TV;
                if (tk + r / (D / 8) >= a.kl) {
                    kreg[u] = half8{};
                    vreg[u] = half8{};
                }
            }
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const uint32_t e = tid + u * THREADS, tile = e / TV, r = e % TV;
            *reinterpret_cast<half8 *>(&ks[buf][tile * KTILE + (r / (D / 8)) * KROW + (r % (D / 8)) * 8]) =
                kreg[u];
            *reinterpret_cast<half8 *>(&vs[buf][tile * VTILE + (r / (D / 8)) * VROW + (r % (D / 8)) * 8]) =
                vreg[u];
        }
    };

    if (t_begin < tiles) {
        fetch(t_begin * kFlashN);
        stash(0, t_begin * kFlashN);
    }
    __syncthreads();
    // step: KS tiles from t0; this wave takes tile t0 + kpart
    for (uint32_t t0 = t_begin, step = 0; t0 < tiles; t0 += KS, ++step) {
        const int buf = step & 1;
        const uint32_t t = t0 + kpart;
        const uint32_t k0 = t * kFlashN;
        const bool more = t0 + KS < tiles;
        if (more) fetch((t0 + KS) * kFlashN);
        if (t < tiles && wave_live && !(a.causal && (uint64_t)k0 > wave_last_key)) {
            // interior tile: every key exists and is visible to every query of
            // the wave, so no per-score bounds or causal test is needed
            const bool interior = k0 + kFlashN <= a.kl &&
                                  (!a.causal || (uint64_t)k0 + kFlashN - 1 <= (uint64_t)qw + a.causal_offset);
            // the two 32-key halves are independent accumulation chains:
            // interleaved, each MFMA's latency is covered by the other's
            float16v st[2];
#pragma unroll
            for (int hblk = 0; hblk < 2; ++hblk)
#pragma unroll
                for (int r = 0; r < 16; ++r) st[hblk][r] = 0.0f;
            mfma_phase_begin();
#pragma unroll
            for (int c = 0; c < KC; ++c)
#pragma unroll
                for (int hblk = 0; hblk < 2; ++hblk) {
                    const half8 kf = *reinterpret_cast<const half8 *>(
                        &ks[buf][kpart * KTILE + (32 * hblk + col) * KROW + 16 * c + 8 * half]);
                    st[hblk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[c], st[hblk], 0, 0, 0);
                }
            lds_read_ahead<2 * KC>();
            mfma_phase_end();
            // Scores are in log2 units: s = raw * scale2 (+ mask * log2 e).
            // Without a mask (and with scale2 > 0) st keeps the raw products
            // and sc = scale2 is applied inside exp2's fma; max_r(raw) * scale2
            // == max_r(raw * scale2) since rounding is monotone. The kMask
            // variant (also run for a scale <= 0, with or without a mask)
            // turns st into s and uses sc = 1 (fma(s, 1, -m) == s - m). The
            // interior test is taken once per tile (inside the unrolled loop
            // it became one branch per score).
            auto score = [&](float raw, uint32_t kk, bool edge) {
                float s = raw * scale2;
                if (mask != nullptr && kk < a.kl && q_live)
                    s = __builtin_fmaf((float)mask[(size_t)qi * a.kl + kk], kLog2e, s);
                if (edge && (kk >= a.kl || (a.causal && (uint64_t)kk > lane_last_key)))
                    s = neg_inf;
                return s;
            };
            // the online-softmax step for scores sv (s = sv * sc): P of the
            // tile into pf, m, l and o updated
            half8 pf[4];
            auto softmax = [&](const float16v (&sv)[2], float sc) {
                // four independent max chains instead of one of 32
                float part_max[4] = {neg_inf, neg_inf, neg_inf, neg_inf};
#pragma unroll
                for (int r = 0; r < 32; ++r) part_max[r % 4] = fmaxf(part_max[r % 4], sv[r / 16][r % 16]);
                const float tile_max =
                    pair_max(fmaxf(fmaxf(part_max[0], part_max[1]), fmaxf(part_max[2], part_max[3]))) * sc;
                // Lazy rescale: the running max m (and with it o and l) moves
                // only when some lane's maximum grows by more than
                // 2^kLazyLog2; until then p = 2^(s - m) <= 2^kLazyLog2, well
                // inside f16's range.
                const float m_cand = fmaxf(m, tile_max);
                if (__builtin_amdgcn_ballot_w64(m_cand > m + kLazyLog2) != 0) {
                    const float alpha = m_cand == neg_inf ? 1.0f : __builtin_amdgcn_exp2f(m - m_cand);
                    l *= alpha;
#pragma unroll
                    for (int tt = 0; tt < VT; ++tt)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[tt][r] *= alpha;
                    m = m_cand;
                }
                const bool none = m == neg_inf;   // nothing visible to this query yet
                if (wave_any(none)) {
                    // a NaN score while nothing is visible is remembered: the
                    // row is NaN if a key becomes visible later (its p, NaN,
                    // also reaches o and l)
                    bool local_nan = false;
#pragma unroll
                    for (int r = 0; r < 32; ++r) local_nan = local_nan || sv[r / 16][r % 16] != sv[r / 16][r % 16];
                    nan_seen = nan_seen || (none && local_nan);
                }
                // with nothing visible every non-NaN score is -inf: p = 2^-inf = 0
                const float m_use = none ? 0.0f : m;
#pragma unroll
                for (int r = 0; r < 32; ++r)
                    pf[r / 8][r % 8] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(sv[r / 16][r % 16], sc, -m_use));
                // the row sum of P as the MFMA sees it (f16), by v_dot2 with {1, 1}
                const half2_t ones = {(_Float16)1.0f, (_Float16)1.0f};
                float part_sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        part_sum[j] = __builtin_amdgcn_fdot2(half2_t{pf[c][2 * j], pf[c][2 * j + 1]}, ones,
                                                             part_sum[j], false);
                l += pair_sum((part_sum[0] + part_sum[1]) + (part_sum[2] + part_sum[3]));
            };
            if constexpr (kMask) {
                float16v sv[2];
                if (interior) {
#pragma unroll
                    for (int hblk = 0; hblk < 2; ++hblk)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            sv[hblk][r] = score(st[hblk][r], k0 + 32 * hblk + 8 * (r / 4) + 4 * half + r % 4, false);
                } else {
#pragma unroll
                    for (int hblk = 0; hblk < 2; ++hblk)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            sv[hblk][r] = score(st[hblk][r], k0 + 32 * hblk + 8 * (r / 4) + 4 * half + r % 4, true);
                }
                softmax(sv, 1.0f);
            } else {
                // raw products, scale2 > 0: keys out of range or past the
                // causal limit become -inf in place
                if (!interior) {
#pragma unroll
                    for (int hblk = 0; hblk < 2; ++hblk)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const uint32_t kk = k0 + 32 * hblk + 8 * (r / 4) + 4 * half + r % 4;
                            if (kk >= a.kl || (a.causal && (uint64_t)kk > lane_last_key)) st[hblk][r] = neg_inf;
                        }
                }
                softmax(st, scale2);
            }
            // the VT output tiles are independent chains: issue them side by side
            mfma_phase_begin();
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int tt = 0; tt < VT; ++tt) {
                    const _Float16 *vp = &vs[buf][kpart * VTILE + 16 * c * VROW + v_lane + 32 * tt];
                    const half4 lo = lds_read_tr(vp), hi = lds_read_tr(vp + 8 * VROW);
                    const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[c], o[tt], 0, 0, 0);
                }
            lds_read_ahead<4 * VT, 2>();
            mfma_phase_end();
        }
        if (more) stash(buf ^ 1, (t0 + KS) * kFlashN);
        __syncthreads();
    }
    nan_seen = nan_seen || __shfl_xor((int)nan_seen, 32, kWave);
    if constexpr (KS == 2) {
        // Merge the two key parts of each query group through LDS (the loop
        // ended on a barrier, so the tile buffers are free): the part-1 wave
        // leaves its (o, m, l, NaN flag), the part-0 wave folds them in with
        // the merge rules of sdpa_combine_kernel and goes on alone.
        static_assert(QW * (VT * 4 + 1) * kWave * 16 <= sizeof(ks), "merge area");
        f32x4 *xch = reinterpret_cast<f32x4 *>(&ks[0][0]) + qgroup * (VT * 4 + 1) * kWave + lane;
        if (kpart == 1) {
#pragma unroll
            for (int tt = 0; tt < VT; ++tt)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    xch[(tt * 4 + g) * kWave] =
                        f32x4{o[tt][4 * g], o[tt][4 * g + 1], o[tt][4 * g + 2], o[tt][4 * g + 3]};
            xch[VT * 4 * kWave] = f32x4{m, l, nan_seen ? 1.0f : 0.0f, 0.0f};
        }
        __syncthreads();
        if (kpart == 1) return;
        const f32x4 other = xch[VT * 4 * kWave];
        const float big = fmaxf(m, other.x);
        // weights 2^(m_s - M); a part that saw nothing (m_s = -inf), and
        // every part of a row whose M is not finite (a zero row), weigh 0
        const bool finite = __builtin_isfinite(big);
        const float w0 = !finite || m == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m - big);
        const float w1 = !finite || other.x == -__builtin_inff() ? 0.0f
                                                                  : __builtin_amdgcn_exp2f(other.x - big);
#pragma unroll
        for (int tt = 0; tt < VT; ++tt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 p = xch[(tt * 4 + g) * kWave];
#pragma unroll
                for (int j = 0; j < 4; ++j) o[tt][4 * g + j] = w0 * o[tt][4 * g + j] + w1 * p[j];
            }
        l = w0 * l + w1 * other.y;
        m = big;
        nan_seen = nan_seen || other.z != 0.0f;
    }
    if (!q_live) return;
    if constexpr (kSplit) {
        if (item.parts > 1) {
            write_partial<D, VT>(a, item.part, (size_t)bh * a.ql + qi, half, o, m, l, nan_seen);
            return;
        }
    }
    const bool zero = !__builtin_isfinite(m);
    const float inverse = l == 0.0f ? 0.0f : 1.0f / l;
    const float nan = __builtin_nanf("");
    _Float16 *orow = out + ((size_t)bh * a.ql + qi) * D;
#pragma unroll
    for (int tt = 0; tt < VT; ++tt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            _Float16 quad[4] __attribute__((aligned(8)));
#pragma unroll
            for (int j = 0; j < 4; ++j)
                quad[j] = (_Float16)(zero ? 0.0f : nan_seen ? nan : o[tt][4 * g + j] * inverse);
            *reinterpret_cast<uint2 *>(orow + 32 * tt + 8 * g + 4 * half) =
                *reinterpret_cast<const uint2 *>(quad);
        }
}

// f32 flash kernel (D = Dv in {64, 128}): v_mfma_f32_32x32x2_f32, one wave
// per 32 queries, BM queries per block, 32-key K and V tiles in LDS
// (row-major, row pitch D + 4 floats: conflict-free 16-byte reads),
// double-buffered.
//   S^T = K Q^T: MFMA c contracts the d pair {c, D/2 + c}: lane half h holds
//   d in [h D/2, (h + 1) D/2), so each lane's K and Q operands are runs of
//   consecutive floats (Q stays in registers for the whole kernel).
//   out^T += V^T P^T: MFMA j contracts the key pair {8(j/4) + j%4, that + 4},
//   exactly the keys that accumulator register j of S^T holds in the two lane
//   halves, so P is the B operand as it stands and V needs no transpose.
// Scores are s * scale (+ mask), causal keys -inf; the online softmax uses
// expf (libm accuracy) and normalises once at the end by the reciprocal of
// the sum, with the special-row rules of the f16 kernel.
constexpr int kFlashN32 = 32;   // keys per f32 tile

template <int D, int BM, bool kMask, bool kSplit, int KS>
__global__ __launch_bounds__(BM * 2 * KS) void sdpa_flash_f32_kernel(const float *__restrict__ q,
                                                                const float *__restrict__ k,
                                                                const float *__restrict__ v,
                                                                const float *__restrict__ mask,
                                                                float *__restrict__ out,
                                                                SdpaArgs a) {
    constexpr int QW = BM / 32;              // query groups of 32: one wave each per key part
    constexpr int THREADS = BM * 2 * KS;
    constexpr int KN = kFlashN32;
    constexpr int ROW = D + 4;               // LDS row (floats)
    constexpr int VT = D / 32;               // 32-row tiles of out^T
    constexpr int QC = D / 2;                // MFMAs of S^T per tile
    constexpr int TILE = KN * ROW;           // LDS floats of one K or V tile
    constexpr int TV = KN * D / 4;           // float4 vectors per K or V tile
    constexpr int VECS = KS * TV;            // per operand and step (KS tiles)
    constexpr int PER = VECS / THREADS;
    static_assert(VECS % THREADS == 0, "tile load split");
    // step buffer b: K tiles at lds[b * 2 KS TILE], V tiles KS TILE further
    __shared__ __attribute__((aligned(16))) float lds[2 * 2 * KS * TILE];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(tid / kWave);
    // wave w takes query group w % QW and key tile kpart of every step
    const uint32_t qgroup = wave % QW, kpart = wave / QW;
    const uint32_t col = lane & 31, half = lane >> 5;
    const FlashItem item = flash_item(a, blockIdx.x);
    const uint32_t qblock = item.qblock, bh = item.bh;
    const uint32_t head = bh % a.qh, b = bh / a.qh;
    const size_t kv_base = ((size_t)b * a.kvh + head / a.group) * a.kl;
    const uint32_t qw = qblock * BM + qgroup * 32;
    const uint32_t qi = qw + col;
    const bool q_live = qi < a.ql;
    const float neg_inf = -__builtin_inff();

    float qf[QC];
    {
        const f32x4 *qrow = reinterpret_cast<const f32x4 *>(
            q + ((size_t)bh * a.ql + (q_live ? qi : 0)) * D + half * QC);
#pragma unroll
        for (int c = 0; c < QC / 4; ++c) {
            const f32x4 t = qrow[c];
            qf[4 * c] = t.x;
            qf[4 * c + 1] = t.y;
            qf[4 * c + 2] = t.z;
            qf[4 * c + 3] = t.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);   // Q ready before the tile loop
    __builtin_amdgcn_sched_barrier(0);
    float16v o[VT];
#pragma unroll
    for (int t = 0; t < VT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
    float m = neg_inf, l = 0.0f;
    bool nan_seen = false;

    const uint32_t all_tiles = flash_tiles(a.ql, a.kl, a.causal != 0, a.causal_offset, BM, KN,
                                           qblock);
    const uint32_t share = (all_tiles + item.parts - 1) / item.parts;
    const uint32_t t_begin = min(item.part * share, all_tiles);
    const uint32_t tiles = min(t_begin + share, all_tiles);
    const bool wave_live = qw < a.ql;
    const uint64_t wave_last_key = (uint64_t)min(qw + 31, a.ql - 1) + a.causal_offset;
    const uint64_t lane_last_key = (uint64_t)qi + a.causal_offset;

    // tile loads of a step (KS tiles from key k0): vector e of a tile is key
    // e / (D/4), floats 4 (e % (D/4)) ...; branch-free (rows past the end
    // clamped onto the last key, zeroed when stored: see the f16 kernel)
    f32x4 kreg[PER], vreg[PER];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const uint32_t e = tid + u * THREADS, tk = k0 + e / TV * KN, r = e % TV;
            const size_t at = (kv_base + min(tk + r / (D / 4), a.kl - 1)) * D + (r % (D / 4)) * 4;
            kreg[u] = *reinterpret_cast<const f32x4 *>(k + at);
            vreg[u] = *reinterpret_cast<const f32x4 *>(v + at);
        }
    };
    auto stash = [&](int buf, uint32_t k0) {
        if (k0 + KS * KN > a.kl) {   // a ragged last step: zero the rows past the end
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const uint32_t e = tid + u * THREADS, tk = k0 + e / TV * KN, r = e % TV;
                if (tk + r / (D / 4) >= a.kl) {
                    kreg[u] = f32x4{0, 0, 0, 0};
                    vreg[u] = f32x4{0, 0, 0, 0};
                }
            }
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const uint32_t e = tid + u * THREADS, r = e % TV;
            const uint32_t at = buf * 2 * KS * TILE + (e / TV) * TILE + (r / (D / 4)) * ROW + (r % (D / 4)) * 4;
            *reinterpret_cast<f32x4 *>(&lds[at]) = kreg[u];
            *reinterpret_cast<f32x4 *>(&lds[at + KS * TILE]) = vreg[u];
        }
    };

    if (t_begin < tiles) {
        fetch(t_begin * KN);
        stash(0, t_begin * KN);
    }
    __syncthreads();
    // step: KS tiles from t0; this wave takes tile t0 + kpart
    for (uint32_t t0 = t_begin, step = 0; t0 < tiles; t0 += KS, ++step) {
        const int buf = step & 1;
        const uint32_t t = t0 + kpart;
        const uint32_t k0 = t * KN;
        const bool more = t0 + KS < tiles;
        if (more) fetch((t0 + KS) * KN);
        const float *kt = &lds[buf * 2 * KS * TILE + kpart * TILE];   // this wave's K tile
        const float *vt = kt + KS * TILE;                              // and V tile
        if (t < tiles && wave_live && !(a.causal && (uint64_t)k0 > wave_last_key)) {
            const bool interior = k0 + KN <= a.kl &&
                                  (!a.causal || (uint64_t)k0 + KN - 1 <= (uint64_t)qw + a.causal_offset);
            // two accumulators (even and odd d pairs) keep two MFMA chains in flight
            float16v acc[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[h2][r] = 0.0f;
            const float *krow = kt + col * ROW + half * QC;
#pragma unroll
            for (int c4 = 0; c4 < QC / 4; ++c4) {
                const f32x4 kf = *reinterpret_cast<const f32x4 *>(krow + 4 * c4);
                acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qf[4 * c4], acc[0], 0, 0, 0);
                acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qf[4 * c4 + 1], acc[1], 0, 0, 0);
                acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qf[4 * c4 + 2], acc[0], 0, 0, 0);
                acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qf[4 * c4 + 3], acc[1], 0, 0, 0);
            }
            float st[16];
            float local_max = neg_inf;
            auto score = [&](float raw, uint32_t kk, bool edge) {
                float s = raw * a.scale;
                if constexpr (kMask) {
                    if (kk < a.kl && q_live) s = s + mask[(size_t)qi * a.kl + kk];
                }
                if (edge && (kk >= a.kl || (a.causal && (uint64_t)kk > lane_last_key)))
                    s = neg_inf;
                return s;
            };
            float part_max[4] = {neg_inf, neg_inf, neg_inf, neg_inf};
            if (interior) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    st[r] = score(acc[0][r] + acc[1][r], k0 + 8 * (r / 4) + 4 * half + r % 4, false);
                    part_max[r % 4] = fmaxf(part_max[r % 4], st[r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    st[r] = score(acc[0][r] + acc[1][r], k0 + 8 * (r / 4) + 4 * half + r % 4, true);
                    part_max[r % 4] = fmaxf(part_max[r % 4], st[r]);
                }
            }
            local_max = fmaxf(fmaxf(part_max[0], part_max[1]), fmaxf(part_max[2], part_max[3]));
            const float m_new = fmaxf(m, pair_max(local_max));
            const bool none = m_new == neg_inf;
            if (wave_any(none)) {
                bool local_nan = false;
#pragma unroll
                for (int r = 0; r < 16; ++r) local_nan = local_nan || st[r] != st[r];
                nan_seen = nan_seen || (none && local_nan);
            }
            const float alpha = none ? 1.0f : expf(m - m_new);
            float part_sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                st[r] = none ? 0.0f : expf(st[r] - m_new);
                part_sum[r % 4] += st[r];
            }
            const float local_sum = (part_sum[0] + part_sum[1]) + (part_sum[2] + part_sum[3]);
            l = l * alpha + pair_sum(local_sum);
            m = m_new;
            if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
                for (int tt = 0; tt < VT; ++tt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[tt][r] *= alpha;
            }
            // the VT output tiles are independent chains: issue them side by side
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float *vrow = vt + (8 * (j / 4) + 4 * half + j % 4) * ROW + col;
#pragma unroll
                for (int tt = 0; tt < VT; ++tt)
                    o[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * tt], st[j], o[tt], 0, 0, 0);
            }
        }
        if (more) stash(buf ^ 1, (t0 + KS) * KN);
        __syncthreads();
    }
    nan_seen = nan_seen || __shfl_xor((int)nan_seen, 32, kWave);
    if constexpr (KS == 2) {
        // the two key parts of each query group merged through LDS, as in
        // the f16 kernel, with natural-exp weights e^(m_s - M)
        static_assert(QW * (VT * 4 + 1) * kWave * 16 <= sizeof(lds), "merge area");
        f32x4 *xch = reinterpret_cast<f32x4 *>(&lds[0]) + qgroup * (VT * 4 + 1) * kWave + lane;
        if (kpart == 1) {
#pragma unroll
            for (int tt = 0; tt < VT; ++tt)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    xch[(tt * 4 + g) * kWave] =
                        f32x4{o[tt][4 * g], o[tt][4 * g + 1], o[tt][4 * g + 2], o[tt][4 * g + 3]};
            xch[VT * 4 * kWave] = f32x4{m, l, nan_seen ? 1.0f : 0.0f, 0.0f};
        }
        __syncthreads();
        if (kpart == 1) return;
        const f32x4 other = xch[VT * 4 * kWave];
        const float big = fmaxf(m, other.x);
        const bool finite = __builtin_isfinite(big);
        const float w0 = !finite || m == -__builtin_inff() ? 0.0f : expf(m - big);
        const float w1 = !finite || other.x == -__builtin_inff() ? 0.0f : expf(other.x - big);
#pragma unroll
        for (int tt = 0; tt < VT; ++tt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 p = xch[(tt * 4 + g) * kWave];
#pragma unroll
                for (int j = 0; j < 4; ++j) o[tt][4 * g + j] = w0 * o[tt][4 * g + j] + w1 * p[j];
            }
        l = w0 * l + w1 * other.y;
        m = big;
        nan_seen = nan_seen || other.z != 0.0f;
    }
    if (!q_live) return;
    if constexpr (kSplit) {
        if (item.parts > 1) {
            write_partial<D, VT>(a, item.part, (size_t)bh * a.ql + qi, half, o, m, l, nan_seen);
            return;
        }
    }
    const bool zero = !__builtin_isfinite(m);
    const float inverse = l == 0.0f ? 0.0f : 1.0f / l;
    const float nan = __builtin_nanf("");
    float *orow = out + ((size_t)bh * a.ql + qi) * D;
#pragma unroll
    for (int tt = 0; tt < VT; ++tt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 quad;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                quad[j] = zero ? 0.0f : nan_seen ? nan : o[tt][4 * g + j] * inverse;
            *reinterpret_cast<f32x4 *>(orow + 32 * tt + 8 * g + 4 * half) = quad;
        }
}

template <typename S>
hipError_t launch_sdpa(const S *q, const S *k, const S *v, const S *mask, S *out,
                       const k::SdpaShape &sh, float scale, bool causal, hipStream_t s) {
    if (sh.batch == 0 || sh.q_heads == 0 || sh.kv_heads == 0 || sh.q_len == 0 ||
        sh.kv_len == 0 || sh.head_dim == 0 || sh.value_dim == 0 ||
        sh.q_heads % sh.kv_heads != 0)
        return hipErrorInvalidValue;
    if (sh.head_dim > (size_t)kMaxRowRegs * kWave || sh.value_dim > (size_t)kMaxRowRegs * kWave)
        return hipErrorInvalidValue;
    const uint64_t lim = 0xffffffffull;
    if (sh.batch > lim || sh.q_heads > lim || sh.kv_heads > lim || sh.q_len > lim ||
        sh.kv_len > lim)
        return hipErrorInvalidValue;
    SdpaArgs a{};
    a.batch = (uint32_t)sh.batch;
    a.qh = (uint32_t)sh.q_heads;
    a.kvh = (uint32_t)sh.kv_heads;
    a.group = (uint32_t)(sh.q_heads / sh.kv_heads);
    a.ql = (uint32_t)sh.q_len;
    a.kl = (uint32_t)sh.kv_len;
    a.dim = (uint32_t)sh.head_dim;
    a.vdim = (uint32_t)sh.value_dim;
    a.causal_offset = a.kl > a.ql ? a.kl - a.ql : 0;
    a.scale = scale;
    a.causal = causal ? 1 : 0;
    const size_t rows = sh.batch * sh.q_heads * sh.q_len;
    const size_t waves_per_block = kBlock / kWave;
    const size_t blocks = (rows + waves_per_block - 1) / waves_per_block;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    constexpr size_t E = Vec16<S>::N;
    if (sh.head_dim % E == 0 && ((uintptr_t)k & 15u) == 0)
        hipLaunchKernelGGL((sdpa_row_kernel<S, true>), dim3((unsigned)blocks), dim3(kBlock), 0, s,
                           q, k, v, mask, out, a);
    else
        hipLaunchKernelGGL((sdpa_row_kernel<S, false>), dim3((unsigned)blocks), dim3(kBlock), 0,
                           s, q, k, v, mask, out, a);
    return hipGetLastError();
}

}  // namespace

namespace {

// Flash path choice for a shape: f16 256-query blocks (8 waves sharing each
// K/V tile) when there are at least 256 of them (32 x 2048^2 D 128 82.8 us
// vs 89.2 with 128-query blocks, 4096^2 causal 164.6 vs 179.9; 4 x 16 x
// 512^2, 128 such blocks, 23.5 vs 20.9), else 128-query blocks (4 waves)
// when there are at least 64 of them, else 64-query blocks (measured:
// 12 x 1024^2 D 64 f16 20.1 us wide vs 22.2 narrow, 4 x 16 x 512^2 D 128
// 21.1 vs 25.6, 32 x 1024^2 causal 33.2 vs 39.0, f32 4 x 16 x 512^2 56.6
// vs 70.6; f32 stays at 128). The work is then cut into items and ordered longest first.
// With a workspace, query blocks whose key range is long against the whole
// launch are split: target split_tiles = max(total key tiles / slots,
// kMinPartTiles), slots measured over 128 .. 3072: f16 128 (a split rarely
// pays for its merge: the vision shape is best in 2 parts, 32 x 2048^2
// causal unsplit; grids of up to 256 blocks of 128 queries take 256 and
// the parts fitted to one round, below), f32 512 (its 32-key tiles of
// 64 MFMAs keep a block busy: 12 x 1024^2 D 64 53 us in 6 parts vs 59 in
// 2 and 103 unsplit; 4 x 16 x 512^2, 256 blocks, is best unsplit). The
// part size grows until a (batch, head)'s items fit kMaxFlashItems; more
// query blocks than that: descending query blocks, no split.
struct FlashPlan {
    bool flash = false;
    uint32_t bm = 64, tk = 64;   // queries per block (64, 128, or 256 for f16), keys per tile
    uint32_t key_parts = 1;      // f16: waves per query group, taking alternate key tiles
    uint32_t qblocks = 0, items = 0;
    uint32_t split_tiles = 0;
    uint32_t max_parts = 1;
    uint32_t first_split = 0;   // first split query block
    bool table = false, xcd_heads = false;
    uint32_t item[kMaxFlashItems] = {};
};

// f16 blocks of 128 queries whose 8 waves split the key tiles in two (see
// sdpa_flash_kernel) pay where a causal launch is about one round of
// 256-query blocks with uneven key ranges: twice as many blocks, each half
// as long, let the longest-first order pair long blocks with short ones on
// a CU, with no merge launch. Measured (us, two-part vs 256-query blocks):
// 32q/8kv 2048^2 D 128 causal 58.4 vs 70.3, D 64 37.3 vs 50.0; 32 x 1024^2
// D 64 causal 17.5 vs 22.4 (128-query blocks). Each two-part step stages
// twice the K/V bytes per wave, so where the key ranges are even, or there
// are several rounds of blocks for the order to balance, they lose: 2048^2
// D 128 non-causal 95 vs 80, 4096^2 causal 187 vs 167, 4 x 2048^2 causal
// 220 vs 189.
// f32: the same in-block split for causal launches of at least one 8-wave
// block per CU with uneven key ranges (measured below)
bool key_parts_pay_f32(const k::SdpaShape &sh, bool causal) {
    const size_t bhs = sh.batch * sh.q_heads;
    if (!causal || ((sh.q_len + 127) / 128) * bhs < 256) return false;
    const uint32_t ql = (uint32_t)sh.q_len, kl = (uint32_t)sh.kv_len;
    const uint32_t offset = kl > ql ? kl - ql : 0, blocks = (ql + 127) / 128;
    // every block up to 1024 of them, else an even sample (the longest,
    // the last block, always in it)
    const uint32_t stride = blocks > 1024 ? blocks / 1024 : 1;
    uint64_t total = 0, most = 0, n = 0;
    for (uint32_t j = blocks - 1;; j -= stride) {
        const uint64_t t = flash_tiles(ql, kl, true, offset, 128, kFlashN32, j);
        total += t;
        most = t > most ? t : most;
        ++n;
        if (j < stride) break;
    }
    return 4 * most * n > 5 * total;
}

bool key_parts_pay(const k::SdpaShape &sh, bool causal) {
    const size_t bhs = sh.batch * sh.q_heads;
    if (!causal || ((sh.q_len + 127) / 128) * bhs < 256 || ((sh.q_len + 255) / 256) * bhs > 256)
        return false;
    // uneven: the longest 256-query block sees > 5/4 of the average key tiles
    const uint32_t ql = (uint32_t)sh.q_len, kl = (uint32_t)sh.kv_len;
    const uint32_t offset = kl > ql ? kl - ql : 0, blocks = (ql + 255) / 256;
    uint64_t total = 0, most = 0;
    for (uint32_t j = 0; j < blocks; ++j) {
        const uint64_t t = flash_tiles(ql, kl, true, offset, 256, kFlashN, j);
        total += t;
        most = t > most ? t : most;
    }
    return 4 * most * blocks > 5 * total;
}

FlashPlan flash_plan(const k::SdpaShape &sh, bool aligned, bool f32, bool causal, bool split) {
    FlashPlan p;
    const uint64_t lim = 0x7fffffffull;
    if (!aligned || sh.head_dim != sh.value_dim || (sh.head_dim != 64 && sh.head_dim != 128) ||
        !sh.batch || !sh.q_heads || !sh.kv_heads || sh.q_heads % sh.kv_heads != 0 ||
        !sh.q_len || sh.q_len > lim || !sh.kv_len || sh.kv_len > lim ||
        sh.batch * sh.q_heads * ((sh.q_len + 63) / 64) > lim / (8 * kMaxKeyParts))
        return p;
    p.flash = true;
    const size_t bhs = sh.batch * sh.q_heads;
    // f16 grids of 64-255 blocks of 128 queries (fewer blocks than CUs)
    // also take two key parts, with the key-range split across blocks kept:
    // twice the waves per block (12 heads x 1024^2 D 64: 18.7 -> 16.9 us).
    // Non-causal ones of at most 128 such blocks over at most 1024 keys take
    // 64-query blocks (4 waves: 2 query groups x 2 key parts) and no split:
    // at most one block per CU, no merge launch (us, same box: 12 heads x
    // 1024^2 D 64 17.4 -> 14.3, D 128 25.9 -> 20.8, 32 heads x 512^2 D 64
    // 11.2 -> 9.6, 8 heads x 1024^2 D 64 15.7 -> 13.8); over 2048 keys, or
    // with more blocks than CUs, the split plan stays faster (4 heads x
    // 2048^2 D 128 31.7 vs 35.7; 20 heads x 1024^2 D 64 17.0 vs 25.9).
    // Exactly 256 such blocks (one per CU; not the 256-query plan) likewise
    // take two key parts: 8 waves per CU instead of 4 (us, same box: 32 x
    // 1024^2 D 64 non-causal 22.8 -> 18.7, 32q/8kv 1024 x 4096 D 128 109 ->
    // 90, causal 32 x 1024 x 4096 D 64 (even key ranges) 77 -> 57; with 384
    // blocks, two rounds, they lose: 48 x 1024^2 D 64 30.1 vs 34.1).
    const uint64_t q128 = ((sh.q_len + 127) / 128) * bhs;
    const bool small_grid = !f32 && q128 >= 64 &&
                            (q128 < 256 || (q128 == 256 && ((sh.q_len + 255) / 256) * bhs < 256));
    const bool small_short = small_grid && !causal && q128 <= 128 && sh.kv_len <= 1024;
    // Grids of fewer than 64 blocks of 128 queries: 64-query blocks of 4
    // waves (2 query groups x 2 key parts), the key range split over blocks
    // as before (us, same box, one-part 64-query blocks -> two-part: f16
    // 32q/8kv 128 x 2048 D 128 causal 33.3 -> 25.3, 8 x 512 x 4096 D 128
    // causal 55.0 -> 39.7, 40q/8kv 64 x 4096 D 128 33.0 -> 25.3, 16 x 256 x
    // 1024 D 64 15.5 -> 12.5, 8 x 512^2 D 128 14.7 -> 13.5; f32 16 x 256 x
    // 1024 D 64 34.7 -> 26.1, 4 x 1024^2 D 64 32.9 -> 24.6, 8 x 512^2 D 128
    // 32.8 -> 25.1). f32 at D 128 over more keys keeps one part (its
    // two-part 64-query block needs ~300 registers, one wave per SIMD:
    // 32q/8kv 128 x 2048 63.6 vs 68.9, 8 x 512 x 4096 causal 103 vs 111).
    const bool tiny_grid = q128 < 64 && (!f32 || sh.head_dim == 64 || sh.kv_len <= 512);
    if (f32 ? key_parts_pay_f32(sh, causal) : key_parts_pay(sh, causal)) {
        p.bm = 128;
        p.key_parts = 2;
    } else if (small_grid) {
        p.bm = small_short ? 64 : 128;
        p.key_parts = 2;
    } else if (tiny_grid) {
        p.bm = 64;
        p.key_parts = 2;
    } else if (!f32) {
        // more than 256 blocks of 128 queries: 256-query blocks, also below
        // one round of them (us, same box, 128-query blocks -> 256: 48 x
        // 1024^2 D 64 30.4 -> 29.7, 32q/8kv 1536^2 D 128 59.4 -> 58.0, causal
        // 48q/8kv 1024 x 4096 D 128 135 -> 132)
        p.bm = 256;
    } else if (q128 >= 64) p.bm = 128;
    else p.bm = 64;
    p.tk = f32 ? 32 : 64;
    p.qblocks = (uint32_t)((sh.q_len + p.bm - 1) / p.bm);
    p.items = p.qblocks;
    p.first_split = p.qblocks;
    p.xcd_heads = (sh.batch * sh.kv_heads) % 8 == 0;
    if (p.qblocks > kMaxFlashItems) return p;
    const uint32_t ql = (uint32_t)sh.q_len, kl = (uint32_t)sh.kv_len;
    const uint32_t offset = kl > ql ? kl - ql : 0;
    auto tiles = [&](uint32_t j) { return flash_tiles(ql, kl, causal, offset, p.bm, p.tk, j); };
    // f32 launches of two key parts in one round (256 blocks of 128
    // queries) split the long blocks' key ranges as well (us, same box:
    // causal 16 x 2048^2 D 64 171 -> 135, D 128 300 -> 228); from two rounds
    // on the longest-first order balances them without the merge's traffic
    const bool f32_round_split = f32 && p.key_parts == 2 && q128 <= 256;
    if (split && (p.key_parts == 1 || (small_grid && !small_short) || tiny_grid || f32_round_split)) {
        uint64_t total = 0;
        for (uint32_t j = 0; j < p.qblocks; ++j) total += tiles(j);
        total *= bhs;
        // f16 grids of up to 256 blocks (one per CU: the two-part blocks
        // take up to 151 KB of LDS) cut their key ranges into the most
        // parts that still fit one round of 256 blocks (us, same box, 128
        // slots before: 32q/8kv decode over 16384 keys 64.5 -> 37.0, 4 x
        // 32q/8kv decode over 2048 keys 34.2 -> 22.5, 32q/8kv 16 x 4096 causal
        // 22.8 -> 16.6, 8 x 512 x 4096 causal 39.5 -> 28.3, 8 x 1024 x 8192
        // 76.7 -> 54.3, 16 x 1024 x 4096 causal 48.7 -> 37.0; others equal)
        const bool fit = !f32 && (tiny_grid || small_grid);
        const uint64_t slots = f32 ? 512 : fit ? 256 : 128;
        const uint64_t target = (total + slots - 1) / slots;
        p.split_tiles = (uint32_t)(target > kMinPartTiles ? target : kMinPartTiles);
        // The smallest part size from there whose items fit the work table
        // (kMaxFlashItems per (batch, head)) and, for `fit`, 256 blocks in
        // all. The item count never grows with the part size, so a binary
        // search; at the largest size every query block is one item.
        auto parts_of = [&](uint32_t st) {
            uint64_t n = 0;
            for (uint32_t j = 0; j < p.qblocks; ++j) n += split_parts(tiles(j), st);
            return n;
        };
        auto fits = [&](uint32_t st) {
            const uint64_t n = parts_of(st);
            return n <= kMaxFlashItems && (!fit || n * bhs <= 256);
        };
        uint32_t lo = p.split_tiles, hi = lo;
        for (uint32_t j = 0; j < p.qblocks; ++j) hi = tiles(j) > hi ? tiles(j) : hi;
        while (lo < hi) {
            const uint32_t mid = lo + (hi - lo) / 2;
            if (fits(mid)) hi = mid;
            else lo = mid + 1;
        }
        p.split_tiles = lo;
    }
    struct Item {
        uint32_t size, qblock, part, parts;
    };
    Item list[kMaxFlashItems];
    uint32_t n = 0;
    for (uint32_t j = 0; j < p.qblocks; ++j) {
        const uint32_t t = tiles(j), parts = split_parts(t, p.split_tiles);
        const uint32_t share = (t + parts - 1) / parts;
        if (n + parts > kMaxFlashItems) {   // too many: descending query blocks, whole
            p.split_tiles = 0;
            p.max_parts = 1;
            p.first_split = p.qblocks;
            return p;
        }
        for (uint32_t q = 0; q < parts; ++q) {
            const uint32_t lo = q * share < t ? q * share : t;
            const uint32_t hi = lo + share < t ? lo + share : t;
            list[n++] = Item{hi - lo, j, q, parts};
        }
        if (parts > p.max_parts) p.max_parts = parts;
        if (parts > 1 && j < p.first_split) p.first_split = j;
    }
    std::stable_sort(list, list + n, [](const Item &x, const Item &y) {
        return x.size != y.size ? x.size > y.size : x.qblock > y.qblock;
    });
    p.items = n;
    p.table = true;
    for (uint32_t r = 0; r < n; ++r)
        p.item[r] = list[r].qblock | list[r].part << 16 | list[r].parts << 24;
    if (p.max_parts == 1) p.split_tiles = 0;
    return p;
}

size_t partial_bytes(const k::SdpaShape &sh, uint32_t parts) {
    const size_t rows = sh.batch * sh.q_heads * sh.q_len;
    return (size_t)parts * rows * (sh.head_dim + 4) * sizeof(float);
}

// The plan for a launch: split only when the caller's workspace holds the
// partial results.
FlashPlan launch_plan(const k::SdpaShape &sh, bool aligned, bool f32, bool causal,
                      size_t workspace_bytes, const void *workspace) {
    const FlashPlan p = flash_plan(sh, aligned, f32, causal, true);
    if (p.max_parts > 1 && (workspace == nullptr || workspace_bytes < partial_bytes(sh, p.max_parts)))
        return flash_plan(sh, aligned, f32, causal, false);
    return p;
}

SdpaArgs flash_args(const FlashPlan &p, const k::SdpaShape &sh, float scale, bool causal,
                    void *workspace) {
    SdpaArgs a{};
    a.batch = (uint32_t)sh.batch;
    a.qh = (uint32_t)sh.q_heads;
    a.kvh = (uint32_t)sh.kv_heads;
    a.group = (uint32_t)(sh.q_heads / sh.kv_heads);
    a.ql = (uint32_t)sh.q_len;
    a.kl = (uint32_t)sh.kv_len;
    a.dim = a.vdim = (uint32_t)sh.head_dim;
    a.causal_offset = a.kl > a.ql ? a.kl - a.ql : 0;
    a.scale = scale;
    a.causal = causal ? 1 : 0;
    a.items = p.items;
    a.qblocks = p.qblocks;
    a.split_tiles = p.split_tiles;
    a.table = p.table ? 1 : 0;
    a.xcd_heads = p.xcd_heads ? 1 : 0;
    for (uint32_t r = 0; r < p.items && p.table; ++r) a.item[r] = p.item[r];
    if (p.max_parts > 1) {
        const size_t rows = sh.batch * sh.q_heads * sh.q_len;
        a.part_o = static_cast<float *>(workspace);
        a.part_ml = reinterpret_cast<f32x4 *>(a.part_o + (size_t)p.max_parts * rows * sh.head_dim);
    }
    return a;
}

template <typename S>
hipError_t combine_splits(const SdpaArgs &a, const FlashPlan &p, S *out, hipStream_t s) {
    const uint32_t first_row = p.first_split * p.bm;
    const size_t n = (size_t)a.batch * a.qh * (a.ql - first_row) * (a.dim / 8);
    const dim3 grid((unsigned)((n + kBlock - 1) / kBlock)), block(kBlock);
    // the part-count bucket: no row of this launch has more parts
    static_assert(kMaxKeyParts <= 8, "combine buckets");
    if (p.max_parts <= 2)
        hipLaunchKernelGGL((sdpa_combine_kernel<S, sizeof(S) == 2, 2>), grid, block, 0, s, a, out,
                           p.bm, p.tk, first_row);
    else if (p.max_parts <= 4)
        hipLaunchKernelGGL((sdpa_combine_kernel<S, sizeof(S) == 2, 4>), grid, block, 0, s, a, out,
                           p.bm, p.tk, first_row);
    else
        hipLaunchKernelGGL((sdpa_combine_kernel<S, sizeof(S) == 2, 8>), grid, block, 0, s, a, out,
                           p.bm, p.tk, first_row);
    return hipGetLastError();
}

}  // namespace

// One flash launch for the plan's (D, BM, KS) with the general (mask) /
// split variant.
#define ICSDK_FLASH_VARIANTS_KS(KERNEL, D, BM, KS, Q, K, V, M, O)                                  \
    do {                                                                                           \
        if (general && split)                                                                      \
            hipLaunchKernelGGL((KERNEL<D, BM, true, true, KS>), grid, block, 0, s, Q, K, V, M, O, a);  \
        else if (general)                                                                          \
            hipLaunchKernelGGL((KERNEL<D, BM, true, false, KS>), grid, block, 0, s, Q, K, V, M, O, a); \
        else if (split)                                                                            \
            hipLaunchKernelGGL((KERNEL<D, BM, false, true, KS>), grid, block, 0, s, Q, K, V, M, O, a); \
        else                                                                                       \
            hipLaunchKernelGGL((KERNEL<D, BM, false, false, KS>), grid, block, 0, s, Q, K, V, M, O, a);\
    } while (0)
// two key parts: the raw-product variants only (the general variant would
// not fit two waves per SIMD at D 128 and runs with one key part)
#define ICSDK_FLASH_VARIANTS_KS2(KERNEL, D, Q, K, V, M, O)                                         \
    do {                                                                                           \
        if (split)                                                                                 \
            hipLaunchKernelGGL((KERNEL<D, 128, false, true, 2>), grid, block, 0, s, Q, K, V, M, O, a); \
        else                                                                                       \
            hipLaunchKernelGGL((KERNEL<D, 128, false, false, 2>), grid, block, 0, s, Q, K, V, M, O, a);\
    } while (0)
// two-part blocks of 64 or 128 queries
#define ICSDK_FLASH_VARIANTS_KS2_BM(KERNEL, D, Q, K, V, M, O)                                     \
    do {                                                                                           \
        if (plan.bm == 64 && split)                                                                \
            hipLaunchKernelGGL((KERNEL<D, 64, false, true, 2>), grid, block, 0, s, Q, K, V, M, O, a); \
        else if (plan.bm == 64)                                                                    \
            hipLaunchKernelGGL((KERNEL<D, 64, false, false, 2>), grid, block, 0, s, Q, K, V, M, O, a); \
        else                                                                                       \
            ICSDK_FLASH_VARIANTS_KS2(KERNEL, D, Q, K, V, M, O);                                    \
    } while (0)
// the f32 kernel: 64- or 128-query blocks, 64- or 128-query blocks with two
// key parts per query group
#define ICSDK_FLASH_SHAPES_F32(KERNEL, Q, K, V, M, O)                                              \
    do {                                                                                           \
        if (shape.head_dim == 64) {                                                                \
            if (ks == 2) ICSDK_FLASH_VARIANTS_KS2_BM(KERNEL, 64, Q, K, V, M, O);                   \
            else if (plan.bm == 128) ICSDK_FLASH_VARIANTS_KS(KERNEL, 64, 128, 1, Q, K, V, M, O);   \
            else ICSDK_FLASH_VARIANTS_KS(KERNEL, 64, 64, 1, Q, K, V, M, O);                        \
        } else {                                                                                   \
            if (ks == 2) ICSDK_FLASH_VARIANTS_KS2_BM(KERNEL, 128, Q, K, V, M, O);                  \
            else if (plan.bm == 128) ICSDK_FLASH_VARIANTS_KS(KERNEL, 128, 128, 1, Q, K, V, M, O);  \
            else ICSDK_FLASH_VARIANTS_KS(KERNEL, 128, 64, 1, Q, K, V, M, O);                       \
        }                                                                                          \
    } while (0)
// the f16 kernel: 64-, 128- or 256-query blocks, 64- or 128-query blocks
// with two key parts per query group
#define ICSDK_FLASH_SHAPES_F16(KERNEL, Q, K, V, M, O)                                              \
    do {                                                                                           \
        const int bm = (int)plan.bm;                                                               \
        if (shape.head_dim == 64) {                                                                \
            if (ks == 2) ICSDK_FLASH_VARIANTS_KS2_BM(KERNEL, 64, Q, K, V, M, O);                      \
            else if (bm == 256) ICSDK_FLASH_VARIANTS_KS(KERNEL, 64, 256, 1, Q, K, V, M, O);        \
            else if (bm == 128) ICSDK_FLASH_VARIANTS_KS(KERNEL, 64, 128, 1, Q, K, V, M, O);        \
            else ICSDK_FLASH_VARIANTS_KS(KERNEL, 64, 64, 1, Q, K, V, M, O);                        \
        } else {                                                                                   \
            if (ks == 2) ICSDK_FLASH_VARIANTS_KS2_BM(KERNEL, 128, Q, K, V, M, O);                     \
            else if (bm == 256) ICSDK_FLASH_VARIANTS_KS(KERNEL, 128, 256, 1, Q, K, V, M, O);       \
            else if (bm == 128) ICSDK_FLASH_VARIANTS_KS(KERNEL, 128, 128, 1, Q, K, V, M, O);       \
            else ICSDK_FLASH_VARIANTS_KS(KERNEL, 128, 64, 1, Q, K, V, M, O);                       \
        }                                                                                          \
    } while (0)

namespace k {

size_t sdpa_workspace_bytes(const SdpaShape &shape, bool f32, bool causal) {
    const FlashPlan p = flash_plan(shape, true, f32, causal, true);
    return p.flash && p.max_parts > 1 ? partial_bytes(shape, p.max_parts) : 0;
}

hipError_t sdpa_f32(const float *q, const float *k, const float *v, const float *mask,
                    float *out, const SdpaShape &shape, float scale, bool causal,
                    void *workspace, size_t workspace_bytes, hipStream_t s) {
    const bool aligned = (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u) == 0;
    const FlashPlan plan = launch_plan(shape, aligned, true, causal, workspace_bytes, workspace);
    if (!plan.flash) return launch_sdpa<float>(q, k, v, mask, out, shape, scale, causal, s);
    const SdpaArgs a = flash_args(plan, shape, scale, causal, workspace);
    const bool split = plan.max_parts > 1;
    const bool general = mask != nullptr;
    const uint32_t ks = general ? 1 : plan.key_parts;
    const dim3 grid((unsigned)(shape.batch * shape.q_heads * plan.items)), block(2 * plan.bm * ks);
    ICSDK_FLASH_SHAPES_F32(sdpa_flash_f32_kernel, q, k, v, mask, out);
    const hipError_t status = hipGetLastError();
    return status != hipSuccess || !split ? status : combine_splits(a, plan, out, s);
}

hipError_t sdpa_f16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                    const uint16_t *mask, uint16_t *out, const SdpaShape &shape, float scale,
                    bool causal, void *workspace, size_t workspace_bytes, hipStream_t s) {
    auto h = [](const uint16_t *p) { return reinterpret_cast<const _Float16 *>(p); };
    _Float16 *o16 = reinterpret_cast<_Float16 *>(out);
    const bool aligned = (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u) == 0;
    const FlashPlan plan = launch_plan(shape, aligned, false, causal, workspace_bytes, workspace);
    if (!plan.flash)
        return launch_sdpa<_Float16>(h(q), h(k), h(v), h(mask), o16, shape, scale, causal, s);
    const SdpaArgs a = flash_args(plan, shape, scale, causal, workspace);
    const bool split = plan.max_parts > 1;
    // the raw-product softmax needs scale > 0; other scales take the general
    // (mask) variant, whose mask may be null
    const bool general = mask != nullptr || !(scale > 0.0f);
    const uint32_t ks = general ? 1 : plan.key_parts;
    const dim3 grid((unsigned)(shape.batch * shape.q_heads * plan.items)), block(2 * plan.bm * ks);
    ICSDK_FLASH_SHAPES_F16(sdpa_flash_kernel, h(q), h(k), h(v), h(mask), o16);
    const hipError_t status = hipGetLastError();
    return status != hipSuccess || !split ? status : combine_splits(a, plan, o16, s);
}

}  // namespace k

#undef ICSDK_FLASH_SHAPES_F16
#undef ICSDK_FLASH_SHAPES_F32
#undef ICSDK_FLASH_VARIANTS_KS2_BM
#undef ICSDK_FLASH_VARIANTS_KS2
#undef ICSDK_FLASH_VARIANTS_KS


}  // namespace icsdk
