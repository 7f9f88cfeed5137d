// Row reductions over the last dimension for gfx950: RMSNorm (optionally
// fused with the residual add), LayerNorm, softmax (optionally causal), row
// sum and row max.
//
// Register path: a row is owned by a group of WPR wave64s (WPR = 1 for rows up
// to 64*8 vectors of 16 bytes, 4 above that). Each lane loads NV 16-byte
// vectors, interleaved so that every load instruction of the group covers a
// contiguous span (coalesced), keeps the widened f32 values in registers,
// reduces them with the DPP wave reduction and, for WPR > 1, combines the
// per-wave partials through LDS. The row is read from HBM exactly once and
// the output written once.
//
// Streaming path (widths that are not a multiple of the 16-byte vector, or
// too wide for registers): one 256-thread block per row, scalar accesses,
// the row re-read for every pass.
//
// Accumulation is f32; the order is per-lane sequential then a tree, which
// differs from the reference's single sequential sum only by rounding.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

// ---- group reductions ----------------------------------------------------

template <int WPR>
__device__ inline float group_sum(float v, float *lds) {
    v = wave_sum(v);
    if constexpr (WPR == 1) {
        return v;
    } else {
        const int wave = threadIdx.x / kWave;
        __syncthreads();
        if ((threadIdx.x & (kWave - 1)) == 0) lds[wave] = v;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < WPR; ++w) total += lds[w];
        return total;
    }
}

template <int WPR>
__device__ inline float group_max(float v, float *lds) {
    v = wave_max(v);
    if constexpr (WPR == 1) {
        return v;
    } else {
        const int wave = threadIdx.x / kWave;
        __syncthreads();
        if ((threadIdx.x & (kWave - 1)) == 0) lds[wave] = v;
        __syncthreads();
        float m = lds[0];
#pragma unroll
        for (int w = 1; w < WPR; ++w) m = fmaxf(m, lds[w]);
        return m;
    }
}

template <int WPR>
__device__ inline int group_sum_i32(int v, float *lds) {
    v = wave_sum_i32(v);
    if constexpr (WPR == 1) {
        return v;
    } else {
        const int wave = threadIdx.x / kWave;
        __syncthreads();
        if ((threadIdx.x & (kWave - 1)) == 0) lds[wave] = __builtin_bit_cast(float, v);
        __syncthreads();
        int total = 0;
#pragma unroll
        for (int w = 0; w < WPR; ++w) total += __builtin_bit_cast(int, lds[w]);
        return total;
    }
}

// Which row this thread group owns and the thread's index inside the group.
template <int WPR>
struct RowSlot {
    size_t row;
    uint32_t t;
    __device__ RowSlot() {
        if constexpr (WPR == 1) {
            // the wave index is wave-uniform; readfirstlane tells the compiler,
            // so the row and its base addresses live in scalar registers
            row = (size_t)blockIdx.x * (kBlock / kWave) +
                  (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
            t = threadIdx.x & (kWave - 1);
        } else {
            row = blockIdx.x;
            t = threadIdx.x;
        }
    }
};

// kExact: the row is exactly NV * WPR * 64 vectors (checked on the host), so
// no lane needs a bounds check.
template <typename S, int NV, int WPR, bool kExact = false>
struct RowRegs {
    static constexpr int E = Vec16<S>::N;
    static constexpr uint32_t T = WPR * kWave;
    float v[NV][E];

    __device__ static inline bool valid(int j, uint32_t t, uint32_t vpr) {
        return kExact || t + j * T < vpr;
    }

    // Every load is issued unconditionally (a lane past the row end re-reads
    // vector 0 of the row) and the fill value selected afterwards: a guarded
    // load becomes a branch after which the compiler waits for it, which
    // would serialise the row's loads.
    __device__ inline void load(const S *row, uint32_t t, uint32_t vpr, float fill) {
        Vec16<S> raw[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) raw[j] = load16_stream(row + (size_t)clamp(j, t, vpr) * E);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const bool ok = valid(j, t, vpr);
#pragma unroll
            for (int e = 0; e < E; ++e) v[j][e] = ok ? Elem<S>::load(raw[j].v[e]) : fill;
        }
    }

    __device__ static inline uint32_t clamp(int j, uint32_t t, uint32_t vpr) {
        const uint32_t vi = t + j * T;
        return kExact || vi < vpr ? vi : 0u;
    }
};

// Unconditional loads of a per-column parameter slice (weights, scale, bias).
template <typename S, int NV, int WPR, bool kExact = false>
__device__ inline void load_params(const S *p, uint32_t t, uint32_t vpr, Vec16<S> (&out)[NV]) {
    using R = RowRegs<S, NV, WPR, kExact>;
#pragma unroll
    for (int j = 0; j < NV; ++j) out[j] = load16(p + (size_t)R::clamp(j, t, vpr) * R::E);
}

// ---- RMSNorm / fused residual + RMSNorm ------------------------------------

// The weight slice is requested first and pinned there (a scheduling
// barrier): it comes from L2, and left to the scheduler its loads sink below
// the row reduction, adding an L2 round trip to every row's critical path.
// Outputs are written through L2 (OutWindow).
template <typename S, int NV, int WPR, bool kResidual, bool kExact>
__global__ __launch_bounds__(kBlock) void rms_norm_kernel(
    const S *__restrict__ x, const S *__restrict__ residual, S *__restrict__ sum_out,
    const S *__restrict__ w, S *__restrict__ y, size_t rows, uint32_t width, float eps) {
    __shared__ float lds[kBlock / kWave];
    using R = RowRegs<S, NV, WPR, kExact>;
    constexpr int E = R::E;
    const RowSlot<WPR> slot;
    // A slot past the last row recomputes the last row and stores nothing
    // (its output windows are 0 bytes long: the hardware drops the stores):
    // no branch waits for `rows` before the loads, so the kernel's argument
    // loads return in one round trip (an early return cost three before the
    // row's first load), and no branch on it lets the compiler sink the
    // weight loads down to the stores.
    const bool live = slot.row < rows;
    const size_t row = live ? slot.row : rows - 1;
    const uint32_t vpr = width / E;
    const size_t base = row * width;
    Vec16<S> wv[NV];
    load_params<S, NV, WPR, kExact>(w, slot.t, vpr, wv);
    __builtin_amdgcn_sched_barrier(0);
    R r;
    r.load(x + base, slot.t, vpr, 0.0f);
    const uint32_t row_bytes = width * (uint32_t)sizeof(S);
    if constexpr (kResidual) {
        Vec16<S> rv[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j)
            rv[j] = load16_stream(residual + base + (size_t)R::clamp(j, slot.t, vpr) * E);
        const OutWindow sums(sum_out + base, live ? row_bytes : 0u);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t vi = slot.t + j * R::T;
            const bool ok = R::valid(j, slot.t, vpr);
            Vec16<S> sum;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                sum.v[e] = Elem<S>::store(r.v[j][e] + Elem<S>::load(rv[j].v[e]));
                r.v[j][e] = ok ? Elem<S>::load(sum.v[e]) : 0.0f;
            }
            if (ok) sums.store16(vi * 16u, sum);
        }
    }
    float squares = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) squares += r.v[j][e] * r.v[j][e];
    squares = group_sum<WPR>(squares, lds);
    const float scale = 1.0f / sqrtf(squares / (float)width + eps);
    const OutWindow out(y + base, live ? row_bytes : 0u);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t vi = slot.t + j * R::T;
        if (R::valid(j, slot.t, vpr)) {
            Vec16<S> o;
#pragma unroll
            for (int e = 0; e < E; ++e)
                o.v[e] = Elem<S>::store(r.v[j][e] * scale * Elem<S>::load(wv[j].v[e]));
            out.store16(vi * 16u, o);
        }
    }
}

template <typename S, bool kResidual>
__global__ __launch_bounds__(kBlock) void rms_norm_stream_kernel(
    const S *__restrict__ x, const S *__restrict__ residual, S *__restrict__ sum_out,
    const S *__restrict__ w, S *__restrict__ y, size_t rows, size_t width, float eps) {
    __shared__ float lds[kBlock / kWave];
    const size_t row = blockIdx.x;
    if (row >= rows) return;
    const size_t base = row * width;
    float squares = 0.0f;
    for (size_t c = threadIdx.x; c < width; c += kBlock) {
        float v = Elem<S>::load(x[base + c]);
        if constexpr (kResidual) {
            const S s = Elem<S>::store(v + Elem<S>::load(residual[base + c]));
            sum_out[base + c] = s;
            v = Elem<S>::load(s);
        }
        squares += v * v;
    }
    squares = group_sum<kBlock / kWave>(squares, lds);
    const float scale = 1.0f / sqrtf(squares / (float)width + eps);
    const S *src = kResidual ? sum_out : x;
    for (size_t c = threadIdx.x; c < width; c += kBlock)
        y[base + c] = Elem<S>::store(Elem<S>::load(src[base + c]) * scale * Elem<S>::load(w[c]));
}

// ---- LayerNorm -----------------------------------------------------------

// kScale / kBias: which affine parameters are present (compile time, so that
// their loads are unconditional and issued first, like RMSNorm's weights).
template <typename S, int NV, int WPR, bool kExact, bool kScale, bool kBias>
__global__ __launch_bounds__(kBlock) void layer_norm_kernel(
    const S *__restrict__ x, const S *__restrict__ scale, const S *__restrict__ bias,
    S *__restrict__ y, size_t rows, uint32_t width, float eps) {
    __shared__ float lds[kBlock / kWave];
    using R = RowRegs<S, NV, WPR, kExact>;
    constexpr int E = R::E;
    const RowSlot<WPR> slot;
    // past the last row: recompute the last row into a 0-byte window (as in
    // rms_norm_kernel), so no branch waits for `rows` before the loads
    const bool live = slot.row < rows;
    const size_t row = live ? slot.row : rows - 1;
    const uint32_t vpr = width / E;
    const size_t base = row * width;
    Vec16<S> sv[NV], bv[NV];
    if constexpr (kScale) load_params<S, NV, WPR, kExact>(scale, slot.t, vpr, sv);
    if constexpr (kBias) load_params<S, NV, WPR, kExact>(bias, slot.t, vpr, bv);
    __builtin_amdgcn_sched_barrier(0);
    R r;
    r.load(x + base, slot.t, vpr, 0.0f);
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) total += r.v[j][e];
    const float mean = group_sum<WPR>(total, lds) / (float)width;
    float variance = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        if (R::valid(j, slot.t, vpr)) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float d = r.v[j][e] - mean;
                variance += d * d;
            }
        }
    variance = group_sum<WPR>(variance, lds);
    const float inverse_std = 1.0f / sqrtf(variance / (float)width + eps);
    const OutWindow out(y + base, live ? width * (uint32_t)sizeof(S) : 0u);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t vi = slot.t + j * R::T;
        if (R::valid(j, slot.t, vpr)) {
            Vec16<S> o;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                float v = (r.v[j][e] - mean) * inverse_std;
                if constexpr (kScale) v *= Elem<S>::load(sv[j].v[e]);
                if constexpr (kBias) v += Elem<S>::load(bv[j].v[e]);
                o.v[e] = Elem<S>::store(v);
            }
            out.store16(vi * 16u, o);
        }
    }
}

template <typename S>
__global__ __launch_bounds__(kBlock) void layer_norm_stream_kernel(
    const S *__restrict__ x, const S *__restrict__ scale, const S *__restrict__ bias,
    S *__restrict__ y, size_t rows, size_t width, float eps) {
    __shared__ float lds[kBlock / kWave];
    const size_t row = blockIdx.x;
    if (row >= rows) return;
    const S *src = x + row * width;
    float total = 0.0f;
    for (size_t c = threadIdx.x; c < width; c += kBlock) total += Elem<S>::load(src[c]);
    const float mean = group_sum<kBlock / kWave>(total, lds) / (float)width;
    float variance = 0.0f;
    for (size_t c = threadIdx.x; c < width; c += kBlock) {
        const float d = Elem<S>::load(src[c]) - mean;
        variance += d * d;
    }
    variance = group_sum<kBlock / kWave>(variance, lds);
    const float inverse_std = 1.0f / sqrtf(variance / (float)width + eps);
    for (size_t c = threadIdx.x; c < width; c += kBlock) {
        float v = (Elem<S>::load(src[c]) - mean) * inverse_std;
        if (scale) v *= Elem<S>::load(scale[c]);
        if (bias) v += Elem<S>::load(bias[c]);
        y[row * width + c] = Elem<S>::store(v);
    }
}

// ---- softmax -------------------------------------------------------------

// exp used for the softmax numerators: the hardware exp2 path for f16
// outputs, the libm-accurate expf for f32 outputs.
template <typename S>
__device__ inline float softmax_exp(float x) {
    if constexpr (sizeof(S) == 2) return fast_exp(x);
    else return expf(x);
}

// Causal masking: key k of query row q is kept when k <= q + offset. A
// vector whose first key is past the limit is never loaded.
// The row's position in its query range is a multiply-high division by
// q_len (q_mul, q_shift: FastDiv) for rows below 2^32, kept in front of the
// loads as a few scalar instructions.
template <typename S, int NV, int WPR>
__global__ __launch_bounds__(kBlock) void softmax_kernel(const S *__restrict__ x,
                                                         S *__restrict__ y, size_t rows,
                                                         uint32_t width, uint32_t q_len,
                                                         uint32_t q_mul, uint32_t q_shift,
                                                         uint32_t causal_offset) {
    __shared__ float lds[kBlock / kWave];
    using R = RowRegs<S, NV, WPR>;
    constexpr int E = R::E;
    const RowSlot<WPR> slot;
    // past the last row: recompute the last row and store nothing, so no
    // branch waits for `rows` before the loads
    const bool live = slot.row < rows;
    const size_t row = live ? slot.row : rows - 1;
    const uint32_t vpr = width / E;
    const size_t base = row * width;
    // keys 0..limit are visible (keys are < width < 2^32, so a limit past
    // 2^32 - 1 is held at that)
    uint32_t limit = width;
    if (q_len) {
        const uint32_t row32 = (uint32_t)row;
        // row-uniform: rows past 2^32 (never at real shapes) take the modulo
        const uint32_t pos = row >> 32 ? (uint32_t)(row % q_len)
                                       : row32 - fast_div(row32, FastDiv{q_len, q_mul, q_shift}) * q_len;
        limit = (uint32_t)min((uint64_t)pos + causal_offset, (uint64_t)0xffffffffu);
    }
    const float neg_inf = -__builtin_inff();
    R r;
    float m = neg_inf;
    // Vectors entirely past the causal limit re-read the row's first vector
    // (already requested by lane 0, so no HBM traffic) instead of branching.
    Vec16<S> raw[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t vi = slot.t + j * R::T;
        const bool use = vi < vpr && vi * (uint32_t)E <= limit;
        raw[j] = load16_stream(x + base + (size_t)(use ? vi : 0u) * E);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t first = (slot.t + j * R::T) * (uint32_t)E;
        const bool row_ok = slot.t + j * R::T < vpr;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float s = Elem<S>::load(raw[j].v[e]);
            s = row_ok && first + e <= limit ? s : neg_inf;
            r.v[j][e] = s;
            m = fmaxf(m, s);
        }
    }
    m = group_max<WPR>(m, lds);
    if (m == neg_inf) {
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < E; ++e) r.v[j][e] = 0.0f;
    } else if (m == __builtin_inff()) {
        // some visible key is +inf (fmaxf passes over NaN, so exactly then):
        // the +inf keys share the row equally; counted only on this path
        // (row-uniform: with several waves per row the block is the row)
        int pos_inf = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < E; ++e) pos_inf += r.v[j][e] == __builtin_inff();
        pos_inf = group_sum_i32<WPR>(pos_inf, lds);
        const float share = 1.0f / (float)pos_inf;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < E; ++e) r.v[j][e] = r.v[j][e] == __builtin_inff() ? share : 0.0f;
    } else {
        float total = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < E; ++e) {
                r.v[j][e] = softmax_exp<S>(r.v[j][e] - m);
                total += r.v[j][e];
            }
        total = group_sum<WPR>(total, lds);
        const float inverse = 1.0f / total;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if constexpr (sizeof(S) == 2) r.v[j][e] = r.v[j][e] * inverse;
                else r.v[j][e] = r.v[j][e] / total;
            }
    }
    // Written through L2 from a row-uniform window (a slot past the last row
    // gets a 0-byte window; lanes past the row's end fall outside it). The
    // output is the whole row while only its visible part was read, so the
    // kernel is write-heavy: at configs[2]'s [65536, 2048] causal shape
    // (134 MB read, 268 MB written) write-through stores measured 1.5-2 us
    // faster than non-temporal ones on MI355X, as a 268 MB write alone is
    // (37.4-38.1 us against 39.4-40.7).
    const OutWindow out(y + base, live ? width * (uint32_t)sizeof(S) : 0u);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t vi = slot.t + j * R::T;
        Vec16<S> o;
#pragma unroll
        for (int e = 0; e < E; ++e) o.v[e] = Elem<S>::store(r.v[j][e]);
        out.store16(vi * 16u, o);
    }
}

template <typename S>
__global__ __launch_bounds__(kBlock) void softmax_stream_kernel(const S *__restrict__ x,
                                                                S *__restrict__ y,
                                                                size_t rows, size_t width,
                                                                size_t q_len,
                                                                size_t causal_offset) {
    __shared__ float lds[kBlock / kWave];
    constexpr int W = kBlock / kWave;
    const size_t row = blockIdx.x;
    if (row >= rows) return;
    const size_t limit = q_len ? row % q_len + causal_offset : width;
    const S *src = x + row * width;
    S *dst = y + row * width;
    const float neg_inf = -__builtin_inff();
    float m = neg_inf;
    int pos_inf = 0;
    for (size_t c = threadIdx.x; c < width; c += kBlock) {
        const float s = c <= limit ? Elem<S>::load(src[c]) : neg_inf;
        m = fmaxf(m, s);
        pos_inf += s == __builtin_inff();
    }
    m = group_max<W>(m, lds);
    pos_inf = group_sum_i32<W>(pos_inf, lds);
    if (m == neg_inf) {
        for (size_t c = threadIdx.x; c < width; c += kBlock) dst[c] = Elem<S>::store(0.0f);
        return;
    }
    if (pos_inf > 0) {
        const float share = 1.0f / (float)pos_inf;
        for (size_t c = threadIdx.x; c < width; c += kBlock) {
            const float s = c <= limit ? Elem<S>::load(src[c]) : neg_inf;
            dst[c] = Elem<S>::store(s == __builtin_inff() ? share : 0.0f);
        }
        return;
    }
    float total = 0.0f;
    for (size_t c = threadIdx.x; c < width; c += kBlock)
        if (c <= limit) total += softmax_exp<S>(Elem<S>::load(src[c]) - m);
    total = group_sum<W>(total, lds);
    for (size_t c = threadIdx.x; c < width; c += kBlock) {
        const float e = c <= limit ? softmax_exp<S>(Elem<S>::load(src[c]) - m) : 0.0f;
        dst[c] = Elem<S>::store(e / total);
    }
}

// ---- row sum / row max -----------------------------------------------------

template <typename S, int NV, int WPR, bool kMax>
__global__ __launch_bounds__(kBlock) void row_reduce_kernel(const S *__restrict__ x,
                                                            float *__restrict__ y,
                                                            size_t rows, uint32_t width) {
    __shared__ float lds[kBlock / kWave];
    using R = RowRegs<S, NV, WPR>;
    constexpr int E = R::E;
    const RowSlot<WPR> slot;
    // past the last row: reduce the last row again and store nothing, so no
    // branch waits for `rows` before the loads
    const bool live = slot.row < rows;
    const size_t row = live ? slot.row : rows - 1;
    const uint32_t vpr = width / E;
    R r;
    r.load(x + row * width, slot.t, vpr, kMax ? -__builtin_inff() : 0.0f);
    float acc = kMax ? -__builtin_inff() : 0.0f;
    bool has_nan = false;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if constexpr (kMax) {
                acc = fmaxf(acc, r.v[j][e]);
                has_nan |= r.v[j][e] != r.v[j][e];
            } else {
                acc += r.v[j][e];
            }
        }
    float result;
    if constexpr (kMax) {
        result = group_max<WPR>(acc, lds);
        const int nan_count = group_sum_i32<WPR>(has_nan ? 1 : 0, lds);
        if (nan_count) result = __builtin_nanf("");
    } else {
        result = group_sum<WPR>(acc, lds);
    }
    if (slot.t == 0 && live) y[row] = result;
}

template <typename S, bool kMax>
__global__ __launch_bounds__(kBlock) void row_reduce_stream_kernel(const S *__restrict__ x,
                                                                   float *__restrict__ y,
                                                                   size_t rows,
                                                                   size_t width) {
    __shared__ float lds[kBlock / kWave];
    constexpr int W = kBlock / kWave;
    const size_t row = blockIdx.x;
    if (row >= rows) return;
    float acc = kMax ? -__builtin_inff() : 0.0f;
    int nan_count = 0;
    for (size_t c = threadIdx.x; c < width; c += kBlock) {
        const float v = Elem<S>::load(x[row * width + c]);
        if constexpr (kMax) {
            acc = fmaxf(acc, v);
            nan_count += v != v;
        } else {
            acc += v;
        }
    }
    float result;
    if constexpr (kMax) {
        result = group_max<W>(acc, lds);
        if (group_sum_i32<W>(nan_count, lds)) result = __builtin_nanf("");
    } else {
        result = group_sum<W>(acc, lds);
    }
    if (threadIdx.x == 0) y[row] = result;
}

// ---- launch-shape selection --------------------------------------------------

inline bool aligned16(const void *p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Register-path shape for a row of `width` elements of size `elem`: returns
// false when the row must take the streaming path.
struct RowShape {
    int nv;
    int wpr;
};

// Waves per row tried first (1 or 4); the first group whose lanes hold the
// row in at most 8 vectors each wins.
inline bool pick_row_shape(size_t width, size_t elem, bool aligned, RowShape *shape,
                           int wpr_first = 1) {
    const size_t per_vec = 16 / elem;
    if (!aligned || width == 0 || width % per_vec != 0 || width > 0xffffffffu) return false;
    const size_t vpr = width / per_vec;
    for (int wpr : {wpr_first, 5 - wpr_first}) {
        const size_t threads = (size_t)wpr * kWave;
        for (int nv : {1, 2, 4, 8}) {
            if ((size_t)nv * threads >= vpr) {
                shape->nv = nv;
                shape->wpr = wpr;
                return true;
            }
        }
    }
    return false;
}

inline dim3 row_grid(size_t rows, int wpr) {
    const size_t per_block = wpr == 1 ? kBlock / kWave : 1;
    return dim3((unsigned)((rows + per_block - 1) / per_block));
}

// Expands a run-time (nv, wpr) into the template instance.
#define ICSDK_ROW_DISPATCH(shape, KERNEL_TMPL, ...)                                      \
    do {                                                                                \
        switch ((shape).wpr * 100 + (shape).nv) {                                        \
            case 101: KERNEL_TMPL(1, 1); break;                                         \
            case 102: KERNEL_TMPL(2, 1); break;                                         \
            case 104: KERNEL_TMPL(4, 1); break;                                         \
            case 108: KERNEL_TMPL(8, 1); break;                                         \
            case 401: KERNEL_TMPL(1, 4); break;                                         \
            case 402: KERNEL_TMPL(2, 4); break;                                         \
            case 404: KERNEL_TMPL(4, 4); break;                                         \
            case 408: KERNEL_TMPL(8, 4); break;                                         \
            default: return hipErrorInvalidValue;                                       \
        }                                                                               \
    } while (0)

template <typename S, bool kResidual>
hipError_t launch_rms(const S *x, const S *residual, S *sum_out, const S *w, S *y,
                      size_t rows, size_t width, float eps, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    RowShape shape;
    const bool aligned = aligned16(x) && aligned16(residual) && aligned16(sum_out) &&
                         aligned16(w) && aligned16(y);
    // Many rows of at least 256 vectors: four waves per row (one vector per
    // lane at width 2048 f16), so the launch streams in more, smaller waves;
    // measured on MI355X at [16384, 2048] f16: 22.0 -> 21.7 us. At 4096 rows
    // the two shapes tie. (The causal softmax keeps one wave per row: four
    // cost it 30%.)
    const int wpr_first = rows >= 8192 && width * sizeof(S) >= 16u * 4 * kWave ? 4 : 1;
    if (pick_row_shape(width, sizeof(S), aligned, &shape, wpr_first)) {
        const bool exact = width / (16 / sizeof(S)) == (size_t)shape.nv * shape.wpr * kWave;
#define ICSDK_RMS(NV, WPR)                                                                 \
    do {                                                                                   \
        if (exact)                                                                         \
            hipLaunchKernelGGL((rms_norm_kernel<S, NV, WPR, kResidual, true>),             \
                               row_grid(rows, WPR), dim3(kBlock), 0, s, x, residual,       \
                               sum_out, w, y, rows, (uint32_t)width, eps);                 \
        else                                                                               \
            hipLaunchKernelGGL((rms_norm_kernel<S, NV, WPR, kResidual, false>),            \
                               row_grid(rows, WPR), dim3(kBlock), 0, s, x, residual,       \
                               sum_out, w, y, rows, (uint32_t)width, eps);                 \
    } while (0)
        ICSDK_ROW_DISPATCH(shape, ICSDK_RMS);
#undef ICSDK_RMS
    } else {
        // one block per row: the grid's x dimension holds at most 2^32 - 1
        if (rows > 0xffffffffu) return hipErrorInvalidValue;
        hipLaunchKernelGGL((rms_norm_stream_kernel<S, kResidual>), dim3((unsigned)rows),
                           dim3(kBlock), 0, s, x, residual, sum_out, w, y, rows, width, eps);
    }
    return hipGetLastError();
}

template <typename S>
hipError_t launch_layer(const S *x, const S *scale, const S *bias, S *y, size_t rows,
                        size_t width, float eps, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    RowShape shape;
    const bool aligned = aligned16(x) && aligned16(scale) && aligned16(bias) && aligned16(y);
    if (pick_row_shape(width, sizeof(S), aligned, &shape)) {
        const bool exact = width / (16 / sizeof(S)) == (size_t)shape.nv * shape.wpr * kWave;
        const int affine = (scale ? 1 : 0) + (bias ? 2 : 0);
#define ICSDK_LN_GO(NV, WPR, EX, SC, BI)                                                    \
    hipLaunchKernelGGL((layer_norm_kernel<S, NV, WPR, EX, SC, BI>), row_grid(rows, WPR),     \
                       dim3(kBlock), 0, s, x, scale, bias, y, rows, (uint32_t)width, eps)
#define ICSDK_LN_AFF(NV, WPR, EX)                                                           \
    do {                                                                                    \
        switch (affine) {                                                                   \
            case 0: ICSDK_LN_GO(NV, WPR, EX, false, false); break;                          \
            case 1: ICSDK_LN_GO(NV, WPR, EX, true, false); break;                           \
            case 2: ICSDK_LN_GO(NV, WPR, EX, false, true); break;                           \
            default: ICSDK_LN_GO(NV, WPR, EX, true, true); break;                           \
        }                                                                                   \
    } while (0)
#define ICSDK_LN(NV, WPR)                                                                   \
    do {                                                                                    \
        if (exact) ICSDK_LN_AFF(NV, WPR, true);                                             \
        else ICSDK_LN_AFF(NV, WPR, false);                                                  \
    } while (0)
        ICSDK_ROW_DISPATCH(shape, ICSDK_LN);
#undef ICSDK_LN
#undef ICSDK_LN_AFF
#undef ICSDK_LN_GO
    } else {
        // one block per row: the grid's x dimension holds at most 2^32 - 1
        if (rows > 0xffffffffu) return hipErrorInvalidValue;
        hipLaunchKernelGGL((layer_norm_stream_kernel<S>), dim3((unsigned)rows), dim3(kBlock),
                           0, s, x, scale, bias, y, rows, width, eps);
    }
    return hipGetLastError();
}

template <typename S>
hipError_t launch_softmax(const S *x, S *y, size_t rows, size_t width, size_t q_len,
                          hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const size_t offset = q_len && width > q_len ? width - q_len : 0;
    RowShape shape;
    const bool aligned = aligned16(x) && aligned16(y);
    if (q_len <= 0xffffffffu && pick_row_shape(width, sizeof(S), aligned, &shape)) {
        const FastDiv qd = make_fast_div(q_len ? (uint32_t)q_len : 1u);
#define ICSDK_SM(NV, WPR)                                                                  \
    hipLaunchKernelGGL((softmax_kernel<S, NV, WPR>), row_grid(rows, WPR), dim3(kBlock), 0, \
                       s, x, y, rows, (uint32_t)width, (uint32_t)q_len, qd.multiplier,      \
                       qd.shift, (uint32_t)offset)
        ICSDK_ROW_DISPATCH(shape, ICSDK_SM);
#undef ICSDK_SM
    } else {
        // one block per row: the grid's x dimension holds at most 2^32 - 1
        if (rows > 0xffffffffu) return hipErrorInvalidValue;
        hipLaunchKernelGGL((softmax_stream_kernel<S>), dim3((unsigned)rows), dim3(kBlock), 0,
                           s, x, y, rows, width, q_len, offset);
    }
    return hipGetLastError();
}

template <typename S, bool kMax>
hipError_t launch_row_reduce(const S *x, float *y, size_t rows, size_t width,
                             hipStream_t s) {
    if (rows == 0) return hipSuccess;
    RowShape shape;
    if (pick_row_shape(width, sizeof(S), aligned16(x), &shape)) {
#define ICSDK_RR(NV, WPR)                                                                  \
    hipLaunchKernelGGL((row_reduce_kernel<S, NV, WPR, kMax>), row_grid(rows, WPR),         \
                       dim3(kBlock), 0, s, x, y, rows, (uint32_t)width)
        ICSDK_ROW_DISPATCH(shape, ICSDK_RR);
#undef ICSDK_RR
    } else {
        // one block per row: the grid's x dimension holds at most 2^32 - 1
        if (rows > 0xffffffffu) return hipErrorInvalidValue;
        hipLaunchKernelGGL((row_reduce_stream_kernel<S, kMax>), dim3((unsigned)rows),
                           dim3(kBlock), 0, s, x, y, rows, width);
    }
    return hipGetLastError();
}

inline const _Float16 *h(const uint16_t *p) { return reinterpret_cast<const _Float16 *>(p); }
inline _Float16 *h(uint16_t *p) { return reinterpret_cast<_Float16 *>(p); }

}  // namespace

namespace k {

hipError_t rms_norm_f32(const float *x, const float *w, float *y, size_t rows,
                        size_t width, float eps, hipStream_t s) {
    return launch_rms<float, false>(x, nullptr, nullptr, w, y, rows, width, eps, s);
}

hipError_t rms_norm_f16(const uint16_t *x, const uint16_t *residual, uint16_t *sum_out,
                        const uint16_t *w, uint16_t *y, size_t rows, size_t width,
                        float eps, hipStream_t s) {
    if (residual)
        return launch_rms<_Float16, true>(h(x), h(residual), h(sum_out), h(w), h(y), rows,
                                          width, eps, s);
    return launch_rms<_Float16, false>(h(x), nullptr, nullptr, h(w), h(y), rows, width,
                                       eps, s);
}

hipError_t layer_norm_f32(const float *x, const float *scale, const float *bias, float *y,
                          size_t rows, size_t width, float eps, hipStream_t s) {
    return launch_layer<float>(x, scale, bias, y, rows, width, eps, s);
}

hipError_t layer_norm_f16(const uint16_t *x, const uint16_t *scale, const uint16_t *bias,
                          uint16_t *y, size_t rows, size_t width, float eps, hipStream_t s) {
    return launch_layer<_Float16>(h(x), h(scale), h(bias), h(y), rows, width, eps, s);
}

hipError_t softmax_f32(const float *x, float *y, size_t rows, size_t width, size_t q_len,
                       hipStream_t s) {
    return launch_softmax<float>(x, y, rows, width, q_len, s);
}

hipError_t softmax_f16(const uint16_t *x, uint16_t *y, size_t rows, size_t width,
                       size_t q_len, hipStream_t s) {
    return launch_softmax<_Float16>(h(x), h(y), rows, width, q_len, s);
}

hipError_t row_sum_f32(const float *x, float *y, size_t rows, size_t width, hipStream_t s) {
    return launch_row_reduce<float, false>(x, y, rows, width, s);
}
hipError_t row_sum_f16(const uint16_t *x, float *y, size_t rows, size_t width,
                       hipStream_t s) {
    return launch_row_reduce<_Float16, false>(h(x), y, rows, width, s);
}
hipError_t row_max_f32(const float *x, float *y, size_t rows, size_t width, hipStream_t s) {
    return launch_row_reduce<float, true>(x, y, rows, width, s);
}
hipError_t row_max_f16(const uint16_t *x, float *y, size_t rows, size_t width,
                       hipStream_t s) {
    return launch_row_reduce<_Float16, true>(h(x), y, rows, width, s);
}

}  // namespace k
}  // namespace icsdk
