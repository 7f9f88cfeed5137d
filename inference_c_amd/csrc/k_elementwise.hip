// Elementwise and row-broadcast kernels for gfx950.
//
// Design: one kernel template per arity. Each lane moves one 16-byte vector
// per operand (global_load_dwordx4 / global_store_dwordx4 with the
// non-temporal hint: every byte is streamed once), on a one-shot grid that
// covers the tensor. The op is a functor on f32 values; f16 inputs are
// widened exactly and outputs rounded to nearest even by the hardware
// conversions.
//
// Math per op (reference semantics cited in the public headers):
//   add / mul             one IEEE op (bit-exact against the CPU reference);
//   silu (f32)            v / (1 + expf(-v)), IEEE divide;
//   silu (f16 output)     v * rcp(1 + exp2(-v log2 e));
//   gelu                  x >= 5 -> x, x <= -5 -> 0, else the reference's
//                         0.5 x (1 + tanh(u)) evaluated as x / (1 + e^(-2u)),
//                         the same function without the cancellation of
//                         1 + tanh(u) for u << 0, u = 0.7978845608 (x + 0.044715 x^3);
//                         f16 outputs form the exponent as one f32 polynomial
//                         and use v_exp_f32 / v_rcp_f32, f32 outputs form u in
//                         double.
#include "kern_common.hpp"
#include "kernels.hpp"

namespace icsdk {
namespace {

// ---- op functors ---------------------------------------------------------

// f32-output path: u in double, then e^(-2u) from a hi/lo split of -2u
// (e^(hi+lo) = e^hi * (1 + lo) to f32 accuracy), so the result is a few f32
// ulps from the exact formula; rounding u itself to f32 would already cost
// ~1e-6 relative where x/(1+e^(-2u)) is steep (x around -3.5).
__device__ inline float gelu_sigmoid_precise(float v) {
    const double vd = v;
    const double u = (double)0.7978845608f * (vd + (double)0.044715f * vd * vd * vd);
    const double t = -2.0 * u;
    const float hi = (float)t;
    const float lo = (float)(t - (double)hi);
    const float e = expf(hi) * (1.0f + lo);
    return v / (1.0f + e);
}

// f16-output path: the exponent -2u log2(e) as one polynomial,
// t = v (c1 + c2 v^2) with c1 = -2 log2(e) 0.7978845608 and c2 = 0.044715 c1,
// three VALU ops instead of seven (the kernel is VALU-bound at this op
// count). t is within a few f32 ulps of the reference's exponent, so the
// result moves by < 1e-5 relative, far inside half an f16 ulp (2.4e-4). The
// x >= 5 clamp is implied here: there exp2(t) < 2^-24, 1 + exp2(t) rounds to
// 1 and the result is x exactly (also for +inf); the x <= -5 clamp stays,
// for the f16 subnormal results it forces to zero and for -inf.
constexpr float kGeluC1 = (float)(-2.0 * 1.4426950408889634 * (double)0.7978845608f);
constexpr float kGeluC2 = (float)((double)kGeluC1 * (double)0.044715f);

template <bool kFast>
__device__ inline float gelu(float v) {
    if constexpr (kFast) {
        // The two products as fmas with a zero addend (equal to the plain
        // products but for the sign of an exact zero, which exp2 ignores):
        // each then reads an f16 input straight from its packed register
        // (v_fma_mix_f32), with no separate conversion to f32.
        const float v2 = __builtin_fmaf(v, v, 0.0f);
        const float t = __builtin_fmaf(v, __builtin_fmaf(kGeluC2, v2, kGeluC1), 0.0f);
        const float r = v * fast_rcp(1.0f + __builtin_amdgcn_exp2f(t));
        return v <= -5.0f ? 0.0f : r;
    } else {
        float r = gelu_sigmoid_precise(v);
        r = v >= 5.0f ? v : r;
        return v <= -5.0f ? 0.0f : r;
    }
}

template <bool kFast>
__device__ inline float silu(float v) {
    // -v log2(e) as an fma with a zero addend: v_fma_mix_f32 reads the f16
    // input directly (same value as the product; exp2 ignores a zero's sign)
    if constexpr (kFast)
        return v * fast_rcp(1.0f + __builtin_amdgcn_exp2f(
                                       __builtin_fmaf(v, -1.4426950408889634f, 0.0f)));
    else return v / (1.0f + expf(-v));
}

template <k::Unary kOp, bool kFast> struct UnaryOp {
    __device__ inline float operator()(float a, float) const {
        if constexpr (kOp == k::Unary::Silu) return silu<kFast>(a);
        else if constexpr (kOp == k::Unary::Gelu) return gelu<kFast>(a);
        else if constexpr (kOp == k::Unary::Relu) return a > 0.0f ? a : 0.0f;
        else return a;
    }
};

template <k::Binary kOp, bool kFast> struct BinaryOp {
    __device__ inline float operator()(float a, float b) const {
        if constexpr (kOp == k::Binary::Add) return a + b;
        else if constexpr (kOp == k::Binary::Mul) return a * b;
        else if constexpr (kOp == k::Binary::SiluMul) return silu<kFast>(a) * b;
        else return gelu<kFast>(a) * b;
    }
};

// ---- same-shape map ------------------------------------------------------

template <typename S, int kArity, class Op>
__device__ inline Vec16<S> apply(const Vec16<S> &a, const Vec16<S> &b, Op op) {
    Vec16<S> out;
#pragma unroll
    for (int e = 0; e < Vec16<S>::N; ++e) {
        const float x = Elem<S>::load(a.v[e]);
        const float y = kArity == 2 ? Elem<S>::load(b.v[e]) : 0.0f;
        out.v[e] = Elem<S>::store(op(x, y));
    }
    return out;
}

// One 16-byte vector per lane and a one-shot grid (one wave per KiB per
// operand). Measured on MI355X this streams at the device's practical
// ceiling (~6.4 TB/s for 128 MiB operands); deeper per-lane unrolling and
// persistent grid-stride loops were 5-20% slower, and cached (temporal)
// loads ~40% slower. A launch covers at most kMaxLaunchVecs vectors (a
// dispatch's work-item count is 32 bits); the host splits longer operands
// into several launches. kThrough selects write-through stores (small
// outputs).
template <typename S, int kArity, class Op, bool kThrough>
__global__ __launch_bounds__(kBlock) void map_vec_kernel(const S *__restrict__ a,
                                                         const S *__restrict__ b,
                                                         S *__restrict__ y, size_t nvec,
                                                         size_t n, Op op) {
    constexpr int E = Vec16<S>::N;
    // One-shot grid (the host covers nvec with one vector per lane): no
    // grid-stride loop, whose stride -- the grid size, a hidden argument --
    // was one more scalar-load round trip before the first vector load.
    const size_t first = (size_t)blockIdx.x * kBlock;
    const size_t i = first + threadIdx.x;
    if (i < nvec) {
        const Vec16<S> va = load16_stream(a + i * E);
        Vec16<S> vb{};
        if constexpr (kArity == 2) vb = load16_stream(b + i * E);
        store_block_vec<kThrough>(y, first * E, apply<S, kArity>(va, vb, op));
    }
    // ragged tail (fewer than one vector)
    if (blockIdx.x == 0 && threadIdx.x < n - nvec * E) {
        const size_t t = nvec * E + threadIdx.x;
        const float x = Elem<S>::load(a[t]);
        const float z = kArity == 2 ? Elem<S>::load(b[t]) : 0.0f;
        y[t] = Elem<S>::store(op(x, z));
    }
}

// Element-at-a-time variant for operands that are not 16-byte aligned.
template <typename S, int kArity, class Op>
__global__ __launch_bounds__(kBlock) void map_scalar_kernel(const S *__restrict__ a,
                                                            const S *__restrict__ b,
                                                            S *__restrict__ y, size_t n,
                                                            Op op) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        const float x = Elem<S>::load(a[i]);
        const float z = kArity == 2 ? Elem<S>::load(b[i]) : 0.0f;
        y[i] = Elem<S>::store(op(x, z));
    }
}

inline bool aligned16(const void *p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Blocks for a grid-stride kernel: one lane per work item, capped so that
// blocks * per_block work-items fit the dispatch's 32-bit count (the kernels
// loop over the rest).
unsigned grid_for(size_t work_items, size_t per_block) {
    size_t blocks = (work_items + per_block - 1) / per_block;
    if (blocks < 1) blocks = 1;
    const size_t cap = size_t{0xffffffff} / per_block;
    if (blocks > cap) blocks = cap;
    return (unsigned)blocks;
}

// Vectors per map_vec_kernel launch: a multiple of kBlock, with the work-item
// count (blocks * kBlock) below 2^32.
constexpr size_t kMaxLaunchVecs = size_t{1} << 31;

template <typename S, int kArity, class Op>
hipError_t launch_map(const S *a, const S *b, S *y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    constexpr int E = Vec16<S>::N;
    if (aligned16(a) && aligned16(b) && aligned16(y)) {
        const size_t nvec = n / E;
        const bool through = write_through_for(n * sizeof(S));
        // each launch covers its part of nvec in one pass of the grid; the
        // last one also takes the ragged tail of fewer than E elements
        size_t done = 0;
        do {
            const size_t part = nvec - done > kMaxLaunchVecs ? kMaxLaunchVecs : nvec - done;
            const bool last = done + part == nvec;
            const size_t part_n = last ? n - done * E : part * E;
            const S *pa = a + done * E;
            const S *pb = b == nullptr ? nullptr : b + done * E;
            S *py = y + done * E;
            const unsigned grid = (unsigned)((part > 0 ? part + kBlock - 1 : kBlock) / kBlock);
            if (through)
                hipLaunchKernelGGL((map_vec_kernel<S, kArity, Op, true>), dim3(grid), dim3(kBlock),
                                   0, s, pa, pb, py, part, part_n, Op{});
            else
                hipLaunchKernelGGL((map_vec_kernel<S, kArity, Op, false>), dim3(grid),
                                   dim3(kBlock), 0, s, pa, pb, py, part, part_n, Op{});
            done += part;
        } while (done < nvec);
    } else {
        hipLaunchKernelGGL((map_scalar_kernel<S, kArity, Op>), dim3(grid_for(n, kBlock)),
                           dim3(kBlock), 0, s, a, b, y, n, Op{});
    }
    return hipGetLastError();
}

template <typename S, bool kFast>
hipError_t unary_dispatch(k::Unary op, const S *x, S *y, size_t n, hipStream_t s) {
    switch (op) {
        case k::Unary::Silu: return launch_map<S, 1, UnaryOp<k::Unary::Silu, kFast>>(x, nullptr, y, n, s);
        case k::Unary::Gelu: return launch_map<S, 1, UnaryOp<k::Unary::Gelu, kFast>>(x, nullptr, y, n, s);
        case k::Unary::Relu: return launch_map<S, 1, UnaryOp<k::Unary::Relu, kFast>>(x, nullptr, y, n, s);
        case k::Unary::Copy: return launch_map<S, 1, UnaryOp<k::Unary::Copy, kFast>>(x, nullptr, y, n, s);
    }
    return hipErrorInvalidValue;
}

template <typename S, bool kFast>
hipError_t binary_dispatch(k::Binary op, const S *a, const S *b, S *y, size_t n,
                           hipStream_t s) {
    switch (op) {
        case k::Binary::Add: return launch_map<S, 2, BinaryOp<k::Binary::Add, kFast>>(a, b, y, n, s);
        case k::Binary::Mul: return launch_map<S, 2, BinaryOp<k::Binary::Mul, kFast>>(a, b, y, n, s);
        case k::Binary::SiluMul: return launch_map<S, 2, BinaryOp<k::Binary::SiluMul, kFast>>(a, b, y, n, s);
        case k::Binary::GeluMul: return launch_map<S, 2, BinaryOp<k::Binary::GeluMul, kFast>>(a, b, y, n, s);
    }
    return hipErrorInvalidValue;
}

// ---- row broadcast (bias) ----------------------------------------------

template <typename S, bool kGelu>
__device__ inline float bias_value(float x, float b) {
    const float v = x + b;
    if constexpr (kGelu) return gelu<sizeof(S) == 2>(v);
    else return v;
}

// Vector path: width % E == 0 and 16-byte aligned operands, nvec < 2^32.
// The column of vector i is i mod (width / E), computed with a multiply-high
// division; the bias vector is re-read from L1/L2 (it is width*sizeof(S) bytes).
template <typename S, bool kGelu, bool kThrough>
__global__ __launch_bounds__(kBlock) void bias_vec_kernel(const S *__restrict__ x,
                                                          const S *__restrict__ bias,
                                                          S *__restrict__ y, uint32_t nvec,
                                                          FastDiv per_row) {
    constexpr int E = Vec16<S>::N;
    // one-shot grid (nvec < 2^32 vectors, one per lane): no grid-stride loop
    // and so no round trip for the grid size before the loads
    const size_t first = (size_t)blockIdx.x * kBlock;
    if (first + threadIdx.x >= nvec) return;
    const uint32_t i = (uint32_t)(first + threadIdx.x);
    const uint32_t row = fast_div(i, per_row);
    const uint32_t col = i - row * per_row.divisor;
    const Vec16<S> vx = load16_stream(x + (size_t)i * E);
    const Vec16<S> vb = load16(bias + (size_t)col * E);
    Vec16<S> out;
#pragma unroll
    for (int e = 0; e < E; ++e)
        out.v[e] = Elem<S>::store(bias_value<S, kGelu>(Elem<S>::load(vx.v[e]),
                                                       Elem<S>::load(vb.v[e])));
    store_block_vec<kThrough>(y, first * E, out);
}

template <typename S, bool kGelu>
__global__ __launch_bounds__(kBlock) void bias_scalar_kernel(const S *__restrict__ x,
                                                             const S *__restrict__ bias,
                                                             S *__restrict__ y, size_t n,
                                                             size_t width) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        y[i] = Elem<S>::store(bias_value<S, kGelu>(Elem<S>::load(x[i]),
                                                   Elem<S>::load(bias[i % width])));
}

template <typename S, bool kGelu>
hipError_t launch_bias(const S *x, const S *bias, S *y, size_t rows, size_t width,
                       hipStream_t s) {
    const size_t n = rows * width;
    if (n == 0) return hipSuccess;
    constexpr int E = Vec16<S>::N;
    const size_t nvec = n / E;
    // the vector kernel is one-shot: its grid must cover nvec within the
    // dispatch's 32-bit work-item count; longer operands take the
    // grid-stride scalar kernel
    if (width % E == 0 && aligned16(x) && aligned16(bias) && aligned16(y) &&
        nvec <= kMaxLaunchVecs) {
        const dim3 grid(grid_for(nvec, kBlock)), block(kBlock);
        const FastDiv per_row = make_fast_div((uint32_t)(width / E));
        if (write_through_for(n * sizeof(S)))
            hipLaunchKernelGGL((bias_vec_kernel<S, kGelu, true>), grid, block, 0, s, x, bias, y,
                               (uint32_t)nvec, per_row);
        else
            hipLaunchKernelGGL((bias_vec_kernel<S, kGelu, false>), grid, block, 0, s, x, bias, y,
                               (uint32_t)nvec, per_row);
    } else {
        hipLaunchKernelGGL((bias_scalar_kernel<S, kGelu>), dim3(grid_for(n, kBlock)),
                           dim3(kBlock), 0, s, x, bias, y, n, width);
    }
    return hipGetLastError();
}

}  // namespace

namespace k {

hipError_t unary_f32(Unary op, const float *x, float *y, size_t n, hipStream_t s) {
    return unary_dispatch<float, false>(op, x, y, n, s);
}

hipError_t unary_f16(Unary op, const uint16_t *x, uint16_t *y, size_t n, hipStream_t s) {
    return unary_dispatch<_Float16, true>(op, reinterpret_cast<const _Float16 *>(x),
                                          reinterpret_cast<_Float16 *>(y), n, s);
}

hipError_t binary_f32(Binary op, const float *a, const float *b, float *y, size_t n,
                      hipStream_t s) {
    return binary_dispatch<float, false>(op, a, b, y, n, s);
}

hipError_t binary_f16(Binary op, const uint16_t *a, const uint16_t *b, uint16_t *y,
                      size_t n, hipStream_t s) {
    return binary_dispatch<_Float16, true>(op, reinterpret_cast<const _Float16 *>(a),
                                           reinterpret_cast<const _Float16 *>(b),
                                           reinterpret_cast<_Float16 *>(y), n, s);
}

hipError_t bias_add_f32(const float *x, const float *bias, float *y, size_t rows,
                        size_t width, bool gelu, hipStream_t s) {
    return gelu ? launch_bias<float, true>(x, bias, y, rows, width, s)
                : launch_bias<float, false>(x, bias, y, rows, width, s);
}

hipError_t bias_add_f16(const uint16_t *x, const uint16_t *bias, uint16_t *y,
                        size_t rows, size_t width, bool gelu, hipStream_t s) {
    const auto *hx = reinterpret_cast<const _Float16 *>(x);
    const auto *hb = reinterpret_cast<const _Float16 *>(bias);
    auto *hy = reinterpret_cast<_Float16 *>(y);
    return gelu ? launch_bias<_Float16, true>(hx, hb, hy, rows, width, s)
                : launch_bias<_Float16, false>(hx, hb, hy, rows, width, s);
}

}  // namespace k
}  // namespace icsdk
