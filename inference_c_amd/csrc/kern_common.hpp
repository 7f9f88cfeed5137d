// Device-side building blocks shared by the gfx950 kernels.
//
// Everything here is written for CDNA4 wave64: 16-byte (dwordx4) vector
// accesses, DPP row/broadcast patterns for wave reductions, and the hardware
// transcendental instructions for the f16-output fast paths.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace icsdk {

constexpr int kWave = 64;
constexpr int kBlock = 256;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---- element types -------------------------------------------------------

// Storage type -> arithmetic in f32. f16 uses the hardware conversions
// (v_cvt_f32_f16 exact widening, v_cvt_f16_f32 round-to-nearest-even with
// subnormals, overflow to infinity).
template <typename T> struct Elem;
template <> struct Elem<float> {
    static constexpr int kPerVec = 4;
    __device__ static inline float load(float v) { return v; }
    __device__ static inline float store(float v) { return v; }
};
template <> struct Elem<_Float16> {
    static constexpr int kPerVec = 8;
    __device__ static inline float load(_Float16 v) { return (float)v; }
    __device__ static inline _Float16 store(float v) { return (_Float16)v; }
};

// 16-byte vector of T with lane access.
template <typename T> struct Vec16 {
    static constexpr int N = 16 / sizeof(T);
    T v[N];
};

template <typename T>
__device__ inline Vec16<T> load16(const T *p) {
    u32x4 raw = *reinterpret_cast<const u32x4 *>(p);
    return __builtin_bit_cast(Vec16<T>, raw);
}

template <typename T>
__device__ inline Vec16<T> load16_stream(const T *p) {
    u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return __builtin_bit_cast(Vec16<T>, raw);
}

template <typename T>
__device__ inline void store16(T *p, const Vec16<T> &value) {
    *reinterpret_cast<u32x4 *>(p) = __builtin_bit_cast(u32x4, value);
}

template <typename T>
__device__ inline void store16_stream(T *p, const Vec16<T> &value) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, value),
                                reinterpret_cast<u32x4 *>(p));
}

// ---- write-through stores (buffer_store_dwordx4 ... sc1) -----------------

// Word 3 of a raw (untyped) buffer resource on gfx9-family parts:
// DATA_FORMAT = 32-bit, everything else zero.
constexpr int kRawBufferWord3 = 0x00020000;
// Cache policy of a store with device scope (SC1): the line is written
// through this XCD's L2 towards memory instead of being left dirty in it.
constexpr int kPolicyDeviceScope = 16;
// Cache policy of a streaming load (NT), as __builtin_nontemporal_load gives
// a global load: the line is not kept for reuse.
constexpr int kPolicyStream = 2;

// A window of at most 4 GiB of output, addressed by 32-bit byte offsets from
// a base that is the same for every lane of the wave (a kernel argument plus
// block-uniform terms: the descriptor lives in scalar registers). Stores at
// or past `range` bytes are dropped by the hardware's range check.
//
// Used for outputs that the kernel never reads back: on MI355X a gather or a
// row kernel whose stores write through L2 finishes sooner than the same
// kernel with non-temporal stores, which leave dirty lines for the
// end-of-kernel writeback.
struct OutWindow {
    __amdgpu_buffer_rsrc_t rsrc;
    __device__ OutWindow(void *uniform_base, uint32_t range)
        : rsrc(__builtin_amdgcn_make_buffer_rsrc(uniform_base, 0, (int)range, kRawBufferWord3)) {}

    template <typename T>
    __device__ inline void store16(uint32_t byte_offset, const Vec16<T> &value) const {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, value), rsrc,
                                               (int)byte_offset, 0, kPolicyDeviceScope);
    }
};

// Which store a streaming kernel uses for an output of `bytes` bytes. Measured
// on MI355X with a three-stream f32 add: writing through L2 is 1-5% faster up
// to 64 MiB of output and ~1.5% slower from 128 MiB, where non-temporal stores
// win.
constexpr size_t kWriteThroughMaxBytes = size_t{96} << 20;
inline bool write_through_for(size_t bytes) { return bytes <= kWriteThroughMaxBytes; }

// Stores one 16-byte vector of a block's contiguous output span: element
// `block_first + threadIdx.x * N` of `y`, where block_first is block-uniform.
template <bool kThrough, typename T>
__device__ inline void store_block_vec(T *y, size_t block_first, const Vec16<T> &value) {
    if constexpr (kThrough) {
        const OutWindow w(y + block_first, kBlock * 16u);
        w.store16(threadIdx.x * 16u, value);
    } else {
        store16_stream(y + block_first + (size_t)threadIdx.x * Vec16<T>::N, value);
    }
}

// ---- fast math for f16-output paths ---------------------------------------

// e^x through v_exp_f32 (2^x). The product x*log2(e) is rounded once, so the
// relative error grows like |x| * 2^-24; for f16 outputs (2^-11 ulp) this is
// invisible except at rounding ties.
__device__ inline float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// 1/x through v_rcp_f32 (1 ulp).
__device__ inline float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ---- wave64 reductions (DPP) --------------------------------------------

template <int kCtrl, int kRowMask = 0xf>
__device__ inline float dpp_f32(float old_value, float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old_value),
                                           __builtin_bit_cast(int, v), kCtrl,
                                           kRowMask, 0xf, false));
}

template <int kCtrl, int kRowMask = 0xf>
__device__ inline int dpp_i32(int old_value, int v) {
    return __builtin_amdgcn_update_dpp(old_value, v, kCtrl, kRowMask, 0xf, false);
}

// DPP controls (GFX9 encoding).
constexpr int kQuadSwap1 = 0xb1;     // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4e;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowBcast15 = 0x142;   // lane 15 of row r -> row r+1
constexpr int kRowBcast31 = 0x143;   // lane 31 -> rows 2 and 3

// Sum over the 64 lanes; every lane receives the total. The first four steps
// reduce within 16-lane rows (all lanes valid), the broadcasts fold rows into
// lane 63, which is then read as a scalar.
__device__ inline float wave_sum(float v) {
    v += dpp_f32<kQuadSwap1>(0.0f, v);
    v += dpp_f32<kQuadSwap2>(0.0f, v);
    v += dpp_f32<kRowHalfMirror>(0.0f, v);
    v += dpp_f32<kRowMirror>(0.0f, v);
    v += dpp_f32<kRowBcast15, 0xa>(0.0f, v);
    v += dpp_f32<kRowBcast31, 0xc>(0.0f, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ inline int wave_sum_i32(int v) {
    v += dpp_i32<kQuadSwap1>(0, v);
    v += dpp_i32<kQuadSwap2>(0, v);
    v += dpp_i32<kRowHalfMirror>(0, v);
    v += dpp_i32<kRowMirror>(0, v);
    v += dpp_i32<kRowBcast15, 0xa>(0, v);
    v += dpp_i32<kRowBcast31, 0xc>(0, v);
    return __builtin_amdgcn_readlane(v, 63);
}

// Max over the 64 lanes (fmaxf semantics: a NaN operand is ignored).
__device__ inline float wave_max(float v) {
    const float lowest = -__builtin_inff();
    v = fmaxf(v, dpp_f32<kQuadSwap1>(lowest, v));
    v = fmaxf(v, dpp_f32<kQuadSwap2>(lowest, v));
    v = fmaxf(v, dpp_f32<kRowHalfMirror>(lowest, v));
    v = fmaxf(v, dpp_f32<kRowMirror>(lowest, v));
    v = fmaxf(v, dpp_f32<kRowBcast15, 0xa>(lowest, v));
    v = fmaxf(v, dpp_f32<kRowBcast31, 0xc>(lowest, v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Double-precision sum over the wave, the same DPP steps as wave_sum with
// each double moved as its two 32-bit halves (a lane outside the row mask
// receives 0.0: both halves 0).
template <int kCtrl, int kRowMask = 0xf>
__device__ inline double dpp_f64(double v) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)bits, kCtrl,
                                                              kRowMask, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(bits >> 32), kCtrl,
                                                              kRowMask, 0xf, false);
    return __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
}

__device__ inline double wave_sum_f64(double v) {
    v += dpp_f64<kQuadSwap1>(v);
    v += dpp_f64<kQuadSwap2>(v);
    v += dpp_f64<kRowHalfMirror>(v);
    v += dpp_f64<kRowMirror>(v);
    v += dpp_f64<kRowBcast15, 0xa>(v);
    v += dpp_f64<kRowBcast31, 0xc>(v);
    const uint64_t bits = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)bits, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(bits >> 32), 63);
    return __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
}

__device__ inline bool wave_any(bool flag) {
    return __builtin_amdgcn_ballot_w64(flag) != 0;
}

// ---- integer division by a run-time constant -----------------------------

// q = n / d for 32-bit n via a precomputed multiplier (Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, the
// round-up variant with a 33-bit multiplier folded as t + n).
struct FastDiv {
    uint32_t divisor;
    uint32_t multiplier;
    uint32_t shift;
};

__host__ inline FastDiv make_fast_div(uint32_t d) {
    FastDiv f{d, 0, 0};
    uint32_t s = 0;
    while ((uint64_t{1} << s) < d) s++;
    f.shift = s;
    f.multiplier = (uint32_t)(((uint64_t{1} << 32) * ((uint64_t{1} << s) - d)) / d + 1);
    return f;
}

__device__ inline uint32_t fast_div(uint32_t n, const FastDiv &f) {
    const uint32_t t = __umulhi(n, f.multiplier);
    return (uint32_t)(((uint64_t)t + n) >> f.shift);
}

}  // namespace icsdk
