// Row gather (embedding lookup) for gfx950:
//     out[i, :] = table[ids[i], :]
// with ids of any of the reference's index types (int16, uint16, int32,
// uint32, int64, uint64). Rows are moved as bytes, so one kernel serves every
// element type.
//
// check  - one 1024-lane block scans the ids (16-byte vectors, several in
//          flight per lane) and writes 1 to `flag` (pinned host memory)
//          and to `skip` (device memory) when any is negative or at/past
//          the table's row count, else 0; one block needs no atomics and no
//          pre-cleared words. The public entry points enqueue the gather
//          right behind it with `skip`, so a rejected call writes no row,
//          and wait only for the check before reading `flag`;
// gather - rows that are whole 16-byte vectors (and aligned): one output
//          vector per lane on a one-shot grid; the lane's row and column
//          come from a multiply-high division, its id from the (cached) id
//          vector, and the table vector is an ordinary cached load, since a
//          token repeated in a batch re-reads its row. An id outside the
//          table yields a zero row (the compute-table slot's semantics);
// scalar - other row widths: one element (2 or 4 bytes) per lane.
#include "kern_common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace icsdk {
namespace {

template <typename I>
__device__ inline bool index_ok(I value, uint64_t rows, uint64_t *id) {
    if constexpr (std::is_signed<I>::value) {
        if (value < 0) return false;
    }
    *id = (uint64_t)value;
    return *id < rows;
}

constexpr int kCheckBlock = 1024;
constexpr int kCheckUnroll = 4;  // 16-byte vectors in flight per lane

// One block scans all ids: each lane keeps kCheckUnroll 16-byte vectors of
// ids in flight per step (a 1024-lane block covers 64 KiB per step), then a
// scalar tail; the verdict is written by lane 0 to `flag` (a word of pinned
// host memory) and to the device word `skip`.
template <typename I>
__global__ __launch_bounds__(kCheckBlock) void embedding_check_kernel(const I *__restrict__ ids,
                                                                      size_t count, uint64_t rows,
                                                                      uint32_t *__restrict__ flag,
                                                                      uint32_t *__restrict__ skip) {
    constexpr int kPer = 16 / sizeof(I);
    // vector part only for a 16-byte aligned id buffer; otherwise all scalar
    const size_t nvec = ((uintptr_t)ids & 15u) ? 0 : count / kPer;
    const u32x4 *vecs = reinterpret_cast<const u32x4 *>(ids);
    int bad = 0;
    for (size_t base = 0; base < nvec; base += (size_t)kCheckBlock * kCheckUnroll) {
        u32x4 raw[kCheckUnroll];
#pragma unroll
        for (int u = 0; u < kCheckUnroll; ++u) {
            const size_t v = base + threadIdx.x + (size_t)u * kCheckBlock;
            raw[u] = v < nvec ? vecs[v] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kCheckUnroll; ++u) {
            const Vec16<I> ids_vec = __builtin_bit_cast(Vec16<I>, raw[u]);
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                uint64_t id;
                bad |= !index_ok(ids_vec.v[e], rows, &id);
            }
        }
    }
    for (size_t i = nvec * kPer + threadIdx.x; i < count; i += kCheckBlock) {
        uint64_t id;
        bad |= !index_ok(ids[i], rows, &id);
    }
    bad = __syncthreads_or(bad);
    // system scope: visible to the host once it has waited for this kernel;
    // the device word is read by the gather that follows on the stream
    if (threadIdx.x == 0) {
        __hip_atomic_store(flag, bad ? 1u : 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        *skip = bad ? 1u : 0u;
    }
}

template <typename I, bool kThrough>
__global__ __launch_bounds__(kBlock) void embedding_gather_kernel(const u32x4 *__restrict__ table,
                                                                  const I *__restrict__ ids,
                                                                  uint32_t *__restrict__ out,
                                                                  uint32_t nvec, FastDiv vpr,
                                                                  uint64_t rows,
                                                                  const uint32_t *__restrict__ skip) {
    if (skip != nullptr && *skip != 0) return;   // the check rejected the call
    const uint32_t first = blockIdx.x * kBlock;
    const uint32_t v = first + threadIdx.x;
    if (v >= nvec) return;
    const uint32_t row = fast_div(v, vpr);
    const uint32_t col = v - row * vpr.divisor;
    uint64_t id = 0;
    const bool ok = index_ok(ids[row], rows, &id);
    u32x4 value = table[(ok ? id : 0) * vpr.divisor + col];
    if (!ok) value = u32x4{0u, 0u, 0u, 0u};
    store_block_vec<kThrough>(out, (size_t)first * 4, __builtin_bit_cast(Vec16<uint32_t>, value));
}

template <typename I, typename E>
__global__ __launch_bounds__(kBlock) void embedding_gather_scalar_kernel(
    const E *__restrict__ table, const I *__restrict__ ids, E *__restrict__ out, size_t n,
    size_t width, uint64_t rows, const uint32_t *__restrict__ skip) {
    if (skip != nullptr && *skip != 0) return;   // the check rejected the call
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        const size_t row = i / width, col = i - row * width;
        uint64_t id = 0;
        const bool ok = index_ok(ids[row], rows, &id);
        out[i] = ok ? table[id * width + col] : E(0);
    }
}

template <typename I>
hipError_t launch_check(const void *ids, size_t count, uint64_t rows, uint32_t *flag,
                        uint32_t *skip, hipStream_t s) {
    hipLaunchKernelGGL((embedding_check_kernel<I>), dim3(1), dim3(kCheckBlock), 0, s,
                       static_cast<const I *>(ids), count, rows, flag, skip);
    return hipGetLastError();
}

template <typename I>
hipError_t launch_gather(const void *table, uint64_t rows, size_t row_bytes, size_t elem_bytes,
                         const void *ids, size_t count, void *out, const uint32_t *skip,
                         hipStream_t s) {
    const size_t out_bytes = count * row_bytes;
    const bool aligned = (((uintptr_t)table | (uintptr_t)out) & 15u) == 0;
    if (row_bytes % 16 == 0 && aligned && out_bytes / 16 < (size_t{1} << 32)) {
        const uint32_t nvec = (uint32_t)(out_bytes / 16);
        const FastDiv vpr = make_fast_div((uint32_t)(row_bytes / 16));
        const dim3 grid((nvec + kBlock - 1) / kBlock), block(kBlock);
        if (write_through_for(out_bytes))
            hipLaunchKernelGGL((embedding_gather_kernel<I, true>), grid, block, 0, s,
                               static_cast<const u32x4 *>(table), static_cast<const I *>(ids),
                               static_cast<uint32_t *>(out), nvec, vpr, rows, skip);
        else
            hipLaunchKernelGGL((embedding_gather_kernel<I, false>), grid, block, 0, s,
                               static_cast<const u32x4 *>(table), static_cast<const I *>(ids),
                               static_cast<uint32_t *>(out), nvec, vpr, rows, skip);
        return hipGetLastError();
    }
    const size_t width = row_bytes / elem_bytes, n = count * width;
    size_t grid = (n + kBlock - 1) / kBlock;
    if (grid > (size_t{1} << 20)) grid = size_t{1} << 20;
    if (elem_bytes == 4)
        hipLaunchKernelGGL((embedding_gather_scalar_kernel<I, uint32_t>), dim3((unsigned)grid),
                           dim3(kBlock), 0, s, static_cast<const uint32_t *>(table),
                           static_cast<const I *>(ids), static_cast<uint32_t *>(out), n, width,
                           rows, skip);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL((embedding_gather_scalar_kernel<I, uint16_t>), dim3((unsigned)grid),
                           dim3(kBlock), 0, s, static_cast<const uint16_t *>(table),
                           static_cast<const I *>(ids), static_cast<uint16_t *>(out), n, width,
                           rows, skip);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// Expands CALL(I) for the index type of `dtype`.
#define ICSDK_WITH_INDEX_TYPE(dtype, CALL)                      \
    switch (dtype) {                                            \
        case TENSOR_DTYPE_I16: return CALL(int16_t);            \
        case TENSOR_DTYPE_U16: return CALL(uint16_t);           \
        case TENSOR_DTYPE_I32: return CALL(int32_t);            \
        case TENSOR_DTYPE_U32: return CALL(uint32_t);           \
        case TENSOR_DTYPE_I64: return CALL(int64_t);            \
        case TENSOR_DTYPE_U64: return CALL(uint64_t);           \
        default: return hipErrorInvalidValue;                   \
    }

}  // namespace

namespace k {

bool embedding_index_type(TensorDType dtype) {
    return dtype == TENSOR_DTYPE_I16 || dtype == TENSOR_DTYPE_U16 ||
           dtype == TENSOR_DTYPE_I32 || dtype == TENSOR_DTYPE_U32 ||
           dtype == TENSOR_DTYPE_I64 || dtype == TENSOR_DTYPE_U64;
}

hipError_t embedding_check(TensorDType index_dtype, const void *ids, size_t count,
                           uint64_t table_rows, uint32_t *flag, uint32_t *skip, hipStream_t s) {
#define ICSDK_CHECK(I) launch_check<I>(ids, count, table_rows, flag, skip, s)
    ICSDK_WITH_INDEX_TYPE(index_dtype, ICSDK_CHECK)
#undef ICSDK_CHECK
}

hipError_t embedding_gather(TensorDType index_dtype, const void *table, uint64_t table_rows,
                            size_t row_bytes, size_t elem_bytes, const void *ids, size_t count,
                            void *out, const uint32_t *skip, hipStream_t s) {
    if (count == 0 || row_bytes == 0) return hipSuccess;
#define ICSDK_GATHER(I) \
    launch_gather<I>(table, table_rows, row_bytes, elem_bytes, ids, count, out, skip, s)
    ICSDK_WITH_INDEX_TYPE(index_dtype, ICSDK_GATHER)
#undef ICSDK_GATHER
}

}  // namespace k
}  // namespace icsdk
