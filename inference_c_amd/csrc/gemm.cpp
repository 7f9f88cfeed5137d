// Library GEMMs through hipBLASLt (gfx950 tensile kernels, f16 or f32 MFMA
// with f32 accumulation) for linear and matmul. The bias is fused as
// hipBLASLt's BIAS epilogue, so a biased linear is one launch and one
// rounding, as in the reference's host loop (src/common/tensor_ops.c:
// 290-307, :389-396); the reference's CUDA backend instead runs cuBLAS and
// then a separate bias kernel (tensor_compute_cuda.cu:174-214, tensor_ops.c:
// 259-268).
//
// Row-major y[rows][cols] is column-major [cols x rows], so every problem is
// posed as D[cols x rows] = op(A) * B with B = x (column-major [inner x
// rows]) and A = the weight: column-major [inner x cols] transposed for
// linear (w[cols][inner] row-major), [cols x inner] as is for matmul.
//
// One plan (descriptors + the heuristic's first algorithm) is cached per
// (kind, dtype, shape, bias); calls run under one mutex because the bias
// pointer is an attribute of the cached descriptor.
#include "gemm.hpp"
#include "kernels.hpp"

#include "sdk.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace icsdk {
namespace {

constexpr size_t kWorkspaceBytes = 32u << 20;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t workspace = 0;
};

using PlanKey = std::tuple<int, int, uint64_t, uint64_t, uint64_t, bool>;

struct GemmState {
    std::mutex mutex;
    hipblasLtHandle_t handle = nullptr;
    std::map<PlanKey, Plan> plans;
};

GemmState &gemm_state() {
    static GemmState *state = new GemmState;  // outlives static destructors
    return *state;
}

const char *status_text(hipblasStatus_t s) {
    switch (s) {
        case HIPBLAS_STATUS_SUCCESS: return "success";
        case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
        case HIPBLAS_STATUS_ALLOC_FAILED: return "allocation failed";
        case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
        case HIPBLAS_STATUS_ARCH_MISMATCH: return "architecture mismatch";
        case HIPBLAS_STATUS_MAPPING_ERROR: return "mapping error";
        case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
        case HIPBLAS_STATUS_INTERNAL_ERROR: return "internal error";
        case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
        default: return "error";
    }
}

void destroy(Plan &p) {
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
    p = Plan{};
}

// Builds the descriptors for D[m x n] = op(A) * B (+ bias[m]), k inner.
bool make_plan(hipblasLtHandle_t handle, GemmKind kind, hipDataType type, uint64_t m,
               uint64_t n, uint64_t k, bool bias, Plan *plan, char *error, size_t capacity) {
    hipblasStatus_t s = hipblasLtMatmulDescCreate(&plan->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    const hipblasOperation_t op_a = kind == GemmKind::kLinear ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    const hipblasOperation_t op_b = HIPBLAS_OP_N;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_a,
                                            sizeof op_a);
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_b,
                                            sizeof op_b);
    if (s == HIPBLAS_STATUS_SUCCESS && bias) {
        const hipblasLtEpilogue_t epilogue = HIPBLASLT_EPILOGUE_BIAS;
        const int32_t bias_type = type;
        s = hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epilogue,
                                            sizeof epilogue);
        if (s == HIPBLAS_STATUS_SUCCESS)
            s = hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE,
                                                &bias_type, sizeof bias_type);
    }
    // A: linear -> w[m][k] row-major = column-major [k x m], transposed;
    //    matmul -> w[k][m] row-major = column-major [m x k]
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = kind == GemmKind::kLinear ? hipblasLtMatrixLayoutCreate(&plan->a, type, k, m, (int64_t)k)
                                      : hipblasLtMatrixLayoutCreate(&plan->a, type, m, k, (int64_t)m);
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatrixLayoutCreate(&plan->b, type, k, n, (int64_t)k);
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatrixLayoutCreate(&plan->d, type, m, n, (int64_t)m);
    if (s != HIPBLAS_STATUS_SUCCESS) {
        set_error(error, capacity, "GEMM descriptor setup failed: %s", status_text(s));
        return false;
    }
    hipblasLtMatmulPreference_t pref = nullptr;
    s = hipblasLtMatmulPreferenceCreate(&pref);
    const uint64_t limit = kWorkspaceBytes;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                  &limit, sizeof limit);
    hipblasLtMatmulHeuristicResult_t results[8];
    int found = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulAlgoGetHeuristic(handle, plan->desc, plan->a, plan->b, plan->d,
                                            plan->d, pref, 8, results, &found);
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    for (int i = 0; s == HIPBLAS_STATUS_SUCCESS && i < found; ++i) {
        if (results[i].state == HIPBLAS_STATUS_SUCCESS && results[i].workspaceSize <= limit) {
            plan->algo = results[i].algo;
            plan->workspace = results[i].workspaceSize;
            return true;
        }
    }
    set_error(error, capacity, "no GEMM kernel for %llu x %llu x %llu: %s",
              (unsigned long long)m, (unsigned long long)n, (unsigned long long)k,
              s == HIPBLAS_STATUS_SUCCESS ? "none returned" : status_text(s));
    return false;
}

}  // namespace

#ifndef ICSDK_GEMV_LINEAR
#define ICSDK_GEMV_LINEAR 1
#endif

bool gemm(GemmKind kind, TensorDType dtype, const void *x, const void *w, const void *bias,
          void *y, size_t rows, size_t inner, size_t cols, hipStream_t stream, char *error,
          size_t capacity) {
    if (ICSDK_GEMV_LINEAR && kind == GemmKind::kLinear && rows <= k::kGemvMaxRows) {
        // decode-sized linears stream the weights through a GEMV kernel
        const hipError_t e = k::linear_gemv(dtype == TENSOR_DTYPE_F32, x, w, bias, y, rows, inner,
                                            cols, stream);
        if (e == hipSuccess) return true;
        if (e != hipErrorNotSupported) {
            set_error(error, capacity, "GEMV launch failed: %s", hipGetErrorString(e));
            return false;
        }
    }
    const hipDataType type = dtype == TENSOR_DTYPE_F32 ? HIP_R_32F : HIP_R_16F;
    GemmState &g = gemm_state();
    std::lock_guard<std::mutex> lock(g.mutex);
    if (g.handle == nullptr) {
        const hipblasStatus_t s = hipblasLtCreate(&g.handle);
        if (s != HIPBLAS_STATUS_SUCCESS) {
            g.handle = nullptr;
            set_error(error, capacity, "hipBLASLt initialisation failed: %s", status_text(s));
            return false;
        }
    }
    const PlanKey key{(int)kind, (int)dtype, cols, rows, inner, bias != nullptr};
    auto it = g.plans.find(key);
    if (it == g.plans.end()) {
        Plan plan;
        if (!make_plan(g.handle, kind, type, cols, rows, inner, bias != nullptr, &plan, error,
                       capacity)) {
            destroy(plan);
            return false;
        }
        it = g.plans.emplace(key, plan).first;
    }
    Plan &plan = it->second;
    if (bias != nullptr) {
        const hipblasStatus_t s = hipblasLtMatmulDescSetAttribute(
            plan.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof bias);
        if (s != HIPBLAS_STATUS_SUCCESS) {
            set_error(error, capacity, "GEMM bias setup failed: %s", status_text(s));
            return false;
        }
    }
    // the workspace comes from the staging pool; later users of the block
    // enqueue on the same stream, after this GEMM
    ScratchBlock workspace(plan.workspace);
    if (plan.workspace != 0 && workspace.get() == nullptr) {
        set_error(error, capacity, "out of device memory for the GEMM workspace");
        return false;
    }
    const float alpha = 1.0f, beta = 0.0f;
    const hipblasStatus_t s = hipblasLtMatmul(g.handle, plan.desc, &alpha, w, plan.a, x, plan.b,
                                              &beta, y, plan.d, y, plan.d, &plan.algo,
                                              plan.workspace ? workspace.get() : nullptr,
                                              plan.workspace, stream);
    if (s != HIPBLAS_STATUS_SUCCESS) {
        set_error(error, capacity, "GEMM launch failed: %s", status_text(s));
        return false;
    }
    return true;
}

void gemm_release() {
    GemmState &g = gemm_state();
    std::lock_guard<std::mutex> lock(g.mutex);
    for (auto &entry : g.plans) destroy(entry.second);
    g.plans.clear();
}

}  // namespace icsdk
