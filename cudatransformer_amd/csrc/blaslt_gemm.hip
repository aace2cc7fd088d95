// Plain row-major GEMMs of the linear layers on hipBLASLt.
//
// The linear layer's three products (y = x W^T + b, dX = dY W, dW += dY^T X) are plain
// library GEMMs: no head-split layouts, no fused attention work.  hipBLASLt's fp32 / bf16 /
// fp16 kernels run them 1.2-1.5x faster than the projection GEMM family at the NanoGPT
// shapes (4096 x {384, 1536} x {384, 1536}), so ctattn_linear_fwd / ctattn_linear_bwd send
// them here and keep the projection family for the head-split products and as the fallback
// (fp64, or whenever hipBLASLt returns no algorithm).  Setting CTATTN_NO_BLASLT=1 in the
// environment turns this path off.
//
// hipBLASLt is column-major; a row-major [R][C] matrix is the column-major C x R matrix with
// leading dimension C, so each product is written as its transpose (see proj_capi.hip).
// Descriptors, layouts and the heuristic's algorithm are cached per problem.  Only algorithms
// that need no workspace are accepted: there is then no scratch shared between calls, so two
// products in flight on different streams cannot race on one, and nothing is allocated.
// Under CTATTN_POLICY_GENERIC the products stay on the library's own GEMM kernels (the
// cross-check path), as they do with CTATTN_NO_BLASLT=1 in the environment.
#include "blaslt_gemm.h"

#include "ctattn.h"

#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

namespace ctattn {
namespace {

constexpr int kMaxDevices = 64;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};

using Key = std::tuple<int, int, int, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int, int>;

struct State {
    std::mutex mu;
    hipblasLtHandle_t handle[kMaxDevices] = {};
    bool failed[kMaxDevices] = {};  // handle creation failed on this device: never retried
    std::map<Key, Plan> plans;
    bool disabled = std::getenv("CTATTN_NO_BLASLT") != nullptr && std::getenv("CTATTN_NO_BLASLT")[0] == '1';
};

State &state() {
    static State *s = new State();  // never destroyed: may be used from static destructors
    return *s;
}

hipDataType data_type(int dtype) {
    switch (dtype) {
        case 0: return HIP_R_32F;
        case 1: return HIP_R_16BF;
        default: return HIP_R_16F;
    }
}

// Column-major rows x cols with leading dimension ld.
bool make_layout(hipblasLtMatrixLayout_t *l, hipDataType t, int64_t rows, int64_t cols, int64_t ld) {
    return hipblasLtMatrixLayoutCreate(l, t, uint64_t(rows), uint64_t(cols), ld) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace

bool blaslt_gemm(int dtype, bool trans_a, bool trans_b, int64_t m, int64_t n, int64_t k, const void *A, int64_t lda,
                 const void *B, int64_t ldb, void *C, int64_t ldc, float beta, const void *bias, hipStream_t stream) {
    if (dtype < 0 || dtype > 2 || m <= 0 || n <= 0 || k <= 0) return false;
    State &s = state();
    if (s.disabled || ctattn_get_policy() == CTATTN_POLICY_GENERIC) return false;
    int dev = 0;
    if ((stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev)) != hipSuccess || dev < 0 ||
        dev >= kMaxDevices)
        return false;
    std::lock_guard<std::mutex> lock(s.mu);
    if (s.handle[dev] == nullptr) {
        if (s.failed[dev]) return false;
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess) return false;
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return false;
        const bool created = hipblasLtCreate(&s.handle[dev]) == HIPBLAS_STATUS_SUCCESS;
        if (cur != dev) (void)hipSetDevice(cur);
        if (!created) {
            s.handle[dev] = nullptr;
            s.failed[dev] = true;
            return false;
        }
    }
    const Key key{dev, dtype, int(trans_a), int(trans_b), m, n, k, lda, ldb, ldc, beta != 0.f, bias != nullptr};
    auto it = s.plans.find(key);
    if (it == s.plans.end()) {
        Plan p;
        const hipDataType t = data_type(dtype);
        bool good = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
        const hipblasOperation_t oa = trans_a ? HIPBLAS_OP_T : HIPBLAS_OP_N, ob = trans_b ? HIPBLAS_OP_T : HIPBLAS_OP_N;
        good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &oa, sizeof(oa)) ==
                           HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &ob, sizeof(ob)) ==
                           HIPBLAS_STATUS_SUCCESS;
        if (good && bias != nullptr) {
            const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
            const int32_t bt = int32_t(t);
            good = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep)) ==
                       HIPBLAS_STATUS_SUCCESS &&
                   hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)) ==
                       HIPBLAS_STATUS_SUCCESS;
        }
        good = good && make_layout(&p.a, t, trans_a ? k : m, trans_a ? m : k, lda);
        good = good && make_layout(&p.b, t, trans_b ? n : k, trans_b ? k : n, ldb);
        good = good && make_layout(&p.c, t, m, n, ldc);
        if (good) {
            hipblasLtMatmulPreference_t pref = nullptr;
            const uint64_t ws = 0;  // algorithms without workspace only
            hipblasLtMatmulHeuristicResult_t res[1];
            int found = 0;
            good = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
                   hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                         sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
                   hipblasLtMatmulAlgoGetHeuristic(s.handle[dev], p.desc, p.a, p.b, p.c, p.c, pref, 1, res, &found) ==
                       HIPBLAS_STATUS_SUCCESS &&
                   found > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize == 0;
            if (pref != nullptr) hipblasLtMatmulPreferenceDestroy(pref);
            if (good) p.algo = res[0].algo;
        }
        p.ok = good;
        it = s.plans.emplace(key, p).first;
    }
    Plan &p = it->second;
    if (!p.ok) return false;
    if (bias != nullptr &&
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) !=
            HIPBLAS_STATUS_SUCCESS)
        return false;
    const float alpha = 1.f;
    return hipblasLtMatmul(s.handle[dev], p.desc, &alpha, A, p.a, B, p.b, &beta, C, p.c, C, p.c, &p.algo, nullptr, 0,
                           stream) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace ctattn
