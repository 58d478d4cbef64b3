// Plain prefill GEMMs on hipBLASLt: C[M][N] = A[M][K] . W[N][K]^T (+ bias[N]) (+ R[M][N]),
// A and W fp16, fp32 accumulation, C and R fp32 (R may be C: the residual added in place).
// These are the prefill F.linear / addmm calls of model.py:177, :213, :235 under the
// reference's CUDA autocast (model.py:147-151) that need no fused epilogue beyond a bias or a
// residual: QKV (+ bias), the o-projection and ffn_down (+ residual). The gate/up product with
// its SiLU epilogue and the attention stay on this library's own MFMA kernels.
//
// Row-major C = A W^T is the column-major product C^T = W A^T: hipBLASLt's matrix "A" is the
// weight buffer (column-major K x N, transposed), "B" the activation buffer (column-major
// K x M), D column-major N x M with leading dimension ldc; the bias epilogue adds a vector
// along D's rows (N), and beta = 1 with C = R adds the residual.
//
// State: one hipBLASLt handle per device and a cache of matmul plans (descriptors, layouts and
// the heuristic's first algorithm) per shape, guarded by a mutex; the workspace is the
// caller's.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "pe_common.h"

namespace {

struct LtPlan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

using LtKey = std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int, int, int64_t>;

std::mutex g_lt_mutex;
std::map<int, hipblasLtHandle_t> g_lt_handles;
std::map<LtKey, LtPlan> g_lt_plans;

constexpr int kMaxLtPlans = 256;

void destroy_plan(LtPlan& p) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.op) hipblasLtMatmulDescDestroy(p.op);
    p = LtPlan{};
}

// The plan of a shape (created and cached on first use; nullptr on any hipBLASLt failure).
const LtPlan* get_plan(hipblasLtHandle_t h, int dev, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldc, int64_t ldr, bool bias, bool res, int64_t ws_bytes) {
    const LtKey key{dev, M, N, K, lda, ldc, ldr, bias ? 1 : 0, res ? 1 : 0, ws_bytes};
    auto it = g_lt_plans.find(key);
    if (it != g_lt_plans.end()) return &it->second;
    if ((int)g_lt_plans.size() >= kMaxLtPlans) {
        for (auto& kv : g_lt_plans) destroy_plan(kv.second);
        g_lt_plans.clear();
    }
    LtPlan p;
    bool ok = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) == HIPBLAS_STATUS_SUCCESS;
    if (bias) {
        const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
        const hipDataType bt = HIP_R_32F;
        ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) == HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)) == HIPBLAS_STATUS_SUCCESS;
    }
    // "A" = W: column-major K x N (ld K); "B" = A: column-major K x M (ld lda); D: N x M (ld ldc)
    ok = ok && hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16F, (uint64_t)K, (uint64_t)N, K) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16F, (uint64_t)K, (uint64_t)M, lda) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, (uint64_t)N, (uint64_t)M, ldc) == HIPBLAS_STATUS_SUCCESS;
    (void)ldr;  // the residual shares C's layout (checked by the caller: ldr == ldc)
    hipblasLtMatmulPreference_t pref = nullptr;
    ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
    const uint64_t wsz = (uint64_t)ws_bytes;
    ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz,
                                                     sizeof(wsz)) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulHeuristicResult_t heur{};
    int found = 0;
    ok = ok && hipblasLtMatmulAlgoGetHeuristic(h, p.op, p.la, p.lb, p.lc, p.lc, pref, 1, &heur, &found) ==
                   HIPBLAS_STATUS_SUCCESS && found > 0;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (!ok) {
        destroy_plan(p);
        return nullptr;
    }
    p.algo = heur.algo;
    return &(g_lt_plans[key] = p);
}

// The device's handle, created on first use (the caller holds g_lt_mutex); nullptr on failure.
hipblasLtHandle_t lt_handle(int dev) {
    auto hit = g_lt_handles.find(dev);
    if (hit != g_lt_handles.end()) return hit->second;
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return nullptr;
    g_lt_handles[dev] = h;
    return h;
}

}  // namespace

using namespace pe;

extern "C" int pe_gemm_lt_init(void) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return PE_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_lt_mutex);
    return lt_handle(dev) ? PE_OK : PE_ERR_LAUNCH;
}

extern "C" int pe_gemm_lt(const void* a, int64_t lda, const void* w, int64_t M, int64_t N, int64_t K,
                          const float* bias, const float* res, int64_t ldr, float* c, int64_t ldc,
                          void* workspace, int64_t workspace_bytes, pe_stream_t stream) {
    if (M < 0 || N <= 0 || K <= 0 || lda < K || ldc < N) return PE_ERR_SHAPE;
    if (res && ldr != ldc) return PE_ERR_SHAPE;
    if (M == 0) return PE_OK;
    if (!a || !w || !c || (workspace_bytes > 0 && !workspace) || workspace_bytes < 0) return PE_ERR_NULL;
    if (!aligned(a, 16) || !aligned(w, 16) || !aligned(c, 16) || !aligned(res, 16) || !aligned(bias, 16) ||
        lda % 8 || ldc % 4 || K % 8 || !aligned(workspace, 256))
        return PE_ERR_ALIGN;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return PE_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_lt_mutex);
    const hipblasLtHandle_t h = lt_handle(dev);
    if (!h) return PE_ERR_LAUNCH;
    const LtPlan* p = get_plan(h, dev, M, N, K, lda, ldc, ldr, bias != nullptr, res != nullptr, workspace_bytes);
    if (!p) return PE_ERR_LAUNCH;
    if (bias && hipblasLtMatmulDescSetAttribute(p->op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) !=
                    HIPBLAS_STATUS_SUCCESS)
        return PE_ERR_LAUNCH;
    const float alpha = 1.0f, beta = res ? 1.0f : 0.0f;
    const void* cin = res ? (const void*)res : (const void*)c;
    const hipblasStatus_t st = hipblasLtMatmul(h, p->op, &alpha, w, p->la, a, p->lb, &beta, cin, p->lc, c, p->lc,
                                               &p->algo, workspace, (size_t)workspace_bytes, (hipStream_t)stream);
    if (st != HIPBLAS_STATUS_SUCCESS) return PE_ERR_LAUNCH;
    return launch_status();
}
