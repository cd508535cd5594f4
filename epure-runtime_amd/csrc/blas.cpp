// Library GEMMs for the backward (hipBLASLt): the two plain dense products
// of the compressed-state backward at large token counts,
//
//   D = A . B     with A, B fp16/bf16 and D f32, f32 accumulation,
//
// i.e. grad_x's gy . W (W materialized to fp16 first) and G = gy^T . x.
// The reference computes both through autograd on the materialized weight
// (epure/runtime.py:84-88: torch matmuls); the LUT kernels here cannot
// beat the library on a dense GEMM, so only these two products go to it,
// with every special step (the materialization, the exact gy prescale,
// the codebook reductions) in this library's own kernels.
//
// One handle per device, created on first use; plans (descriptors, layouts
// and an algorithm) cached per shape.  The algorithm: the heuristic's
// candidates are each timed once on the call's own operands when the plan
// is made (the first call for a shape, outside stream capture; a plan made
// during capture takes the heuristic's first choice), the fastest kept.
// Matrices are column-major in hipBLASLt's terms; callers pass row-major
// buffers as their transposes.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <mutex>
#include <vector>

#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {

struct Plan {
    int dev, ta, tb, ab_dtype;
    int64_t m, n, k, lda, ldb, ldd;
    size_t ws;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
    hipblasLtMatmulAlgo_t algo;
};

std::mutex g_mu;
hipblasLtHandle_t g_handle[64] = {};
std::vector<Plan> g_plans;

const char *status_name(hipblasStatus_t s)
{
    switch (s) {
    case HIPBLAS_STATUS_SUCCESS:
        return "success";
    case HIPBLAS_STATUS_NOT_INITIALIZED:
        return "not initialized";
    case HIPBLAS_STATUS_ALLOC_FAILED:
        return "alloc failed";
    case HIPBLAS_STATUS_INVALID_VALUE:
        return "invalid value";
    case HIPBLAS_STATUS_NOT_SUPPORTED:
        return "not supported";
    case HIPBLAS_STATUS_EXECUTION_FAILED:
        return "execution failed";
    default:
        return "error";
    }
}

#define EP_BLAS_CHECK(expr)                                                                    \
    do {                                                                                       \
        hipblasStatus_t _s = (expr);                                                           \
        if (_s != HIPBLAS_STATUS_SUCCESS)                                                      \
            return set_error(EP_ERR_HIP, "%s: %s", #expr, status_name(_s));                   \
    } while (0)

int handle_for(int dev, hipblasLtHandle_t *h)
{
    if (dev < 0 || dev >= 64)
        return set_error(EP_ERR_ARG, "device %d", dev);
    if (!g_handle[dev])
        EP_BLAS_CHECK(hipblasLtCreate(&g_handle[dev]));
    *h = g_handle[dev];
    return EP_OK;
}

// Mean time of `reps` runs of one algorithm (after one untimed run), or a
// negative value when it does not run.
float time_algo(hipblasLtHandle_t h, const Plan &p, const hipblasLtMatmulAlgo_t &algo, const float *alpha,
                const void *A, const void *B, float *D, void *ws, size_t ws_bytes, hipStream_t stream,
                hipEvent_t e0, hipEvent_t e1)
{
    const float beta = 0.0f;
    constexpr int reps = 3;
    if (hipblasLtMatmul(h, p.desc, alpha, A, p.la, B, p.lb, &beta, D, p.ld, D, p.ld, &algo, ws, ws_bytes,
                        stream) != HIPBLAS_STATUS_SUCCESS)
        return -1.0f;
    if (hipEventRecord(e0, stream) != hipSuccess)
        return -1.0f;
    for (int r = 0; r < reps; ++r)
        if (hipblasLtMatmul(h, p.desc, alpha, A, p.la, B, p.lb, &beta, D, p.ld, D, p.ld, &algo, ws, ws_bytes,
                            stream) != HIPBLAS_STATUS_SUCCESS)
            return -1.0f;
    float ms = -1.0f;
    if (hipEventRecord(e1, stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
        return -1.0f;
    return ms / reps;
}

int make_plan(Plan &p, hipblasLtHandle_t h, const float *alpha, const void *A, const void *B, float *D,
              void *ws, hipStream_t stream)
{
    const hipDataType ab = p.ab_dtype == EP_F16 ? HIP_R_16F : HIP_R_16BF;
    EP_BLAS_CHECK(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t opa = p.ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    const hipblasOperation_t opb = p.tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    EP_BLAS_CHECK(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa)));
    EP_BLAS_CHECK(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb)));
    EP_BLAS_CHECK(hipblasLtMatrixLayoutCreate(&p.la, ab, p.ta ? p.k : p.m, p.ta ? p.m : p.k, p.lda));
    EP_BLAS_CHECK(hipblasLtMatrixLayoutCreate(&p.lb, ab, p.tb ? p.n : p.k, p.tb ? p.k : p.n, p.ldb));
    EP_BLAS_CHECK(hipblasLtMatrixLayoutCreate(&p.ld, HIP_R_32F, p.m, p.n, p.ldd));
    hipblasLtMatmulPreference_t pref;
    EP_BLAS_CHECK(hipblasLtMatmulPreferenceCreate(&pref));
    uint64_t wsz = p.ws;
    hipblasStatus_t s = hipblasLtMatmulPreferenceSetAttribute(
        pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz, sizeof(wsz));
    constexpr int kCand = 8;
    hipblasLtMatmulHeuristicResult_t res[kCand];
    int nres = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.ld, p.ld, pref, kCand, res, &nres);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS)
        return set_error(EP_ERR_HIP, "hipblasLtMatmulAlgoGetHeuristic: %s", status_name(s));
    if (nres < 1)
        return set_error(EP_DECLINE_SHAPE, "hipBLASLt has no algorithm for this GEMM");
    p.algo = res[0].algo;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (nres < 2 || hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
        return EP_OK;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        float best = -1.0f;
        for (int i = 0; i < nres; ++i) {
            const float t = time_algo(h, p, res[i].algo, alpha, A, B, D, ws, p.ws, stream, e0, e1);
            if (t > 0.0f && (best < 0.0f || t < best)) {
                best = t;
                p.algo = res[i].algo;
            }
        }
    }
    if (e0)
        (void)hipEventDestroy(e0);
    if (e1)
        (void)hipEventDestroy(e1);
    (void)hipGetLastError();  // a candidate that failed leaves no error behind
    return EP_OK;
}

}  // namespace

size_t blas_workspace_bytes() { return (size_t)32 << 20; }

// D[m x n] (f32, column-major, ldd) = alpha * op(A) . op(B); op(A) is m x k.
int blas_gemm_f32out(int ta, int tb, int64_t m, int64_t n, int64_t k, int ab_dtype, const void *A,
                     int64_t lda, const void *B, int64_t ldb, float *D, int64_t ldd, float alpha,
                     void *ws, size_t ws_bytes, hipStream_t stream)
{
    if (ab_dtype != EP_F16 && ab_dtype != EP_BF16)
        return set_error(EP_DECLINE_SHAPE, "library GEMM: fp16 or bf16 operands");
    int dev = 0;
    EP_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_mu);
    hipblasLtHandle_t h;
    int rc = handle_for(dev, &h);
    if (rc != EP_OK)
        return rc;
    Plan *plan = nullptr;
    for (Plan &p : g_plans)
        if (p.dev == dev && p.ta == ta && p.tb == tb && p.ab_dtype == ab_dtype && p.m == m && p.n == n &&
            p.k == k && p.lda == lda && p.ldb == ldb && p.ldd == ldd && p.ws == ws_bytes)
            plan = &p;
    if (!plan) {
        Plan p;
        p.dev = dev;
        p.ta = ta;
        p.tb = tb;
        p.ab_dtype = ab_dtype;
        p.m = m;
        p.n = n;
        p.k = k;
        p.lda = lda;
        p.ldb = ldb;
        p.ldd = ldd;
        p.ws = ws_bytes;
        rc = make_plan(p, h, &alpha, A, B, D, ws, stream);
        if (rc != EP_OK)
            return rc;
        g_plans.push_back(p);
        plan = &g_plans.back();
    }
    const float beta = 0.0f;
    EP_BLAS_CHECK(hipblasLtMatmul(h, plan->desc, &alpha, A, plan->la, B, plan->lb, &beta, D, plan->ld,
                                  D, plan->ld, &plan->algo, ws, ws_bytes, stream));
    return EP_OK;
}

}  // namespace ep
