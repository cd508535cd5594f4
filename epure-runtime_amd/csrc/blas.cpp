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
// One handle per device, created on first use outside stream capture
// (blas_ready() tells a caller under capture whether one exists).  Plans
// (descriptors, layouts and an algorithm) are cached per exact shape, at
// most kMaxPlans of them (the least recently used is destroyed to make
// room), so callers with a new token count on every call do not grow it
// without bound.  The algorithm: the heuristic's candidates are timed once
// per shape bucket (each dimension rounded up to a power of two) on the
// first call of the bucket outside stream capture -- that call waits for
// its timing runs on the host -- and the fastest is kept for the bucket;
// later shapes of the bucket take it when the heuristic offers it for
// them, else the heuristic's first choice, with no timing and no host
// wait.  A plan made during capture takes the heuristic's first choice.
// Matrices are column-major in hipBLASLt's terms; callers pass row-major
// buffers as their transposes.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstring>
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
    uint64_t used = 0;  // last use (g_clock)
};

// The timed choice of one shape bucket.
struct Timed {
    int dev, ta, tb, ab_dtype;
    int64_t bm, bn, bk;
    size_t ws;
    hipblasLtMatmulAlgo_t algo;
};

constexpr size_t kMaxPlans = 64;
constexpr size_t kMaxTimed = 256;

std::mutex g_mu;
hipblasLtHandle_t g_handle[64] = {};
std::vector<Plan> g_plans;
std::vector<Timed> g_timed;
uint64_t g_clock = 0;

int64_t bucket(int64_t v)
{
    int64_t b = 1;
    while (b < v)
        b <<= 1;
    return b;
}

void destroy_plan(Plan &p)
{
    if (p.desc)
        hipblasLtMatmulDescDestroy(p.desc);
    if (p.la)
        hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb)
        hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.ld)
        hipblasLtMatrixLayoutDestroy(p.ld);
    p.desc = nullptr;
    p.la = p.lb = p.ld = nullptr;
}

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

int handle_for(int dev, hipStream_t stream, hipblasLtHandle_t *h)
{
    if (dev < 0 || dev >= 64)
        return set_error(EP_ERR_ARG, "device %d", dev);
    if (!g_handle[dev]) {
        // creating the handle allocates device memory: never under capture
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
            return set_error(EP_DECLINE_SHAPE, "library GEMM: no hipBLASLt handle yet (first call under capture)");
        EP_BLAS_CHECK(hipblasLtCreate(&g_handle[dev]));
    }
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
    // the bucket's timed choice, where the heuristic offers it for this shape
    const int64_t bm = bucket(p.m), bn = bucket(p.n), bk = bucket(p.k);
    for (const Timed &t : g_timed) {
        if (t.dev != p.dev || t.ta != p.ta || t.tb != p.tb || t.ab_dtype != p.ab_dtype || t.bm != bm ||
            t.bn != bn || t.bk != bk || t.ws != p.ws)
            continue;
        for (int i = 0; i < nres; ++i)
            if (std::memcmp(res[i].algo.data, t.algo.data, sizeof(t.algo.data)) == 0)
                p.algo = res[i].algo;
        return EP_OK;
    }
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
        if (best > 0.0f && g_timed.size() < kMaxTimed)
            g_timed.push_back(Timed{p.dev, p.ta, p.tb, p.ab_dtype, bm, bn, bk, p.ws, p.algo});
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

bool blas_ready(int dev)
{
    std::lock_guard<std::mutex> lock(g_mu);
    return dev >= 0 && dev < 64 && g_handle[dev] != nullptr;
}

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
    int rc = handle_for(dev, stream, &h);
    if (rc != EP_OK)
        return rc;
    Plan *plan = nullptr;
    for (Plan &p : g_plans)
        if (p.dev == dev && p.ta == ta && p.tb == tb && p.ab_dtype == ab_dtype && p.m == m && p.n == n &&
            p.k == k && p.lda == lda && p.ldb == ldb && p.ldd == ldd && p.ws == ws_bytes)
            plan = &p;
    if (!plan) {
        if (g_plans.size() >= kMaxPlans) {
            // room for the new plan: destroy the least recently used one
            size_t lru = 0;
            for (size_t i = 1; i < g_plans.size(); ++i)
                if (g_plans[i].used < g_plans[lru].used)
                    lru = i;
            destroy_plan(g_plans[lru]);
            g_plans.erase(g_plans.begin() + (std::ptrdiff_t)lru);
        }
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
        if (rc != EP_OK) {
            destroy_plan(p);
            return rc;
        }
        g_plans.push_back(p);
        plan = &g_plans.back();
    }
    plan->used = ++g_clock;
    const float beta = 0.0f;
    EP_BLAS_CHECK(hipblasLtMatmul(h, plan->desc, &alpha, A, plan->la, B, plan->lb, &beta, D, plan->ld,
                                  D, plan->ld, &plan->algo, ws, ws_bytes, stream));
    return EP_OK;
}

}  // namespace ep
