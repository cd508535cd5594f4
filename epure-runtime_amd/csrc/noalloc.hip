// ep_dequant_matmul_noalloc: the fused dequant-matmul for callers that
// cannot allocate device memory (code being captured into a HIP graph,
// serving loops that forbid allocation).  Its workspace is a file-scope
// device array of fixed size, `scratch`, which every GPU the library runs
// on holds until the process ends; no entry point here allocates.
//
// The array's name is a host-side stand-in, not a device address: host code
// uses only the per-device address hipGetSymbolAddress returns, fetched once
// per device (with that device current) on the first call there.  Every
// call on one GPU shares that GPU's array; the kernels behind
// ep_dequant_matmul overwrite every workspace byte they later read (split
// partials, row exponents, staged activations), so nothing has to start at
// zero -- but two calls in flight on one GPU at the same time (different
// streams, or different threads) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "epure_hip.h"
#include "ep_internal.h"

namespace ep {
namespace {

constexpr size_t kScratchBytes = (size_t)32 << 20;  // 32 MiB per GPU
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// Device address of this device's `scratch` (looked up once per device).
int scratch_address(void **out)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return set_error(EP_ERR_HIP, "noalloc: no current device (or device id %d >= %d)", dev,
                         kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != hipSuccess || !p)
            return set_error(EP_ERR_HIP, "noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                             dev, hipGetErrorString(rc));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return EP_OK;
}

}  // namespace
}  // namespace ep

using namespace ep;

extern "C" {

size_t ep_noalloc_scratch_bytes(void) { return kScratchBytes; }

int ep_dequant_matmul_noalloc(const void *x, int x_dtype, int64_t ldx, const uint8_t *packed,
                              const void *scale, int scale_dtype, int64_t ld_scale,
                              const void *cb, int cb_dtype, int levels, int group, int64_t M,
                              int64_t N, int64_t K, void *y, int y_dtype, int64_t ldy, int flags,
                              void *stream)
{
    if (M < 0 || N < 0 || K < 0)
        return set_error(EP_ERR_ARG, "noalloc: negative shape M=%lld N=%lld K=%lld",
                         (long long)M, (long long)N, (long long)K);
    const size_t need = ep_dequant_matmul_workspace(M, N, K, levels, group);
    if (need > kScratchBytes)
        return set_error(EP_ERR_WORKSPACE,
                         "noalloc: M=%lld N=%lld K=%lld needs %zu bytes of workspace, the static "
                         "scratch holds %zu; use ep_dequant_matmul with a caller workspace",
                         (long long)M, (long long)N, (long long)K, need, kScratchBytes);
    void *ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc != EP_OK)
        return rc;
    return ep_dequant_matmul(x, x_dtype, ldx, packed, scale, scale_dtype, ld_scale, cb, cb_dtype,
                             levels, group, M, N, K, y, y_dtype, ldy, flags, ws, kScratchBytes,
                             stream);
}

}  // extern "C"
