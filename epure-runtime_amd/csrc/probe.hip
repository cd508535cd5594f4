// Streaming-read probe: the practical HBM read ceiling the dequant kernels
// are judged against (the intended analogue of the reference's diagnostic
// kernel with "the same traffic", epure/kernels/_triton.py:188-236
// dequant_nolut).  It reads a buffer exactly once with the load shape of
// the GEMV and the decode step -- each workgroup streams one contiguous
// slice (as a CU streams its share of rows), 16-byte non-temporal loads,
// eight per lane in flight, 512 threads per workgroup -- and folds what it
// read into one XOR word per workgroup, so no load can be dropped and the
// result is checkable (the XOR of the sink words is the XOR of the
// buffer's words).
#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {

constexpr int kProbeThreads = 512;
constexpr int kProbeDepth = 8;  // 16-byte loads in flight per lane

__global__ void __launch_bounds__(kProbeThreads) read_probe_kernel(const u32x4_t *__restrict__ buf,
                                                                   int64_t n16, uint32_t *sink)
{
    __shared__ uint32_t part[kProbeThreads / 64];
    // slice [beg, end) of the 16-byte elements, whole 512-element rows
    const int64_t per = (n16 + (int64_t)gridDim.x * kProbeThreads - 1) / ((int64_t)gridDim.x * kProbeThreads) *
                        kProbeThreads;
    const int64_t beg = (int64_t)blockIdx.x * per;
    const int64_t end = beg + per < n16 ? beg + per : n16;
    constexpr int64_t stride = kProbeThreads;
    int64_t i = beg + threadIdx.x;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    for (; i + (kProbeDepth - 1) * stride < end; i += kProbeDepth * stride) {
        u32x4_t v[kProbeDepth];
#pragma unroll
        for (int k = 0; k < kProbeDepth; ++k)
            v[k] = __builtin_nontemporal_load(buf + i + k * stride);
#pragma unroll
        for (int k = 0; k < kProbeDepth; ++k)
            acc ^= v[k];
    }
    for (; i < end; i += stride)
        acc ^= __builtin_nontemporal_load(buf + i);
    uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        x ^= (uint32_t)__shfl_xor((int)x, o, 64);
    if ((threadIdx.x & 63) == 0)
        part[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < kProbeThreads / 64; ++w)
            s ^= part[w];
        sink[blockIdx.x] = s;
    }
}

}  // namespace

int launch_read_probe(const void *buf, int64_t bytes, uint32_t *sink, int grid, hipStream_t stream)
{
    if (bytes < 0 || bytes % 16 != 0 || ((uintptr_t)buf & 15) != 0)
        return set_error(EP_DECLINE_SHAPE, "read probe: %lld bytes at %p (16-byte multiples)",
                         (long long)bytes, buf);
    if (grid < 1 || grid > 65535 || !sink || (bytes > 0 && !buf))
        return set_error(EP_ERR_ARG, "read probe: grid %d, null buffer or sink", grid);
    hipLaunchKernelGGL(read_probe_kernel, dim3(grid), dim3(kProbeThreads), 0, stream,
                       (const u32x4_t *)buf, bytes / 16, sink);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

}  // namespace ep

extern "C" int ep_read_probe(const void *buf, int64_t bytes, uint32_t *sink, int grid, void *stream)
{
    return ep::launch_read_probe(buf, bytes, sink, grid, (hipStream_t)stream);
}
