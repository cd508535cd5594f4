// Index unpack and dequantized-tile kernels.
//
// unpack:  the flat nibble stream -> one uint8 per index
//          (epure/runtime.py:48-54 _unpack4; identity copy above 16 levels).
// dequant: W[n, k] = cb[idx] * scale[n, k / group] with the rounding of
//          epure/runtime.py:78-89 materialize(dtype):
//            f32:       f32(cb) * f32(scale)      (container.py:70-88)
//            f16/bf16:  dtype(dtype(cb) * dtype(scale))
//          The exact product of two fp16 (or two bf16) values fits in fp32,
//          so computing it in fp32 and rounding once is the torch result.
// embedding rows: the dequant of selected rows (PackedEmbedding).
// All read indices through the same flat-stream addressing as the GEMV
// fallback, so odd K with 4-bit packing is covered.
#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {

__global__ void __launch_bounds__(256) unpack_kernel(const uint8_t *__restrict__ packed, int64_t n,
                                                     int four, uint8_t *__restrict__ idx)
{
    // Each thread expands 8 indices (4 packed bytes for 4-bit).
    const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (base >= n)
        return;
    uint8_t out[8];
    if (four) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t p = base + 2 * i;
            const uint8_t b = p < n ? packed[p >> 1] : 0;
            out[2 * i] = b & 0x0f;
            out[2 * i + 1] = b >> 4;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            out[i] = base + i < n ? packed[base + i] : 0;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (base + i < n)
            idx[base + i] = out[i];
}

__device__ __forceinline__ float round_to(int dt, float v)
{
    if (dt == EP_F16)
        return (float)(f16_t)v;
    if (dt == EP_BF16)
        return bf16_to_f32(f32_to_bf16(v));
    return v;
}

struct TileArgs {
    const uint8_t *packed;
    const void *scale;
    int scale_dtype;
    int64_t lds;
    const void *cb;
    int cb_dtype;
    int levels;
    int group;
    int64_t N, K;
    void *out;
    int out_dtype;
    int64_t ldo;
};

// Element (n, k) of the dequantized weight in out_dtype's rounding.
__device__ __forceinline__ float dequant_elem(const TileArgs &a, int64_t n, int64_t k)
{
    const bool four = a.levels <= 16;
    const int64_t p = n * a.K + k;
    const uint8_t byte = a.packed[four ? (p >> 1) : p];
    const int idx = four ? ((p & 1) ? (byte >> 4) : (byte & 15)) : byte;
    const float c = idx < a.levels ? load_as_f32(a.cb, a.cb_dtype, idx) : 0.0f;
    const float s = load_as_f32(a.scale, a.scale_dtype, n * a.lds + k / a.group);
    return round_to(a.out_dtype, c) * round_to(a.out_dtype, s);
}

__global__ void __launch_bounds__(256) dequant_tile_kernel(TileArgs a)
{
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= a.K)
        return;
    for (int64_t n = blockIdx.y; n < a.N; n += gridDim.y)
        store_from_f32(a.out, a.out_dtype, n * a.ldo + k, dequant_elem(a, n, k));
}

// The same tile for 4-bit rows of whole 16-byte chunks (K % 32 == 0, groups
// of 32·2^i): one thread per 16 packed bytes (32 weights, one group scale),
// the codebook pre-rounded in LDS, 16-byte stores.  Same arithmetic as
// dequant_elem (round(c) * round(s) in fp32, rounded once).
constexpr int kTile4 = 1;
template <int DT>
__global__ void __launch_bounds__(256) dequant_tile4_kernel(TileArgs a)
{
    __shared__ float tab[16];
    if (threadIdx.x < 16)
        tab[threadIdx.x] = threadIdx.x < a.levels ? round_to(DT, load_as_f32(a.cb, a.cb_dtype, threadIdx.x)) : 0.0f;
    __syncthreads();
    const int64_t cpr = a.K / 32;  // chunks per row
    const int64_t total = a.N * cpr;
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    // kTile4 chunks per thread, all loaded before the first is expanded
    u32x4_t wv[kTile4];
    float scv[kTile4];
#pragma unroll
    for (int j = 0; j < kTile4; ++j) {
        const int64_t i = i0 + j * stride < total ? i0 + j * stride : 0;
        const int64_t n = i / cpr, c = i % cpr;
        wv[j] = *(const u32x4_t *)(a.packed + n * (a.K / 2) + c * 16);
        scv[j] = load_as_f32(a.scale, a.scale_dtype, n * a.lds + (c * 32) / a.group);
    }
#pragma unroll
    for (int j = 0; j < kTile4; ++j) {
    const int64_t i = i0 + j * stride;
    if (i >= total)
        break;
    const int64_t n = i / cpr, c = i % cpr;
    const u32x4_t w = wv[j];
    const float sc = round_to(DT, scv[j]);
    float v[32];
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int t = 0; t < 8; ++t)
            v[d * 8 + t] = tab[(w[d] >> (4 * t)) & 15] * sc;
    char *dst = (char *)a.out + (n * a.ldo + c * 32) * (DT == EP_F32 ? 4 : 2);
    if constexpr (DT == EP_F32) {
#pragma unroll
        for (int q = 0; q < 8; ++q)
            ((f32x4_t *)dst)[q] = (f32x4_t){v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4_t o;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float lo = v[8 * q + 2 * t], hi = v[8 * q + 2 * t + 1];
                if constexpr (DT == EP_F16)
                    o[t] = (uint32_t)f16_bits((f16_t)lo) | ((uint32_t)f16_bits((f16_t)hi) << 16);
                else
                    o[t] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
            }
            ((u32x4_t *)dst)[q] = o;
        }
    }
    }
}

// out[i, :] = dequantized row ids[i] (epure/runtime.py:139-156
// PackedEmbedding.forward: only the rows a batch asks for are expanded);
// an id outside [0, N) gives a row of zeros.
__global__ void __launch_bounds__(256) embedding_rows_kernel(TileArgs a, const int64_t *ids, int64_t n_ids)
{
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= a.K)
        return;
    for (int64_t i = blockIdx.y; i < n_ids; i += gridDim.y) {
        const int64_t n = ids[i];
        const float w = (n >= 0 && n < a.N) ? dequant_elem(a, n, k) : 0.0f;
        store_from_f32(a.out, a.out_dtype, i * a.ldo + k, w);
    }
}

}  // namespace

int launch_unpack(const uint8_t *packed, int64_t n, int levels, uint8_t *idx, hipStream_t stream)
{
    if (n <= 0)
        return EP_OK;
    const int64_t threads = (n + 7) / 8;
    const int64_t grid = (threads + 255) / 256;
    hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)grid), dim3(256), 0, stream, packed, n,
                       levels <= 16 ? 1 : 0, idx);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

int launch_dequant_tile(const PackedDesc &w, void *out, int out_dtype, int64_t ldo,
                        hipStream_t stream)
{
    if (w.N <= 0 || w.K <= 0)
        return EP_OK;
    TileArgs a{w.packed, w.scale, w.scale_dtype, w.ld_scale, w.cb, w.cb_dtype, w.levels,
               w.group, w.N, w.K, out, out_dtype, ldo};
    const int esz = out_dtype == EP_F32 ? 4 : 2;
    const bool fast = w.levels <= 16 && w.K % 32 == 0 && w.group % 32 == 0 &&
                      ((uintptr_t)w.packed & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                      (ldo * esz) % 16 == 0 && (w.N * (w.K / 32) + 255) / 256 < 0x7fffffff &&
                      w.N * (w.K / 32) >= 1;
    if (fast) {
        const dim3 grid((unsigned)((w.N * (w.K / 32) + 256 * kTile4 - 1) / (256 * kTile4)));
        if (out_dtype == EP_F16)
            hipLaunchKernelGGL(dequant_tile4_kernel<EP_F16>, grid, dim3(256), 0, stream, a);
        else if (out_dtype == EP_BF16)
            hipLaunchKernelGGL(dequant_tile4_kernel<EP_BF16>, grid, dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL(dequant_tile4_kernel<EP_F32>, grid, dim3(256), 0, stream, a);
        EP_HIP_CHECK(hipGetLastError());
        return EP_OK;
    }
    dim3 grid((unsigned)((w.K + 255) / 256), (unsigned)(w.N < 65535 ? w.N : 65535));
    hipLaunchKernelGGL(dequant_tile_kernel, grid, dim3(256), 0, stream, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

int launch_embedding_rows(const PackedDesc &w, const int64_t *ids, int64_t n_ids, void *out,
                          int out_dtype, int64_t ldo, hipStream_t stream)
{
    if (n_ids <= 0 || w.K <= 0)
        return EP_OK;
    TileArgs a{w.packed, w.scale, w.scale_dtype, w.ld_scale, w.cb, w.cb_dtype, w.levels,
               w.group, w.N, w.K, out, out_dtype, ldo};
    dim3 grid((unsigned)((w.K + 255) / 256), (unsigned)(n_ids < 65535 ? n_ids : 65535));
    hipLaunchKernelGGL(embedding_rows_kernel, grid, dim3(256), 0, stream, a, ids, n_ids);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

}  // namespace ep
