// Batch-1 / small-M fused codebook dequant-GEMV for gfx950.
//
// y[m, n] = sum_g scale[n, g] * sum_{k in g} fp16(x[m, k]) * fp16(cb[idx[n, k]])
// with fp32 accumulation; the dense weight is never written anywhere.
//
// Reference behaviour this serves: the packed-linear forward at small M,
// epure/kernels/_triton.py:54-107 (table kernel) / :317-377 (GEMV) and
// kernel/src/lib.rs:47-88 (row_dot).  The decode here is exact for the
// codebook: fp16(cb[l]) for fp16-valued codebooks, as the Rust LUT.
//
// Design (see the module header of the C ABI for the operand contract):
//  * Every packed byte holds two 4-bit indices (low nibble = even k).  An LDS
//    "pair table" maps the byte value b to the half2 (cb[b & 15], cb[b >> 4]),
//    so one ds_read_b32 + one v_dot2_f32_f16 consumes two weights.  8-bit
//    indices use the same table shape holding one fp16 per byte value and
//    two reads per v_dot2.
//  * The table is replicated 64x with lane l reading slot l, so each of the
//    64 lanes of a ds_read_b32 hits its own bank: no bank conflicts despite
//    random byte values.  Address = (byte << 8) | (lane << 2), one v_perm.
//  * 16 lanes cover 256 contiguous bytes of a row with 16-byte loads (fully
//    coalesced); a wave covers 4 rows x 256 bytes per load instruction and
//    the waves of a workgroup split the row's bytes into 256-byte slabs, so
//    each lane keeps the fp16 activations of its slabs in registers for the
//    whole kernel.
//  * The group scale is applied once per 32 weights (a 16-byte chunk never
//    straddles a group: group % 32 == 0 for 4-bit, % 16 for 8-bit).
//  * x is converted to fp16 after an exact per-row power-of-two rescale
//    computed in-kernel, so large activations cannot overflow fp16; the
//    result is scaled back exactly.
//  * Workgroups are persistent over 16-row blocks; each builds the 64 KiB
//    table once.  Cross-lane and cross-wave sums run in a fixed order, so
//    results are deterministic run to run.
#include <stdarg.h>

#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {

constexpr int kRepl = 64;                // table replicas (one per lane)
constexpr int kTabDwords = 256 * kRepl;  // 64 KiB
constexpr int kSlabBytes = 256;          // bytes of a row covered by 16 lanes
constexpr int kMaxWaves = 16;

struct GemvArgs {
    const void *x;
    int x_dtype;
    int64_t ldx;
    int M;
    const uint8_t *packed;
    int64_t row_bytes;
    const void *scale;
    int scale_dtype;
    int64_t lds;
    const void *cb;
    int cb_dtype;
    int levels;
    void *y;
    int y_dtype;
    int64_t ldy;
    int accumulate;
    int N;
    int64_t K;
    int group;
};

template <int BITS>
EP_DEV void build_table(uint32_t *tab, const void *cb, int cb_dtype, int levels)
{
    for (int e4 = threadIdx.x; e4 < kTabDwords / 4; e4 += blockDim.x) {
        const int b = (e4 * 4) / kRepl;
        uint32_t v;
        if constexpr (BITS == 4) {
            const int lo = b & 15, hi = b >> 4;
            const float clo = lo < levels ? load_as_f32(cb, cb_dtype, lo) : 0.0f;
            const float chi = hi < levels ? load_as_f32(cb, cb_dtype, hi) : 0.0f;
            v = (uint32_t)f16_bits((f16_t)clo) | ((uint32_t)f16_bits((f16_t)chi) << 16);
        } else {
            const float c = b < levels ? load_as_f32(cb, cb_dtype, b) : 0.0f;
            const uint32_t h = f16_bits((f16_t)c);
            v = h | (h << 16);
        }
        ((u32x4_t *)tab)[e4] = (u32x4_t){v, v, v, v};
    }
}

// v_perm selectors building the LDS byte address (byte_i << 8) | lane4:
// result byte0 = lane4 (src1 byte 0), byte1 = byte i of the packed word
// (src0 byte i = selector 4 + i), bytes 2-3 = 0 (selector 12).
constexpr uint32_t kSelByte[4] = {0x0c0c0400u, 0x0c0c0500u, 0x0c0c0600u, 0x0c0c0700u};

EP_DEV uint32_t lds_read_u32(const uint32_t *base, uint32_t byte_addr)
{
    return *(const uint32_t *)((const char *)base + byte_addr);
}

// Sum over the 16 lanes of a DPP row (lanes 16r..16r+15).
EP_DEV float row16_sum(float v)
{
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
}

// Two raw 16-bit activations (bf16 or fp16, per XDT) -> scaled fp16 pair.
template <int XDT>
EP_DEV f16x2_t cvt_pair(uint32_t raw, float pw)
{
    float lo, hi;
    if constexpr (XDT == EP_BF16) {
        lo = __uint_as_float(raw << 16);
        hi = __uint_as_float(raw & 0xffff0000u);
    } else {
        lo = (float)f16_from_bits((uint16_t)(raw & 0xffffu));
        hi = (float)f16_from_bits((uint16_t)(raw >> 16));
    }
    return (f16x2_t){(f16_t)(lo * pw), (f16_t)(hi * pw)};
}

template <int XDT>
EP_DEV float pair_amax(uint32_t raw)
{
    float lo, hi;
    if constexpr (XDT == EP_BF16) {
        lo = __uint_as_float(raw << 16);
        hi = __uint_as_float(raw & 0xffff0000u);
    } else {
        lo = (float)f16_from_bits((uint16_t)(raw & 0xffffu));
        hi = (float)f16_from_bits((uint16_t)(raw >> 16));
    }
    return fmaxf(fabsf(lo), fabsf(hi));
}

template <int BITS, int MT, int RQ, int SPW, int XDT>
__global__ void __launch_bounds__(1024) gemv_lut_kernel(GemvArgs a)
{
    constexpr int PAIRS = BITS == 4 ? 16 : 8;  // weight pairs per 16-byte chunk
    constexpr int ROWS = 4 * RQ;                // rows per block

    // Static LDS: the table sits at a compile-time address, so a lookup is
    // one v_perm for the address and the base folds into ds_read's offset.
    __shared__ __align__(16) uint32_t tab[kTabDwords];
    __shared__ float red[kMaxWaves * ROWS * MT];   // [W][ROWS][MT]
    __shared__ float s_amax[kMaxWaves * MT];       // [W][MT]
    __shared__ int s_exp[MT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int W = blockDim.x >> 6;
    const int rq = lane >> 4, c = lane & 15;
    const int64_t KB = BITS == 4 ? a.K / 2 : a.K;
    const int S = (int)((KB + kSlabBytes - 1) / kSlabBytes);

    // ---- stage this lane's activation chunks (raw) and their amax -------
    f16x2_t xh[SPW][MT][PAIRS];
    uint32_t xraw[SPW][MT][PAIRS];
    float amax[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
        amax[m] = 0.0f;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
        const int s = wave + j * W;
        const int64_t byte0 = (int64_t)s * kSlabBytes + c * 16;
        const bool act = s < S && byte0 < KB;
        const int64_t k0 = BITS == 4 ? byte0 * 2 : byte0;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const bool live = act && m < a.M;
            if constexpr (XDT == EP_F32) {
                const float *xp = (const float *)a.x + (int64_t)m * a.ldx + k0;
#pragma unroll
                for (int p = 0; p < PAIRS; p += 2) {
                    f32x4_t v = live ? *(const f32x4_t *)(xp + 2 * p) : (f32x4_t){0, 0, 0, 0};
                    amax[m] = fmaxf(amax[m], fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])),
                                                   fmaxf(fabsf(v[2]), fabsf(v[3]))));
                }
            } else {
                const uint16_t *xp = (const uint16_t *)a.x + (int64_t)m * a.ldx + k0;
#pragma unroll
                for (int p = 0; p < PAIRS; p += 4) {
                    u32x4_t v = live ? *(const u32x4_t *)(xp + 2 * p) : (u32x4_t){0, 0, 0, 0};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        xraw[j][m][p + t] = v[t];
                        amax[m] = fmaxf(amax[m], pair_amax<XDT>(v[t]));
                    }
                }
            }
        }
    }

    build_table<BITS>(tab, a.cb, a.cb_dtype, a.levels);

#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const float v = wave_max(amax[m]);
        if (lane == 0)
            s_amax[wave * MT + m] = v;
    }
    __syncthreads();
    if (tid < MT) {
        float v = 0.0f;
        for (int w = 0; w < W; ++w)
            v = fmaxf(v, s_amax[w * MT + tid]);
        s_exp[tid] = row_exponent(v);
    }
    __syncthreads();

    // ---- convert to scaled fp16 pairs ------------------------------------
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const float pw = ldexpf(1.0f, -s_exp[m]);
#pragma unroll
        for (int j = 0; j < SPW; ++j) {
            if constexpr (XDT == EP_F32) {
                const int s = wave + j * W;
                const int64_t byte0 = (int64_t)s * kSlabBytes + c * 16;
                const bool live = s < S && byte0 < KB && m < a.M;
                const int64_t k0 = BITS == 4 ? byte0 * 2 : byte0;
                const float *xp = (const float *)a.x + (int64_t)m * a.ldx + k0;
#pragma unroll
                for (int p = 0; p < PAIRS; p += 2) {
                    f32x4_t v = live ? *(const f32x4_t *)(xp + 2 * p) : (f32x4_t){0, 0, 0, 0};
                    xh[j][m][p] = (f16x2_t){(f16_t)(v[0] * pw), (f16_t)(v[1] * pw)};
                    xh[j][m][p + 1] = (f16x2_t){(f16_t)(v[2] * pw), (f16_t)(v[3] * pw)};
                }
            } else {
#pragma unroll
                for (int p = 0; p < PAIRS; ++p)
                    xh[j][m][p] = cvt_pair<XDT>(xraw[j][m][p], pw);
            }
        }
    }

    const uint32_t lane4 = (uint32_t)lane << 2;
    const int nblk = (a.N + ROWS - 1) / ROWS;

    for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
        const int row0 = blk * ROWS;
        float acc[RQ][MT];
#pragma unroll
        for (int q = 0; q < RQ; ++q)
#pragma unroll
            for (int m = 0; m < MT; ++m)
                acc[q][m] = 0.0f;

#pragma unroll
        for (int j = 0; j < SPW; ++j) {
            const int s = wave + j * W;
            const int64_t byte0 = (int64_t)s * kSlabBytes + c * 16;
            const bool act = s < S && byte0 < KB;
            const int64_t k0 = BITS == 4 ? byte0 * 2 : byte0;
            const int g = act ? (int)(k0 / a.group) : 0;

            // Unconditional loads from clamped addresses (an out-of-range lane
            // reads row 0 / byte 0 and is zeroed through its scale), so the
            // compiler issues all RQ loads back to back.
            const uint32_t bsafe = act ? (uint32_t)byte0 : 0u;
            u32x4_t wq[RQ];
            uint32_t soff[RQ];
            float sc[RQ];
#pragma unroll
            for (int q = 0; q < RQ; ++q) {
                const int row = row0 + 4 * q + rq;
                const uint32_t rsafe = row < a.N ? (uint32_t)row : 0u;
                // 32-bit offsets: the host guarantees N * row_bytes < 2^31.
                wq[q] = __builtin_nontemporal_load(
                    (const u32x4_t *)(a.packed + (rsafe * (uint32_t)a.row_bytes + bsafe)));
                soff[q] = rsafe * (uint32_t)a.lds + (uint32_t)g;
            }
            if (a.scale_dtype == EP_F16) {
#pragma unroll
                for (int q = 0; q < RQ; ++q)
                    sc[q] = (float)((const f16_t *)a.scale)[soff[q]];
            } else if (a.scale_dtype == EP_F32) {
#pragma unroll
                for (int q = 0; q < RQ; ++q)
                    sc[q] = ((const float *)a.scale)[soff[q]];
            } else {
#pragma unroll
                for (int q = 0; q < RQ; ++q)
                    sc[q] = bf16_to_f32(((const uint16_t *)a.scale)[soff[q]]);
            }
#pragma unroll
            for (int q = 0; q < RQ; ++q)
                if (!act || row0 + 4 * q + rq >= a.N)
                    sc[q] = 0.0f;

#pragma unroll
            for (int q = 0; q < RQ; ++q) {
                float part[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    part[m] = 0.0f;
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    const uint32_t w = wq[q][wd];
                    if constexpr (BITS == 4) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t ad = __builtin_amdgcn_perm(w, lane4, kSelByte[i]);
                            const uint32_t t = lds_read_u32(tab, ad);
                            const f16x2_t wv = __builtin_bit_cast(f16x2_t, t);
#pragma unroll
                            for (int m = 0; m < MT; ++m)
                                part[m] = __builtin_amdgcn_fdot2(wv, xh[j][m][wd * 4 + i], part[m],
                                                                 false);
                        }
                    } else {
#pragma unroll
                        for (int p = 0; p < 2; ++p) {
                            const uint32_t a0 = __builtin_amdgcn_perm(w, lane4, kSelByte[2 * p]);
                            const uint32_t a1 = __builtin_amdgcn_perm(w, lane4, kSelByte[2 * p + 1]);
                            const uint32_t t0 = lds_read_u32(tab, a0);
                            const uint32_t t1 = lds_read_u32(tab, a1);
                            const uint32_t pr = __builtin_amdgcn_perm(t1, t0, 0x07060100u);
                            const f16x2_t wv = __builtin_bit_cast(f16x2_t, pr);
#pragma unroll
                            for (int m = 0; m < MT; ++m)
                                part[m] = __builtin_amdgcn_fdot2(wv, xh[j][m][wd * 2 + p], part[m],
                                                                 false);
                        }
                    }
                }
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    acc[q][m] = fmaf(part[m], sc[q], acc[q][m]);
            }
        }

#pragma unroll
        for (int q = 0; q < RQ; ++q)
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float v = row16_sum(acc[q][m]);
                if (c == 0)
                    red[(wave * ROWS + 4 * q + rq) * MT + m] = v;
            }
        __syncthreads();
        for (int t = tid; t < ROWS * MT; t += blockDim.x) {
            const int r = t / MT, m = t % MT;
            const int row = row0 + r;
            if (row < a.N && m < a.M) {
                float v = 0.0f;
                for (int w = 0; w < W; ++w)
                    v += red[(w * ROWS + r) * MT + m];
                v = ldexpf(v, s_exp[m]);
                const int64_t off = (int64_t)m * a.ldy + row;
                if (a.accumulate)
                    v += load_as_f32(a.y, a.y_dtype, off);
                store_from_f32(a.y, a.y_dtype, off, v);
            }
        }
        __syncthreads();
    }
}

// Any shape, any stride, any M: one wave per output row, fp32 arithmetic
// (w = f32(cb[idx]) * f32(scale), fma into fp32).  Flat-stream indexing
// (position n*K + k), so odd K with 4-bit packing is served too.
__global__ void __launch_bounds__(256) gemv_generic_kernel(GemvArgs a)
{
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= a.N)
        return;
    const bool four = a.levels <= 16;
    for (int m = 0; m < a.M; ++m) {
        float acc = 0.0f;
        for (int64_t k = lane; k < a.K; k += 64) {
            const int64_t p = row * a.K + k;
            const uint8_t byte = a.packed[four ? (p >> 1) : p];
            const int idx = four ? ((p & 1) ? (byte >> 4) : (byte & 15)) : byte;
            const float cbv = idx < a.levels ? load_as_f32(a.cb, a.cb_dtype, idx) : 0.0f;
            const float w = cbv * load_as_f32(a.scale, a.scale_dtype, row * a.lds + k / a.group);
            acc = fmaf(load_as_f32(a.x, a.x_dtype, (int64_t)m * a.ldx + k), w, acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            const int64_t off = (int64_t)m * a.ldy + row;
            float v = acc;
            if (a.accumulate)
                v += load_as_f32(a.y, a.y_dtype, off);
            store_from_f32(a.y, a.y_dtype, off, v);
        }
    }
}

template <int BITS, int MT, int RQ, int SPW, int XDT>
int launch_lut(const GemvArgs &a, int waves, hipStream_t stream)
{
    constexpr int ROWS = 4 * RQ;
    constexpr size_t smem = (size_t)kTabDwords * 4 + (size_t)kMaxWaves * ROWS * MT * 4 +
                            (size_t)kMaxWaves * MT * 4 + (size_t)MT * 4;
    auto kern = gemv_lut_kernel<BITS, MT, RQ, SPW, XDT>;
    static int num_cu = 0;
    if (num_cu == 0) {
        int dev = 0;
        EP_HIP_CHECK(hipGetDevice(&dev));
        EP_HIP_CHECK(hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, dev));
    }
    const int nblk = (a.N + ROWS - 1) / ROWS;
    const int per_cu = 160 * 1024 / (int)smem;  // workgroups resident per CU by LDS
    int grid = num_cu * (per_cu > 0 ? per_cu : 1);
    if (grid > nblk)
        grid = nblk;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(waves * 64), 0, stream, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

template <int BITS, int MT, int SPW>
int dispatch_xdt(const GemvArgs &a, int xdt, int waves, hipStream_t s)
{
    switch (xdt) {
    case EP_BF16:
        return launch_lut<BITS, MT, 4, SPW, EP_BF16>(a, waves, s);
    case EP_F16:
        return launch_lut<BITS, MT, 4, SPW, EP_F16>(a, waves, s);
    default:
        return launch_lut<BITS, MT, 4, SPW, EP_F32>(a, waves, s);
    }
}

template <int BITS, int MT>
int dispatch_spw(const GemvArgs &a, int xdt, int spw, int waves, hipStream_t s)
{
    switch (spw) {
    case 1:
        return dispatch_xdt<BITS, MT, 1>(a, xdt, waves, s);
    case 2:
        return dispatch_xdt<BITS, MT, 2>(a, xdt, waves, s);
    default:
        return dispatch_xdt<BITS, MT, 4>(a, xdt, waves, s);
    }
}

GemvArgs make_args(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y)
{
    GemvArgs a;
    a.x = x.ptr;
    a.x_dtype = x.dtype;
    a.ldx = x.ld;
    a.M = (int)M;
    a.packed = w.packed;
    a.row_bytes = w.bits() == 4 ? w.K / 2 : w.K;
    a.scale = w.scale;
    a.scale_dtype = w.scale_dtype;
    a.lds = w.ld_scale;
    a.cb = w.cb;
    a.cb_dtype = w.cb_dtype;
    a.levels = w.levels;
    a.y = y.ptr;
    a.y_dtype = y.dtype;
    a.ldy = y.ld;
    a.accumulate = y.accumulate;
    a.N = (int)w.N;
    a.K = w.K;
    a.group = w.group;
    return a;
}

// Slabs per wave and waves per workgroup for a row of KB bytes.
void plan(int64_t KB, int &spw, int &waves)
{
    const int S = (int)((KB + kSlabBytes - 1) / kSlabBytes);
    spw = 1;
    while ((S + spw - 1) / spw > kMaxWaves)
        spw *= 2;
    waves = (S + spw - 1) / spw;
    if (waves < 1)
        waves = 1;
}

}  // namespace

bool gemv_serves(const PackedDesc &w, const ActDesc &x, int64_t M)
{
    const int bits = w.bits();
    if (M < 1 || M > 4 || w.N < 1 || w.N > INT32_MAX || w.K < 1)
        return false;
    const int64_t rb = bits == 4 ? w.K / 2 : w.K;
    if (w.N * rb >= ((int64_t)1 << 31) || w.N * w.ld_scale >= ((int64_t)1 << 31))
        return false;
    if (bits == 4 ? (w.K % 32 != 0 || w.group % 32 != 0) : (w.K % 16 != 0 || w.group % 16 != 0))
        return false;
    if (((uintptr_t)w.packed & 15) != 0)
        return false;
    const int esz = x.dtype == EP_F32 ? 4 : 2;
    if (((uintptr_t)x.ptr & 15) != 0 || (M > 1 && (x.ld * esz) % 16 != 0))
        return false;
    int spw, waves;
    plan(bits == 4 ? w.K / 2 : w.K, spw, waves);
    if (spw > 4)
        return false;
    const int mt = M == 1 ? 1 : (M == 2 ? 2 : 4);
    return spw * mt <= 8;
}

int launch_gemv(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                hipStream_t stream)
{
    if (!gemv_serves(w, x, M))
        return EP_DECLINE_SHAPE;
    const GemvArgs a = make_args(w, x, M, y);
    int spw, waves;
    plan(a.row_bytes, spw, waves);
    const int mt = M == 1 ? 1 : (M == 2 ? 2 : 4);
    if (w.bits() == 4) {
        if (mt == 1)
            return dispatch_spw<4, 1>(a, x.dtype, spw, waves, stream);
        if (mt == 2)
            return dispatch_spw<4, 2>(a, x.dtype, spw, waves, stream);
        return dispatch_spw<4, 4>(a, x.dtype, spw, waves, stream);
    }
    if (mt == 1)
        return dispatch_spw<8, 1>(a, x.dtype, spw, waves, stream);
    if (mt == 2)
        return dispatch_spw<8, 2>(a, x.dtype, spw, waves, stream);
    return dispatch_spw<8, 4>(a, x.dtype, spw, waves, stream);
}

int launch_gemv_generic(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                        hipStream_t stream)
{
    if (M < 1 || w.N < 1 || w.K < 1)
        return EP_OK;
    const GemvArgs a = make_args(w, x, M, y);
    const int rows_per_wg = 4;
    const int64_t grid = (w.N + rows_per_wg - 1) / rows_per_wg;
    hipLaunchKernelGGL(gemv_generic_kernel, dim3((unsigned)grid), dim3(rows_per_wg * 64), 0,
                       stream, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

}  // namespace ep
