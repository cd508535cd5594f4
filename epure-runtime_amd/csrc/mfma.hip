// Small-M / prefill fused dequant-matmul on gfx950 MFMA.
//
// y[M, N] = x[M, K] . W[N, K]^T for M large enough that the contraction is
// compute-bound.  Reference behaviour: the tiled table kernel
// epure/kernels/_triton.py:54-107 (operands in fp16, fp32 accumulation).
//
// Per K-step of 64:
//  * the packed bytes of a BN x 64 weight tile are read once (16-byte loads),
//    expanded through a 256-entry LDS pair table and multiplied by the group
//    scale with v_pk_mul_f16, giving fp16(fp16(cb[idx]) * fp16(scale)) --
//    the reference's materialize(float16) tile, bit for bit -- written to LDS;
//  * the BM x 64 activation tile is converted to fp16 after the exact
//    per-row power-of-two rescale (exponents from a one-pass pre-kernel in the
//    workspace) and written to LDS;
//  * each wave runs v_mfma_f32_32x32x16_f16 over its sub-tile from LDS.
// The next step's global loads are issued before the MFMAs of the current
// one.  The dense weight never reaches global memory.
#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {

constexpr int BK = 64;
constexpr int LDT = BK + 8;  // halfs per LDS tile row (padding keeps b128 reads conflict-free)

struct MmArgs {
    const void *x;
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
    const int *rexp;
};

// One wave per activation row: exponent of the row's largest |x|.
__global__ void __launch_bounds__(256)
    row_exp_kernel(const void *x, int xdt, int64_t ldx, int M, int64_t K, int *rexp)
{
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M)
        return;
    float amax = 0.0f;
    for (int64_t k = lane; k < K; k += 64)
        amax = fmaxf(amax, fabsf(load_as_f32(x, xdt, row * ldx + k)));
    amax = wave_max_bfly(amax);
    if (lane == 0)
        rexp[row] = row_exponent(amax);
}

template <int BITS, int BM, int BN, int WM, int WN, int XDT>
__global__ void __launch_bounds__(256) mm_kernel(MmArgs a)
{
    static_assert(WM * WN == 4, "four waves");
    constexpr int TM = BM / WM / 32;  // 32x32 MFMA tiles per wave along M
    constexpr int TN = BN / WN / 32;  // ... along N
    constexpr int XCH = BM * (BK / 8) / 256;                        // 8-element x chunks / thread
    constexpr int WPR = BITS == 4 ? BK / 32 : BK / 16;              // 16-byte W chunks per row
    constexpr int WCH = BN * WPR / 256;                             // W chunks / thread
    constexpr int KPC = BITS == 4 ? 32 : 16;                        // k per W chunk
    static_assert(XCH >= 1 && WCH >= 1, "tile too small for 256 threads");

    __shared__ __align__(16) f16_t As[BM * LDT];
    __shared__ __align__(16) f16_t Bs[BN * LDT];
    __shared__ uint32_t tab[256];
    __shared__ float s_pw[BM];
    __shared__ int s_e[BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    {
        const int b = tid;  // 256 threads, 256 table entries
        uint32_t v;
        if constexpr (BITS == 4) {
            const int lo = b & 15, hi = b >> 4;
            const float clo = lo < a.levels ? load_as_f32(a.cb, a.cb_dtype, lo) : 0.0f;
            const float chi = hi < a.levels ? load_as_f32(a.cb, a.cb_dtype, hi) : 0.0f;
            v = (uint32_t)f16_bits((f16_t)clo) | ((uint32_t)f16_bits((f16_t)chi) << 16);
        } else {
            const float c = b < a.levels ? load_as_f32(a.cb, a.cb_dtype, b) : 0.0f;
            v = f16_bits((f16_t)c);
        }
        tab[b] = v;
    }
    for (int r = tid; r < BM; r += 256) {
        const int m = m0 + r;
        const int e = m < a.M ? a.rexp[m] : 0;
        s_e[r] = e;
        s_pw[r] = ldexpf(1.0f, -e);
    }

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[i][j][r] = 0.0f;

    // register staging of one K-step
    u32x4_t xr[XCH][XDT == EP_F32 ? 2 : 1];
    u32x4_t wr[WCH];
    float wsc[WCH];

    auto load_step = [&](int kt) {
        const int64_t kbase = (int64_t)kt * BK;
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / (BK / 8), col = (c % (BK / 8)) * 8;
            const int m = m0 + r;
            if constexpr (XDT == EP_F32) {
                const float *p = (const float *)a.x + (int64_t)m * a.ldx + kbase + col;
                xr[i][0] = m < a.M ? *(const u32x4_t *)p : (u32x4_t){0, 0, 0, 0};
                xr[i][1] = m < a.M ? *(const u32x4_t *)(p + 4) : (u32x4_t){0, 0, 0, 0};
            } else {
                const uint16_t *p = (const uint16_t *)a.x + (int64_t)m * a.ldx + kbase + col;
                xr[i][0] = m < a.M ? *(const u32x4_t *)p : (u32x4_t){0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int i = 0; i < WCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / WPR, part = c % WPR;
            const int n = n0 + r;
            const int64_t k0 = kbase + part * KPC;
            const int64_t byte0 = BITS == 4 ? k0 / 2 : k0;
            if (n < a.N) {
                wr[i] = __builtin_nontemporal_load(
                    (const u32x4_t *)(a.packed + (int64_t)n * a.row_bytes + byte0));
                wsc[i] = load_as_f32(a.scale, a.scale_dtype, (int64_t)n * a.lds + k0 / a.group);
            } else {
                wr[i] = (u32x4_t){0, 0, 0, 0};
                wsc[i] = 0.0f;
            }
        }
    };

    auto store_step = [&]() {
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / (BK / 8), col = (c % (BK / 8)) * 8;
            const float pw = s_pw[r];
            f16x8_t h;
            if constexpr (XDT == EP_F32) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    h[t] = (f16_t)(__uint_as_float(xr[i][0][t]) * pw);
                    h[4 + t] = (f16_t)(__uint_as_float(xr[i][1][t]) * pw);
                }
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t raw = xr[i][0][t];
                    float lo, hi;
                    if constexpr (XDT == EP_BF16) {
                        lo = __uint_as_float(raw << 16);
                        hi = __uint_as_float(raw & 0xffff0000u);
                    } else {
                        lo = (float)f16_from_bits((uint16_t)(raw & 0xffffu));
                        hi = (float)f16_from_bits((uint16_t)(raw >> 16));
                    }
                    h[2 * t] = (f16_t)(lo * pw);
                    h[2 * t + 1] = (f16_t)(hi * pw);
                }
            }
            *(f16x8_t *)&As[r * LDT + col] = h;
        }
#pragma unroll
        for (int i = 0; i < WCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / WPR, part = c % WPR;
            const f16_t sh = (f16_t)wsc[i];
            const f16x2_t s2 = (f16x2_t){sh, sh};
            f16x2_t o[KPC / 2];
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                const uint32_t w = wr[i][wd];
                if constexpr (BITS == 4) {
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const uint32_t t = tab[(w >> (8 * b)) & 0xffu];
                        o[wd * 4 + b] = as_f16x2(t) * s2;
                    }
                } else {
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const uint32_t t0 = tab[(w >> (16 * p)) & 0xffu];
                        const uint32_t t1 = tab[(w >> (16 * p + 8)) & 0xffu];
                        const f16x2_t pr =
                            as_f16x2((t0 & 0xffffu) | (t1 << 16));
                        o[wd * 2 + p] = pr * s2;
                    }
                }
            }
            f16_t *dst = &Bs[r * LDT + part * KPC];
#pragma unroll
            for (int v = 0; v < KPC / 8; ++v) {
                f16x8_t h;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    h[2 * t] = o[v * 4 + t][0];
                    h[2 * t + 1] = o[v * 4 + t][1];
                }
                *(f16x8_t *)(dst + v * 8) = h;
            }
        }
    };

    const int KT = (int)(a.K / BK);
    __syncthreads();  // table and row scales ready
    load_step(0);
    for (int kt = 0; kt < KT; ++kt) {
        store_step();
        __syncthreads();
        if (kt + 1 < KT)
            load_step(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            f16x8_t af[TM], bfr[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *(const f16x8_t *)&As[(wm * TM * 32 + i * 32 + (lane & 31)) * LDT +
                                               kk * 16 + (lane >> 5) * 8];
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bfr[j] = *(const f16x8_t *)&Bs[(wn * TN * 32 + j * 32 + (lane & 31)) * LDT +
                                                kk * 16 + (lane >> 5) * 8];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bfr[j], acc[i][j], 0,
                                                                       0, 0);
        }
        __syncthreads();
    }

    // epilogue: D[row][col] lives in lane col + 32 * ((row / 4) % 2),
    // register (row % 4) + 4 * (row / 8).
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * TM * 32 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                const int col = wn * TN * 32 + j * 32 + (lane & 31);
                const int m = m0 + row, n = n0 + col;
                if (m < a.M && n < a.N) {
                    float v = ldexpf(acc[i][j][r], s_e[row]);
                    const int64_t off = (int64_t)m * a.ldy + n;
                    if (a.accumulate)
                        v += load_as_f32(a.y, a.y_dtype, off);
                    store_from_f32(a.y, a.y_dtype, off, v);
                }
            }
}

template <int BITS, int BM, int BN, int WM, int WN>
int launch_cfg(const MmArgs &a, int xdt, hipStream_t s)
{
    dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM));
    switch (xdt) {
    case EP_BF16:
        hipLaunchKernelGGL((mm_kernel<BITS, BM, BN, WM, WN, EP_BF16>), grid, dim3(256), 0, s, a);
        break;
    case EP_F16:
        hipLaunchKernelGGL((mm_kernel<BITS, BM, BN, WM, WN, EP_F16>), grid, dim3(256), 0, s, a);
        break;
    default:
        hipLaunchKernelGGL((mm_kernel<BITS, BM, BN, WM, WN, EP_F32>), grid, dim3(256), 0, s, a);
        break;
    }
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

template <int BITS>
int launch_bits(const MmArgs &a, int xdt, hipStream_t s)
{
    if (a.M <= 32)
        return launch_cfg<BITS, 32, 128, 1, 4>(a, xdt, s);
    if (a.M <= 64)
        return launch_cfg<BITS, 64, 128, 1, 4>(a, xdt, s);
    return launch_cfg<BITS, 128, 128, 2, 2>(a, xdt, s);
}

}  // namespace

size_t mfma_workspace(int64_t M) { return (size_t)((M * 4 + 255) / 256 * 256); }

bool mfma_serves(const PackedDesc &w, const ActDesc &x, int64_t M)
{
    if (M < 1 || M > INT32_MAX || w.N < 1 || w.N > INT32_MAX || w.K < BK || w.K % BK != 0)
        return false;
    if (w.bits() == 4 ? (w.group % 32 != 0) : (w.group % 16 != 0))
        return false;
    if (((uintptr_t)w.packed & 15) != 0 || ((uintptr_t)x.ptr & 15) != 0)
        return false;
    const int esz = x.dtype == EP_F32 ? 4 : 2;
    return (x.ld * esz) % 16 == 0;
}

int launch_mfma(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y, void *ws,
                size_t ws_bytes, hipStream_t stream)
{
    if (!mfma_serves(w, x, M))
        return EP_DECLINE_SHAPE;
    if (!ws || ws_bytes < mfma_workspace(M))
        return set_error(EP_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given",
                         mfma_workspace(M), ws_bytes);
    int *rexp = (int *)ws;
    hipLaunchKernelGGL(row_exp_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream, x.ptr,
                       x.dtype, x.ld, (int)M, w.K, rexp);
    EP_HIP_CHECK(hipGetLastError());
    MmArgs a;
    a.x = x.ptr;
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
    a.rexp = rexp;
    return w.bits() == 4 ? launch_bits<4>(a, x.dtype, stream) : launch_bits<8>(a, x.dtype, stream);
}

}  // namespace ep
