// Compressed-state backward of y = x . W^T, W = cb[idx] * scale, indices
// frozen (fine-tuning/README.md:62-68; the reference gets these from
// autograd through materialize(), runtime.py:84-88):
//
//   grad_x     = gy . W                              (dx kernel)
//   grad_scale[n, g] = sum_{k in g} G[n, k] * cb[idx[n, k]]
//   grad_cb[l]       = sum_{idx[n,k] == l} G[n, k] * scale[n, g(k)]
//   with G = gy^T . x, which is never written to memory  (dw kernel)
//
// dx: MFMA over 128x128 (m, k) tiles, contraction over n in steps of 32.
//     gy enters as fp16 after the exact per-row power-of-two rescale (as in
//     the forward); each W tile is read once from the packed bytes,
//     expanded to fp16(cb * scale) and written transposed into LDS.
// dw: MFMA (bf16 operands: gy and x are bf16, products exact in fp32) over
//     128x128 (k, n) tiles of G, contraction over the token dimension m in
//     steps of 32.  The epilogue never stores G: each value is multiplied by
//     cb[idx] and summed over its group (grad_scale is complete inside the
//     tile, one plain store per (n, g)), and multiplied by its scale and
//     added into a per-thread private LDS histogram over the 16 codebook
//     levels; histograms are reduced in a fixed order per workgroup and
//     across workgroups by a final kernel.  No float atomics race, so the
//     result is deterministic.  `packed` is only read.
#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int T = 128;   // output tile (both dims)
constexpr int KS = 32;   // contraction step
constexpr int LD = KS + 8;  // LDS row length (elements), padded

struct BwdArgs {
    const void *gy;
    int gy_dtype;
    int64_t ldgy;
    const void *x;
    int64_t ldx;
    const uint8_t *packed;
    const void *scale;
    int scale_dtype;
    int64_t lds;
    const void *cb;
    int cb_dtype;
    int levels;
    int group;
    int M, N, K;
    void *gx;
    int gx_dtype;
    int64_t ldgx;
    float *gscale;
    int64_t ldgs;
    const int *rexp;     // [M] per-row exponents of gy
    float *gc_part;      // [num dw workgroups][16]
};

__global__ void __launch_bounds__(256)
    row_exp_gy_kernel(const void *gy, int dt, int64_t ld, int M, int N, int *rexp)
{
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M)
        return;
    float amax = 0.0f;
    for (int64_t n = lane; n < N; n += 64)
        amax = fmaxf(amax, fabsf(load_as_f32(gy, dt, row * ld + n)));
    amax = wave_max_bfly(amax);
    if (lane == 0)
        rexp[row] = row_exponent(amax);
}

// grad_x[m, k] = sum_n gy[m, n] W[n, k]
template <int BITS>
__global__ void __launch_bounds__(256) dx_kernel(BwdArgs a)
{
    __shared__ __align__(16) f16_t As[T * LD];  // gy tile [m][n]
    __shared__ __align__(16) f16_t Bs[T * LD];  // W^T tile [k][n]
    __shared__ uint32_t tab[256];
    __shared__ float s_pw[T];
    __shared__ int s_e[T];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wk = wave & 1;
    const int m0 = blockIdx.y * T, k0 = blockIdx.x * T;
    {
        const int b = tid;
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
    if (tid < T) {
        const int m = m0 + tid;
        const int e = m < a.M ? a.rexp[m] : 0;
        s_e[tid] = e;
        s_pw[tid] = ldexpf(1.0f, -e);
    }

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[i][j][r] = 0.0f;

    // staging registers for one contraction step
    float gv[16];          // gy: 128 rows x 32 n = 16 values per thread
    u32x4_t wr;            // W: 32 rows x 128 k; 4-bit: 16 bytes/thread (128 threads)
    float wsc = 0.0f;      //    8-bit: 16 bytes/thread (256 threads)
    constexpr int WTHREADS = BITS == 4 ? 128 : 256;
    constexpr int KPC = BITS == 4 ? 32 : 16;   // k per 16-byte chunk

    auto load = [&](int n0) {
        // gy: thread -> row tid/2, 16 consecutive n
        const int r = tid >> 1, c0 = (tid & 1) * 16;
        const int m = m0 + r;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int n = n0 + c0 + e;
            gv[e] = (m < a.M && n < a.N) ? load_as_f32(a.gy, a.gy_dtype, (int64_t)m * a.ldgy + n)
                                         : 0.0f;
        }
        if (tid < WTHREADS) {
            const int per_row = T / KPC;             // chunks per W row in the tile
            const int wrow = tid / per_row, part = tid % per_row;
            const int n = n0 + wrow;
            const int64_t kk = (int64_t)k0 + part * KPC;
            const int64_t byte0 = BITS == 4 ? kk / 2 : kk;
            if (n < a.N) {
                wr = *(const u32x4_t *)(a.packed + (int64_t)n * (BITS == 4 ? a.K / 2 : a.K) + byte0);
                wsc = load_as_f32(a.scale, a.scale_dtype, (int64_t)n * a.lds + kk / a.group);
            } else {
                wr = (u32x4_t){0, 0, 0, 0};
                wsc = 0.0f;
            }
        }
    };
    auto store = [&]() {
        {
            const int r = tid >> 1, c0 = (tid & 1) * 16;
            const float pw = s_pw[r];
            f16x8_t h0, h1;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                h0[e] = (f16_t)(gv[e] * pw);
                h1[e] = (f16_t)(gv[8 + e] * pw);
            }
            *(f16x8_t *)&As[r * LD + c0] = h0;
            *(f16x8_t *)&As[r * LD + c0 + 8] = h1;
        }
        if (tid < WTHREADS) {
            const int per_row = T / KPC;
            const int wrow = tid / per_row, part = tid % per_row;
            const f16_t sh = (f16_t)wsc;
            const f16x2_t s2 = (f16x2_t){sh, sh};
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                const uint32_t w = wr[wd];
                if constexpr (BITS == 4) {
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const f16x2_t v =
                            as_f16x2(tab[(w >> (8 * b)) & 0xffu]) * s2;
                        const int kl = part * KPC + (wd * 4 + b) * 2;
                        Bs[kl * LD + wrow] = v[0];
                        Bs[(kl + 1) * LD + wrow] = v[1];
                    }
                } else {
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const f16x2_t v = as_f16x2(tab[(w >> (8 * b)) & 0xffu] & 0xffffu) * s2;
                        const int kl = part * KPC + wd * 4 + b;
                        Bs[kl * LD + wrow] = v[0];
                    }
                }
            }
        }
    };

    const int steps = (a.N + KS - 1) / KS;
    __syncthreads();
    load(0);
    for (int st = 0; st < steps; ++st) {
        store();
        __syncthreads();
        if (st + 1 < steps)
            load((st + 1) * KS);
#pragma unroll
        for (int kk = 0; kk < KS / 16; ++kk) {
            f16x8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *(const f16x8_t *)&As[(wm * 64 + i * 32 + (lane & 31)) * LD + kk * 16 +
                                               (lane >> 5) * 8];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *(const f16x8_t *)&Bs[(wk * 64 + j * 32 + (lane & 31)) * LD + kk * 16 +
                                               (lane >> 5) * 8];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                const int col = wk * 64 + j * 32 + (lane & 31);
                const int m = m0 + row, k = k0 + col;
                if (m < a.M && k < a.K)
                    store_from_f32(a.gx, a.gx_dtype, (int64_t)m * a.ldgx + k,
                                   ldexpf(acc[i][j][r], s_e[row]));
            }
}

// G tile (k x n) = x^T . gy, reduced into grad_scale and per-workgroup
// codebook-gradient partials.  4-bit indices (levels <= 16), bf16 gy / x.
__global__ void __launch_bounds__(256) dw_kernel(BwdArgs a)
{
    __shared__ __align__(16) __bf16 Xs[T * LD];   // x^T  [k][m]
    __shared__ __align__(16) __bf16 Gs[T * LD];   // gy^T [n][m]
    __shared__ uint8_t Ps[T * (T / 2)];           // packed bytes of the tile [n][k/2]
    __shared__ float Ss[T * 4];                   // scale[n][g] for the tile's groups
    __shared__ float cbf[16];
    __shared__ float hist[16 * 256];              // private per-thread level histograms
    __shared__ float gsp[2][T * 4];               // grad_scale partials per k-wave

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wk = wave >> 1, wn = wave & 1;
    const int k0 = blockIdx.x * T, n0 = blockIdx.y * T;
    const int gpt = T / a.group;  // groups per tile (1, 2 or 4)

    if (tid < 16)
        cbf[tid] = tid < a.levels ? load_as_f32(a.cb, a.cb_dtype, tid) : 0.0f;
    for (int i = tid; i < 16 * 256; i += 256)
        hist[i] = 0.0f;
    for (int i = tid; i < T * gpt; i += 256) {
        const int nl = i / gpt, gi = i % gpt;
        const int n = n0 + nl;
        Ss[nl * 4 + gi] =
            n < a.N ? load_as_f32(a.scale, a.scale_dtype, (int64_t)n * a.lds + k0 / a.group + gi)
                    : 0.0f;
    }
    for (int i = tid; i < T * (T / 2) / 16; i += 256) {
        const int nl = i / (T / 32), part = i % (T / 32);
        const int n = n0 + nl;
        u32x4_t v = (u32x4_t){0, 0, 0, 0};
        if (n < a.N)
            v = *(const u32x4_t *)(a.packed + (int64_t)n * (a.K / 2) + k0 / 2 + part * 16);
        *(u32x4_t *)&Ps[nl * (T / 2) + part * 16] = v;
    }

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[i][j][r] = 0.0f;

    // staging: x tile [32 m x 128 k] and gy tile [32 m x 128 n], bf16;
    // thread -> row m = tid / 8, 16 consecutive columns (two 16-byte loads)
    u32x4_t xr[2], gr[2];
    auto load = [&](int mb) {
        const int r = tid >> 3, c0 = (tid & 7) * 16;
        const int m = mb + r;
        const bool ok = m < a.M;
        const uint16_t *xp = (const uint16_t *)a.x + (int64_t)m * a.ldx + k0 + c0;
        const uint16_t *gp = (const uint16_t *)a.gy + (int64_t)m * a.ldgy + n0 + c0;
        xr[0] = ok ? *(const u32x4_t *)xp : (u32x4_t){0, 0, 0, 0};
        xr[1] = ok ? *(const u32x4_t *)(xp + 8) : (u32x4_t){0, 0, 0, 0};
        const bool okn = ok && n0 + c0 < a.N;
        gr[0] = okn ? *(const u32x4_t *)gp : (u32x4_t){0, 0, 0, 0};
        gr[1] = okn ? *(const u32x4_t *)(gp + 8) : (u32x4_t){0, 0, 0, 0};
    };
    auto store = [&]() {
        const int r = tid >> 3, c0 = (tid & 7) * 16;
        uint16_t *xs = (uint16_t *)Xs, *gs = (uint16_t *)Gs;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = c0 + h * 8 + 2 * e;
                xs[c * LD + r] = (uint16_t)(xr[h][e] & 0xffffu);
                xs[(c + 1) * LD + r] = (uint16_t)(xr[h][e] >> 16);
                gs[c * LD + r] = (uint16_t)(gr[h][e] & 0xffffu);
                gs[(c + 1) * LD + r] = (uint16_t)(gr[h][e] >> 16);
            }
    };

    const int steps = (a.M + KS - 1) / KS;
    __syncthreads();
    load(0);
    for (int st = 0; st < steps; ++st) {
        store();
        __syncthreads();
        if (st + 1 < steps)
            load((st + 1) * KS);
#pragma unroll
        for (int kk = 0; kk < KS / 16; ++kk) {
            bf16x8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *(const bf16x8_t *)&Xs[(wk * 64 + i * 32 + (lane & 31)) * LD + kk * 16 +
                                                (lane >> 5) * 8];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *(const bf16x8_t *)&Gs[(wn * 64 + j * 32 + (lane & 31)) * LD + kk * 16 +
                                                (lane >> 5) * 8];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // ---- epilogue: G[k][n] -> grad_scale partials and level histograms ----
    // D[row][col] of a 32x32 tile sits in lane col + 32 * ((row / 4) % 2),
    // register (row % 4) + 4 * (row / 8); rows are k, cols are n.
    float *my_hist = hist + tid;  // slot [level * 256 + tid]
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int nl = wn * 64 + j * 32 + (lane & 31);
        float gs_acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kl = wk * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                const uint8_t byte = Ps[nl * (T / 2) + (kl >> 1)];
                const int lev = (kl & 1) ? (byte >> 4) : (byte & 15);
                const float g = acc[i][j][r];
                const int gi = kl / a.group;
                gs_acc[gi] = fmaf(g, cbf[lev], gs_acc[gi]);
                my_hist[lev * 256] += g * Ss[nl * 4 + gi];
            }
        // lanes l and l + 32 hold the same n
#pragma unroll
        for (int gi = 0; gi < 4; ++gi)
            gs_acc[gi] += __shfl_xor(gs_acc[gi], 32, 64);
        if (lane < 32)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi)
                gsp[wk][nl * 4 + gi] = gs_acc[gi];
    }
    __syncthreads();
    for (int i = tid; i < T * gpt; i += 256) {
        const int nl = i / gpt, gi = i % gpt;
        const int n = n0 + nl;
        if (n < a.N)
            a.gscale[(int64_t)n * a.ldgs + k0 / a.group + gi] =
                gsp[0][nl * 4 + gi] + gsp[1][nl * 4 + gi];
    }
    if (tid < 16) {
        float s = 0.0f;
        for (int t = 0; t < 256; ++t)
            s += hist[tid * 256 + t];
        a.gc_part[((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * 16 + tid] = s;
    }
}

// grad_cb[l] = sum over workgroups (fixed order) of the partials.
__global__ void __launch_bounds__(256) gc_final_kernel(const float *part, int nwg, int levels,
                                                       float *gcb)
{
    __shared__ float red[256];
    const int lev = blockIdx.x, t = threadIdx.x;
    float s = 0.0f;
    for (int w = t; w < nwg; w += 256)
        s += part[(int64_t)w * 16 + lev];
    red[t] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (t < o)
            red[t] += red[t + o];
        __syncthreads();
    }
    if (t == 0 && lev < levels)
        gcb[lev] = red[0];
}

}  // namespace

size_t backward_workspace(int64_t M, int64_t N, int64_t K, int levels, int group)
{
    (void)levels;
    (void)group;
    const int64_t nwg = ((K + T - 1) / T) * ((N + T - 1) / T);
    return (size_t)((M * 4 + 255) / 256 * 256) + (size_t)nwg * 16 * sizeof(float);
}

bool backward_serves(const PackedDesc &w, int gy_dtype, int x_dtype)
{
    // gy is staged in 16-column chunks, so N % 16 == 0 keeps every load in its row.
    return w.levels <= 16 && w.K % T == 0 && T % w.group == 0 && T / w.group <= 4 &&
           w.N % 16 == 0 && gy_dtype == EP_BF16 && x_dtype == EP_BF16 && w.N <= INT32_MAX &&
           w.K <= INT32_MAX;
}

int launch_backward(const PackedDesc &w, const ActDesc &gy, const ActDesc &x, int64_t M,
                    const OutDesc &gx, float *grad_cb, float *grad_scale, int64_t ld_gscale,
                    void *ws, size_t ws_bytes, hipStream_t stream)
{
    if (!backward_serves(w, gy.dtype, x.dtype))
        return set_error(EP_DECLINE_SHAPE,
                         "fused backward serves levels <= 16, K %% 128 == 0, N %% 16 == 0, group "
                         "in {32, 64, 128}, bf16 gy and x");
    if (M <= 0 || w.N <= 0)
        return EP_OK;
    const size_t need = backward_workspace(M, w.N, w.K, w.levels, w.group);
    if (!ws || ws_bytes < need)
        return set_error(EP_ERR_WORKSPACE, "backward workspace of %zu bytes needed, %zu given",
                         need, ws_bytes);
    if (((uintptr_t)gy.ptr & 15) || ((uintptr_t)x.ptr & 15) || (gy.ld % 8) || (x.ld % 8) ||
        ((uintptr_t)w.packed & 15))
        return set_error(EP_DECLINE_SHAPE, "fused backward needs 16-byte aligned rows");
    BwdArgs a{};
    a.gy = gy.ptr;
    a.gy_dtype = gy.dtype;
    a.ldgy = gy.ld;
    a.x = x.ptr;
    a.ldx = x.ld;
    a.packed = w.packed;
    a.scale = w.scale;
    a.scale_dtype = w.scale_dtype;
    a.lds = w.ld_scale;
    a.cb = w.cb;
    a.cb_dtype = w.cb_dtype;
    a.levels = w.levels;
    a.group = w.group;
    a.M = (int)M;
    a.N = (int)w.N;
    a.K = (int)w.K;
    a.gx = gx.ptr;
    a.gx_dtype = gx.dtype;
    a.ldgx = gx.ld;
    a.gscale = grad_scale;
    a.ldgs = ld_gscale;
    a.rexp = (const int *)ws;
    a.gc_part = (float *)((char *)ws + (M * 4 + 255) / 256 * 256);
    if (gx.ptr) {
        hipLaunchKernelGGL(row_exp_gy_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream,
                           gy.ptr, gy.dtype, gy.ld, (int)M, (int)w.N, (int *)ws);
        EP_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(dx_kernel<4>, dim3((unsigned)((w.K + T - 1) / T), (unsigned)((M + T - 1) / T)),
                           dim3(256), 0, stream, a);
        EP_HIP_CHECK(hipGetLastError());
    }
    if (grad_cb || grad_scale) {
        float *gs_dummy = nullptr;
        if (!grad_scale)
            return set_error(EP_ERR_ARG, "grad_cb without grad_scale is not served");
        (void)gs_dummy;
        const dim3 grid((unsigned)(w.K / T), (unsigned)((w.N + T - 1) / T));
        hipLaunchKernelGGL(dw_kernel, grid, dim3(256), 0, stream, a);
        EP_HIP_CHECK(hipGetLastError());
        if (grad_cb) {
            hipLaunchKernelGGL(gc_final_kernel, dim3(16), dim3(256), 0, stream, a.gc_part,
                               (int)(grid.x * grid.y), w.levels, grad_cb);
            EP_HIP_CHECK(hipGetLastError());
        }
    }
    return EP_OK;
}

}  // namespace ep
