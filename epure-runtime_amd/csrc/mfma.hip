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
#include "gemv_core.h"

#include <type_traits>

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
    // grouped experts (mm_kernel<..., true>): row tile blockIdx.y is entry
    // tiles[4 y ..] = (expert, first sorted row, rows, 0) while y < *ntiles;
    // sorted row p is token perm[p] (its x row, y row and exponent); the
    // expert's weight rows start estride_w bytes / estride_s scales further
    const int *perm;
    const int *tiles;
    const int *ntiles;
    int64_t estride_w, estride_s;
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

template <int BITS, int BM, int BN, int WM, int WN, int XDT, bool GR = false>
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
    __shared__ int s_row[GR ? BM : 1];  // grouped: token of each tile row (-1: none)

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    int gstart = 0, gcount = 0;
    if constexpr (GR) {
        // tiles past the sorted expert runs do nothing (uniform exit)
        if ((int)blockIdx.y >= *a.ntiles)
            return;
        const int *tl = a.tiles + 4 * blockIdx.y;
        const int e = tl[0];
        gstart = tl[1];
        gcount = tl[2];
        a.packed += (int64_t)e * a.estride_w;
        a.scale = (const char *)a.scale + e * a.estride_s * (a.scale_dtype == EP_F32 ? 4 : 2);
    }

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
        int e;
        if constexpr (GR) {
            const int t = r < gcount ? a.perm[gstart + r] : -1;
            s_row[r] = t;
            e = t >= 0 ? a.rexp[t] : 0;
        } else {
            const int m = m0 + r;
            e = m < a.M ? a.rexp[m] : 0;
        }
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

    // register staging, PD K-steps of loads in flight: every load goes out
    // unconditionally (a row past M or N reads row 0 of its buffer and is
    // zeroed at the store), and the scale's raw bits are converted at the
    // store, so no wait for a load sits before the MFMAs of the steps ahead
    constexpr int PD = 3;
    constexpr int XW = XDT == EP_F32 ? 2 : 1;
    u32x4_t xr[PD][XCH][XW];
    u32x4_t wr[PD][WCH];
    uint32_t wsr[PD][WCH];
    const int KT = (int)(a.K / BK);

    auto load_step = [&](int kt, auto dc) {
        constexpr int d = decltype(dc)::value;
        const int64_t kbase = (int64_t)(kt < KT ? kt : KT - 1) * BK;
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / (BK / 8), col = (c % (BK / 8)) * 8;
            const int m = GR ? s_row[r] : m0 + r;
            const bool ok = GR ? m >= 0 : m < a.M;
            const int64_t mm = ok ? m : 0;
            if constexpr (XDT == EP_F32) {
                const float *p = (const float *)a.x + mm * a.ldx + kbase + col;
                xr[d][i][0] = *(const u32x4_t *)p;
                xr[d][i][1] = *(const u32x4_t *)(p + 4);
            } else {
                const uint16_t *p = (const uint16_t *)a.x + mm * a.ldx + kbase + col;
                xr[d][i][0] = *(const u32x4_t *)p;
            }
        }
#pragma unroll
        for (int i = 0; i < WCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / WPR, part = c % WPR;
            const int n = n0 + r < a.N ? n0 + r : 0;
            const int64_t k0 = kbase + part * KPC;
            const int64_t byte0 = BITS == 4 ? k0 / 2 : k0;
            wr[d][i] = __builtin_nontemporal_load((const u32x4_t *)(a.packed + (int64_t)n * a.row_bytes + byte0));
            const int64_t e = (int64_t)n * a.lds + k0 / a.group;
            wsr[d][i] = a.scale_dtype == EP_F32 ? ((const uint32_t *)a.scale)[e]
                                                : (uint32_t)((const uint16_t *)a.scale)[e];
        }
    };

    auto store_step = [&](auto dc) {
        constexpr int d = decltype(dc)::value;
        u32x4_t (&xrd)[XCH][XW] = xr[d];
        u32x4_t (&wrd)[WCH] = wr[d];
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / (BK / 8);
            const int m = GR ? s_row[r] : m0 + r;
            if (!(GR ? m >= 0 : m < a.M)) {
#pragma unroll
                for (int w = 0; w < XW; ++w)
                    xrd[i][w] = (u32x4_t){0u, 0u, 0u, 0u};
            }
        }
        float wsc[WCH];
#pragma unroll
        for (int i = 0; i < WCH; ++i) {
            const int c = tid + i * 256;
            const int r = c / WPR;
            const uint32_t raw = wsr[d][i];
            const float sv = a.scale_dtype == EP_F32 ? __uint_as_float(raw)
                             : (a.scale_dtype == EP_BF16 ? bf16_to_f32((uint16_t)raw)
                                                         : (float)f16_from_bits((uint16_t)raw));
            const bool nok = n0 + r < a.N;
            wsc[i] = nok ? sv : 0.0f;
            if (!nok)
                wrd[i] = (u32x4_t){0u, 0u, 0u, 0u};
        }
        u32x4_t (&xr)[XCH][XW] = xrd;
        u32x4_t (&wr)[WCH] = wrd;
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

    __syncthreads();  // table and row scales ready
    load_step(0, std::integral_constant<int, 0>{});
    load_step(1, std::integral_constant<int, 1>{});
    // one K-step on register set D: step kt + PD - 1's loads into the set
    // the previous step left, then this step's tiles into LDS and its MFMAs
    auto kstep = [&](int kt, auto dc) {
        constexpr int D = decltype(dc)::value;
        load_step(kt + PD - 1, std::integral_constant<int, (D + PD - 1) % PD>{});
        store_step(dc);
        __syncthreads();
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
    };
    for (int kt = 0; kt < KT; kt += PD) {
        kstep(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < KT)
            kstep(kt + 1, std::integral_constant<int, 1>{});
        if (kt + 2 < KT)
            kstep(kt + 2, std::integral_constant<int, 2>{});
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
                const int m = GR ? s_row[row] : m0 + row, n = n0 + col;
                if ((GR ? m >= 0 : m < a.M) && n < a.N) {
                    float v = ldexpf(acc[i][j][r], s_e[row]);
                    const int64_t off = (int64_t)m * a.ldy + n;
                    if (a.accumulate)
                        v += load_as_f32(a.y, a.y_dtype, off);
                    store_from_f32(a.y, a.y_dtype, off, v);
                }
            }
}

// Tokens grouped by expert on the device: a stable counting sort of the T
// ids (clamped into [0, E)) into perm (sorted row p -> token) and the row
// tiles of BM rows of each expert's run (tiles[4 i ..] = expert, first
// sorted row, rows, 0; *ntiles of them).  One wave per expert in both
// kernels: expert_count_kernel counts the expert's tokens (a ballot per 64
// ids); expert_place_kernel sums the counts of the experts before it (its
// run's start and first tile), writes its tiles, then walks the ids again
// in token order and stores each of its tokens at start + its rank (the
// popcount of the ballot below its lane), so equal ids keep their token
// order.  Every id is read once per expert from L2; deterministic, no
// atomics.
constexpr int kSortWavesPerWg = 4;
constexpr int kIdBatches = 16;  // batches of 64 ids read at once per wave
constexpr int kMaxExperts = 1024;

EP_DEV int clamp_expert(int e, int E) { return e < 0 ? 0 : (e >= E ? E - 1 : e); }

__global__ void __launch_bounds__(64 * kSortWavesPerWg)
    expert_count_kernel(const int *ids, int T, int E, int *counts)
{
    const int lane = threadIdx.x & 63;
    const int e = (int)blockIdx.x * kSortWavesPerWg + (int)(threadIdx.x >> 6);
    if (e >= E)
        return;  // a whole wave
    const auto rs = buffer_rsrc(ids, (uint32_t)T * 4u);  // ids past T read 0 (masked below)
    int c = 0;
    for (int b = 0; b < T; b += 64 * kIdBatches) {
        int v[kIdBatches];  // 16 loads in flight per lane, no branch around them
#pragma unroll
        for (int u = 0; u < kIdBatches; ++u)
            v[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs, (b + 64 * u + lane) * 4, 0, 0);
#pragma unroll
        for (int u = 0; u < kIdBatches; ++u) {
            const int t = b + 64 * u + lane;
            v[u] = t < T ? clamp_expert(v[u], E) : -1;
        }
#pragma unroll
        for (int u = 0; u < kIdBatches; ++u)
            c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(v[u] == e));
    }
    if (lane == 0)
        counts[e] = c;
}

__global__ void __launch_bounds__(64 * kSortWavesPerWg)
    expert_place_kernel(const int *ids, int T, int E, int BM, const int *counts, int *perm, int *tiles,
                        int *ntiles)
{
    const int lane = threadIdx.x & 63;
    const int e = (int)blockIdx.x * kSortWavesPerWg + (int)(threadIdx.x >> 6);
    if (e >= E)
        return;  // a whole wave
    // rows and tiles of the experts before e (lanes stride over them)
    int rows = 0, tl = 0;
    for (int f = lane; f < e; f += 64) {
        const int c = counts[f];
        rows += c;
        tl += (c + BM - 1) / BM;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        rows += __shfl_xor(rows, o, 64);
        tl += __shfl_xor(tl, o, 64);
    }
    const int cnt = counts[e];
    const int nt = (cnt + BM - 1) / BM;
    for (int j = lane; j < nt; j += 64) {
        int *d = tiles + 4 * (tl + j);
        d[0] = e;
        d[1] = rows + j * BM;
        d[2] = cnt - j * BM < BM ? cnt - j * BM : BM;
        d[3] = 0;
    }
    if (e == E - 1 && lane == 0)
        *ntiles = tl + nt;
    int pos = rows;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));  // lanes under this one
    const auto rs = buffer_rsrc(ids, (uint32_t)T * 4u);  // ids past T read 0 (masked below)
    for (int b = 0; b < T && pos < rows + cnt; b += 64 * kIdBatches) {
        int v[kIdBatches];  // 16 loads in flight per lane, then the batches in token order
#pragma unroll
        for (int u = 0; u < kIdBatches; ++u)
            v[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs, (b + 64 * u + lane) * 4, 0, 0);
#pragma unroll
        for (int u = 0; u < kIdBatches; ++u) {
            const int t = b + 64 * u + lane;
            v[u] = t < T ? clamp_expert(v[u], E) : -1;
        }
#pragma unroll
        for (int u = 0; u < kIdBatches; ++u) {
            const bool hit = v[u] == e;
            const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
            if (hit)
                perm[pos + __builtin_popcountll(m & below)] = b + 64 * u + lane;
            pos += __builtin_popcountll(m);
        }
    }
}

// Row exponents (row_exponent of the largest |x|) for 16-bit activation
// rows with 16-byte aligned starts: one wave per row, 16-byte loads, four
// in flight per lane.
template <int XDT>
__global__ void __launch_bounds__(256) row_exp16_kernel(const void *x, int64_t ldx, int M, int64_t K, int *rexp)
{
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M)
        return;
    const char *base = (const char *)x + row * ldx * 2;
    const int64_t pieces = K / 8;  // 16-byte pieces (K % 8 == 0)
    float amax = 0.0f;
    for (int64_t p0 = lane; p0 < pieces; p0 += 256) {
        u32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t p = p0 + 64 * u;
            v[u] = p < pieces ? *(const __attribute__((address_space(1))) u32x4_t *)(base + p * 16)
                              : (u32x4_t){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float lo, hi;
                unpack_pair<XDT>(v[u][q], lo, hi);
                amax = fmaxf(amax, fmaxf(fabsf(lo), fabsf(hi)));
            }
    }
    amax = wave_max_bfly(amax);
    if (lane == 0)
        rexp[row] = row_exponent(amax);
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

template <int BITS, int BM, int BN, int WM, int WN>
int launch_grouped_cfg(const MmArgs &a, int xdt, unsigned tiles_y, hipStream_t s)
{
    dim3 grid((unsigned)((a.N + BN - 1) / BN), tiles_y);
    switch (xdt) {
    case EP_BF16:
        hipLaunchKernelGGL((mm_kernel<BITS, BM, BN, WM, WN, EP_BF16, true>), grid, dim3(256), 0, s, a);
        break;
    case EP_F16:
        hipLaunchKernelGGL((mm_kernel<BITS, BM, BN, WM, WN, EP_F16, true>), grid, dim3(256), 0, s, a);
        break;
    default:
        hipLaunchKernelGGL((mm_kernel<BITS, BM, BN, WM, WN, EP_F32, true>), grid, dim3(256), 0, s, a);
        break;
    }
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

// Row tile of the grouped launch from the mean rows per expert: 32 rows up
// to 32 tokens per expert, 64 up to 64, else 128 (2 x 2 waves).
int grouped_bm(int64_t T, int64_t E)
{
    const int64_t avg = (T + E - 1) / E;
    return avg <= 32 ? 32 : (avg <= 64 ? 64 : 128);
}
int64_t grouped_max_tiles(int64_t T, int64_t E, int bm) { return (T + bm - 1) / bm + (E < T ? E : T); }

template <int BITS>
int launch_grouped_bits(const MmArgs &a, int xdt, int bm, unsigned tiles_y, hipStream_t s)
{
    if (bm == 32)
        return launch_grouped_cfg<BITS, 32, 128, 1, 4>(a, xdt, tiles_y, s);
    if (bm == 64)
        return launch_grouped_cfg<BITS, 64, 128, 1, 4>(a, xdt, tiles_y, s);
    return launch_grouped_cfg<BITS, 128, 128, 2, 2>(a, xdt, tiles_y, s);
}

}  // namespace

// Workspace of the grouped expert launch: perm [T] | tiles [T / 32 + E][4]
// | counts [E] | ntiles | the row exponents [T] and, for the prefill
// kernel, the fp16 copy of the token rows [T][K] (every part 256-byte
// aligned).
static size_t al256(int64_t b) { return (size_t)((b + 255) / 256 * 256); }
size_t expert_grouped_workspace(int64_t T, int64_t E, int64_t K)
{
    if (T <= 0 || E <= 0 || K <= 0)
        return 0;
    return al256(T * 4) + al256(grouped_max_tiles(T, E, 32) * 16) + al256(E * 4) + 256 +
           prefill_grouped_workspace(T, K);
}

bool expert_grouped_serves(const PackedDesc &w, const ActDesc &x, int64_t T, int64_t E)
{
    return E >= 1 && E <= kMaxExperts && T >= 1 && T <= (int64_t)1 << 24 && mfma_serves(w, x, T);
}

// The prefill kernel (the whole K per workgroup; 128-row tiles where the
// experts average 128 tokens or more, 64 from 32, else 32: a tile's MFMAs
// cover all of its rows, live or not) wherever its shape rules hold (fp16
// scales; at 16 / 128 / 512 / 2048 tokens of a 128 x 768 x 2048 stack,
// top-8: 46 / 67 / 87 / 215 us against 58 / 76 / 134 / 216 on the generic
// kernel; 32-row tiles against 64 at 16 / 128 tokens: 46 / 67 against 52 /
// 74 us); the generic MFMA kernel (32- or 64-row tiles) for the rest.
int launch_expert_grouped(const PackedDesc &w, const ActDesc &x, int64_t T, const int *ids, int E,
                          const OutDesc &y, void *ws, size_t ws_bytes, hipStream_t stream)
{
    if (!expert_grouped_serves(w, x, T, E))
        return set_error(EP_DECLINE_SHAPE,
                         "grouped experts: 1 <= E <= %d, T <= 2^24, K %% 64 == 0, 16-byte aligned rows", kMaxExperts);
    const size_t need = expert_grouped_workspace(T, E, w.K);
    if (!ws || ws_bytes < need)
        return set_error(EP_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws_bytes);
    char *base = (char *)ws;
    int *perm = (int *)base;
    base += al256(T * 4);
    int *tiles = (int *)base;
    base += al256(grouped_max_tiles(T, E, 32) * 16);
    int *counts = (int *)base;
    base += al256((int64_t)E * 4);
    int *ntiles = (int *)base;
    base += 256;
    int *rexp = (int *)base;  // (the prefill kernel's exponents and fp16 rows start here too)
    const int64_t avg = (T + E - 1) / E;
    const bool pf = prefill_grouped_serves(w, x, T);
    const int bm = pf ? (avg >= 128 ? 128 : avg >= 32 ? 64 : 32) : grouped_bm(T, E);
    const dim3 sg((unsigned)((E + kSortWavesPerWg - 1) / kSortWavesPerWg)), sb(64 * kSortWavesPerWg);
    hipLaunchKernelGGL(expert_count_kernel, sg, sb, 0, stream, ids, (int)T, E, counts);
    EP_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(expert_place_kernel, sg, sb, 0, stream, ids, (int)T, E, bm, counts, perm, tiles, ntiles);
    EP_HIP_CHECK(hipGetLastError());
    const unsigned ty = (unsigned)grouped_max_tiles(T, E, bm);
    if (pf)
        return launch_prefill_grouped(w, x, T, perm, tiles, ntiles, bm, ty, y, rexp, stream);
    const dim3 rg((unsigned)((T + 3) / 4));
    if (x.dtype == EP_BF16)
        hipLaunchKernelGGL(row_exp16_kernel<EP_BF16>, rg, dim3(256), 0, stream, x.ptr, x.ld, (int)T, w.K, rexp);
    else if (x.dtype == EP_F16)
        hipLaunchKernelGGL(row_exp16_kernel<EP_F16>, rg, dim3(256), 0, stream, x.ptr, x.ld, (int)T, w.K, rexp);
    else
        hipLaunchKernelGGL(row_exp_kernel, rg, dim3(256), 0, stream, x.ptr, x.dtype, x.ld, (int)T, w.K, rexp);
    EP_HIP_CHECK(hipGetLastError());
    MmArgs a{};
    a.x = x.ptr;
    a.ldx = x.ld;
    a.M = (int)T;
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
    a.accumulate = 0;
    a.N = (int)w.N;
    a.K = w.K;
    a.group = w.group;
    a.rexp = rexp;
    a.perm = perm;
    a.tiles = tiles;
    a.ntiles = ntiles;
    a.estride_w = w.N * a.row_bytes;
    a.estride_s = w.N * w.ld_scale;
    return w.bits() == 4 ? launch_grouped_bits<4>(a, x.dtype, bm, ty, stream)
                         : launch_grouped_bits<8>(a, x.dtype, bm, ty, stream);
}

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
