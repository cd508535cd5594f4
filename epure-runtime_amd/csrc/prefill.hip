// Prefill (M > 64 rows) fused codebook dequant-matmul on gfx950 MFMA.
//
// y[M, N] = x[M, K] . W[N, K]^T, W[n, k] = cb[idx[n, k]] * scale[n, k / group],
// for row counts where the contraction is compute-bound.  Reference
// behaviour: the table kernel epure/kernels/_triton.py:54-107 (fp16 operands,
// fp32 accumulation) and, for the dense tile, materialize(float16)
// (runtime.py:78-89): the weight enters the product as fp16(fp16(cb) * fp16(scale)).
//
// Layout of the work (v_mfma_f32_32x32x16_f16):
//  * a workgroup is 4 waves and covers 4 x 32 NT weight rows x BM activation
//    rows; each wave owns NT 32-row N tiles and all BM rows, so every weight
//    is dequantized exactly once per workgroup, in registers, straight into
//    the B operand -- the dense weight never reaches LDS or global memory.
//    Dequantization is the VALU-heavy part, so the MFMAs per dequantized
//    weight (BM / 32) set the pace: 8-bit at M >= 256 runs BM = 128 with one
//    N tile per wave (64 accumulators; two N tiles would not fit 256 VGPRs),
//    ~1.25x the 64 x 2-tile layout; 4-bit runs 128 x 1 at M = 256..1023 and
//    128 x 2 from 1024;
//  * lane (j = lane & 31, h = lane >> 5) of a wave holds, per 64-k step and
//    N tile, 32 consecutive weights of row j (k = 32 h .. 32 h + 31 of the
//    step: one 16-byte load at 4 bits, two at 8 bits); MFMA sub-step s takes
//    weights 8 s .. 8 s + 7 of them as its k slots 8 h .. 8 h + 7, and the
//    activation operand is read from LDS with the same k mapping;
//  * dequantization is one LDS lookup per packed byte in a 256-entry table
//    replicated 32 times (lane & 31 reads its own copy: no bank conflicts),
//    then the group scale is applied in fp16 (v_pk_mul_f16);
//  * activations are converted once to fp16 after the exact per-row
//    power-of-two rescale by a pre-kernel (pf_prep_kernel, into the
//    workspace) and staged in LDS as they are, double buffered: step k + 1
//    is stored while step k is multiplied;
//  * weight loads run PD steps ahead in registers (buffer loads: a row past
//    N or a step past K reads zeros without touching memory);
//  * when the grid of (N / 256) x (M / BM) workgroups cannot fill the device,
//    K is split and the f32 partials are summed in split order by the
//    reduction shared with the small-M path (deterministic).
#include "ep_common.h"
#include "ep_internal.h"
#include "gemv_core.h"

#include <type_traits>

namespace ep {
namespace {

constexpr int kPfThreads = 256;        // 4 waves
constexpr int kPfWaves = 4;            // waves per workgroup, 32 * NT weight rows each
constexpr int kPfBK = 64;              // k per step
constexpr int kPfCopies = 32;          // LDS table replicas
constexpr uint32_t kPfOut = 0x7ffffff0u;  // a buffer offset past every buffer's end

struct PfArgs {
    const void *x;
    int64_t ldx;
    int M;
    const uint8_t *packed;
    uint32_t row_bytes;
    const void *scale;
    int64_t lds;
    const void *cb;
    int cb_dtype;
    int levels;
    int N;
    int K;
    int group;
    int ksteps;   // k steps per split (a multiple of the unroll)
    const int *rexp;
    uint32_t xbytes, wbytes, sbytes, cbbytes;
    void *y;
    int y_dtype;
    int64_t ldy;
    int accumulate;  // with one split: y += result (read in the epilogue)
    float *part;     // [S][M][N] partials (null: results go straight to y)
};

EP_DEV __amdgpu_buffer_rsrc_t pf_rsrc(const void *p, uint32_t bytes)
{
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((uint64_t)hi << 32) | lo), 0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Per-row exponent of the largest |x| (row_exponent), then the row rescaled
// by 2^-e and rounded to fp16 into xh [M][K] (one wave per row, 16-byte
// loads, four in flight per lane; the second pass re-reads the row from the
// caches).  Converting once here saves the main kernel a conversion per
// N tile.
__global__ void __launch_bounds__(256)
    pf_prep_kernel(const void *x, int xdt, int64_t ldx, int M, int K, int *rexp, f16_t *xh)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M)
        return;
    const int esz = xdt == EP_F32 ? 4 : 2;
    const int pieces = K * esz / 16;
    const char *base = (const char *)x + (int64_t)row * ldx * esz;
    float amax = 0.0f;
    for (int p0 = lane; p0 < pieces; p0 += 256) {
        u32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int p = p0 + 64 * u;
            v[u] = p < pieces ? *(const __attribute__((address_space(1))) u32x4_t *)(base + (int64_t)p * 16)
                              : (u32x4_t){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t r = v[u][t];
                if (xdt == EP_F32) {
                    amax = fmaxf(amax, fabsf(__uint_as_float(r)));
                } else {
                    float lo, hi;
                    if (xdt == EP_BF16)
                        unpack_pair<EP_BF16>(r, lo, hi);
                    else
                        unpack_pair<EP_F16>(r, lo, hi);
                    amax = fmaxf(amax, fmaxf(fabsf(lo), fabsf(hi)));
                }
            }
    }
    amax = wave_max(amax);
    const int e = row_exponent(amax);
    if (lane == 0)
        rexp[row] = e;
    const float pw = ldexpf(1.0f, -e);
    // output pieces of 8 values: 16 input bytes (2-byte types) or 32 (f32)
    f16x8_t *dst = (f16x8_t *)(xh + (int64_t)row * K);
    for (int q = lane; q < K / 8; q += 64) {
        float v[8];
        if (xdt == EP_F32) {
            const u32x4_t a0 = *(const __attribute__((address_space(1))) u32x4_t *)(base + (int64_t)q * 32);
            const u32x4_t a1 = *(const __attribute__((address_space(1))) u32x4_t *)(base + (int64_t)q * 32 + 16);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                v[t] = __uint_as_float(a0[t]);
                v[4 + t] = __uint_as_float(a1[t]);
            }
        } else {
            const u32x4_t a0 = *(const __attribute__((address_space(1))) u32x4_t *)(base + (int64_t)q * 16);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (xdt == EP_BF16)
                    unpack_pair<EP_BF16>(a0[t], v[2 * t], v[2 * t + 1]);
                else
                    unpack_pair<EP_F16>(a0[t], v[2 * t], v[2 * t + 1]);
            }
        }
        f16x8_t h;
#pragma unroll
        for (int t = 0; t < 8; ++t)
            h[t] = (f16_t)(v[t] * pw);
        dst[q] = h;
    }
}

template <int BITS, int BM, int PD, int NT>
__global__ void __launch_bounds__(kPfThreads, 2) pf_kernel(PfArgs a)
{
    constexpr int MT = BM / 32;                  // 32-row M tiles per wave
    constexpr int XLD = kPfBK + 8;               // halfs per staged activation row
    constexpr int TPR = kPfThreads / BM;         // staging threads per activation row
    constexpr int VPT = kPfBK / TPR;             // values per staging thread and step
    constexpr int XE = 2;  // activations: fp16, pre-scaled per row (pf_prep_kernel)
    constexpr int XP = VPT * XE / 16;            // 16-byte pieces per staging thread
    constexpr int WL = BITS == 4 ? 1 : 2;        // 16-byte weight loads per lane, N tile and step
    constexpr int NB = (PD > 2 ? PD : 2) + 1;    // register sets (weights PD, activations 2 steps ahead)
    static_assert(VPT % 8 == 0, "staging in 8-value pieces");
    static_assert(kPfThreads == 256, "one table entry per thread");

    __shared__ __align__(16) uint32_t tab[256 * kPfCopies];
    __shared__ __align__(16) f16_t xs[2][BM * XLD];
    __shared__ uint32_t s_cbraw[kPfThreads];
    __shared__ uint16_t s_cb16[256];
    __shared__ int s_e[BM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int nw = blockIdx.x * (kPfWaves * 32 * NT) + wave * (32 * NT);  // the wave's first weight row
    const int m0 = blockIdx.y * BM;
    const int kt0 = blockIdx.z * a.ksteps;
    const int nk = a.K / kPfBK;
    const auto rx = pf_rsrc(a.x, a.xbytes), rw = pf_rsrc(a.packed, a.wbytes);
    const auto rs = pf_rsrc(a.scale, a.sbytes), rcb = pf_rsrc(a.cb, a.cbbytes);

    // ---- first loads: codebook, row exponents, step 0's activations
    const uint32_t cbraw = __builtin_amdgcn_raw_buffer_load_b32(rcb, tid * 4, 0, 0);
    const int xr = tid / TPR, xq = tid % TPR;
    const int xm = m0 + xr;
    const int ex = *(const __attribute__((address_space(1))) int *)(a.rexp + (xm < a.M ? xm : 0));

    auto issue_x = [&](int kt, u32x4_t (&xv)[XP]) {
        const int k = kt * kPfBK + xq * VPT;
        const bool ok = xm < a.M && kt < nk && kt < kt0 + a.ksteps;
        const uint32_t off = (uint32_t)(((int64_t)xm * a.ldx + k) * XE);
#pragma unroll
        for (int p = 0; p < XP; ++p)
            xv[p] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (int)(off + 16 * p) : (int)kPfOut, 0, 0);
    };
    auto issue_w = [&](int kt, u32x4_t (&w)[NT][WL], uint32_t (&sr)[NT][WL]) {
        const bool kok = kt < nk && kt < kt0 + a.ksteps;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = nw + nt * 32 + j;
            const bool ok = kok && n < a.N;
#pragma unroll
            for (int l = 0; l < WL; ++l) {
                const int k = kt * kPfBK + 32 * h + 16 * l;  // first k of the 16-byte piece (8-bit) / 32 (4-bit)
                const uint32_t off = (uint32_t)n * a.row_bytes + (uint32_t)(BITS == 4 ? k / 2 : k);
                w[nt][l] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? (int)off : (int)kPfOut, 0, 0);
                const uint32_t soff = (uint32_t)(((int64_t)n * a.lds + k / a.group) * 2);
                sr[nt][l] = __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? (int)soff : (int)kPfOut, 0, 0);
            }
        }
    };

    // NB register sets, rotated with static indices: weights run PD steps
    // ahead, activations two steps ahead (stored to LDS one step ahead)
    u32x4_t xv[NB][XP];
    u32x4_t wb[NB][NT][WL];
    uint32_t sb[NB][NT][WL];
    issue_x(kt0, xv[0]);
    issue_x(kt0 + 1, xv[1]);
#pragma unroll
    for (int d = 0; d < PD; ++d)
        issue_w(kt0 + d, wb[d], sb[d]);
    __builtin_amdgcn_sched_barrier(0);

    auto store_x = [&](const u32x4_t (&v4)[XP], f16_t *dst) {
#pragma unroll
        for (int p = 0; p < XP; ++p)
            *(u32x4_t *)(dst + 8 * p) = v4[p];
    };

    // codebook -> fp16 -> the replicated table; step 0's activations -> LDS
    s_cbraw[tid] = cbraw;
    if (tid < BM)
        s_e[tid] = 0;
    lds_barrier();
    {
        float c = 0.0f;
        if (tid < a.levels) {
            if (a.cb_dtype == EP_F32) {
                c = __uint_as_float(s_cbraw[tid]);
            } else {
                const uint16_t hb = (uint16_t)(s_cbraw[tid >> 1] >> (16 * (tid & 1)));
                c = a.cb_dtype == EP_F16 ? (float)f16_from_bits(hb) : bf16_to_f32(hb);
            }
        }
        // fp16 bits of the entries (past levels: 0, the Rust LUT's zeros)
        s_cb16[tid] = tid < a.levels ? f16_bits((f16_t)c) : (uint16_t)0;
        lds_barrier();
        // entry t: (cb[t & 15], cb[t >> 4]) at 4 bits, cb[t] twice at 8 bits
        const uint32_t v = BITS == 4 ? ((uint32_t)s_cb16[tid & 15] | ((uint32_t)s_cb16[tid >> 4] << 16))
                                     : ((uint32_t)s_cb16[tid] | ((uint32_t)s_cb16[tid] << 16));
        u32x4_t *row = (u32x4_t *)(tab + tid * kPfCopies);
#pragma unroll
        for (int i = 0; i < kPfCopies / 4; ++i)
            row[i] = (u32x4_t){v, v, v, v};
    }
    if (tid % TPR == 0 && xm < a.M)
        s_e[xr] = ex;
    store_x(xv[0], xs[0] + xr * XLD + xq * VPT);
    lds_barrier();

    f32x16_t acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[mt][nt][r] = 0.0f;

    const uint32_t c8 = (uint32_t)(lane & 31) << 3;  // (copy << 2) << 1: the address is halved below
    // One step (register set r = (kt - kt0) % NB): issue step kt + 2's
    // activations and step kt + PD's weights, multiply step kt, store step
    // kt + 1's activations.
    auto step = [&](int kt, auto rc) {
        constexpr int r = decltype(rc)::value;
        issue_x(kt + 2, xv[(r + 2) % NB]);
        issue_w(kt + PD, wb[(r + PD) % NB], sb[(r + PD) % NB]);
        // the loads above stay here, ahead of the work below (the scheduler
        // would otherwise sink them next to their use)
        __builtin_amdgcn_sched_barrier(0);
        const f16_t *xa = xs[(kt - kt0) & 1];
        u32x4_t (&wc)[NT][WL] = wb[r];
        uint32_t (&sc)[NT][WL] = sb[r];
        f16x2_t pr[NT][16];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
            for (int l = 0; l < WL; ++l) {
                const f16_t s16 = f16_from_bits((uint16_t)sc[nt][l]);
                const f16x2_t s2 = (f16x2_t){s16, s16};
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    const uint32_t word = wc[nt][l][wd];
                    if constexpr (BITS == 4) {
#pragma unroll
                        for (int b = 0; b < 4; ++b)
                            pr[nt][wd * 4 + b] =
                                as_f16x2(lds_read_u32(tab, __builtin_amdgcn_perm(word, c8, kSelByte[b]) >> 1)) * s2;
                    } else {
                        const uint32_t t0 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c8, kSelByte[0]) >> 1);
                        const uint32_t t1 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c8, kSelByte[1]) >> 1);
                        const uint32_t t2 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c8, kSelByte[2]) >> 1);
                        const uint32_t t3 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c8, kSelByte[3]) >> 1);
                        pr[nt][l * 8 + wd * 2] = as_f16x2(__builtin_amdgcn_perm(t1, t0, 0x05040100u)) * s2;
                        pr[nt][l * 8 + wd * 2 + 1] = as_f16x2(__builtin_amdgcn_perm(t3, t2, 0x05040100u)) * s2;
                    }
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            f16x8_t av[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                av[mt] = *(const f16x8_t *)(xa + (mt * 32 + j) * XLD + 32 * h + 8 * s);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f16x8_t bv = {pr[nt][4 * s][0],     pr[nt][4 * s][1],     pr[nt][4 * s + 1][0],
                                    pr[nt][4 * s + 1][1], pr[nt][4 * s + 2][0], pr[nt][4 * s + 2][1],
                                    pr[nt][4 * s + 3][0], pr[nt][4 * s + 3][1]};
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv, acc[mt][nt], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        store_x(xv[(r + 1) % NB], xs[(kt + 1 - kt0) & 1] + xr * XLD + xq * VPT);
        // LDS-only barrier: __syncthreads() would also wait for the loads
        // in flight
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    // ksteps is a multiple of NB; steps past K read zeros and add nothing
    for (int kt = kt0; kt < kt0 + a.ksteps; kt += NB) {
        step(kt, std::integral_constant<int, 0>{});
        step(kt + 1, std::integral_constant<int, 1>{});
        step(kt + 2, std::integral_constant<int, 2>{});
        if constexpr (NB > 3)
            step(kt + 3, std::integral_constant<int, 3 % NB>{});
        if constexpr (NB > 4)
            step(kt + 4, std::integral_constant<int, 4 % NB>{});
    }

    // D[row][col] of a 32x32 tile: lane col + 32 * ((row / 4) % 2), register
    // (row % 4) + 4 * (row / 8)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = nw + nt * 32 + j;
            if (n >= a.N)
                continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = mt * 32 + (r % 4) + 4 * h + 8 * (r / 4);
                const int m = m0 + row;
                if (m >= a.M)
                    continue;
                const float v = ldexpf(acc[mt][nt][r], s_e[row]);
                if (a.part) {
                    *(__attribute__((address_space(1))) float *)(a.part + ((int64_t)blockIdx.z * a.M + m) * a.N + n) = v;
                } else {
                    const int64_t off = (int64_t)m * a.ldy + n;
                    store_from_f32(a.y, a.y_dtype, off, a.accumulate ? v + load_as_f32(a.y, a.y_dtype, off) : v);
                }
            }
        }
}

// Tile rows, weight prefetch depth and K split for a shape.
// 8-bit tiling knobs (measured: weight prefetch depth 2-4 within 1%)
#ifndef EP_PF_BIG8_M
#define EP_PF_BIG8_M 256  // M from which 8-bit runs BM = 128, one N tile per wave
#endif
#ifndef EP_PF_PD8
#define EP_PF_PD8 3
#endif
struct PfPlan {
    int bm, pd, nt, S, ksteps;
};

PfPlan pf_plan(int bits, int64_t M, int64_t N, int64_t K)
{
    PfPlan p;
    if (bits == 4) {
        // measured: 128 x 2 tiles lead from M = 1024, 128 x 1 at 256..1023
        p.bm = M >= 256 ? 128 : 64;
        p.nt = M >= 256 && M < 1024 ? 1 : 2;
        p.pd = p.bm == 128 && p.nt == 2 ? 2 : 4;
    } else if (M >= EP_PF_BIG8_M) {
        p.bm = 128;
        p.pd = EP_PF_PD8;
        p.nt = 1;
    } else {
        p.bm = 64;
        p.pd = 3;
        p.nt = 2;
    }
    const int nb = (p.pd > 2 ? p.pd : 2) + 1;
    const int bn = kPfWaves * 32 * p.nt;
    const int64_t tiles = ((N + bn - 1) / bn) * ((M + p.bm - 1) / p.bm);
    const int nk = (int)(K / kPfBK);
    const int target = 2 * device_cus();  // two resident workgroups per CU
    int S = 1;
    while (tiles * S < target && S < 8 && nk / (S * 2) >= 8)
        S *= 2;
    int ks = (nk + S - 1) / S;
    ks = (ks + nb - 1) / nb * nb;
    p.S = (nk + ks - 1) / ks;
    p.ksteps = ks;
    return p;
}

template <int BITS, int BM, int PD, int NT>
int pf_launch(const PfArgs &a, const PfPlan &p, hipStream_t s)
{
    constexpr int BN = kPfWaves * 32 * NT;
    const dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM), (unsigned)p.S);
    hipLaunchKernelGGL((pf_kernel<BITS, BM, PD, NT>), grid, dim3(kPfThreads), 0, s, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

}  // namespace

bool prefill_serves(const PackedDesc &w, const ActDesc &x, int64_t M)
{
    const int bits = w.bits();
    if (M < 1 || M > ((int64_t)1 << 24) || w.N < 1 || w.K < kPfBK || w.K % kPfBK != 0)
        return false;
    if (w.scale_dtype != EP_F16 || w.group % (bits == 4 ? 32 : 16) != 0)
        return false;
    const int esz = x.dtype == EP_F32 ? 4 : 2;
    const int64_t rb = bits == 4 ? w.K / 2 : w.K;
    const int64_t G = (w.K + w.group - 1) / w.group;
    if (w.N * rb > kPfOut || ((M - 1) * x.ld + w.K) * esz > kPfOut || ((w.N - 1) * w.ld_scale + G) * 2 > kPfOut)
        return false;
    if (((uintptr_t)w.packed & 15) != 0 || ((uintptr_t)x.ptr & 15) != 0)
        return false;
    return (x.ld * esz) % 16 == 0;
}

// Workspace: row exponents, the fp16 activations, then the split partials.
size_t prefill_workspace(int64_t M, int64_t N, int64_t K, int levels)
{
    const PfPlan p = pf_plan(levels <= 16 ? 4 : 8, M, N, K);
    const size_t ex = (size_t)((M * 4 + 255) / 256 * 256);
    const size_t xh = (size_t)((M * K * 2 + 255) / 256 * 256);
    return ex + xh + (p.S > 1 ? (size_t)p.S * (size_t)M * (size_t)N * sizeof(float) : 0);
}

int launch_prefill(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y, void *ws,
                   size_t ws_bytes, hipStream_t stream)
{
    if (!prefill_serves(w, x, M))
        return EP_DECLINE_SHAPE;
    const int bits = w.bits();
    const PfPlan p = pf_plan(bits, M, w.N, w.K);
    const bool partials = p.S > 1;
    const size_t ex = (size_t)((M * 4 + 255) / 256 * 256);
    const size_t xhb = (size_t)((M * w.K * 2 + 255) / 256 * 256);
    const size_t need = ex + xhb + (partials ? (size_t)p.S * (size_t)M * (size_t)w.N * sizeof(float) : 0);
    if (!ws || ws_bytes < need)
        return set_error(EP_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws_bytes);
    int *rexp = (int *)ws;
    f16_t *xh = (f16_t *)((char *)ws + ex);
    hipLaunchKernelGGL(pf_prep_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream, x.ptr, x.dtype,
                       x.ld, (int)M, (int)w.K, rexp, xh);
    EP_HIP_CHECK(hipGetLastError());
    PfArgs a{};
    a.xbytes = (uint32_t)(M * w.K * 2);
    a.wbytes = (uint32_t)(w.N * (bits == 4 ? w.K / 2 : w.K));
    a.sbytes = (uint32_t)(((w.N - 1) * w.ld_scale + (w.K + w.group - 1) / w.group) * 2);
    a.cbbytes = (uint32_t)(w.levels * (w.cb_dtype == EP_F32 ? 4 : 2));
    a.x = xh;
    a.ldx = w.K;
    a.M = (int)M;
    a.packed = w.packed;
    a.row_bytes = (uint32_t)(bits == 4 ? w.K / 2 : w.K);
    a.scale = w.scale;
    a.lds = w.ld_scale;
    a.cb = w.cb;
    a.cb_dtype = w.cb_dtype;
    a.levels = w.levels;
    a.N = (int)w.N;
    a.K = (int)w.K;
    a.group = w.group;
    a.ksteps = p.ksteps;
    a.rexp = rexp;
    a.y = y.ptr;
    a.y_dtype = y.dtype;
    a.ldy = y.ld;
    a.accumulate = y.accumulate;
    a.part = partials ? (float *)((char *)ws + ex + xhb) : nullptr;
    int rc;
    if (bits == 4)
        rc = p.nt == 1 ? pf_launch<4, 128, 4, 1>(a, p, stream)
             : p.bm == 128 ? pf_launch<4, 128, 2, 2>(a, p, stream) : pf_launch<4, 64, 4, 2>(a, p, stream);
    else
        rc = p.nt == 1 ? pf_launch<8, 128, EP_PF_PD8, 1>(a, p, stream) : pf_launch<8, 64, 3, 2>(a, p, stream);
    if (rc != EP_OK || !partials)
        return rc;
    return launch_split_reduce(a.part, p.S, M, w.N, y, stream);
}

}  // namespace ep
