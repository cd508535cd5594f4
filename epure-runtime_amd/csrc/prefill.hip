// Prefill (M > 64 rows) fused codebook dequant-matmul on gfx950 MFMA.
//
// y[M, N] = x[M, K] . W[N, K]^T, W[n, k] = cb[idx[n, k]] * scale[n, k / group],
// for row counts where the contraction is compute-bound.  Reference
// behaviour: the table kernel epure/kernels/_triton.py:54-107 (fp16 operands,
// fp32 accumulation) and, for the dense tile, materialize(float16)
// (runtime.py:78-89): the weight enters the product as fp16(fp16(cb) * fp16(scale)).
//
// Layout of the work (v_mfma_f32_32x32x16_f16):
//  * a workgroup is WAVES waves and covers WAVES x 32 NT weight rows x BM
//    activation rows; each wave owns NT 32-row N tiles and all BM rows, so
//    every weight is dequantized exactly once per workgroup, in registers,
//    straight into the B operand -- the dense weight never reaches LDS or
//    global memory.  From M = 128 (8-bit) or 160 (4-bit): 8 waves x BM = 128
//    (8-bit: one N tile per wave, as two would not fit 256 VGPRs; 4-bit: one
//    tile at M < 1024, two from 1024), one workgroup per CU.  What bounds these tilings is the
//    bytes a CU pulls from L2 per k step (weights + the activation tile: a
//    CU keeps ~32 KiB of loads in flight), so wider workgroups -- more weight
//    rows per staged activation tile -- measured faster than 4-wave ones
//    (8-bit 1.1-1.15x) and than two weight tiles at 64 activation rows
//    (8-bit 1.25x); smaller M runs 4 waves x BM = 64 x two tiles;
//  * lane (j = lane & 31, h = lane >> 5) of a wave holds, per 64-k step and
//    N tile, 32 consecutive weights of row j (k = 32 h .. 32 h + 31 of the
//    step: one 16-byte load at 4 bits, two at 8 bits); MFMA sub-step s takes
//    weights 8 s .. 8 s + 7 of them as its k slots 8 h .. 8 h + 7, and the
//    activation operand is read from LDS with the same k mapping;
//  * dequantization is one LDS lookup per packed byte in a 256-entry table
//    replicated 32 times (lane & 31 reads its own copy: no bank conflicts),
//    addressed by one v_perm of the packed word, then the group scale is
//    applied in fp16 (v_pk_mul_f16);
//  * activations are converted once to fp16 after the exact per-row
//    power-of-two rescale by a pre-kernel (pf_prep_kernel, into the
//    workspace) and staged in LDS as they are, double buffered: step k + 1
//    is stored while step k is multiplied;
//  * weight loads run PD steps ahead in registers (buffer loads: a row past
//    N or a step past K reads zeros without touching memory);
//  * when the grid of (N / (32 WAVES NT)) x (M / BM) workgroups cannot fill the device,
//    K is split and the f32 partials are summed in split order by the
//    reduction shared with the small-M path (deterministic).
#include "ep_common.h"
#include "ep_internal.h"
#include "gemv_core.h"

#include <type_traits>

namespace ep {
namespace {

// A workgroup is WAVES waves (4 or 8), 32 * NT weight rows each.
constexpr int kPfBK = 64;              // k per step
constexpr int kPfCopies = 32;          // LDS table replicas
// A buffer offset past every buffer's end (buffers are at most this long);
// sums of two such parts plus a piece offset stay below 2^32.
constexpr uint32_t kPfOut = 0x7fffff00u;

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
    int gk_mul, gk_shift;  // k step kt starts in group (kt * gk_mul) >> gk_shift
    int ksteps;   // k steps per split (a multiple of the unroll)
    const int *rexp;
    uint32_t xbytes, wbytes, sbytes, cbbytes;
    void *y;
    int y_dtype;
    int64_t ldy;
    int accumulate;  // with one split: y += result (read in the epilogue)
    float *part;     // [S][M][N] partials (null: results go straight to y)
    // grouped experts (pf_kernel<..., true>): row tile blockIdx.y is entry
    // tiles[4 y ..] = (expert, first sorted row, rows, 0) while y < *ntiles;
    // sorted row p is token perm[p]; expert e's weight rows start
    // e * estride_w bytes and its scales e * estride_s elements further
    const int *perm;
    const int *tiles;
    const int *ntiles;
    int64_t estride_w, estride_s;
};

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

template <int BITS, int BM, int PD, int NT, int WAVES, bool GR = false>
__global__ void __launch_bounds__(WAVES * 64, 8 / WAVES) pf_kernel(PfArgs a)
{
    constexpr int MT = BM / 32;                  // 32-row M tiles per wave
    constexpr int THREADS = WAVES * 64;
    constexpr int TPR = THREADS / BM;            // staging threads per activation row
    constexpr int VPT = kPfBK / TPR;             // values per staging thread and step
    constexpr int XE = 2;  // activations: fp16, pre-scaled per row (pf_prep_kernel)
    constexpr int XP = VPT * XE / 16;            // 16-byte pieces per staging thread
    constexpr int WL = BITS == 4 ? 1 : 2;        // 16-byte weight loads per lane, N tile and step
    constexpr int NB = (PD > 2 ? PD : 2) + 1;    // register sets (weights PD, activations 2 steps ahead)
    static_assert(VPT % 8 == 0, "staging in 8-value pieces");
    static_assert(THREADS >= 256, "one table entry per thread");
    static_assert(BM <= 128, "two activation buffers in the table's gaps");

    // 256-byte table entries: the lower 128 bytes hold entry b's 32 copies
    // (copy c at byte (b << 8) | (c << 2), the address one v_perm builds from
    // the packed byte); the upper 128 bytes of entry q * 128 + r hold row r
    // of activation buffer q (64 fp16 values), 16-byte piece p at position
    // p ^ (r & 7) so a 32-row operand read and the staging stores are free
    // of bank conflicts.
    __shared__ __align__(16) uint32_t tab[256 * 64];
    __shared__ uint32_t s_cbraw[256];
    __shared__ uint16_t s_cb16[256];
    __shared__ int s_e[BM];
    __shared__ int s_row[GR ? BM : 1];  // grouped: token of each tile row (-1: none)

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int nw = blockIdx.x * (WAVES * 32 * NT) + wave * (32 * NT);  // the wave's first weight row
    const int m0 = blockIdx.y * BM;
    const int kt0 = blockIdx.z * a.ksteps;
    const int nk = a.K / kPfBK;
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
        a.scale = (const char *)a.scale + e * a.estride_s * 2;
    }
    const auto rx = buffer_rsrc(a.x, a.xbytes), rw = buffer_rsrc(a.packed, a.wbytes);
    const auto rs = buffer_rsrc(a.scale, a.sbytes), rcb = buffer_rsrc(a.cb, a.cbbytes);

    // ---- first loads: codebook, row exponents, step 0's activations
    const uint32_t cbraw = __builtin_amdgcn_raw_buffer_load_b32(rcb, tid * 4, 0, 0);
    const int xr = tid / TPR, xq = tid % TPR;
    int xm;
    if constexpr (GR)
        xm = xr < gcount ? a.perm[gstart + xr] : -1;
    else
        xm = m0 + xr < a.M ? m0 + xr : -1;
    const int ex = *(const __attribute__((address_space(1))) int *)(a.rexp + (xm >= 0 ? xm : 0));

    // Load offsets = a per-lane part fixed for the whole loop (kPfOut for a
    // row past M or N) + a per-step part that is uniform (kPfOut for a step
    // past K or the split): one add per load.  Both parts stay below 2^31,
    // so a sum with either at kPfOut is past the buffer and reads zeros
    // (the bounds check covers the per-lane offset, which holds the sum).
    const uint32_t xlo = xm >= 0 ? (uint32_t)(((int64_t)xm * a.ldx + xq * VPT) * XE) : kPfOut;
    uint32_t wlo[NT][WL], slo[NT][WL];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int n = nw + nt * 32 + j;
#pragma unroll
        for (int l = 0; l < WL; ++l) {
            const int kl = 32 * h + 16 * l;  // first k of the piece within the step
            wlo[nt][l] = n < a.N ? (uint32_t)n * a.row_bytes + (uint32_t)(BITS == 4 ? kl / 2 : kl) : kPfOut;
            // the group divides 64 or is 64 * 2^i: the piece's group is the
            // step's (kt * gk_mul) >> gk_shift plus kl / group
            slo[nt][l] = n < a.N ? (uint32_t)(((int64_t)n * a.lds + kl / a.group) * 2) : kPfOut;
        }
    }
    auto kstep_ok = [&](int kt) { return kt < nk && kt < kt0 + a.ksteps; };
    auto issue_x = [&](int kt, u32x4_t (&xv)[XP]) {
        const uint32_t ks = kstep_ok(kt) ? (uint32_t)(kt * kPfBK * XE) : kPfOut;
#pragma unroll
        for (int p = 0; p < XP; ++p)
            xv[p] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(xlo + ks + 16 * p), 0, 0);
    };
    auto issue_w = [&](int kt, u32x4_t (&w)[NT][WL], uint32_t (&sr)[NT][WL]) {
        const bool kok = kstep_ok(kt);
        const uint32_t kw = kok ? (uint32_t)(kt * (BITS == 4 ? kPfBK / 2 : kPfBK)) : kPfOut;
        const uint32_t kg = kok ? (uint32_t)(((kt * a.gk_mul) >> a.gk_shift) * 2) : kPfOut;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int l = 0; l < WL; ++l) {
                w[nt][l] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(wlo[nt][l] + kw), 0, 0);
                sr[nt][l] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)(slo[nt][l] + kg), 0, 0);
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

    // staged activation row r, buffer q, 16-byte piece p (see the layout above)
    auto xs_off = [](int q, int r, int p) -> uint32_t {
        return ((uint32_t)(q * 128 + r) << 8) + 128u + ((uint32_t)(p ^ (r & 7)) << 4);
    };
    auto store_x = [&](const u32x4_t (&v4)[XP], int q) {
#pragma unroll
        for (int p = 0; p < XP; ++p)
            *(u32x4_t *)((char *)tab + xs_off(q, xr, xq * XP + p)) = v4[p];
    };

    // codebook -> fp16 -> the replicated table; step 0's activations -> LDS
    if (tid < 256)
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
        if (tid < 256)
            s_cb16[tid] = tid < a.levels ? f16_bits((f16_t)c) : (uint16_t)0;
        lds_barrier();
        // entry t: (cb[t & 15], cb[t >> 4]) at 4 bits, cb[t] twice at 8 bits
        if (tid < 256) {
            const uint32_t v = BITS == 4 ? ((uint32_t)s_cb16[tid & 15] | ((uint32_t)s_cb16[tid >> 4] << 16))
                                         : ((uint32_t)s_cb16[tid] | ((uint32_t)s_cb16[tid] << 16));
            u32x4_t *row = (u32x4_t *)(tab + tid * 64);
#pragma unroll
            for (int i = 0; i < kPfCopies / 4; ++i)
                row[i] = (u32x4_t){v, v, v, v};
        }
    }
    if (tid % TPR == 0) {
        if (xm >= 0)
            s_e[xr] = ex;
        if constexpr (GR)
            s_row[xr] = xm;
    }
    store_x(xv[0], 0);
    lds_barrier();

    f32x16_t acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[mt][nt][r] = 0.0f;

    const uint32_t c4 = (uint32_t)(lane & 31) << 2;  // the lane's table copy
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
        // activation buffer of step kt: static when the unroll is even
        const int q = NB % 2 == 0 ? (r & 1) : ((kt - kt0) & 1);
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
                                as_f16x2(lds_read_u32(tab, __builtin_amdgcn_perm(word, c4, kSelByte[b]))) * s2;
                    } else {
                        const uint32_t t0 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c4, kSelByte[0]));
                        const uint32_t t1 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c4, kSelByte[1]));
                        const uint32_t t2 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c4, kSelByte[2]));
                        const uint32_t t3 = lds_read_u32(tab, __builtin_amdgcn_perm(word, c4, kSelByte[3]));
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
                av[mt] = *(const f16x8_t *)((const char *)tab + xs_off(q, mt * 32 + j, 4 * h + s));
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
        store_x(xv[(r + 1) % NB], q ^ 1);
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
                const int m = GR ? s_row[row] : m0 + row;
                if (GR ? m < 0 : m >= a.M)
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
// M from which the 8-wave 128-row tilings run (measured: 8-bit gains from
// M = 128, 4-bit only above it)
#ifndef EP_PF_BIG4_M
#define EP_PF_BIG4_M 160
#endif
#ifndef EP_PF_BIG8_M
#define EP_PF_BIG8_M 128
#endif
#ifndef EP_PF_PD8
#define EP_PF_PD8 3
#endif
struct PfPlan {
    int bm, pd, nt, waves, S, ksteps;
};

PfPlan pf_plan(int bits, int64_t M, int64_t N, int64_t K)
{
    PfPlan p;
    if (bits == 4) {
        // measured: 128 x 2 tiles lead from M = 1024, 128 x 1 at 256..1023
        p.bm = M >= EP_PF_BIG4_M ? 128 : 64;
        p.nt = M >= EP_PF_BIG4_M && M < 1024 ? 1 : 2;
        p.pd = p.bm == 128 && p.nt == 2 ? 2 : 4;
        p.waves = M >= EP_PF_BIG4_M ? 8 : 4;
    } else if (M >= EP_PF_BIG8_M) {
        p.bm = 128;
        p.pd = EP_PF_PD8;
        p.nt = 1;
        p.waves = 8;
    } else {
        p.bm = 64;
        p.pd = 3;
        p.nt = 2;
        p.waves = 4;
    }
    const int nb = (p.pd > 2 ? p.pd : 2) + 1;
    const int bn = p.waves * 32 * p.nt;
    const int64_t tiles = ((N + bn - 1) / bn) * ((M + p.bm - 1) / p.bm);
    const int nk = (int)(K / kPfBK);
    // K split in two while the grid stays within one round of resident
    // workgroups (8 waves per CU): a split past that only adds partials
    // (14336 x 4096 at M = 512, 224 tiles: 132.7 us with 2 splits, 110.5
    // with none; M = 256, 112 tiles: 93.6 us with 4, 80.9 with 2)
    const int target = 8 / p.waves * device_cus();
    int S = 1;
    while (tiles * S * 2 <= target && S < 8 && nk / (S * 2) >= 8)
        S *= 2;
    int ks = (nk + S - 1) / S;
    ks = (ks + nb - 1) / nb * nb;
    p.S = (nk + ks - 1) / ks;
    p.ksteps = ks;
    return p;
}

template <int BITS, int BM, int PD, int NT, int WAVES>
int pf_launch(const PfArgs &a, const PfPlan &p, hipStream_t s)
{
    constexpr int BN = WAVES * 32 * NT;
    const dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM), (unsigned)p.S);
    hipLaunchKernelGGL((pf_kernel<BITS, BM, PD, NT, WAVES>), grid, dim3(WAVES * 64), 0, s, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

template <int BITS, int BM, int PD, int NT, int WAVES>
int pf_launch_grouped(const PfArgs &a, unsigned tiles_y, hipStream_t s)
{
    constexpr int BN = WAVES * 32 * NT;
    const dim3 grid((unsigned)((a.N + BN - 1) / BN), tiles_y, 1u);
    hipLaunchKernelGGL((pf_kernel<BITS, BM, PD, NT, WAVES, true>), grid, dim3(WAVES * 64), 0, s, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

}  // namespace

bool prefill_grouped_serves(const PackedDesc &w, const ActDesc &x, int64_t T)
{
    // one expert's rows and scales, and the T token rows of x, in buffer range
    return prefill_serves(w, x, T);
}

size_t prefill_grouped_workspace(int64_t T, int64_t K)
{
    return (size_t)((T * 4 + 255) / 256 * 256) + (size_t)((T * K * 2 + 255) / 256 * 256);
}

// Stacked experts grouped by expert (tiles from the device sort): the fp16
// copy of every token row, then pf_kernel over each expert's row tiles (bm
// 64 or 128 rows, the whole K per workgroup), results at the tokens' rows.
int launch_prefill_grouped(const PackedDesc &w, const ActDesc &x, int64_t T, const int *perm,
                           const int *tiles, const int *ntiles, int bm, unsigned tiles_y, const OutDesc &y,
                           void *ws, hipStream_t stream)
{
    const int bits = w.bits();
    int *rexp = (int *)ws;
    f16_t *xh = (f16_t *)((char *)ws + (T * 4 + 255) / 256 * 256);
    hipLaunchKernelGGL(pf_prep_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, stream, x.ptr, x.dtype,
                       x.ld, (int)T, (int)w.K, rexp, xh);
    EP_HIP_CHECK(hipGetLastError());
    PfArgs a{};
    a.xbytes = (uint32_t)(T * w.K * 2);
    a.wbytes = (uint32_t)(w.N * (bits == 4 ? w.K / 2 : w.K));
    a.sbytes = (uint32_t)(((w.N - 1) * w.ld_scale + (w.K + w.group - 1) / w.group) * 2);
    a.cbbytes = (uint32_t)(w.levels * (w.cb_dtype == EP_F32 ? 4 : 2));
    a.x = xh;
    a.ldx = w.K;
    a.M = (int)T;
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
    a.gk_mul = w.group <= kPfBK ? kPfBK / w.group : 1;
    a.gk_shift = 0;
    while (w.group > kPfBK && (kPfBK << a.gk_shift) < w.group)
        ++a.gk_shift;
    const int nk = (int)(w.K / kPfBK);
    a.rexp = rexp;
    a.y = y.ptr;
    a.y_dtype = y.dtype;
    a.ldy = y.ld;
    a.accumulate = 0;
    a.part = nullptr;
    a.perm = perm;
    a.tiles = tiles;
    a.ntiles = ntiles;
    a.estride_w = w.N * (int64_t)a.row_bytes;
    a.estride_s = w.N * w.ld_scale;
    // the whole K per workgroup: steps rounded up to the register-set count
    auto ks = [&](int pd) {
        const int nb = (pd > 2 ? pd : 2) + 1;
        return (nk + nb - 1) / nb * nb;
    };
    if (bits == 4) {
        if (bm == 128) {
            a.ksteps = ks(4);
            return pf_launch_grouped<4, 128, 4, 1, 8>(a, tiles_y, stream);
        }
        a.ksteps = ks(4);
        if (bm == 32)
            return pf_launch_grouped<4, 32, 4, 2, 4>(a, tiles_y, stream);
        return pf_launch_grouped<4, 64, 4, 2, 4>(a, tiles_y, stream);
    }
    if (bm == 128) {
        a.ksteps = ks(EP_PF_PD8);
        return pf_launch_grouped<8, 128, EP_PF_PD8, 1, 8>(a, tiles_y, stream);
    }
    a.ksteps = ks(3);
    if (bm == 32)
        return pf_launch_grouped<8, 32, 3, 2, 4>(a, tiles_y, stream);
    return pf_launch_grouped<8, 64, 3, 2, 4>(a, tiles_y, stream);
}

bool prefill_serves(const PackedDesc &w, const ActDesc &x, int64_t M)
{
    const int bits = w.bits();
    if (M < 1 || M > ((int64_t)1 << 24) || w.N < 1 || w.K < kPfBK || w.K % kPfBK != 0)
        return false;
    if (w.scale_dtype != EP_F16 || w.group % (bits == 4 ? 32 : 16) != 0)
        return false;
    // groups that divide the 64-wide k step or are 64 * 2^i (others: the
    // generic MFMA path)
    if (64 % w.group != 0 && (w.group % 64 != 0 || ((w.group / 64) & (w.group / 64 - 1)) != 0))
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
    a.gk_mul = w.group <= kPfBK ? kPfBK / w.group : 1;
    a.gk_shift = 0;
    while (w.group > kPfBK && (kPfBK << a.gk_shift) < w.group)
        ++a.gk_shift;
    a.ksteps = p.ksteps;
    a.rexp = rexp;
    a.y = y.ptr;
    a.y_dtype = y.dtype;
    a.ldy = y.ld;
    a.accumulate = y.accumulate;
    a.part = partials ? (float *)((char *)ws + ex + xhb) : nullptr;
    int rc;
    if (bits == 4)
        rc = p.nt == 1 ? pf_launch<4, 128, 4, 1, 8>(a, p, stream)
             : p.bm == 128 ? pf_launch<4, 128, 2, 2, 8>(a, p, stream)
                           : pf_launch<4, 64, 4, 2, 4>(a, p, stream);
    else
        rc = p.nt == 1 ? pf_launch<8, 128, EP_PF_PD8, 1, 8>(a, p, stream)
                       : pf_launch<8, 64, 3, 2, 4>(a, p, stream);
    if (rc != EP_OK || !partials)
        return rc;
    return launch_split_reduce(a.part, p.S, M, w.N, y, stream);
}

}  // namespace ep
