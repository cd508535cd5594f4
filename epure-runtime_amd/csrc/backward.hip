// Compressed-state backward of y = x . W^T, W = cb[idx] * scale, indices
// frozen (fine-tuning/README.md:62-68; the reference gets these from
// autograd through materialize(), runtime.py:84-88):
//
//   grad_x     = gy . W                              (dx kernel)
//   grad_scale[n, g] = sum_{k in g} G[n, k] * cb[idx[n, k]]
//   grad_cb[l]       = sum_{idx[n,k] == l} G[n, k] * scale[n, g(k)]
//   with G = gy^T . x, which is never written to memory  (dw kernel)
//
// dx: MFMA over 128x128 (m, k) tiles, contraction over n in steps of 128
//     (split in up to 8 parts, summed in split order, when the tiles alone
//     cannot fill the device).  gy enters as fp16 after the exact per-row
//     power-of-two rescale (as in the forward); W is dequantized per 8x8
//     block to fp16(cb) * fp16(scale) and transposed in registers, so the
//     W^T tile goes to LDS as 16-byte rows.
// dw: MFMA (bf16 operands: gy and x are bf16, products exact in fp32) over
//     128x128 (k, n) tiles of G, contraction over the token dimension m in
//     steps of 64 (x and gy transposed per 8x8 block in registers, LDS
//     double-buffered).  The epilogue never stores G: each value is multiplied by
//     cb[idx] and summed over its group (grad_scale is complete inside the
//     tile, one plain store per (n, g)), and multiplied by its scale and
//     added into a per-thread private LDS histogram over the 16 codebook
//     levels; histograms are reduced in a fixed order per workgroup and
//     across workgroups by a final kernel.  No float atomics race, so the
//     result is deterministic.  `packed` is only read.
#include <array>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int T = 128;        // output tile (both dims)
constexpr int CS = 64;        // dx: contraction step over n
constexpr int MS = 64;        // dw: contraction step over m
constexpr int LDX = CS + 8;   // dx LDS row length (halfs), padded
constexpr int LDW = MS + 8;   // dw LDS row length (halfs), padded

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
    const f16_t *gy16;   // [M][N] fp16(gy * 2^-rexp), written by gy_prep_kernel
    float *gc_part;      // [num dw workgroups][16]
    int dx_steps;        // contraction steps per dx split
    float *dx_part;      // [splits][M][K] f32 partials (null: one split, results go to gx)
};

// A buffer offset past the end of every descriptor (buffer_rsrc: loads
// there read zeros); sums of two such parts stay below 2^32.
constexpr uint32_t kBwOut = 0x7fffff00u;

EP_DEV uint32_t bits_of(f16x2_t v)
{
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}

// 8x8 transpose of 16-bit elements: r[i] is row i (dword d holds elements
// 2d and 2d + 1), c[j] becomes column j (dword d holds rows 2d and 2d + 1).
// 32 byte permutes; lets a thread write whole 16-byte rows of a transposed
// LDS tile instead of 64 two-byte stores.
EP_DEV void tr8x8(const u32x4_t (&r)[8], u32x4_t (&c)[8])
{
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int d = 0; d < 4; ++d)
            c[j][d] = __builtin_amdgcn_perm(r[2 * d + 1][j >> 1], r[2 * d][j >> 1],
                                            (j & 1) ? 0x07060302u : 0x05040100u);
}

// Per-row exponent of the largest |gy| (row_exponent) and the rescaled
// fp16 copy of the row, converted once here instead of once per k tile of
// the dx kernel: one wave per row of bf16 values, 16-byte loads, four in
// flight per lane (rows are 16-byte aligned and N % 16 == 0); the second
// pass re-reads the row from the caches.
__global__ void __launch_bounds__(256)
    gy_prep_kernel(const uint16_t *gy, int64_t ld, int M, int N, int *rexp, f16_t *gy16)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M)
        return;
    const u32x4_t *p = (const u32x4_t *)(gy + (int64_t)row * ld);
    const int pieces = N / 8;
    float amax = 0.0f;
    for (int i0 = lane; i0 < pieces; i0 += 256) {
        u32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            v[u] = i0 + 64 * u < pieces ? p[i0 + 64 * u] : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(v[u][t] << 16)),
                                         fabsf(__uint_as_float(v[u][t] & 0xffff0000u))));
    }
    amax = wave_max(amax);
    const int e = row_exponent(amax);
    if (lane == 0)
        rexp[row] = e;
    const float pw = ldexpf(1.0f, -e);
    f16x8_t *q = (f16x8_t *)(gy16 + (int64_t)row * N);
    for (int i0 = lane; i0 < pieces; i0 += 256) {
        u32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            v[u] = i0 + 64 * u < pieces ? p[i0 + 64 * u] : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            f16x8_t h;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                h[2 * t] = (f16_t)(__uint_as_float(v[u][t] << 16) * pw);
                h[2 * t + 1] = (f16_t)(__uint_as_float(v[u][t] & 0xffff0000u) * pw);
            }
            if (i0 + 64 * u < pieces)
                q[i0 + 64 * u] = h;
        }
    }
}

// grad_x[m, k] = sum_n gy[m, n] W[n, k] over a 128 x 128 (m, k) tile,
// contraction over n in steps of CS (blockIdx.z: the split of the steps).
// Staging per step: gy rows (already fp16, rescaled by 2^-e per row) go to
// LDS as they are ([m][n]); W is dequantized by 8 x 8 blocks (8 rows n x 8
// columns k: one packed dword per row, fp16(cb) pairs from the LDS table
// times the fp16 scale, i.e. materialize(float16)), transposed in registers
// and written as W^T rows ([k][n]), so both MFMA operands are 16-byte LDS
// reads.  The next step's global loads are in flight during the MFMAs.
template <int SDT>  // scale dtype
__global__ void __launch_bounds__(256, 2) dx_kernel(BwdArgs a)
{
    __shared__ __align__(16) f16_t Gs[T * LDX];  // gy tile [m][n]
    __shared__ __align__(16) f16_t Ws[T * LDX];  // W^T tile [k][n]
    __shared__ uint32_t tab[256];
    __shared__ int s_e[T];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wk = wave & 1;
    const int m0 = blockIdx.y * T, k0 = blockIdx.x * T;
    const int nsteps = (a.N + CS - 1) / CS;
    const int st0 = blockIdx.z * a.dx_steps;
    const int st1 = st0 + a.dx_steps < nsteps ? st0 + a.dx_steps : nsteps;
    {
        const int lo = tid & 15, hi = tid >> 4;
        const float clo = lo < a.levels ? load_as_f32(a.cb, a.cb_dtype, lo) : 0.0f;
        const float chi = hi < a.levels ? load_as_f32(a.cb, a.cb_dtype, hi) : 0.0f;
        tab[tid] = (uint32_t)f16_bits((f16_t)clo) | ((uint32_t)f16_bits((f16_t)chi) << 16);
    }
    if (tid < T) {
        const int m = m0 + tid;
        s_e[tid] = m < a.M ? a.rexp[m] : 0;
    }

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[i][j][r] = 0.0f;

    // gy: rows 32 p + (tid >> 3), columns 8 (tid & 7) .. + 7 (p = 0..3);
    // W (threads below 128, waves 0-1): the 8 x 8 block of rows nb * 8 ..,
    // columns kb * 8 ..
    // Loads never branch: buffer descriptors over the tile's gy rows (rows
    // past M read zeros), the packed weights and the scales; an element past
    // N, or any element of a step past this split's end, gets an offset
    // past every buffer.
    const int gr0 = tid >> 3, gc = 8 * (tid & 7);
    const bool wthr = tid < 128;  // wave-uniform
    const int nb = tid & 7, kb = (tid >> 3) & 15;
    const uint32_t rowb = (uint32_t)(a.K / 2);
    constexpr int SE = SDT == EP_F32 ? 4 : 2;
    const int64_t gleft = (int64_t)(a.M - m0) * a.N * 2;
    const auto rg = buffer_rsrc(a.gy16 + (int64_t)m0 * a.N, gleft < kBwOut ? (uint32_t)gleft : kBwOut);
    const auto rw = buffer_rsrc(a.packed, (uint32_t)((int64_t)a.N * rowb));
    const auto rs = buffer_rsrc(a.scale, (uint32_t)(((int64_t)(a.N - 1) * a.lds + a.K / a.group) * SE));
    const uint32_t kbyte = (uint32_t)((k0 + kb * 8) / 2);
    const int kgrp = (k0 + kb * 8) / a.group;
    u32x4_t gva[4], gvb[4];
    uint32_t wva[8], wvb[8], sca[8], scb[8];
    auto load = [&](int st, u32x4_t (&gv)[4], uint32_t (&wv)[8], uint32_t (&sc)[8]) {
        const bool kok = st < st1;  // uniform
        const int n0 = st * CS;
        {
            const int n = n0 + gc;
            const bool ok = kok && n < a.N;
#pragma unroll
            for (int p = 0; p < 4; ++p)
                gv[p] = __builtin_amdgcn_raw_buffer_load_b128(
                    rg, ok ? (int)(((32 * p + gr0) * a.N + n) * 2) : (int)kBwOut, 0, 0);
        }
        // every wave issues them (waves 2-3 out of range: no memory traffic),
        // so no load sits in a branch and the waits stay exact
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int n = n0 + nb * 8 + i;
            const bool ok = wthr && kok && n < a.N;
            wv[i] = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? (int)((uint32_t)n * rowb + kbyte) : (int)kBwOut,
                                                        0, 0);
            const int so = (int)(((int64_t)n * a.lds + kgrp) * SE);
            if constexpr (SE == 4)
                sc[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? so : (int)kBwOut, 0, 0);
            else
                sc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? so : (int)kBwOut, 0, 0);
        }
    };
    auto store = [&](const u32x4_t (&gv)[4], const uint32_t (&wv)[8], const uint32_t (&sc)[8]) {
#pragma unroll
        for (int p = 0; p < 4; ++p)
            *(u32x4_t *)&Gs[(32 * p + gr0) * LDX + gc] = gv[p];
        if (wthr) {
            u32x4_t rw8[8], cw[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float sf = SDT == EP_F32 ? __uint_as_float(sc[i])
                                 : SDT == EP_BF16 ? bf16_to_f32((uint16_t)sc[i])
                                                  : (float)f16_from_bits((uint16_t)sc[i]);
                const f16_t sh = (f16_t)sf;
                const f16x2_t s2 = (f16x2_t){sh, sh};
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    rw8[i][d] = bits_of(as_f16x2(tab[(wv[i] >> (8 * d)) & 0xffu]) * s2);
            }
            tr8x8(rw8, cw);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *(u32x4_t *)&Ws[(kb * 8 + j) * LDX + nb * 8] = cw[j];
        }
    };
    auto step = [&](int st, u32x4_t (&gv)[4], uint32_t (&wv)[8], uint32_t (&sc)[8]) {
        store(gv, wv, sc);
        lds_barrier();
        load(st + 2, gv, wv, sc);
        // keep the loads here and the next step's staging out of this one
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < CS / 16; ++kk) {
            f16x8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *(const f16x8_t *)&Gs[(wm * 64 + i * 32 + (lane & 31)) * LDX + kk * 16 +
                                               (lane >> 5) * 8];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *(const f16x8_t *)&Ws[(wk * 64 + j * 32 + (lane & 31)) * LDX + kk * 16 +
                                               (lane >> 5) * 8];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    lds_barrier();  // tab, s_e
    // two register sets, loads two steps ahead; the step count is rounded up
    // to even (a padding step reads zeros) so the sets rotate with static
    // indices and every wait counts exactly the younger set's loads
    load(st0, gva, wva, sca);
    __builtin_amdgcn_sched_barrier(0);
    load(st0 + 1, gvb, wvb, scb);
    __builtin_amdgcn_sched_barrier(0);
    const int stend = st0 + ((st1 - st0 + 1) & ~1);
    for (int st = st0; st < stend; st += 2) {
        step(st, gva, wva, sca);
        step(st + 1, gvb, wvb, scb);
    }

    // D[row][col] of a 32x32 tile: lane col + 32 * ((row / 4) % 2),
    // register (row % 4) + 4 * (row / 8); rows m, columns k
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                const int col = wk * 64 + j * 32 + (lane & 31);
                const int m = m0 + row, k = k0 + col;
                if (m >= a.M)
                    continue;
                const float v = ldexpf(acc[i][j][r], s_e[row]);
                if (a.dx_part)
                    a.dx_part[((int64_t)blockIdx.z * a.M + m) * a.K + k] = v;
                else
                    store_from_f32(a.gx, a.gx_dtype, (int64_t)m * a.ldgx + k, v);
            }
}

// G tile (k x n) = x^T . gy, reduced into grad_scale and per-workgroup
// codebook-gradient partials.  4-bit indices (levels <= 16), bf16 gy / x.
// Staging per step of MS rows m: waves 0-1 take x, waves 2-3 gy, each
// thread one 8 x 8 block (8 rows m x 8 columns), transposed in registers
// and written as 16-byte rows of x^T [k][m] / gy^T [n][m]; the next step's
// loads are in flight during the MFMAs.  Single-buffered (37 KB of LDS):
// three workgroups per CU.  The epilogue reuses the staging space.
constexpr int kDwStage = 2 * T * LDW * 2;  // [x^T | gy^T] bf16
__global__ void __launch_bounds__(256, 3) dw_kernel(BwdArgs a)
{
    __shared__ __align__(16) char smem[kDwStage];
    // epilogue views of the same space
    uint8_t *Ps = (uint8_t *)smem;                    // packed bytes of the tile [n][k/2]
    float *Ss = (float *)(smem + T * (T / 2));        // scale[n][g] for the tile's groups
    float *cbf = Ss + T * 4;                          // [16]
    float *hist = cbf + 16;                           // [16][256] private per-thread histograms
    float *gsp = hist + 16 * 256;                     // [2][T * 4] grad_scale partials per k-wave
    static_assert(T * (T / 2) + (T * 4 + 16 + 16 * 256 + 2 * T * 4) * 4 <= kDwStage, "epilogue fits");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wk = wave >> 1, wn = wave & 1;
    const int k0 = blockIdx.x * T, n0 = blockIdx.y * T;
    const int gpt = T / a.group;  // groups per tile (1, 2 or 4)

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[i][j][r] = 0.0f;

    // this thread's 8 x 8 staging block: rows (blk & 7) * 8 .. of the step,
    // columns (blk >> 3) * 8 .. of the tile.  The step rows vary fastest
    // over the lanes: a 16-byte LDS store of transposed row bc + j lands at
    // dword (bc + j) * LDW / 2 + br / 2, i.e. banks 4 j + br / 2 (mod 32),
    // so the 8 lanes of one store cycle cover 8 distinct bank quads
    // (columns varying fastest put all 8 on the same banks).
    const bool isx = tid < 128;  // wave-uniform
    const int blk = tid & 127;
    const int br = (blk & 7) * 8, bc = (blk >> 3) * 8;
    // Loads never branch: each step reads through a buffer descriptor based
    // at the step's first row and sized to the bytes left from there, so rows
    // past M (and a step past the end) read zeros; a column past N is sent
    // out of range by its per-lane offset.
    const char *base = isx ? (const char *)a.x : (const char *)a.gy;  // wave-uniform
    const int64_t rowb = (isx ? a.ldx : a.ldgy) * 2;
    const int64_t total = ((int64_t)(a.M - 1) * (isx ? a.ldx : a.ldgy) + (isx ? a.K : a.N)) * 2;
    const bool colok = isx ? true : n0 + bc < a.N;
    const uint32_t off0 = colok ? (uint32_t)(br * rowb + (int64_t)((isx ? k0 : n0) + bc) * 2) : kBwOut;
    const uint32_t offr = (uint32_t)rowb;
    auto load = [&](int mb, u32x4_t (&rr)[8]) {
        const int64_t left = total - (int64_t)mb * rowb;
        const auto rsrc = buffer_rsrc(base + (left > 0 ? (int64_t)mb * rowb : 0),
                                  left > 0 ? (left < kBwOut ? (uint32_t)left : kBwOut) : 0u);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            rr[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, colok ? (int)(off0 + i * offr) : (int)kBwOut, 0, 0);
    };
    auto store = [&](const u32x4_t (&rr)[8], int buf) {
        u32x4_t cc[8];
        tr8x8(rr, cc);
        __bf16 *dst = (__bf16 *)smem + (buf * 2 + (isx ? 0 : 1)) * T * LDW;  // buf is 0
#pragma unroll
        for (int j = 0; j < 8; ++j)
            *(u32x4_t *)&dst[(bc + j) * LDW + br] = cc[j];
    };

    // One register set (a second one costs the third resident workgroup,
    // measured slower): the next step's loads are issued right after the
    // set is staged and waited for only at the next staging, so they overlap
    // this step's MFMAs (the barriers wait for LDS operations only).
    const int steps = (a.M + MS - 1) / MS;
    const __bf16 *Xs = (const __bf16 *)smem;
    const __bf16 *Gs = Xs + T * LDW;
    u32x4_t rra[8];
    load(0, rra);
    auto step = [&](int st, u32x4_t (&rr)[8]) {
        store(rr, 0);
        lds_barrier();
        load((st + 1) * MS, rr);
        // keep the loads here and the next step's transpose out of this one
        // (either move makes a wait cover the younger register set)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < MS / 16; ++kk) {
            bf16x8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *(const bf16x8_t *)&Xs[(wk * 64 + i * 32 + (lane & 31)) * LDW + kk * 16 +
                                                (lane >> 5) * 8];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *(const bf16x8_t *)&Gs[(wn * 64 + j * 32 + (lane & 31)) * LDW + kk * 16 +
                                                (lane >> 5) * 8];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int st = 0; st < steps; ++st)
        step(st, rra);

    // ---- epilogue: G[k][n] -> grad_scale partials and level histograms ----
    // the tile's packed bytes, scales and the codebook (loaded only now:
    // registers held across the main loop would spill)
    u32x4_t pk[2];
    float sv[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int c = tid + 256 * q;  // 16-byte piece: row c >> 2, part c & 3
        const int n = n0 + (c >> 2);
        pk[q] = n < a.N ? *(const u32x4_t *)(a.packed + (int64_t)n * (a.K / 2) + k0 / 2 + (c & 3) * 16)
                        : (u32x4_t){0u, 0u, 0u, 0u};
        const int nl = c / gpt, gi = c % gpt;
        sv[q] = (c < T * gpt && n0 + nl < a.N)
                    ? load_as_f32(a.scale, a.scale_dtype, (int64_t)(n0 + nl) * a.lds + k0 / a.group + gi)
                    : 0.0f;
    }
    const float cbv = tid < a.levels ? load_as_f32(a.cb, a.cb_dtype, tid) : 0.0f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int c = tid + 256 * q;
        *(u32x4_t *)&Ps[(c >> 2) * (T / 2) + (c & 3) * 16] = pk[q];
        if (c < T * gpt)
            Ss[(c / gpt) * 4 + c % gpt] = sv[q];
    }
    if (tid < 16)
        cbf[tid] = cbv;
    for (int i = tid; i < 16 * 256; i += 256)
        hist[i] = 0.0f;
    __syncthreads();
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
                gsp[wk * T * 4 + nl * 4 + gi] = gs_acc[gi];
    }
    __syncthreads();
    for (int i = tid; i < T * gpt; i += 256) {
        const int nl = i / gpt, gi = i % gpt;
        const int n = n0 + nl;
        if (n < a.N)
            a.gscale[(int64_t)n * a.ldgs + k0 / a.group + gi] = gsp[nl * 4 + gi] + gsp[T * 4 + nl * 4 + gi];
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
    // thread t sums the partial rows t, t + 256, ... (16 levels each, four
    // 16-byte loads per row, four rows in flight); then level l = t / 16 is
    // summed by 16 threads over 16 slots each and across their lanes.
    // Fixed order throughout: deterministic.
    __shared__ float red[16 * 257];
    const int t = threadIdx.x;
    const float4 *p4 = reinterpret_cast<const float4 *>(part);
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        acc[j] = 0.0f;
    int w = t;
    for (; w + 3 * 256 < nwg; w += 4 * 256) {
        float4 v[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                v[r][q] = p4[(int64_t)(w + r * 256) * 4 + q];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[4 * q] += v[r][q].x;
                acc[4 * q + 1] += v[r][q].y;
                acc[4 * q + 2] += v[r][q].z;
                acc[4 * q + 3] += v[r][q].w;
            }
    }
    for (; w < nwg; w += 256) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = p4[(int64_t)w * 4 + q];
            acc[4 * q] += v.x;
            acc[4 * q + 1] += v.y;
            acc[4 * q + 2] += v.z;
            acc[4 * q + 3] += v.w;
        }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
        red[j * 257 + t] = acc[j];
    __syncthreads();
    const int l = t >> 4, slot = t & 15;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
        s += red[l * 257 + slot * 16 + j];
    s += dpp_mov<0x128>(s);  // row_ror 8
    s += dpp_mov<0x124>(s);  // row_ror 4
    s += dpp_mov<0x4e>(s);   // lanes ^ 2
    s += dpp_mov<0xb1>(s);   // lanes ^ 1
    if (slot == 0 && l < levels)
        gcb[l] = s;
}

// rows x cols f32 zeros (row stride ld): 4 rows per workgroup of 256
__global__ void __launch_bounds__(256) zero_rows_kernel(float *p, int rows, int cols, int64_t ld)
{
    const int r = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (r >= rows)
        return;
    for (int c = (int)(threadIdx.x & 63); c < cols; c += 64)
        p[(int64_t)r * ld + c] = 0.0f;
}

// ---- library route (large token counts): gy . W and G = gy^T . x run as
// hipBLASLt GEMMs (blas.cpp); these kernels finish them.

// grad_x[m, k] = D[m, k] * 2^rexp[m] in gx's dtype, D f32 row-major [M][K]
// (the GEMM's column-major K x M result).  Four values per thread.
__global__ void __launch_bounds__(256)
    dx_finish_kernel(const float *D, const int *rexp, int M, int K, void *gx, int gx_dtype, int64_t ldgx)
{
    const int64_t k0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (k0 >= K)
        return;
    for (int m = blockIdx.y; m < M; m += gridDim.y) {
        const int e = rexp[m];
        const float *src = D + (int64_t)m * K + k0;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (k0 + t < K)
                store_from_f32(gx, gx_dtype, (int64_t)m * ldgx + k0 + t, ldexpf(src[t], e));
    }
}

// From G [N][K] (f32, row-major): grad_scale[n, g] = sum_{k in g} G[n, k]
// cb[idx[n, k]] (one plain store per (n, g)) and per-workgroup codebook
// partials grad_cb[l] = sum_{idx == l} G[n, k] scale[n, g(k)], each thread
// adding into its own LDS histogram (slot [level][thread]: no two lanes on
// one bank), summed in thread order at the end; gc_final_kernel sums the
// workgroups in order.  Deterministic, no atomics.  One row per workgroup:
// its 4 waves take alternate 256-value steps of the row (many small
// workgroups per CU hide the histogram's LDS round trips); a lane takes 4
// consecutive k of a step, with the loads of kEpiU steps in flight; group
// sums over the lanes of a group through DPP and v_permlane16_swap.
constexpr int kEpiRows = 1;
constexpr int kEpiU = 6;
template <int LPG>  // lanes per group: group / 4 (8, 16 or 32)
EP_DEV float group_lane_sum(float v)
{
    v += dpp_mov<0xb1>(v);  // lanes ^ 1
    v += dpp_mov<0x4e>(v);  // lanes ^ 2
    if constexpr (LPG == 8) {
        v += dpp_mov<0x141>(v);  // row_half_mirror: the other quad of the 8
    } else {
        v += dpp_mov<0x124>(v);  // row_ror 4
        v += dpp_mov<0x128>(v);  // row_ror 8: the 16-lane row
        if constexpr (LPG == 32)
            v = xor16_sum(v);
    }
    return v;
}

template <int LPG>
__global__ void __launch_bounds__(256)
    gw_epilogue_kernel(const float *G, const uint8_t *packed, const void *scale, int scale_dtype,
                       int64_t lds, const void *cb, int cb_dtype, int levels, int N, int K,
                       float *gscale, int64_t ldgs, float *gc_part)
{
    __shared__ float hist[16 * 256];
    __shared__ float cbf[16];
    constexpr int LG = LPG == 8 ? 5 : (LPG == 16 ? 6 : 7);  // log2(group)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 16 * 256; i += 256)
        hist[i] = 0.0f;
    if (tid < 16)
        cbf[tid] = tid < levels ? load_as_f32(cb, cb_dtype, tid) : 0.0f;
    __syncthreads();
    float *my = hist + tid;
    {
        const int n = blockIdx.x;
        const float *grow = G + (int64_t)n * K;
        const uint16_t *prow = (const uint16_t *)(packed + (int64_t)n * (K / 2));
        for (int kb = 256 * wave; kb < K; kb += 256 * 4 * kEpiU) {
            f32x4_t g4[kEpiU];
            uint32_t b2[kEpiU];
            float sc[kEpiU];
#pragma unroll
            for (int u = 0; u < kEpiU; ++u) {  // every load first (clamped: a step past K reads k = 0)
                const int k = kb + 1024 * u + 4 * lane;
                const int kc = k < K ? k : 0;
                g4[u] = *(const f32x4_t *)(grow + kc);
                b2[u] = prow[kc / 4];  // the 2 bytes at byte offset kc / 2 (kc % 4 == 0)
                sc[u] = load_as_f32(scale, scale_dtype, (int64_t)n * lds + (kc >> LG));
            }
#pragma unroll
            for (int u = 0; u < kEpiU; ++u) {
                const int k = kb + 1024 * u + 4 * lane;
                const bool ok = k < K;
                float gs = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int lev = (b2[u] >> (4 * t)) & 15;
                    const float g = ok ? g4[u][t] : 0.0f;
                    gs = fmaf(g, cbf[lev], gs);
                    if (ok)
                        my[lev * 256] += g * sc[u];
                }
                gs = group_lane_sum<LPG>(gs);  // every lane of the group holds the sum
                if (ok && (lane & (LPG - 1)) == 0)
                    gscale[(int64_t)n * ldgs + (k >> LG)] = gs;
            }
        }
    }
    __syncthreads();
    // level l = tid / 16: 16 threads sum 16 slots each, then the 16 partial
    // sums are added across their lanes (DPP, fixed order)
    {
        const int l = tid >> 4, part = tid & 15;
        const float *src = hist + l * 256 + part * 16;
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            v[j] = src[j];
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            s += v[j];
        s += dpp_mov<0x128>(s);  // row_ror 8
        s += dpp_mov<0x124>(s);  // row_ror 4
        s += dpp_mov<0x4e>(s);   // lanes ^ 2
        s += dpp_mov<0xb1>(s);   // lanes ^ 1
        if (part == 0)
            gc_part[(int64_t)blockIdx.x * 16 + l] = s;
    }
}

}  // namespace

// Splits of the dx contraction: enough work items for the three resident
// workgroups per CU where the (m, k) tiles alone cannot provide them, at
// least 4 steps per split.
static int dx_splits(int64_t M, int64_t N, int64_t K)
{
    const int64_t tiles = ((K + T - 1) / T) * ((M + T - 1) / T);
    if (tiles <= 0)
        return 1;
    const int64_t nsteps = (N + CS - 1) / CS;
    const int64_t slots = 3 * (int64_t)device_cus();
    int64_t S = (slots + tiles - 1) / tiles;
    if (S > 8)
        S = 8;
    while (S > 1 && nsteps / S < 4)
        --S;
    return (int)S;
}

// Token counts from which grad_x and G run as library GEMMs (hipBLASLt
// reaches ~2x the fused kernels' MFMA rate on these plain products; below,
// materializing W costs more than it saves).
// EPURE_BWD_FUSED=1 in the environment (read on the first call) keeps every
// token count on the fused kernels: no W or grad_W in memory, no hipBLASLt
// handle, no host wait, at about half the library route's rate at 2048
// tokens.
constexpr int64_t kBlasMinM = 512;
static bool fused_forced()
{
    static const bool forced = [] {
        const char *v = std::getenv("EPURE_BWD_FUSED");
        return v != nullptr && v[0] != '\0' && v[0] != '0';
    }();
    return forced;
}
static bool blas_route(int64_t M, int64_t N, int64_t K)
{
    return M >= kBlasMinM && N >= 256 && K >= 256 && !fused_forced();
}
static size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// Library-route workspace: rexp [M] | gc partials [N / kEpiRows][16] | gy16
// [M][N] | W16 [N][K] | f32 [M][K] (grad_x's GEMM result) | f32 [N][K] (G) |
// two hipBLASLt workspaces (the two chains may run at once).
struct BlasWs {
    size_t rexp, gc, gy16, w16, f32buf, gbuf, blas, blas2, total;
};
static BlasWs blas_ws(int64_t M, int64_t N, int64_t K)
{
    BlasWs w;
    size_t o = 0;
    w.rexp = o;
    o += al256((size_t)M * 4);
    w.gc = o;
    o += al256((size_t)((N + kEpiRows - 1) / kEpiRows) * 16 * 4);
    w.gy16 = o;
    o += al256((size_t)M * N * 2);
    w.w16 = o;
    o += al256((size_t)N * K * 2);
    w.f32buf = o;
    o += al256((size_t)M * K * 4);
    w.gbuf = o;
    o += al256((size_t)N * K * 4);
    w.blas = o;
    o += blas_workspace_bytes();
    w.blas2 = o;
    o += blas_workspace_bytes();
    w.total = o;
    return w;
}

// The library route's two chains -- grad_x (gy prescale, materialize, GEMM,
// finish) and the scale/codebook gradients (GEMM G, epilogue, final sum) --
// are independent: the second runs on a side stream forked from and joined
// back into the caller's stream with events (both work under stream
// capture), so the memory-bound kernels of one overlap the other's GEMM.
// Each caller stream gets its own side stream (default priority) and two
// events, created on its first call outside capture (at most kMaxSides
// per process; further caller streams run the chains in order):
// a capture on one caller stream then never joins a side stream that
// another thread's eager calls use.  The first call of a shape bucket (the
// one whose library GEMM plans time their candidate algorithms) runs both
// chains in order on the caller's stream, undisturbed.
struct SideStream {
    int dev = -1;
    hipStream_t caller = nullptr, s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    std::mutex mu;  // held across fork, G chain and join (callers sharing a caller stream)
};
constexpr int kMaxSides = 32;
constexpr size_t kMaxSeen = 1024;
static std::mutex g_side_mu;
static SideStream g_side[kMaxSides];
static int g_nside = 0;
static std::vector<std::array<int64_t, 4>> g_bwd_seen;  // (device, shape bucket) run once

static int64_t pow2_ceil(int64_t v)
{
    int64_t b = 1;
    while (b < v)
        b <<= 1;
    return b;
}

// The side stream to fork to, or nullptr (run in order).
static SideStream *side_for(hipStream_t stream, int64_t M, int64_t N, int64_t K)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0)
        return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess)
        return nullptr;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lk(g_side_mu);
    // the caller stream's side stream, created on its first call outside
    // capture -- also when that call runs in order (a bucket's first call),
    // so that a capture right after one eager call still forks
    SideStream *sd = nullptr;
    for (int i = 0; i < g_nside && !sd; ++i)
        if (g_side[i].dev == dev && g_side[i].caller == stream)
            sd = &g_side[i];
    if (!sd && !capturing && g_nside < kMaxSides) {
        sd = &g_side[g_nside++];
        sd->dev = dev;
        sd->caller = stream;
        if (hipStreamCreateWithFlags(&sd->s, hipStreamNonBlocking) != hipSuccess) {
            sd->s = nullptr;
            (void)hipGetLastError();
        } else if (hipEventCreateWithFlags(&sd->fork, hipEventDisableTiming) != hipSuccess ||
                   hipEventCreateWithFlags(&sd->join, hipEventDisableTiming) != hipSuccess) {
            sd->join = nullptr;
            (void)hipGetLastError();
        }
    }
    const std::array<int64_t, 4> key{dev, pow2_ceil(M), pow2_ceil(N), pow2_ceil(K)};
    bool seen = g_bwd_seen.size() >= kMaxSeen;
    for (const auto &k : g_bwd_seen)
        seen = seen || k == key;
    if (!seen) {
        if (!capturing)
            g_bwd_seen.push_back(key);
        return nullptr;
    }
    return sd && sd->s && sd->join ? sd : nullptr;
}

// Whether the library route can run on `stream` now: always outside
// capture; under capture only once the device has a hipBLASLt handle
// (creating one allocates device memory), else the fused kernels serve.
static bool blas_usable(hipStream_t stream)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess)
        return false;
    if (cs == hipStreamCaptureStatusNone)
        return true;
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess && blas_ready(dev);
}

// Workspace of the fused kernels: rexp [M] | gc partials | gy16 [M][N] |
// grad_x split partials.
static size_t fused_ws(int64_t M, int64_t N, int64_t K)
{
    const int64_t nwg = ((K + T - 1) / T) * ((N + T - 1) / T);
    const int S = dx_splits(M, N, K);
    return (size_t)((M * 4 + 255) / 256 * 256) + (size_t)nwg * 16 * sizeof(float) +
           (size_t)((M * N * 2 + 255) / 256 * 256) +
           (S > 1 ? (size_t)S * (size_t)M * (size_t)K * sizeof(float) : 0);
}

size_t backward_workspace(int64_t M, int64_t N, int64_t K, int levels, int group)
{
    (void)levels;
    (void)group;
    if (M <= 0 || N <= 0 || K <= 0)
        return 0;
    const size_t f = fused_ws(M, N, K);
    if (blas_route(M, N, K)) {
        const size_t b = blas_ws(M, N, K).total;
        return b > f ? b : f;  // either route may run (the fused one under capture)
    }
    return f;
}

bool backward_serves(const PackedDesc &w, int gy_dtype, int x_dtype)
{
    // gy is staged in 16-column chunks, so N % 16 == 0 keeps every load in its row.
    // buffer offsets stay below kBwOut: packed bytes, scales, 128 gy rows
    const int64_t sbytes = ((w.N - 1) * w.ld_scale + w.K / w.group) * (w.scale_dtype == EP_F32 ? 4 : 2);
    return w.levels <= 16 && w.K % T == 0 && T % w.group == 0 && T / w.group <= 4 &&
           w.N % 16 == 0 && gy_dtype == EP_BF16 && x_dtype == EP_BF16 && w.N <= INT32_MAX &&
           w.K <= INT32_MAX && w.N * (w.K / 2) < kBwOut && sbytes < kBwOut && w.N * T * 2 < kBwOut;
}

int launch_backward(const PackedDesc &w, const ActDesc &gy, const ActDesc &x, int64_t M,
                    const OutDesc &gx, float *grad_cb, float *grad_scale, int64_t ld_gscale,
                    void *ws, size_t ws_bytes, hipStream_t stream)
{
    if (!backward_serves(w, gy.dtype, x.dtype))
        return set_error(EP_DECLINE_SHAPE,
                         "fused backward serves levels <= 16, K %% 128 == 0, N %% 16 == 0, group "
                         "in {32, 64, 128}, bf16 gy and x");
    if (M <= 0 || w.N <= 0) {
        // no tokens: grad_x is empty, grad_cb and grad_scale are sums over
        // nothing (zeros, written by a kernel so the call stays capturable)
        const int G = (int)((w.K + w.group - 1) / w.group);
        if (grad_scale && w.N > 0 && G > 0)
            hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)((w.N + 3) / 4)), dim3(256), 0,
                               stream, grad_scale, (int)w.N, G, ld_gscale);
        if (grad_cb)
            hipLaunchKernelGGL(zero_rows_kernel, dim3(1), dim3(256), 0, stream, grad_cb, 1,
                               w.levels, (int64_t)w.levels);
        EP_HIP_CHECK(hipGetLastError());
        return EP_OK;
    }
    const bool lib = blas_route(M, w.N, w.K) && blas_usable(stream);
    const size_t need = lib ? blas_ws(M, w.N, w.K).total : fused_ws(M, w.N, w.K);
    if (!ws || ws_bytes < need)
        return set_error(EP_ERR_WORKSPACE, "backward workspace of %zu bytes needed, %zu given",
                         need, ws_bytes);
    if (((uintptr_t)gy.ptr & 15) || ((uintptr_t)x.ptr & 15) || (gy.ld % 8) || (x.ld % 8) ||
        ((uintptr_t)w.packed & 15))
        return set_error(EP_DECLINE_SHAPE, "fused backward needs 16-byte aligned rows");
    if (64 * gy.ld * 2 >= kBwOut || 64 * x.ld * 2 >= kBwOut)
        return set_error(EP_DECLINE_SHAPE, "fused backward: row strides of gy and x below 16M elements");
    if (lib) {
        // grad_x = (gy16 . W16) * 2^rexp per row; G = gy^T . x -> grad_scale, grad_cb
        const BlasWs L = blas_ws(M, w.N, w.K);
        char *base = (char *)ws;
        int *rexp = (int *)(base + L.rexp);
        float *gcp = (float *)(base + L.gc);
        f16_t *gy16 = (f16_t *)(base + L.gy16);
        f16_t *w16 = (f16_t *)(base + L.w16);
        float *buf = (float *)(base + L.f32buf);
        float *gbuf = (float *)(base + L.gbuf);
        const bool want_g = grad_cb || grad_scale;
        if (want_g && !grad_scale)
            return set_error(EP_ERR_ARG, "grad_cb without grad_scale is not served");
        SideStream *side = gx.ptr && want_g ? side_for(stream, M, w.N, w.K) : nullptr;
        const hipStream_t gs = side ? side->s : stream;  // the G chain's stream
        std::unique_lock<std::mutex> side_lock;
        if (side) {
            side_lock = std::unique_lock<std::mutex>(side->mu);
            EP_HIP_CHECK(hipEventRecord(side->fork, stream));
            EP_HIP_CHECK(hipStreamWaitEvent(side->s, side->fork, 0));
        }
        // both chains; the side stream is joined back whatever they return
        auto chains = [&]() -> int {
            if (want_g) {
                // column-major: G^T (K x N) = x (K x M) . gy^T (M x N): G row-major [N][K]
                int rc = blas_gemm_f32out(0, 1, w.K, w.N, M, EP_BF16, x.ptr, x.ld, gy.ptr, gy.ld, gbuf, w.K, 1.0f,
                                          base + L.blas2, blas_workspace_bytes(), gs);
                if (rc != EP_OK)
                    return rc;
                const int nwg = (int)((w.N + kEpiRows - 1) / kEpiRows);
                if (w.group == 32)
                    hipLaunchKernelGGL(gw_epilogue_kernel<8>, dim3((unsigned)nwg), dim3(256), 0, gs, gbuf,
                                       w.packed, w.scale, w.scale_dtype, w.ld_scale, w.cb, w.cb_dtype, w.levels,
                                       (int)w.N, (int)w.K, grad_scale, ld_gscale, gcp);
                else if (w.group == 64)
                    hipLaunchKernelGGL(gw_epilogue_kernel<16>, dim3((unsigned)nwg), dim3(256), 0, gs, gbuf,
                                       w.packed, w.scale, w.scale_dtype, w.ld_scale, w.cb, w.cb_dtype, w.levels,
                                       (int)w.N, (int)w.K, grad_scale, ld_gscale, gcp);
                else
                    hipLaunchKernelGGL(gw_epilogue_kernel<32>, dim3((unsigned)nwg), dim3(256), 0, gs, gbuf,
                                       w.packed, w.scale, w.scale_dtype, w.ld_scale, w.cb, w.cb_dtype, w.levels,
                                       (int)w.N, (int)w.K, grad_scale, ld_gscale, gcp);
                EP_HIP_CHECK(hipGetLastError());
                if (grad_cb) {
                    hipLaunchKernelGGL(gc_final_kernel, dim3(1), dim3(256), 0, gs, gcp, nwg, w.levels, grad_cb);
                    EP_HIP_CHECK(hipGetLastError());
                }
            }
            if (gx.ptr) {
                hipLaunchKernelGGL(gy_prep_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream,
                                   (const uint16_t *)gy.ptr, gy.ld, (int)M, (int)w.N, rexp, gy16);
                EP_HIP_CHECK(hipGetLastError());
                int rc = launch_dequant_tile(w, w16, EP_F16, w.K, stream);  // materialize(float16)
                if (rc != EP_OK)
                    return rc;
                // column-major: D (K x M) = W16 (K x N) . gy16 (N x M)
                rc = blas_gemm_f32out(0, 0, w.K, M, w.N, EP_F16, w16, w.K, gy16, w.N, buf, w.K, 1.0f, base + L.blas,
                                      blas_workspace_bytes(), stream);
                if (rc != EP_OK)
                    return rc;
                hipLaunchKernelGGL(dx_finish_kernel, dim3((unsigned)((w.K + 1023) / 1024), (unsigned)(M < 65535 ? M : 65535)), dim3(256),
                                   0, stream, buf, rexp, (int)M, (int)w.K, gx.ptr, gx.dtype, gx.ld);
                EP_HIP_CHECK(hipGetLastError());
            }
            return EP_OK;
        };
        const int rc = chains();
        if (side) {
            EP_HIP_CHECK(hipEventRecord(side->join, side->s));
            EP_HIP_CHECK(hipStreamWaitEvent(stream, side->join, 0));
        }
        return rc;
    }
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
        const size_t nwg_bytes = (size_t)((w.K + T - 1) / T) * ((w.N + T - 1) / T) * 16 * sizeof(float);
        f16_t *gy16 = (f16_t *)((char *)a.gc_part + nwg_bytes);
        a.gy16 = gy16;
        hipLaunchKernelGGL(gy_prep_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream,
                           (const uint16_t *)gy.ptr, gy.ld, (int)M, (int)w.N, (int *)ws, gy16);
        EP_HIP_CHECK(hipGetLastError());
        const int S = dx_splits(M, w.N, w.K);
        const int nsteps = (int)((w.N + CS - 1) / CS);
        a.dx_steps = (nsteps + S - 1) / S;
        const int Sused = (nsteps + a.dx_steps - 1) / a.dx_steps;
        a.dx_part = Sused > 1 ? (float *)((char *)gy16 + (size_t)((M * w.N * 2 + 255) / 256 * 256)) : nullptr;
        const dim3 grid((unsigned)((w.K + T - 1) / T), (unsigned)((M + T - 1) / T), (unsigned)Sused);
        if (w.scale_dtype == EP_F32)
            hipLaunchKernelGGL(dx_kernel<EP_F32>, grid, dim3(256), 0, stream, a);
        else if (w.scale_dtype == EP_BF16)
            hipLaunchKernelGGL(dx_kernel<EP_BF16>, grid, dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL(dx_kernel<EP_F16>, grid, dim3(256), 0, stream, a);
        EP_HIP_CHECK(hipGetLastError());
        if (Sused > 1) {
            const int rc = launch_split_reduce(a.dx_part, Sused, M, w.K, OutDesc{gx.ptr, gx.dtype, gx.ld, 0}, stream);
            if (rc != EP_OK)
                return rc;
        }
    }
    if (grad_cb || grad_scale) {
        if (!grad_scale)
            return set_error(EP_ERR_ARG, "grad_cb without grad_scale is not served");
        const dim3 grid((unsigned)(w.K / T), (unsigned)((w.N + T - 1) / T));
        hipLaunchKernelGGL(dw_kernel, grid, dim3(256), 0, stream, a);
        EP_HIP_CHECK(hipGetLastError());
        if (grad_cb) {
            hipLaunchKernelGGL(gc_final_kernel, dim3(1), dim3(256), 0, stream, a.gc_part,
                               (int)(grid.x * grid.y), w.levels, grad_cb);
            EP_HIP_CHECK(hipGetLastError());
        }
    }
    return EP_OK;
}

}  // namespace ep
