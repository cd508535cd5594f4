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
//  * The table is replicated 32x with lane l reading copy l & 31, so the
//    32 lanes a ds_read_b32 serves per cycle hit 32 banks: no bank conflicts
//    despite random byte values.  Address = (byte << 8) | ((lane & 31) << 2),
//    one v_perm.
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
#include "gemv_core.h"

namespace ep {
namespace {

// Tuning knobs (compile-time; the defaults are the measured choice).
#ifndef EP_GEMV_NT_LOADS
#define EP_GEMV_NT_LOADS 1      // weight loads marked non-temporal (streamed once)
#endif
#ifndef EP_GEMV_RQ1
#define EP_GEMV_RQ1 4           // row quads per block when a wave holds one slab
#endif
#ifndef EP_GEMV_PER_CU
#define EP_GEMV_PER_CU 2        // workgroups per CU for one-slab variants
#endif
#ifndef EP_GEMV_ROW_WAVES
#define EP_GEMV_ROW_WAVES 8     // waves per workgroup of gemv_row_kernel
#endif

constexpr int kMaxWaves = 8;   // 512 threads: up to 256 VGPRs per lane
constexpr int kMaxSeg = 3;

// Where the activation row comes from (template XS).
constexpr int XS_PLAIN = 0;    // x[m, k] in x_dtype
constexpr int XS_RMSNORM = 1;  // x = rmsnorm(h) * w: h f32 [K] (x), w bf16 [K] (x2), eps
constexpr int XS_SWIGLU = 2;   // x = silu(g) * u: g f32 [K] (x), u f32 [K] (x2)

// One weight sharing K / group / levels / dtypes with the others of a launch
// (e.g. q, k and v of one layer); workgroups [wg_begin, wg_end) serve it.
struct Seg {
    const uint8_t *packed;
    const void *scale;
    const void *cb;
    void *y;
    int N;
    int wg_begin, wg_end;
};

struct GemvArgs {
    const void *x;
    int x_dtype;
    int64_t ldx;
    int M;
    const void *x2;
    float eps;
    int64_t row_bytes;
    int scale_dtype;
    int64_t lds;
    int cb_dtype;
    int levels;
    int y_dtype;
    int64_t ldy;
    int accumulate;
    int64_t K;
    int group;
    int nseg;
    Seg seg[kMaxSeg];
    // Gathered rows (stacked experts): when gidx is set, grid row y serves
    // token y -- x row y, y row y -- with the rows of expert gidx[y] of a
    // stack of E weights, each estride_w packed bytes and estride_s scale
    // bytes after the previous one (seg[0] points at expert 0).
    const int *gidx;
    int E, ntok;
    int64_t estride_w, estride_s;
};

// Writes one chunk of 2 * PAIRS activations (already multiplied by the
// chunk's power of two pw) as fp16 pairs, and with HL their lo terms.
template <bool HL, int PAIRS>
EP_DEV void stage_chunk(const float *v, float pw, uint32_t *hi, uint32_t *lo)
{
#pragma unroll
    for (int p = 0; p < PAIRS; p += 4) {
        u32x4_t q4, l4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float a0 = v[2 * (p + t)] * pw, a1 = v[2 * (p + t) + 1] * pw;
            const f16_t h0 = (f16_t)a0, h1 = (f16_t)a1;
            q4[t] = (uint32_t)f16_bits(h0) | ((uint32_t)f16_bits(h1) << 16);
            l4[t] = (uint32_t)f16_bits((f16_t)(a0 - (float)h0)) |
                    ((uint32_t)f16_bits((f16_t)(a1 - (float)h1)) << 16);
        }
        *(u32x4_t *)(hi + p) = q4;
        if constexpr (HL)
            *(u32x4_t *)(lo + p) = l4;
    }
}

template <int BITS, int MT, int RQ, int SPW, int XDT, int XS, bool DB, int XCAP>
__global__ void __launch_bounds__(512) gemv_lut_kernel(GemvArgs a)
{
    constexpr int PAIRS = BITS == 4 ? 16 : 8;  // weight pairs per 16-byte chunk
    constexpr int KPC = 2 * PAIRS;              // k values per chunk
    constexpr int ROWS = 4 * RQ;                // rows per block
    static_assert(XS == XS_PLAIN || MT == 1, "fused activation sources serve M = 1");

    // Static LDS: the table sits at a compile-time address, so a lookup is
    // one v_perm for the address and the base folds into ds_read's offset.
    __shared__ __align__(16) uint32_t tab[kTabDwords];
    __shared__ float red[kMaxWaves * ROWS * MT];   // [W][ROWS][MT]
    __shared__ float s_part[kMaxWaves];            // sum-of-squares partials
    __shared__ uint16_t s_cb[256];                 // codebook as fp16 bits
    __shared__ float s_rinv;
    // f32 activations are carried as two fp16 terms, hi = fp16(x) and
    // lo = fp16(x - hi) (~22 significant bits together, after the chunk's
    // power-of-two factor): every table lookup feeds two dot products, so
    // an f32 row is not narrowed to fp16.  16-bit rows are exact in hi.
    constexpr bool HL = XDT == EP_F32;
    __shared__ __align__(16) uint32_t xs[XCAP * MT];      // staged activations, fp16 pairs
    __shared__ __align__(16) uint32_t xl[HL ? XCAP * MT : 4];  // their lo terms
    __shared__ float xf[(2 * XCAP / (BITS == 4 ? 32 : 16)) * MT];  // 2^e per chunk

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int W = blockDim.x >> 6;
    const int rq = lane >> 4, c = lane & 15;
    const int64_t KB = BITS == 4 ? a.K / 2 : a.K;
    const int S = (int)((KB + kSlabBytes - 1) / kSlabBytes);

    // Segment of this workgroup; kept in scalar registers (readfirstlane)
    // so every per-segment pointer below is uniform.
    const int bid = (int)blockIdx.x;
    const int si = __builtin_amdgcn_readfirstlane(
        (a.nseg > 2 && bid >= a.seg[2].wg_begin) ? 2 : ((a.nseg > 1 && bid >= a.seg[1].wg_begin) ? 1 : 0));
    const Seg &s0 = a.seg[0], &s1 = a.seg[1], &s2 = a.seg[2];
    const uint8_t *packed = si == 0 ? s0.packed : (si == 1 ? s1.packed : s2.packed);
    const void *scale = si == 0 ? s0.scale : (si == 1 ? s1.scale : s2.scale);
    const void *cbp = si == 0 ? s0.cb : (si == 1 ? s1.cb : s2.cb);
    void *yseg = si == 0 ? s0.y : (si == 1 ? s1.y : s2.y);
    const int N = si == 0 ? s0.N : (si == 1 ? s1.N : s2.N);
    const int wg_begin = si == 0 ? s0.wg_begin : (si == 1 ? s1.wg_begin : s2.wg_begin);
    const int wg_end = si == 0 ? s0.wg_end : (si == 1 ? s1.wg_end : s2.wg_end);
    const int nwg = wg_end - wg_begin;
    const int nblk = (N + ROWS - 1) / ROWS;
    int blk = bid - wg_begin;
    const char *xbase = (const char *)a.x;
    if (a.gidx) {
        // the token's expert (clamped into the stack: ids are checked on the
        // host where the caller can be synchronized)
        int e = __builtin_amdgcn_readfirstlane(a.gidx[blockIdx.y]);
        e = e < 0 ? 0 : (e >= a.E ? a.E - 1 : e);
        packed += (int64_t)e * a.estride_w;
        scale = (const char *)scale + (int64_t)e * a.estride_s;
        xbase += (int64_t)blockIdx.y * a.ldx * (XDT == EP_F32 ? 4 : 2);
        yseg = (char *)yseg + (int64_t)blockIdx.y * a.ldy * (a.y_dtype == EP_F32 ? 4 : 2);
    }

    // This lane's 16-byte chunk of each of its slabs (fixed for the kernel).
    uint32_t cbyte[SPW];
    bool act[SPW];
    int gidx[SPW];
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
        const int s = wave + j * W;
        const int64_t b0 = (int64_t)s * kSlabBytes + c * 16;
        act[j] = s < S && b0 < KB;
        cbyte[j] = act[j] ? (uint32_t)b0 : 0u;
        const int64_t k0 = BITS == 4 ? b0 * 2 : b0;
        gidx[j] = act[j] ? (int)(k0 / a.group) : 0;
    }

    // Issue the loads of one row block: all SPW x RQ 16-byte chunks and
    // their scales, from clamped addresses (an out-of-range row reads row 0
    // and is zeroed through its scale), so they go out back to back.
    auto load_block = [&](int b, u32x4_t (&wq)[SPW][RQ], float (&sc)[SPW][RQ]) {
        const int row0 = b * ROWS;
        uint32_t soff[SPW][RQ];
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int q = 0; q < RQ; ++q) {
                const int row = row0 + 4 * q + rq;
                const uint32_t rs = row < N ? (uint32_t)row : 0u;
                // 32-bit offsets: the host guarantees N * row_bytes < 2^31.
#if EP_GEMV_NT_LOADS
                wq[j][q] = __builtin_nontemporal_load(
                    (const u32x4_t *)(packed + (rs * (uint32_t)a.row_bytes + cbyte[j])));
#else
                wq[j][q] = *(const u32x4_t *)(packed + (rs * (uint32_t)a.row_bytes + cbyte[j]));
#endif
                soff[j][q] = rs * (uint32_t)a.lds + (uint32_t)gidx[j];
            }
        if (a.scale_dtype == EP_F16) {
#pragma unroll
            for (int j = 0; j < SPW; ++j)
#pragma unroll
                for (int q = 0; q < RQ; ++q)
                    sc[j][q] = (float)((const f16_t *)scale)[soff[j][q]];
        } else if (a.scale_dtype == EP_F32) {
#pragma unroll
            for (int j = 0; j < SPW; ++j)
#pragma unroll
                for (int q = 0; q < RQ; ++q)
                    sc[j][q] = ((const float *)scale)[soff[j][q]];
        } else {
#pragma unroll
            for (int j = 0; j < SPW; ++j)
#pragma unroll
                for (int q = 0; q < RQ; ++q)
                    sc[j][q] = bf16_to_f32(((const uint16_t *)scale)[soff[j][q]]);
        }
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int q = 0; q < RQ; ++q)
                if (!act[j] || row0 + 4 * q + rq >= N)
                    sc[j][q] = 0.0f;
    };

    u32x4_t wqA[SPW][RQ], wqB[SPW][RQ];
    float scA[SPW][RQ], scB[SPW][RQ];
    // FAST (one plain activation row, one slab per wave, one block per
    // workgroup -- the batch-1 decode shape): every load is issued at entry,
    // this thread's chunk of x and its codebook entry first, then the
    // weights and their raw scale halves, all unconditionally from clamped
    // addresses and in the global address space, so the compiler's waits
    // count them exactly;
    // staging and the table build then overlap the weight round trip and
    // the scales are converted only at use (a conversion right after the
    // load would wait for every load in flight).  Other variants hold too
    // many registers for this and keep the plain order.
    constexpr bool FAST = XS == XS_PLAIN && MT == 1 && SPW == 1 && !DB;
    constexpr int XPC = (XDT == EP_F32 ? 4 : 2) * KPC / 16;  // 16-byte pieces per chunk
    uint32_t scR[FAST ? SPW : 1][FAST ? RQ : 1][2];
    u32x4_t xraw[FAST ? XPC : 1];
    uint32_t cb_lo = 0, cb_hi = 0;
    const bool sc_f32 = a.scale_dtype == EP_F32;
    auto load_fast = [&](int b) {
        const int row0 = b * ROWS;
        const auto *sp = (const __attribute__((address_space(1))) uint16_t *)scale;
#pragma unroll
        for (int q = 0; q < RQ; ++q) {
            const int row = row0 + 4 * q + rq;
            const uint32_t rs = row < N ? (uint32_t)row : 0u;
            const auto *wp = (const __attribute__((address_space(1))) u32x4_t *)(
                packed + (rs * (uint32_t)a.row_bytes + cbyte[0]));
#if EP_GEMV_NT_LOADS
            wqA[0][q] = __builtin_nontemporal_load(wp);
#else
            wqA[0][q] = *wp;
#endif
        }
        // both halves of an f32 scale, the one half (twice) of a 16-bit one:
        // the same two loads on every path
#pragma unroll
        for (int q = 0; q < RQ; ++q) {
            const int row = row0 + 4 * q + rq;
            const uint32_t rs = row < N ? (uint32_t)row : 0u;
            const uint32_t e = rs * (uint32_t)a.lds + (uint32_t)gidx[0];
            scR[0][q][0] = sp[sc_f32 ? 2 * e : e];
            scR[0][q][1] = sp[sc_f32 ? 2 * e + 1 : e];
        }
    };
    float cbv = 0.0f;
    if constexpr (FAST) {
        const int xc = tid < (int)(a.K / KPC) ? tid : 0;
        const auto *xp = (const __attribute__((address_space(1))) u32x4_t *)(
            xbase + (int64_t)xc * KPC * (XDT == EP_F32 ? 4 : 2));
#pragma unroll
        for (int p = 0; p < XPC; ++p)
            xraw[p] = xp[p];
        const bool cb32 = a.cb_dtype == EP_F32;
        const uint32_t ci = (uint32_t)(tid < a.levels ? tid : a.levels - 1);
        const auto *cp = (const __attribute__((address_space(1))) uint16_t *)cbp;
        cb_lo = cp[cb32 ? 2 * ci : ci];
        cb_hi = cp[cb32 ? 2 * ci + 1 : ci];
        // the weights last: results return in order, so a load issued after
        // them could not be used before they have all arrived
        load_fast(blk < nblk ? blk : 0);  // a workgroup past the last block never uses it
        __builtin_amdgcn_sched_barrier(0);  // every load goes out before any use
    } else {
        if (blk < nblk)
            load_block(blk, wqA, scA);  // in flight while the table and x are staged
        // the codebook load goes out now too (its own round trip otherwise)
        if (tid < a.levels)
            cbv = load_as_f32(cbp, a.cb_dtype, tid);
    }

    // ---- stage activations ----------------------------------------------
    // The workgroup converts the activation row(s) once, cooperatively: one
    // chunk of KPC values per thread, scaled by an exact power of two chosen
    // from the chunk's largest value and stored to LDS as fp16 pairs; the
    // factor 2^e is folded into the group scale of the chunk's partial sums,
    // so no cross-lane agreement is needed.  RMSNorm's 1/rms is a scalar
    // and is applied to the finished dot products.
    constexpr int NCH = 2 * XCAP / KPC;  // chunk slots per activation row
    const int nchunk = (int)(a.K / KPC);
    float ssq = 0.0f;
    if constexpr (FAST) {
        // straight-line code after the loads, run and stored by every thread
        // (a thread past the last chunk loaded chunk 0 and writes exactly
        // chunk 0's values again): no branch the compiler could sink the x
        // loads into, behind the weight loads.  One chunk per thread covers
        // the row (blockDim = 64 x slabs >= K / KPC).
        float v[KPC];
        if constexpr (XDT == EP_F32) {
#pragma unroll
            for (int p = 0; p < XPC; ++p)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    v[4 * p + t] = __uint_as_float(xraw[p][t]);
        } else {
#pragma unroll
            for (int p = 0; p < XPC; ++p)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    unpack_pair<XDT>(xraw[p][t], v[8 * p + 2 * t], v[8 * p + 2 * t + 1]);
        }
        const int cc = tid < nchunk ? tid : 0;
        float am = 0.0f;
#pragma unroll
        for (int t = 0; t < KPC; ++t)
            am = fmaxf(am, fabsf(v[t]));
        const int e = row_exponent(am);
        const float pw = ldexpf(1.0f, -e);
        stage_chunk<HL, PAIRS>(v, pw, xs + cc * PAIRS, xl + cc * PAIRS);
        xf[cc] = ldexpf(1.0f, e);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const bool live_m = m < a.M;
        for (int cc = tid + (FAST ? (int)blockDim.x : 0); cc < nchunk; cc += blockDim.x) {
            const int64_t k0 = (int64_t)cc * KPC;
            float v[KPC];
            if constexpr (XS == XS_RMSNORM) {
                const float *hp = (const float *)xbase + k0;
                const uint16_t *wp = (const uint16_t *)a.x2 + k0;
#pragma unroll
                for (int p = 0; p < KPC; p += 8) {
                    const f32x4_t h0 = *(const f32x4_t *)(hp + p);
                    const f32x4_t h1 = *(const f32x4_t *)(hp + p + 4);
                    const u32x4_t wv = *(const u32x4_t *)(wp + p);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        float w0, w1;
                        unpack_pair<EP_BF16>(wv[t], w0, w1);
                        const float x0 = t < 2 ? h0[2 * t] : h1[2 * t - 4];
                        const float x1 = t < 2 ? h0[2 * t + 1] : h1[2 * t - 3];
                        ssq = fmaf(x0, x0, fmaf(x1, x1, ssq));
                        v[p + 2 * t] = x0 * w0;
                        v[p + 2 * t + 1] = x1 * w1;
                    }
                }
            } else if constexpr (XS == XS_SWIGLU) {
                const float *gp = (const float *)xbase + k0;
                const float *up = (const float *)a.x2 + k0;
#pragma unroll
                for (int p = 0; p < KPC; p += 4) {
                    const f32x4_t g = *(const f32x4_t *)(gp + p);
                    const f32x4_t u = *(const f32x4_t *)(up + p);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        v[p + t] = silu_mul(g[t], u[t]);
                }
            } else if constexpr (XDT == EP_F32) {
                const float *xp = (const float *)xbase + (int64_t)(live_m ? m : 0) * a.ldx + k0;
#pragma unroll
                for (int p = 0; p < KPC; p += 4) {
                    const f32x4_t t4 = *(const f32x4_t *)(xp + p);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        v[p + t] = live_m ? t4[t] : 0.0f;
                }
            } else {
                const uint16_t *xp = (const uint16_t *)xbase + (int64_t)(live_m ? m : 0) * a.ldx + k0;
#pragma unroll
                for (int p = 0; p < PAIRS; p += 4) {
                    const u32x4_t t4 = *(const u32x4_t *)(xp + 2 * p);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        unpack_pair<XDT>(live_m ? t4[t] : 0u, v[2 * (p + t)], v[2 * (p + t) + 1]);
                }
            }
            float am = 0.0f;
#pragma unroll
            for (int t = 0; t < KPC; ++t)
                am = fmaxf(am, fabsf(v[t]));
            const int e = row_exponent(am);
            const float pw = ldexpf(1.0f, -e);
            stage_chunk<HL, PAIRS>(v, pw, xs + m * XCAP + cc * PAIRS,
                                   xl + (HL ? m * XCAP + cc * PAIRS : 0));
            xf[m * NCH + cc] = ldexpf(1.0f, e);
        }
    }

    // codebook -> fp16 bits in LDS, then the pair table
    if constexpr (FAST) {
        cbv = a.cb_dtype == EP_F32 ? __uint_as_float(cb_lo | (cb_hi << 16))
              : (a.cb_dtype == EP_F16 ? (float)f16_from_bits((uint16_t)cb_lo) : bf16_to_f32((uint16_t)cb_lo));
        if (tid < 256)
            s_cb[tid] = tid < a.levels ? f16_bits((f16_t)cbv) : 0;
        if (blockDim.x < 256) {
            // small workgroups load the remaining entries (the waits for
            // these loads stay inside this branch)
            for (int i = tid + (int)blockDim.x; i < 256; i += blockDim.x)
                s_cb[i] = i < a.levels ? f16_bits((f16_t)load_as_f32(cbp, a.cb_dtype, i)) : 0;
        }
    } else {
        for (int i = tid; i < 256; i += blockDim.x)
            s_cb[i] = i < a.levels ? f16_bits((f16_t)(i == tid ? cbv : load_as_f32(cbp, a.cb_dtype, i)))
                                   : 0;
    }
    if constexpr (XS == XS_RMSNORM) {
        const float v = wave_sum_bfly(ssq);
        if (lane == 0)
            s_part[wave] = v;
    }
    lds_barrier();
    build_table<BITS>(tab, s_cb);
    if constexpr (XS == XS_RMSNORM) {
        if (tid == 0) {
            float q = 0.0f;
            for (int w = 0; w < W; ++w)
                q += s_part[w];
            s_rinv = rsqrtf(q / (float)a.K + a.eps);
        }
    }
    // this lane's activation chunks, from LDS into registers
    f16x2_t xh[SPW][MT][PAIRS];
    f16x2_t xlo[HL ? SPW : 1][HL ? MT : 1][HL ? PAIRS : 1];
    float fexp[SPW][MT];
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
        const int cc = act[j] ? (int)(cbyte[j] / 16) : 0;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const uint32_t *src = xs + m * XCAP + cc * PAIRS;
#pragma unroll
            for (int p = 0; p < PAIRS; p += 4) {
                const u32x4_t q4 = *(const u32x4_t *)(src + p);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    xh[j][m][p + t] = as_f16x2(q4[t]);
                if constexpr (HL) {
                    const u32x4_t l4 = *(const u32x4_t *)(xl + m * XCAP + cc * PAIRS + p);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        xlo[j][m][p + t] = as_f16x2(l4[t]);
                }
            }
            fexp[j][m] = act[j] ? xf[m * NCH + cc] : 0.0f;
        }
    }
    lds_barrier();

    const uint32_t lane4 = ((uint32_t)lane & 31) << 2;  // the lane's table copy
    // scale of (slab j, quad q) of the current block (0 past the row end)
    auto scale_at = [&](int j, int q) {
        if constexpr (FAST) {
            const uint32_t raw = scR[0][q][0] | (scR[0][q][1] << 16);
            const float v = sc_f32 ? __uint_as_float(raw)
                                   : (a.scale_dtype == EP_F16 ? (float)f16_from_bits((uint16_t)raw)
                                                              : bf16_to_f32((uint16_t)raw));
            return (act[0] && blk * ROWS + 4 * q + rq < N) ? v : 0.0f;
        } else {
            return scA[j][q];
        }
    };

    for (; blk < nblk; blk += nwg) {
        const int nxt = blk + nwg;
        if constexpr (DB) {
            if (nxt < nblk)
                load_block(nxt, wqB, scB);  // next block in flight during this one
        }

        float acc[RQ][MT];
#pragma unroll
        for (int q = 0; q < RQ; ++q)
#pragma unroll
            for (int m = 0; m < MT; ++m)
                acc[q][m] = 0.0f;

#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int q = 0; q < RQ; ++q) {
                float part[MT], plo[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    part[m] = plo[m] = 0.0f;
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    const uint32_t w = wqA[j][q][wd];
                    if constexpr (BITS == 4) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t t =
                                lds_read_u32(tab, __builtin_amdgcn_perm(w, lane4, kSelByte[i]));
                            const f16x2_t wv = as_f16x2(t);
#pragma unroll
                            for (int m = 0; m < MT; ++m) {
                                part[m] = __builtin_amdgcn_fdot2(wv, xh[j][m][wd * 4 + i], part[m],
                                                                 false);
                                if constexpr (HL)
                                    plo[m] = __builtin_amdgcn_fdot2(wv, xlo[j][m][wd * 4 + i],
                                                                    plo[m], false);
                            }
                        }
                    } else {
#pragma unroll
                        for (int p = 0; p < 2; ++p) {
                            const uint32_t t0 =
                                lds_read_u32(tab, __builtin_amdgcn_perm(w, lane4, kSelByte[2 * p]));
                            const uint32_t t1 = lds_read_u32(
                                tab, __builtin_amdgcn_perm(w, lane4, kSelByte[2 * p + 1]));
                            const uint32_t pr = __builtin_amdgcn_perm(t1, t0, 0x07060100u);
                            const f16x2_t wv = as_f16x2(pr);
#pragma unroll
                            for (int m = 0; m < MT; ++m) {
                                part[m] = __builtin_amdgcn_fdot2(wv, xh[j][m][wd * 2 + p], part[m],
                                                                 false);
                                if constexpr (HL)
                                    plo[m] = __builtin_amdgcn_fdot2(wv, xlo[j][m][wd * 2 + p],
                                                                    plo[m], false);
                            }
                        }
                    }
                }
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    acc[q][m] = fmaf(HL ? part[m] + plo[m] : part[m], scale_at(j, q) * fexp[j][m],
                                     acc[q][m]);
            }

        const int row0 = blk * ROWS;
#pragma unroll
        for (int q = 0; q < RQ; ++q)
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float v = row16_sum(acc[q][m]);
                if (c == 0)
                    red[(wave * ROWS + 4 * q + rq) * MT + m] = v;
            }
        lds_barrier();
        for (int t = tid; t < ROWS * MT; t += blockDim.x) {
            const int r = t / MT, m = t % MT;
            const int row = row0 + r;
            if (row < N && m < a.M) {
                float v = 0.0f;
                for (int w = 0; w < W; ++w)
                    v += red[(w * ROWS + r) * MT + m];
                if constexpr (XS == XS_RMSNORM)
                    v *= s_rinv;
                const int64_t off = (int64_t)m * a.ldy + row;
                if (a.accumulate)
                    v += load_as_f32(yseg, a.y_dtype, off);
                store_from_f32(yseg, a.y_dtype, off, v);
            }
        }
        if (nxt < nblk)
            lds_barrier();  // red is reused (the last block leaves at once)

        if (nxt < nblk) {
            if constexpr (DB) {
#pragma unroll
                for (int j = 0; j < SPW; ++j)
#pragma unroll
                    for (int q = 0; q < RQ; ++q) {
                        wqA[j][q] = wqB[j][q];
                        scA[j][q] = scB[j][q];
                    }
            } else if constexpr (FAST) {
                load_fast(nxt);
            } else {
                load_block(nxt, wqA, scA);
            }
        }
    }
}

// Batch-1 GEMV over rows of S = 4 .. 64 slabs, a multiple of 4 (served: 4,
// 8, 12, 16, 24, 28, 32 and, with 8-bit indices, 56: K = 2048 .. 16384 with
// 4-bit indices, 1024 .. 14336 with 8-bit), one block of ROWS rows per
// workgroup (4, 2 or 1 rows per wave; S / 4 16-byte loads per lane and row):
// wave w owns rows RW w .. RW w + RW - 1 across the whole row (each 16-byte
// load of a lane covers 4 slabs of one row: lane (sl, c) reads chunk c of
// slab 4 j + sl), so each row's dot product is summed inside one wave (DPP
// and permlane) and stored by it -- no cross-wave reduction and no barrier
// after the loads.  The one barrier orders the pair table and the staged
// activations (one chunk per thread, as gemv_lut_kernel's) before their
// reads.  The thread's activation chunk and codebook entries are loaded at
// entry, and the weights and their scale halves only once the chunk is
// staged and the table built: issued at entry they went out with every
// CU's weight burst, the small loads queued behind it and the staging
// waited (config 0: 5.30 -> 4.59 us per launch; weights issued between the
// staging and the table build: 4.85).  SC32: f32 group scales; otherwise one
// 16-bit load per scale (fp16 or bf16), not the two halves of a word
// (4.61 -> 4.48 us).
template <int BITS, int XDT, int S, bool SC32, int MT>
__global__ void __launch_bounds__(64 * EP_GEMV_ROW_WAVES) gemv_row_kernel(GemvArgs a)
{
    constexpr int NW = EP_GEMV_ROW_WAVES;       // waves per workgroup
    constexpr int NT = 64 * NW;
    constexpr int PAIRS = BITS == 4 ? 16 : 8;  // weight pairs per 16-byte chunk
    constexpr int KPC = 2 * PAIRS;              // k values per chunk
    constexpr int LPR = S / 4;                  // 16-byte loads of a lane per row
    constexpr int RW = LPR < 4 && 4 % LPR == 0 ? 4 / LPR : 1;  // rows per wave
    constexpr int NL = LPR * RW;                // 16-byte weight loads per lane
    constexpr int ROWS = NW * RW;
    constexpr int NPC = 2048 / NT;              // table pieces per thread
    constexpr int NCH = S * 16;                 // chunks per activation row
    constexpr int CPT = (NCH * MT + NT - 1) / NT;  // chunks staged per thread
    constexpr bool HL = XDT == EP_F32;          // f32 rows: hi and lo fp16 terms
    constexpr int ESZ = XDT == EP_F32 ? 4 : 2;
    constexpr int XPC = ESZ * KPC / 16;         // 16-byte pieces of x per chunk
    // one activation row with up to 4 loads per lane keeps its chunks in
    // registers for all its rows; otherwise each chunk is read from LDS at
    // its load
    constexpr bool XPRE = MT == 1 && (RW > 1 || LPR <= 4);
    static_assert(S % 4 == 0 && S >= 4 && S <= 64, "rows of a multiple of 4 slabs, at most 64");
    static_assert(MT == 1 || MT == 2 || MT == 4, "1, 2 or 4 activation rows");
    __shared__ __align__(16) uint32_t tab[kTabDwords];
    __shared__ __align__(16) uint32_t xs[MT * NCH * PAIRS];
    __shared__ __align__(16) uint32_t xl[HL ? MT * NCH * PAIRS : 4];
    __shared__ float xf[MT * NCH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sl = lane >> 4, c = lane & 15;
    const uint8_t *packed = a.seg[0].packed;
    const void *scale = a.seg[0].scale;
    const void *cbp = a.seg[0].cb;
    void *yp = a.seg[0].y;
    const int N = a.seg[0].N;
    const char *xbase = (const char *)a.x;
    if (a.gidx) {
        // the token's expert (clamped into the stack, as gemv_lut_kernel)
        int e = __builtin_amdgcn_readfirstlane(a.gidx[blockIdx.y]);
        e = e < 0 ? 0 : (e >= a.E ? a.E - 1 : e);
        packed += (int64_t)e * a.estride_w;
        scale = (const char *)scale + (int64_t)e * a.estride_s;
        xbase += (int64_t)blockIdx.y * a.ldx * ESZ;
        yp = (char *)yp + (int64_t)blockIdx.y * a.ldy * (a.y_dtype == EP_F32 ? 4 : 2);
    }
    const int row0 = (int)blockIdx.x * ROWS + wave * RW;

    // ---- the activation chunk and codebook loads (the weights follow the
    // table build); chunk ch is chunk ch % NCH of activation row ch / NCH
    u32x4_t xraw[CPT][XPC];
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
        const int ch = tid + NT * q;
        const int m = ch / NCH;
        const bool ok = ch < NCH * MT && m < a.M;
        const auto *xp = (const __attribute__((address_space(1))) u32x4_t *)(
            xbase + (ok ? ((int64_t)m * a.ldx + (int64_t)(ch % NCH) * KPC) * ESZ : 0));
#pragma unroll
        for (int p = 0; p < XPC; ++p)
            xraw[q][p] = xp[p];
    }
    // codebook entries of this thread's NPC table stores (store i = tid +
    // NT k writes a 16-byte piece of entry b = i >> 3): 4-bit: cb[b & 15]
    // (the same for every k) and cb[b >> 4]; 8-bit: cb[b]
    const bool cb32 = a.cb_dtype == EP_F32;
    const auto *cp = (const __attribute__((address_space(1))) uint16_t *)cbp;
    auto cb_at = [&](int i, uint32_t &lo, uint32_t &hi) {
        const uint32_t ci = (uint32_t)(i < a.levels ? i : 0);
        lo = cp[cb32 ? 2 * ci : ci];
        hi = cp[cb32 ? 2 * ci + 1 : ci];
    };
    constexpr int NCB = BITS == 4 ? NPC + 1 : NPC;
    uint32_t cbr[NCB][2];
    int cbi[NCB];
#pragma unroll
    for (int k = 0; k < NCB; ++k) {
        const int b = (tid + NT * k) >> 3;
        if constexpr (BITS == 4)
            cbi[k] = k == NPC ? b & 15 : b >> 4;
        else
            cbi[k] = b;
        cb_at(cbi[k], cbr[k][0], cbr[k][1]);
    }

    // ---- stage the activation chunks and the pair table, one barrier
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
        const int ch = tid + NT * q;
        const bool live = ch / NCH < a.M;  // rows past M stage zeros (never stored)
        float v[KPC];
        if constexpr (XDT == EP_F32) {
#pragma unroll
            for (int p = 0; p < XPC; ++p)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    v[4 * p + t] = live ? __uint_as_float(xraw[q][p][t]) : 0.0f;
        } else {
#pragma unroll
            for (int p = 0; p < XPC; ++p)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    unpack_pair<XDT>(live ? xraw[q][p][t] : 0u, v[8 * p + 2 * t], v[8 * p + 2 * t + 1]);
        }
        float am = 0.0f;
#pragma unroll
        for (int t = 0; t < KPC; ++t)
            am = fmaxf(am, fabsf(v[t]));
        const int e = row_exponent(am);
        if (ch < NCH * MT) {
            stage_chunk<HL, PAIRS>(v, ldexpf(1.0f, -e), xs + ch * PAIRS, xl + (HL ? ch * PAIRS : 0));
            xf[ch] = ldexpf(1.0f, e);
        }
    }
    {
        auto cb16 = [&](int k) -> uint32_t {
            const float f = cb32 ? __uint_as_float(cbr[k][0] | (cbr[k][1] << 16))
                                 : (a.cb_dtype == EP_F16 ? (float)f16_from_bits((uint16_t)cbr[k][0])
                                                         : bf16_to_f32((uint16_t)cbr[k][0]));
            return cbi[k] < a.levels ? (uint32_t)f16_bits((f16_t)f) : 0u;
        };
#pragma unroll
        for (int k = 0; k < NPC; ++k) {
            uint32_t v;
            if constexpr (BITS == 4)
                v = cb16(NPC) | (cb16(k) << 16);
            else
                v = cb16(k) | (cb16(k) << 16);
            // entry b = (tid + NT k) >> 3 at byte b << 8, its 16-byte piece tid & 7
            // (the 32 copies fill the entry's first 128 bytes: gemv_core.h)
            ((u32x4_t *)tab)[(((tid + NT * k) >> 3) << 4) + (tid & 7)] = (u32x4_t){v, v, v, v};
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // weights: load i covers row r = i / LPR, slabs 4 (i % LPR) .. + 3
    u32x4_t wq[NL];
    uint32_t sraw[NL];  // the scale's bits: f32 (SC32) or fp16 / bf16
    {
        const auto *sp = (const __attribute__((address_space(1))) uint16_t *)scale;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int row = row0 + i / LPR;
            const uint32_t rs = row < N ? (uint32_t)row : 0u;
            const uint32_t b0 = (uint32_t)((i % LPR) * 4 + sl) * kSlabBytes + (uint32_t)c * 16;
            const auto *wp = (const __attribute__((address_space(1))) u32x4_t *)(
                packed + (rs * (uint32_t)a.row_bytes + b0));
#if EP_GEMV_NT_LOADS
            wq[i] = __builtin_nontemporal_load(wp);
#else
            wq[i] = *wp;
#endif
            const uint32_t e = rs * (uint32_t)a.lds + (BITS == 4 ? 2 * b0 : b0) / (uint32_t)a.group;
            if constexpr (SC32)
                sraw[i] = ((const __attribute__((address_space(1))) uint32_t *)scale)[e];
            else
                sraw[i] = sp[e];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the weight loads go out before the barrier
    lds_barrier();

    // ---- the lane's activation chunks (slab 4 j + sl, chunk c; row m)
    constexpr int XR = XPRE ? LPR : 1;  // chunks held in registers
    f16x2_t xh[XR][MT][PAIRS];
    f16x2_t xlo[HL ? XR : 1][HL ? MT : 1][HL ? PAIRS : 1];
    float fexp[XR][MT];
    auto read_x = [&](int j, int slot) {
        const int cc = (j * 4 + sl) * 16 + c;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int ch = m * NCH + cc;
#pragma unroll
            for (int p = 0; p < PAIRS; p += 4) {
                const u32x4_t q4 = *(const u32x4_t *)(xs + ch * PAIRS + p);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    xh[slot][m][p + t] = as_f16x2(q4[t]);
                if constexpr (HL) {
                    const u32x4_t l4 = *(const u32x4_t *)(xl + ch * PAIRS + p);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        xlo[slot][m][p + t] = as_f16x2(l4[t]);
                }
            }
            fexp[slot][m] = xf[ch];
        }
    };
    if constexpr (XPRE) {
#pragma unroll
        for (int j = 0; j < LPR; ++j)
            read_x(j, j);
    }

    // ---- dot products: load i adds to row i / LPR of every activation row
    const uint32_t lane4 = ((uint32_t)lane & 31) << 2;  // the lane's table copy
    float acc[RW][MT];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m)
            acc[r][m] = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int r = i / LPR, j = i % LPR;
        if constexpr (!XPRE)
            read_x(j, 0);
        const int xj = XPRE ? j : 0;  // the chunk's register slot
        float part[MT], plo[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m)
            part[m] = plo[m] = 0.0f;
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            const uint32_t w = wq[i][wd];
            if constexpr (BITS == 4) {
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const f16x2_t wv = as_f16x2(lds_read_u32(tab, __builtin_amdgcn_perm(w, lane4, kSelByte[b])));
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        part[m] = __builtin_amdgcn_fdot2(wv, xh[xj][m][wd * 4 + b], part[m], false);
                        if constexpr (HL)
                            plo[m] = __builtin_amdgcn_fdot2(wv, xlo[xj][m][wd * 4 + b], plo[m], false);
                    }
                }
            } else {
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const uint32_t t0 = lds_read_u32(tab, __builtin_amdgcn_perm(w, lane4, kSelByte[2 * p]));
                    const uint32_t t1 = lds_read_u32(tab, __builtin_amdgcn_perm(w, lane4, kSelByte[2 * p + 1]));
                    const f16x2_t wv = as_f16x2(__builtin_amdgcn_perm(t1, t0, 0x07060100u));
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        part[m] = __builtin_amdgcn_fdot2(wv, xh[xj][m][wd * 2 + p], part[m], false);
                        if constexpr (HL)
                            plo[m] = __builtin_amdgcn_fdot2(wv, xlo[xj][m][wd * 2 + p], plo[m], false);
                    }
                }
            }
        }
        const uint32_t raw = sraw[i];
        const float sc = SC32 ? __uint_as_float(raw)
                              : (a.scale_dtype == EP_F16 ? (float)f16_from_bits((uint16_t)raw)
                                                         : bf16_to_f32((uint16_t)raw));
        const float scr = row0 + r < N ? sc : 0.0f;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            acc[r][m] = fmaf(HL ? part[m] + plo[m] : part[m], scr * fexp[xj][m], acc[r][m]);
    }
    // ---- each row's sums inside the wave; lane 0 stores them
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float v = wave_sum(acc[r][m]);
            const int row = row0 + r;
            if (lane == 0 && row < N && m < a.M) {
                const int64_t off = (int64_t)m * a.ldy + row;
                float o = v;
                if (a.accumulate)
                    o += load_as_f32(yp, a.y_dtype, off);
                store_from_f32(yp, a.y_dtype, off, o);
            }
        }
}

// Any shape, any stride, any M: one wave per output row, fp32 arithmetic
// (w = f32(cb[idx]) * f32(scale), fma into fp32).  Flat-stream indexing
// (position n*K + k), so odd K with 4-bit packing is served too.
__global__ void __launch_bounds__(256) gemv_generic_kernel(GemvArgs a)
{
    const int lane = threadIdx.x & 63;
    const Seg &sg = a.seg[0];
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= sg.N)
        return;
    const bool four = a.levels <= 16;
    for (int m = 0; m < a.M; ++m) {
        float acc = 0.0f;
        for (int64_t k = lane; k < a.K; k += 64) {
            const int64_t p = row * a.K + k;
            const uint8_t byte = sg.packed[four ? (p >> 1) : p];
            const int idx = four ? ((p & 1) ? (byte >> 4) : (byte & 15)) : byte;
            const float cbv = idx < a.levels ? load_as_f32(sg.cb, a.cb_dtype, idx) : 0.0f;
            const float w = cbv * load_as_f32(sg.scale, a.scale_dtype, row * a.lds + k / a.group);
            acc = fmaf(load_as_f32(a.x, a.x_dtype, (int64_t)m * a.ldx + k), w, acc);
        }
        acc = wave_sum_bfly(acc);
        if (lane == 0) {
            const int64_t off = (int64_t)m * a.ldy + row;
            float v = acc;
            if (a.accumulate)
                v += load_as_f32(sg.y, a.y_dtype, off);
            store_from_f32(sg.y, a.y_dtype, off, v);
        }
    }
}

// Row quads per block for a given number of slabs per wave: keeps the
// 16-byte loads in flight per lane (SPW * RQ, double-buffered) at 8.
// f32 rows (hi and lo activation terms) take half the row quads from two
// slabs per wave up, to stay in registers.
constexpr int rq_for(int spw, bool hl = false)
{
    return spw >= 8 ? 1 : (spw >= 4 ? (hl ? 1 : 2) : (spw >= 2 ? (hl ? 2 : 4) : EP_GEMV_RQ1));
}

// Activation registers (SPW * MT * pairs-per-chunk, twice that for f32
// rows: hi and lo terms) stay within 64 VGPRs (128 for one f32 row), and
// several activation rows are served with one slab per wave (the other
// variants spill).
constexpr bool fits(int bits, int spw, int mt, bool hl = false)
{
    const int regs = spw * mt * (bits == 4 ? 16 : 8) * (hl ? 2 : 1);
    return regs <= (hl && mt == 1 ? 128 : 64) && (mt == 1 || spw == 1) && !(hl && spw >= 8);
}

// Splits the persistent grid across segments in proportion to their row
// blocks (every segment gets at least one workgroup).
void assign_workgroups(GemvArgs &a, int rows_per_block, int per_cu)
{
    int blocks[kMaxSeg] = {0, 0, 0};
    int total = 0;
    for (int i = 0; i < a.nseg; ++i) {
        blocks[i] = (a.seg[i].N + rows_per_block - 1) / rows_per_block;
        total += blocks[i];
    }
    int grid = device_cus() * per_cu;
    if (grid > total)
        grid = total;
    if (grid < a.nseg)
        grid = a.nseg;
    int begin = 0;
    for (int i = 0; i < a.nseg; ++i) {
        int share = (int)((int64_t)grid * blocks[i] / (total > 0 ? total : 1));
        if (share < 1)
            share = 1;
        if (share > blocks[i] && blocks[i] > 0)
            share = blocks[i];
        if (i == a.nseg - 1 && begin + share < grid && grid - begin <= blocks[i])
            share = grid - begin;
        a.seg[i].wg_begin = begin;
        a.seg[i].wg_end = begin + share;
        begin += share;
    }
    for (int i = a.nseg; i < kMaxSeg; ++i)
        a.seg[i].wg_begin = a.seg[i].wg_end = begin;
}

// LDS bytes of one workgroup of a variant (table + staged activations).
constexpr size_t lds_bytes(int bits, int mt, int rq, int xcap, bool hl)
{
    return (size_t)kTabDwords * 4 + (size_t)kMaxWaves * 4 * rq * mt * 4 +
           (size_t)xcap * mt * 4 * (hl ? 2 : 1) +
           (size_t)(2 * xcap / (bits == 4 ? 32 : 16)) * mt * 4 + 1024;
}

template <int BITS, int MT, int SPW, int XDT, int XS, int XCAP>
int launch_xcap(GemvArgs a, int waves, hipStream_t stream)
{
    constexpr int RQ = rq_for(SPW, XDT == EP_F32);
    constexpr size_t lds = lds_bytes(BITS, MT, RQ, XCAP, XDT == EP_F32);
    static_assert(lds <= 160 * 1024, "LDS budget");
    // persistent grid: as many workgroups per CU as LDS and registers allow
    int per_cu = (int)((160 * 1024) / lds);
    if (per_cu > EP_GEMV_PER_CU)
        per_cu = EP_GEMV_PER_CU;
    if (SPW >= 2 || MT >= 2)
        per_cu = 1;  // ~200+ VGPRs: one 8-wave workgroup per CU
    if (per_cu < 1)
        per_cu = 1;
    assign_workgroups(a, 4 * RQ, per_cu);
    const int grid = a.seg[a.nseg - 1].wg_end;
    // Double-buffer the next block's loads only when a workgroup has more
    // than one block; otherwise the extra registers buy nothing.
    bool multi = false;
    for (int i = 0; i < a.nseg; ++i)
        multi |= (a.seg[i].N + 4 * RQ - 1) / (4 * RQ) > a.seg[i].wg_end - a.seg[i].wg_begin;
    const dim3 g3((unsigned)grid, a.gidx ? (unsigned)a.ntok : 1u);
    if (multi)
        hipLaunchKernelGGL((gemv_lut_kernel<BITS, MT, RQ, SPW, XDT, XS, true, XCAP>), g3,
                           dim3(waves * 64), 0, stream, a);
    else
        hipLaunchKernelGGL((gemv_lut_kernel<BITS, MT, RQ, SPW, XDT, XS, false, XCAP>), g3,
                           dim3(waves * 64), 0, stream, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

template <int BITS, int MT, int SPW, int XDT, int XS>
int launch_lut(GemvArgs a, int waves, hipStream_t stream)
{
    if constexpr (!fits(BITS, SPW, MT, XDT == EP_F32)) {
        return set_error(EP_DECLINE_SHAPE, "GEMV variant does not fit registers");
    } else {
        const int64_t pairs = a.K / 2;
        if (pairs <= 2048)
            return launch_xcap<BITS, MT, SPW, XDT, XS, 2048>(a, waves, stream);
        if constexpr (MT == 1 || (MT == 2 && XDT != EP_F32)) {  // LDS: f32 rows stage twice
            if (pairs <= 8192)
                return launch_xcap<BITS, MT, SPW, XDT, XS, 8192>(a, waves, stream);
        }
        return set_error(EP_DECLINE_SHAPE, "GEMV: K=%lld x M too large to stage",
                         (long long)a.K);
    }
}

template <int BITS, int MT, int SPW>
int dispatch_xdt(const GemvArgs &a, int xdt, int waves, hipStream_t s)
{
    switch (xdt) {
    case EP_BF16:
        return launch_lut<BITS, MT, SPW, EP_BF16, XS_PLAIN>(a, waves, s);
    case EP_F16:
        return launch_lut<BITS, MT, SPW, EP_F16, XS_PLAIN>(a, waves, s);
    default:
        return launch_lut<BITS, MT, SPW, EP_F32, XS_PLAIN>(a, waves, s);
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
    case 4:
        return dispatch_xdt<BITS, MT, 4>(a, xdt, waves, s);
    default:
        return dispatch_xdt<BITS, MT, 8>(a, xdt, waves, s);
    }
}

template <int BITS, int XS>
int dispatch_fused(const GemvArgs &a, int spw, int waves, hipStream_t s)
{
    switch (spw) {
    case 1:
        return launch_lut<BITS, 1, 1, EP_F32, XS>(a, waves, s);
    case 2:
        return launch_lut<BITS, 1, 2, EP_F32, XS>(a, waves, s);
    case 4:
        return launch_lut<BITS, 1, 4, EP_F32, XS>(a, waves, s);
    default:
        return launch_lut<BITS, 1, 8, EP_F32, XS>(a, waves, s);
    }
}

GemvArgs make_args(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y)
{
    GemvArgs a{};
    a.x = x.ptr;
    a.x_dtype = x.dtype;
    a.ldx = x.ld;
    a.M = (int)M;
    a.row_bytes = w.bits() == 4 ? w.K / 2 : w.K;
    a.scale_dtype = w.scale_dtype;
    a.lds = w.ld_scale;
    a.cb_dtype = w.cb_dtype;
    a.levels = w.levels;
    a.y_dtype = y.dtype;
    a.ldy = y.ld;
    a.accumulate = y.accumulate;
    a.K = w.K;
    a.group = w.group;
    a.nseg = 1;
    a.seg[0] = Seg{w.packed, w.scale, w.cb, y.ptr, (int)w.N, 0, 0};
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

// hl: the activations are f32 (hi + lo terms, twice the registers).
bool shape_ok(int bits, int64_t N, int64_t K, int group, int64_t ld_scale, bool hl)
{
    if (N < 1 || N > INT32_MAX || K < 1)
        return false;
    if (bits == 4 ? (K % 32 != 0 || group % 32 != 0) : (K % 16 != 0 || group % 16 != 0))
        return false;
    const int64_t rb = bits == 4 ? K / 2 : K;
    if (N * rb >= ((int64_t)1 << 31) || N * ld_scale >= ((int64_t)1 << 31))
        return false;
    if (K > 16384)
        return false;
    int spw, waves;
    plan(rb, spw, waves);
    return spw <= 8 && fits(bits, spw, 1, hl);
}

}  // namespace

// The most activation rows the row kernel takes at once, with 16-bit
// activations and rows of 4, 8 or 16 slabs: 4 with 4-bit indices (4096^2
// at M = 2 / 3 / 4: 7.65 / 10.1 / 10.2 -> 5.8 / 7.9 / 8.3 us against
// gemv_lut_kernel; 2 for rows of 16 slabs, whose four would spill), 2 with
// 8-bit ones (10.1 -> 9.4 us at M = 2; at M = 3 and 4 the MFMA small-M
// kernel is faster: 10.2 against 11.3 and 11.5); else 1
constexpr int row_max_mt(int bits, int S, int xdt)
{
    return xdt == EP_F32 || (S != 4 && S != 8 && S != 16) ? 1 : (bits == 8 || S == 16 ? 2 : 4);
}

// The row lengths gemv_row_kernel serves, in 256-byte slabs (against
// gemv_lut_kernel at config 3's 8-bit M = 1: 4096^2 8.23 -> 5.84 us,
// 14336 x 4096 21.6 -> 17.5 us, 4096 x 14336 22.6 -> 19.1 us).
static int row_slabs(int64_t row_bytes, int bits)
{
    if (row_bytes % kSlabBytes != 0)
        return 0;
    const int s = (int)(row_bytes / kSlabBytes);
    const bool ok = s == 4 || s == 8 || s == 12 || s == 16 || s == 24 || s == 28 || s == 32 || (s == 56 && bits == 8);
    return ok ? s : 0;
}
// M = 1 at every served length; with 16-bit activations at rows of 4, 8 or
// 16 slabs also M = 2 (and M = 3, 4 with 4-bit indices, but 2 at 16 slabs):
// row_max_mt.
static bool row_serves_shape(int bits, int64_t row_bytes, int xdt, int64_t M)
{
    const int s = row_slabs(row_bytes, bits);
    return s != 0 && M <= row_max_mt(bits, s, xdt);
}

bool gemv_serves(const PackedDesc &w, const ActDesc &x, int64_t M)
{
    const int bits = w.bits();
    if (M < 1 || M > 4 || !shape_ok(bits, w.N, w.K, w.group, w.ld_scale, x.dtype == EP_F32))
        return false;
    if (((uintptr_t)w.packed & 15) != 0)
        return false;
    const int esz = x.dtype == EP_F32 ? 4 : 2;
    if (((uintptr_t)x.ptr & 15) != 0 || (M > 1 && (x.ld * esz) % 16 != 0))
        return false;
    if (row_serves_shape(bits, bits == 4 ? w.K / 2 : w.K, x.dtype, M))
        return true;
    int spw, waves;
    plan(bits == 4 ? w.K / 2 : w.K, spw, waves);
    const int mt = M == 1 ? 1 : (M == 2 ? 2 : 4);
    if (mt > 2 && w.K > 4096)
        return false;  // activations of 4 rows staged in LDS: K <= 4096
    return fits(bits, spw, mt, x.dtype == EP_F32);
}

static int row_kernel_slabs(const GemvArgs &a, int bits) { return row_slabs(a.row_bytes, bits); }
static bool row_serves(const GemvArgs &a, int bits, int xdt, int64_t M)
{
    return row_serves_shape(bits, a.row_bytes, xdt, M);
}

template <int BITS, int XDT, int S, int MT>
static void launch_row_sc(const GemvArgs &a, dim3 g, dim3 b, hipStream_t stream)
{
    if (a.scale_dtype == EP_F32)
        hipLaunchKernelGGL((gemv_row_kernel<BITS, XDT, S, true, MT>), g, b, 0, stream, a);
    else
        hipLaunchKernelGGL((gemv_row_kernel<BITS, XDT, S, false, MT>), g, b, 0, stream, a);
}

template <int BITS, int XDT, int S>
static void launch_row_x(const GemvArgs &a, dim3 g, dim3 b, hipStream_t stream)
{
    constexpr int MX = row_max_mt(BITS, S, XDT);
    if constexpr (MX >= 4) {
        if (a.M > 2) {
            launch_row_sc<BITS, XDT, S, 4>(a, g, b, stream);
            return;
        }
    }
    if constexpr (MX >= 2) {
        if (a.M == 2) {
            launch_row_sc<BITS, XDT, S, 2>(a, g, b, stream);
            return;
        }
    }
    launch_row_sc<BITS, XDT, S, 1>(a, g, b, stream);
}

template <int BITS, int S>
static int launch_row(const GemvArgs &a, int xdt, hipStream_t stream)
{
    constexpr int LPR = S / 4;
    const int rows = EP_GEMV_ROW_WAVES * (LPR < 4 && 4 % LPR == 0 ? 4 / LPR : 1);
    const dim3 g((unsigned)((a.seg[0].N + rows - 1) / rows), a.gidx ? (unsigned)a.ntok : 1u);
    const dim3 b(64 * EP_GEMV_ROW_WAVES);
    if (xdt == EP_BF16)
        launch_row_x<BITS, EP_BF16, S>(a, g, b, stream);
    else if (xdt == EP_F16)
        launch_row_x<BITS, EP_F16, S>(a, g, b, stream);
    else
        launch_row_x<BITS, EP_F32, S>(a, g, b, stream);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

template <int BITS>
static int dispatch_row_bits(const GemvArgs &a, int S, int xdt, hipStream_t stream)
{
    switch (S) {
    case 4:
        return launch_row<BITS, 4>(a, xdt, stream);
    case 8:
        return launch_row<BITS, 8>(a, xdt, stream);
    case 12:
        return launch_row<BITS, 12>(a, xdt, stream);
    case 16:
        return launch_row<BITS, 16>(a, xdt, stream);
    case 24:
        return launch_row<BITS, 24>(a, xdt, stream);
    case 28:
        return launch_row<BITS, 28>(a, xdt, stream);
    case 32:
        return launch_row<BITS, 32>(a, xdt, stream);
    default:
        if constexpr (BITS == 8)
            return launch_row<BITS, 56>(a, xdt, stream);  // 8-bit K = 14336
        return set_error(EP_DECLINE_SHAPE, "row GEMV: %d slabs", S);
    }
}

static int dispatch_row(const GemvArgs &a, int bits, int xdt, hipStream_t stream)
{
    const int S = row_kernel_slabs(a, bits);
    return bits == 4 ? dispatch_row_bits<4>(a, S, xdt, stream) : dispatch_row_bits<8>(a, S, xdt, stream);
}

int launch_gemv(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                hipStream_t stream)
{
    if (!gemv_serves(w, x, M))
        return EP_DECLINE_SHAPE;
    const GemvArgs a = make_args(w, x, M, y);
    if (row_serves(a, w.bits(), x.dtype, M))
        return dispatch_row(a, w.bits(), x.dtype, stream);
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

int launch_gemv_gather(const PackedDesc &w, const ActDesc &x, int64_t T, const int *ids, int E,
                       const OutDesc &y, hipStream_t stream)
{
    if (!gemv_serves(w, x, 1) || y.accumulate)
        return EP_DECLINE_SHAPE;
    // token y's activations are read with 16-byte loads at x + y * ldx
    const int esz = x.dtype == EP_F32 ? 4 : 2;
    if (T > 1 && (x.ld * esz) % 16 != 0)
        return set_error(EP_DECLINE_SHAPE, "gathered GEMV: x row stride not a multiple of 16 bytes");
    if (T > 65535)
        return set_error(EP_DECLINE_SHAPE, "gathered GEMV: at most 65535 tokens per launch");
    GemvArgs a = make_args(w, x, 1, y);
    a.ldx = x.ld;
    a.ldy = y.ld;
    a.gidx = ids;
    a.E = E;
    a.ntok = (int)T;
    a.estride_w = w.N * a.row_bytes;
    a.estride_s = w.N * w.ld_scale * (w.scale_dtype == EP_F32 ? 4 : 2);
    if (row_kernel_slabs(a, w.bits()) != 0)
        return dispatch_row(a, w.bits(), x.dtype, stream);
    int spw, waves;
    plan(a.row_bytes, spw, waves);
    if (w.bits() == 4)
        return dispatch_spw<4, 1>(a, x.dtype, spw, waves, stream);
    return dispatch_spw<8, 1>(a, x.dtype, spw, waves, stream);
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

int launch_gemv_fused(const FusedGemv &f, hipStream_t stream)
{
    if (f.nseg < 1 || f.nseg > kMaxSeg)
        return set_error(EP_ERR_ARG, "fused GEMV: nseg=%d outside 1..%d", f.nseg, kMaxSeg);
    if (f.xsrc != XS_RMSNORM && f.xsrc != XS_SWIGLU && f.xsrc != XS_PLAIN)
        return set_error(EP_ERR_ARG, "fused GEMV: unknown activation source %d", f.xsrc);
    const int bits = f.levels <= 16 ? 4 : 8;
    GemvArgs a{};
    a.x = f.x;
    a.x_dtype = f.xsrc == XS_PLAIN ? f.x_dtype : EP_F32;
    a.ldx = f.K;
    a.M = 1;
    a.x2 = f.x2;
    a.eps = f.eps;
    a.row_bytes = bits == 4 ? f.K / 2 : f.K;
    a.scale_dtype = f.scale_dtype;
    a.lds = (f.K + f.group - 1) / f.group;
    a.cb_dtype = f.cb_dtype;
    a.levels = f.levels;
    a.y_dtype = f.y_dtype;
    a.ldy = 0;
    a.accumulate = f.accumulate;
    a.K = f.K;
    a.group = f.group;
    a.nseg = f.nseg;
    for (int i = 0; i < f.nseg; ++i) {
        if (!shape_ok(bits, f.seg[i].N, f.K, f.group, a.lds, a.x_dtype == EP_F32))
            return set_error(EP_DECLINE_SHAPE, "fused GEMV: segment %d shape not served", i);
        if (((uintptr_t)f.seg[i].packed & 15) != 0)
            return set_error(EP_DECLINE_SHAPE, "fused GEMV: packed not 16-byte aligned");
        a.seg[i] = Seg{f.seg[i].packed, f.seg[i].scale, f.seg[i].cb, f.seg[i].y, (int)f.seg[i].N,
                       0, 0};
    }
    if (((uintptr_t)f.x & 15) != 0 || (f.x2 && ((uintptr_t)f.x2 & 15) != 0))
        return set_error(EP_DECLINE_SHAPE, "fused GEMV: activations not 16-byte aligned");
    int spw, waves;
    plan(a.row_bytes, spw, waves);
    if (f.xsrc == XS_PLAIN)
        return bits == 4 ? dispatch_spw<4, 1>(a, a.x_dtype, spw, waves, stream)
                         : dispatch_spw<8, 1>(a, a.x_dtype, spw, waves, stream);
    if (f.xsrc == XS_RMSNORM)
        return bits == 4 ? dispatch_fused<4, XS_RMSNORM>(a, spw, waves, stream)
                         : dispatch_fused<8, XS_RMSNORM>(a, spw, waves, stream);
    return bits == 4 ? dispatch_fused<4, XS_SWIGLU>(a, spw, waves, stream)
                     : dispatch_fused<8, XS_SWIGLU>(a, spw, waves, stream);
}

}  // namespace ep
