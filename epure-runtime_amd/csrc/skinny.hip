// Small-M (2 <= M <= 64) fused codebook dequant-matmul on gfx950 MFMA.
//
// y[M, N] = x[M, K] . W[N, K]^T with W[n, k] = cb[idx[n, k]] * scale[n, k / group],
// for the row counts between the batch-1 GEMV and the compute-bound prefill
// tiles.  Reference behaviour: the table kernel epure/kernels/_triton.py:54-107
// (fp16 operands, fp32 accumulation; its grid had one program per 16x64
// output tile, too few at small M, _triton.py:260-263) and the reference's
// split-K experiments (_triton.py:239-315, :317-400).
//
// At these M the contraction is HBM-bound: the packed bytes must stream at
// full rate while the MFMA units and LDS are mostly idle.  So:
//  * a workgroup (8 waves) owns one K split of KS values and up to TPW row
//    tiles of 128 rows (16 per wave); its activation and codebook loads go
//    out at entry, half of its weight loads (16 bytes per lane, LD per
//    tile, 16 in all) once the activations are staged, so those first
//    loads do not queue behind every CU's weight burst, the other half
//    right after the table build (all at once, they would hold the waves at
//    the issue until most had landed);
//  * weights are dequantized in registers straight into the B operand of
//    v_mfma_f32_16x16x32_f16: lane (j = lane & 15, q = lane >> 4) loads 16
//    bytes of row j -- 32 (4-bit) or 16 (8-bit) consecutive weights -- looks
//    each byte up in the 64-replica LDS pair table of gemv_core.h and
//    multiplies by the chunk's group scale in fp16 (the tile of
//    materialize(float16), runtime.py:78-89); the MFMA's k index of lane q,
//    element e maps to the weight 8 s + e of the lane's chunk (sub-step s),
//    and the activation operand is read from LDS with the same mapping;
//  * activations of the split (M rows x KS) are staged once in LDS as fp16
//    after an exact power-of-two rescale per row (exponent of the row's
//    largest |x| within the split), and the partial sums are scaled back
//    exactly before they leave the workgroup;
//  * with one split the results go straight to y; otherwise each split
//    writes f32 partials [S][M][N] and sk_reduce_kernel sums them in split
//    order (deterministic; no atomics, no counters);
//  * with 16-bit activations, enough 16-row tiles to fill the CUs and M at
//    most 16 per tile of a workgroup (8-bit indices up to M = 64, 4-bit up
//    to M = 8), sk1_kernel instead: a workgroup owns 1, 2 or 4 row tiles
//    over the whole of K, one launch, no partials (its comment has the
//    layout); bf16 activations with 8-bit indices take its bf16 path (raw
//    bf16 operands, the codebook as exact bf16 hi + lo terms);
//  * with 8-bit indices at 33 <= M <= 64, and at 17 <= M <= 32 on layers
//    of at least 2^25 weights, sk2_kernel instead: K slices of 2048 or
//    4096 values, each
//    wave's activation columns held in registers for all of its
//    workgroup's row tiles (its comment has the layout).
#include <algorithm>

#include "ep_common.h"
#include "ep_internal.h"
#include "gemv_core.h"

namespace ep {
namespace {

constexpr int kSkThreads = 512;
constexpr int kSkWaves = kSkThreads / 64;
constexpr int kSkRows = 16 * kSkWaves;  // rows of a row tile
// 16-byte weight loads per lane and row tile (LD: 4, 8 or 16) and row
// tiles per workgroup (16 / LD: 16 loads per lane in flight).  A longer K
// split means fewer f32 partials [S][M][N] and fewer rounds of loads in the
// ordered reduction; the launch takes the longest split whose grid still
// fills every CU.  The staged activation tile (16 MT rows x K split, fp16)
// stays within ~66 KiB next to the 64 KiB table: sk_ld_max.
constexpr int sk_ld_max(int bits, int mt)
{
    return bits == 8 ? (mt <= 2 ? 16 : 8) : (mt == 1 ? 16 : (mt == 2 ? 8 : 4));
}

template <int BITS>
constexpr int sk_kpl()
{
    return BITS == 4 ? 32 : 16;  // weights per 16-byte load
}
template <int BITS, int LD>
constexpr int sk_ks()
{
    return LD * 4 * sk_kpl<BITS>();  // K per split: LD x 64 bytes of a row
}

constexpr uint32_t kOut = 0x7ffffff0u;  // a buffer offset past every buffer's end

// The B operand of one lane's 16-byte chunk: its KPL weights dequantized
// through the pair table and multiplied by the chunk's fp16 group scale (the
// tile of materialize(float16), runtime.py:78-89), as KPL / 8 pieces of
// eight (piece s = weights 8 s .. 8 s + 7 of the chunk).
template <int BITS>
EP_DEV void dequant_chunk(const uint32_t *tab, u32x4_t w, uint32_t sraw, uint32_t lane4, f16x8_t *bv)
{
    constexpr int KPL = sk_kpl<BITS>();
    const f16_t s16 = f16_from_bits((uint16_t)sraw);
    const f16x2_t s2 = (f16x2_t){s16, s16};
    f16x2_t pr[KPL / 2];
    if constexpr (BITS == 4) {
#pragma unroll
        for (int wd = 0; wd < 4; ++wd)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                pr[wd * 4 + b] = as_f16x2(lds_read_u32(tab, __builtin_amdgcn_perm(w[wd], lane4, kSelByte[b]))) * s2;
    } else {
#pragma unroll
        for (int wd = 0; wd < 4; ++wd)
#pragma unroll
            for (int b = 0; b < 4; b += 2) {
                const uint32_t t0 = lds_read_u32(tab, __builtin_amdgcn_perm(w[wd], lane4, kSelByte[b]));
                const uint32_t t1 = lds_read_u32(tab, __builtin_amdgcn_perm(w[wd], lane4, kSelByte[b + 1]));
                pr[wd * 2 + b / 2] = as_f16x2(__builtin_amdgcn_perm(t1, t0, 0x05040100u)) * s2;
            }
    }
#pragma unroll
    for (int s = 0; s < KPL / 8; ++s)
        bv[s] = (f16x8_t){pr[4 * s][0],     pr[4 * s][1],     pr[4 * s + 1][0], pr[4 * s + 1][1],
                          pr[4 * s + 2][0], pr[4 * s + 2][1], pr[4 * s + 3][0], pr[4 * s + 3][1]};
}

struct SkArgs {
    uint32_t xbytes, wbytes, sbytes, cbbytes;  // extents of x, packed, scale, cb
    const void *x;
    int64_t ldx;
    int M;
    const uint8_t *packed;
    uint32_t row_bytes;
    const void *scale;
    int scale_dtype;
    int64_t lds;
    const void *cb;
    int cb_dtype;
    int levels;
    int N;
    int K;
    int group;
    int tiles;   // row tiles, ceil(N / 128)
    int gtiles;  // workgroups along the row tiles (gridDim.x)
    void *y;
    int y_dtype;
    int64_t ldy;
    int accumulate;
    float *part;  // [S][M][N] partials (null: results go straight to y)
};

template <int BITS, int MT, int XDT, int LD>
__global__ void __launch_bounds__(kSkThreads) sk_kernel(SkArgs a)
{
    constexpr int KPL = sk_kpl<BITS>();
    static_assert(LD <= sk_ld_max(BITS, MT), "activation tile within LDS");
    constexpr int TPW = 16 / LD;
    constexpr int KS = sk_ks<BITS, LD>();
    constexpr int SUB = KPL / 8;          // MFMA sub-steps per load
    constexpr int MR = 16 * MT;           // staged activation rows
    constexpr int XLD = KS + 8;           // halfs per staged row (padding: conflict-free reads)
    constexpr int TPR = kSkThreads / MR;  // staging threads per row
    constexpr int VPT = KS / TPR;         // values per staging thread
    constexpr int XE = XDT == EP_F32 ? 4 : 2;
    constexpr int XP = VPT * XE / 16;     // 16-byte activation pieces per thread
    static_assert(VPT % 8 == 0, "staging in 8-value pieces");

    __shared__ __align__(16) uint32_t tab[kTabDwords];
    __shared__ __align__(16) f16_t xs[MR * XLD];
    __shared__ float s_pw[MR];
    __shared__ uint32_t s_cbraw[kSkThreads];
    __shared__ uint16_t s_cb[256];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int split = blockIdx.y;
    const int ka = split * KS;
    const uint32_t kbyte = BITS == 4 ? (uint32_t)ka / 2 : (uint32_t)ka;
    const auto rx = buffer_rsrc(a.x, a.xbytes), rw = buffer_rsrc(a.packed, a.wbytes);
    const auto rs = buffer_rsrc(a.scale, a.sbytes), rcb = buffer_rsrc(a.cb, a.cbbytes);

    // ---- loads, in the order they are needed: vector-memory results return
    // in order, so a wait for the activations must not also wait for the
    // weights.  Every load is a buffer load; a masked lane gets an offset past
    // the buffer's end and reads 0 (no select on a loaded value, which the
    // compiler would turn into a load at the point of use).
    const uint32_t cbraw = __builtin_amdgcn_raw_buffer_load_b32(rcb, tid < 256 ? tid * 4 : kOut, 0, 0);
    const int xr = tid / TPR, xk0 = (tid % TPR) * VPT;
    u32x4_t xv[XP];
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        const int k = ka + xk0 + p * (16 / XE);
        const bool ok = xr < a.M && k < a.K;  // K % 16 == 0: pieces are whole
        const uint32_t off = ok ? (uint32_t)(((int64_t)xr * a.ldx + k) * XE) : kOut;
        xv[p] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
    }
    // The weights in two halves: the first half after the activation
    // staging, the second after the table build.  A workgroup's weights (up
    // to 128 KB) are more than a CU keeps in flight, so issuing them all at
    // once would hold the waves at the issue until most had landed; this way
    // the table build overlaps the stream.
    constexpr int LH = LD / 2;
    u32x4_t w[TPW][LD];
    uint32_t sraw[TPW][LD];  // fp16 scale bits; 0 where the chunk is masked
    auto issue = [&](int l0, int l1) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const int tile = (int)blockIdx.x + t * a.gtiles;
            const int n = tile * kSkRows + wave * 16 + j;
            const bool live = tile < a.tiles && n < a.N;
#pragma unroll
            for (int l = 0; l < LD; ++l) {
                if (l < l0 || l >= l1)
                    continue;
                const int kc = ka + KPL * (4 * l + q);  // first k of the lane's chunk
                const bool ok = live && kc < a.K;
                const uint32_t off = (uint32_t)n * a.row_bytes + kbyte + (uint32_t)(16 * (4 * l + q));
                w[t][l] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? (int)off : (int)kOut, 0, 2);
                const uint32_t soff = (uint32_t)(((int64_t)n * a.lds + kc / a.group) * 2);
                sraw[t][l] = __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? (int)soff : (int)kOut, 0, 0);
            }
        }
    };

    // ---- codebook -> fp16 bits; activations of the split -> LDS as fp16
    // after the row's exact power-of-two rescale
    s_cbraw[tid] = cbraw;  // unconditional: a conditional use would sink the load
    {
        float v[VPT];
#pragma unroll
        for (int p = 0; p < XP; ++p) {
            if constexpr (XDT == EP_F32) {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    v[4 * p + t] = __uint_as_float(xv[p][t]);
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    unpack_pair<XDT>(xv[p][t], v[8 * p + 2 * t], v[8 * p + 2 * t + 1]);
            }
        }
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
            am = fmaxf(am, fabsf(v[i]));
#pragma unroll
        for (int o = 1; o < TPR; o <<= 1)
            am = fmaxf(am, __shfl_xor(am, o, 64));
        const int e = row_exponent(am);
        const float pw = ldexpf(1.0f, -e);
        f16_t *dst = xs + xr * XLD + xk0;
#pragma unroll
        for (int p = 0; p < VPT; p += 8) {
            f16x8_t h;
#pragma unroll
            for (int t = 0; t < 8; ++t)
                h[t] = (f16_t)(v[p + t] * pw);
            *(f16x8_t *)(dst + p) = h;
        }
        if (tid % TPR == 0)
            s_pw[xr] = ldexpf(1.0f, e);
    }
    // the first half of the weights only now, after the activations have
    // landed: issued at entry they queue with every CU's weight burst and
    // hold the staging back (4096^2 at M = 64: 19.6 -> 19.1 us)
    __builtin_amdgcn_sched_barrier(0);
    issue(0, LH);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    if (tid < 256) {
        float c = 0.0f;
        if (tid < a.levels) {
            if (a.cb_dtype == EP_F32) {
                c = __uint_as_float(s_cbraw[tid]);
            } else {
                const uint16_t h = (uint16_t)(s_cbraw[tid >> 1] >> (16 * (tid & 1)));
                c = a.cb_dtype == EP_F16 ? (float)f16_from_bits(h) : bf16_to_f32(h);
            }
        }
        s_cb[tid] = f16_bits((f16_t)c);
    }
    lds_barrier();
    build_table<BITS>(tab, s_cb);
    issue(LH, LD);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();

    const uint32_t lane4 = ((uint32_t)lane & 31) << 2;  // the lane's table copy
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int tile = (int)blockIdx.x + t * a.gtiles;
        if (tile >= a.tiles)
            break;
        f32x4_t acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            acc[mt] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int l = 0; l < LD; ++l) {
            f16x8_t bv[SUB];
            dequant_chunk<BITS>(tab, w[t][l], sraw[t][l], lane4, bv);
#pragma unroll
            for (int s = 0; s < SUB; ++s) {
                const int kx = KPL * (4 * l + q) + 8 * s;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const f16x8_t av = *(const f16x8_t *)(xs + (16 * mt + j) * XLD + kx);
                    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv[s], acc[mt], 0, 0, 0);
                }
            }
        }
        // D[row][col] of a 16x16 tile: lane col + 16 * (row / 4), register
        // row % 4.  Stores only (y is never read here: accumulation goes
        // through the reduction).
        const int n = tile * kSkRows + wave * 16 + j;
        if (n < a.N) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = 16 * mt + 4 * q + r;
                    if (m < a.M) {
                        const float v = acc[mt][r] * s_pw[m];
                        if (a.part) {
                            *(__attribute__((address_space(1))) float *)(a.part + ((int64_t)split * a.M + m) * a.N + n) = v;
                        } else {
                            const int64_t off = (int64_t)m * a.ldy + n;
                            if (a.y_dtype == EP_F32)
                                *(__attribute__((address_space(1))) float *)((float *)a.y + off) = v;
                            else if (a.y_dtype == EP_F16)
                                *(__attribute__((address_space(1))) uint16_t *)((uint16_t *)a.y + off) = f16_bits((f16_t)v);
                            else
                                *(__attribute__((address_space(1))) uint16_t *)((uint16_t *)a.y + off) = f32_to_bf16(v);
                        }
                    }
                }
        }
    }
}

// One launch for small M with fp16/bf16 activations.  A
// workgroup owns T row tiles of 16 rows (tiles blockIdx.x + t * gridDim.x)
// over the whole of K, so its sums are final: no partials, no second
// launch.  Its 16 waves at one tile (four per SIMD, to hide the latency of
// the table lookups; 8 where the tiles' weights or more activation blocks
// need the registers) split K into contiguous runs of rounds; a round is RK = 4 KPL P
// values of K.  In a round, lane (j, q) loads P 16-byte pieces of row j
// (piece c at chunk 4 c + q of the round: each load instruction covers 64
// bytes of 16 rows, the P of a round, issued back to back, 64 P contiguous
// bytes of each) for each of the T tiles -- the B operand, dequantized
// through the table -- and the KPL activations of row j at each piece's k
// -- the A operand, straight from global memory: x is small and stays in
// L2, and one load serves the T tiles.  fp16 activations are the operand
// as they are; bf16 ones become fp16 after the power-of-two rescale of the
// row's largest |x| in the round (bf16_operand), and each round's MFMA sums
// are scaled back exactly before they join the running f32 sums.  Loads
// run D rounds ahead of the MFMAs.  At the end the waves' sums meet in LDS
// (over the table, which is no longer needed) and are added in wave order.
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

EP_DEV uint32_t max_over_row_lanes(uint32_t v)  // max over lanes l, l ^ 16, l ^ 32, l ^ 48
{
    const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max(b[0], b[1]);
}

// bf16 activations -> the fp16 A operand times 2^-e, e the row's exponent
// over its four lanes' pieces (returned; the same in the four lanes).  On
// the bit patterns, two values per instruction: |x| as a 15-bit integer
// orders like |x|; e = (largest exponent field of the row) - 140 puts the
// row's largest |x| * 2^-e in [2^13, 2^14); the exponent field drops by
// 112 + e and the 7-bit mantissa moves up 3 bits, exactly (values below
// 2^-14 after the rescale, 2^-27 of the row's largest, flush to 0).  With
// inf, NaN or |x| >= 2^124 anywhere in the wave, in floats instead, where
// fp16 overflows to inf as it would unscaled.
template <int SUB>
EP_DEV int bf16_operand(const u32x4_t *xv, f16x8_t *av)
{
    u16x2_t mx = {0, 0};
#pragma unroll
    for (int p = 0; p < SUB; ++p)
#pragma unroll
        for (int t = 0; t < 4; ++t)
            mx = __builtin_elementwise_max(mx, __builtin_bit_cast(u16x2_t, xv[p][t] & 0x7fff7fffu));
    const uint32_t em = max_over_row_lanes(max((uint32_t)mx[0], (uint32_t)mx[1]));
    int e = em == 0 ? 0 : (int)(em >> 7) - 140;
    e = e < -110 ? -110 : e;
    if (__builtin_amdgcn_ballot_w64(e > 110) == 0) {
        const uint16_t sub = (uint16_t)((112 + e) << 7);
        const u16x2_t sub2 = {sub, sub};
#pragma unroll
        for (int p = 0; p < SUB; ++p) {
            u32x4_t h;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t u = xv[p][t];
                u16x2_t m = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2_t, u & 0x7fff7fffu), sub2);
                m = m << (u16x2_t){3, 3};
                h[t] = __builtin_bit_cast(uint32_t, m) | (u & 0x80008000u);
            }
            av[p] = __builtin_bit_cast(f16x8_t, h);
        }
        return e;
    }
    e = row_exponent(__uint_as_float(em << 16));  // em: the row's largest |x| as bf16 bits
    const float pw = ldexpf(1.0f, -e);
#pragma unroll
    for (int p = 0; p < SUB; ++p)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float lo, hi;
            unpack_pair<EP_BF16>(xv[p][t], lo, hi);
            av[p][2 * t] = (f16_t)(lo * pw);
            av[p][2 * t + 1] = (f16_t)(hi * pw);
        }
    return e;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// The 8-bit table of the bf16 path: entry b holds fp16(cb[b]) as two bf16
// terms, hi = its top 8 significant bits (truncated) in the low half and
// lo = fp16(cb[b]) - hi (at most 3 significant bits, so exact) in the high
// half: hi + lo is the fp16 value exactly.  Same layout as build_table.
EP_DEV void build_table_hl(uint32_t *tab, const uint16_t *cb16)
{
#pragma unroll 4
    for (int i = threadIdx.x; i < 256 * kTabCopies / 4; i += blockDim.x) {
        const int b = i >> 3;
        const float f = (float)f16_from_bits(cb16[b]);
        const uint32_t hi = __float_as_uint(f) & 0xffff0000u;
        const float lo = f - __uint_as_float(hi);
        const uint32_t v = (hi >> 16) | (__float_as_uint(lo) & 0xffff0000u);
        ((u32x4_t *)tab)[b * 16 + (i & 7)] = (u32x4_t){v, v, v, v};
    }
}

// The bf16 path's B operands of one lane's 16-byte chunk (8-bit indices):
// the hi and the lo terms of weights 8 s .. 8 s + 7 as eight bf16 each (no
// group scale: it multiplies the piece's sums).
EP_DEV void dequant_chunk_hl(const uint32_t *tab, u32x4_t w, uint32_t lane4, u32x4_t *bh, u32x4_t *bl)
{
#pragma unroll
    for (int wd = 0; wd < 4; ++wd)
#pragma unroll
        for (int b = 0; b < 4; b += 2) {
            const uint32_t t0 = lds_read_u32(tab, __builtin_amdgcn_perm(w[wd], lane4, kSelByte[b]));
            const uint32_t t1 = lds_read_u32(tab, __builtin_amdgcn_perm(w[wd], lane4, kSelByte[b + 1]));
            const int p = wd * 2 + b / 2;  // weights 2 p, 2 p + 1: piece p / 4, dword p % 4
            bh[p >> 2][p & 3] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
            bl[p >> 2][p & 3] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
        }
}

// HL (8-bit indices, bf16 activations, groups of a multiple of 64 values):
// the bf16 path -- the raw bf16 x is the A operand of
// v_mfma_f32_16x16x32_bf16 (no conversion, no rescale: bf16 has f32's
// range), the codebook value the B operand as its exact hi + lo bf16 terms
// (two MFMAs), and the group scale multiplies each piece's f32 sums (a
// piece's 4 x 16 values lie in one group).  The products x * fp16(cb) are
// exact in f32 and summed in f32; the f32 group scale then applies the
// dequantized weight cb * scale without its rounding to fp16 (closer to
// the f32 reference, not farther).
template <int BITS, int XDT, int T, int D, int P, int MT, int NT, bool HL>
__global__ void __launch_bounds__(NT) sk1_kernel(SkArgs a)
{
    constexpr int NW = NT / 64;      // waves
    constexpr int KPL = sk_kpl<BITS>();
    constexpr int RK = 4 * KPL * P;  // P pieces of 16 bytes per lane and tile: 64 P bytes of a row
    constexpr int SUB = KPL / 8;     // MFMA sub-steps per piece = 16-byte x loads per lane and piece
    static_assert(NW * MT * 256 <= kTabDwords, "one tile's wave sums fit over the table");
    static_assert(XDT != EP_F32, "16-bit activations");
    static_assert(!HL || (BITS == 8 && XDT == EP_BF16), "the bf16 path: 8-bit indices, bf16 x");

    __shared__ __align__(16) uint32_t tab[kTabDwords];
    __shared__ uint32_t s_cbraw[NT];
    __shared__ uint16_t s_cb[256];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int nr = (a.K + RK - 1) / RK;
    const int rb = wave * nr / NW, re = (wave + 1) * nr / NW;
    const auto rx = buffer_rsrc(a.x, a.xbytes), rw = buffer_rsrc(a.packed, a.wbytes);
    const auto rs = buffer_rsrc(a.scale, a.sbytes), rcb = buffer_rsrc(a.cb, a.cbbytes);

    const uint32_t cbraw = __builtin_amdgcn_raw_buffer_load_b32(rcb, tid < 256 ? tid * 4 : kOut, 0, 0);
    // Loads of round r into slot d (masked lanes read 0 from past the
    // buffer's end; rounds past the wave's run are all masked, so every
    // slot sees the same number of loads).  Piece c of a round is chunk
    // 4 c + q: a load instruction covers 64 bytes of each of 16 rows, and
    // the P instructions of a round, issued back to back, 64 P contiguous
    // bytes of each.  Activation rows 16 mt + j, mt < MT.
    u32x4_t xv[D][MT][P][SUB];
    u32x4_t wv[D][P][T];
    uint32_t sv[D][P][T];
    auto issue = [&](int d, int r) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int c = 0; c < P; ++c) {
                const int kc = r * RK + KPL * (4 * c + q), m = 16 * mt + j;
                const bool xok = r < re && kc < a.K && m < a.M;  // K % KPL == 0: chunks are whole
#pragma unroll
                for (int p = 0; p < SUB; ++p) {
                    const uint32_t off = xok ? (uint32_t)(((int64_t)m * a.ldx + kc + 8 * p) * 2) : kOut;
                    xv[d][mt][c][p] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
                }
            }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int tile = (int)blockIdx.x + t * (int)gridDim.x;
            const int n = tile * 16 + j;
#pragma unroll
            for (int c = 0; c < P; ++c) {
                const int kc = r * RK + KPL * (4 * c + q);
                const bool ok = r < re && kc < a.K && tile < a.tiles && n < a.N;
                const uint32_t woff = (uint32_t)n * a.row_bytes + (uint32_t)(BITS == 4 ? kc / 2 : kc);
                wv[d][c][t] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? (int)woff : (int)kOut, 0, 2);
            }
#pragma unroll
            for (int c = 0; c < P; ++c) {
                // HL: the piece's group (its first chunk's), the same in the
                // four lanes of a row whose sums the scale multiplies
                const int kc = r * RK + KPL * (HL ? 4 * c : 4 * c + q);
                const bool ok = r < re && kc < a.K && tile < a.tiles && n < a.N;
                const uint32_t soff = (uint32_t)(((int64_t)n * a.lds + kc / a.group) * 2);
                sv[d][c][t] = __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? (int)soff : (int)kOut, 0, 0);
            }
        }
    };
    // Each wave's codebook entry has landed before its first weight load
    // goes out (issued together with the chip-wide weight burst, it would
    // queue behind it and hold the table build: 4096^2 at M = 4, 11.1 ->
    // 10.5 us); then the first half of the prologue's rounds, the table
    // build, and the rest after it, each wave on its own.
    __builtin_amdgcn_sched_barrier(0);
    s_cbraw[tid] = cbraw;
    __builtin_amdgcn_sched_barrier(0);
    constexpr int DH = D / 2;
#pragma unroll
    for (int d = 0; d < DH; ++d)
        issue(d, rb + d);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    if (tid < 256) {
        float c = 0.0f;
        if (tid < a.levels) {
            if (a.cb_dtype == EP_F32) {
                c = __uint_as_float(s_cbraw[tid]);
            } else {
                const uint16_t h = (uint16_t)(s_cbraw[tid >> 1] >> (16 * (tid & 1)));
                c = a.cb_dtype == EP_F16 ? (float)f16_from_bits(h) : bf16_to_f32(h);
            }
        }
        s_cb[tid] = f16_bits((f16_t)c);
    }
    lds_barrier();
    if constexpr (HL)
        build_table_hl(tab, s_cb);
    else
        build_table<BITS>(tab, s_cb);
    lds_barrier();
#pragma unroll
    for (int d = DH; d < D; ++d)
        issue(d, rb + d);

    const uint32_t lane4 = ((uint32_t)lane & 31) << 2;  // the lane's table copy
    f32x4_t acc[T][MT];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            acc[t][mt] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
    for (int r0 = rb; r0 < re; r0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (HL && r0 + d < re) {
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int c = 0; c < P; ++c) {
                        u32x4_t bh[SUB], bl[SUB];
                        dequant_chunk_hl(tab, wv[d][c][t], lane4, bh, bl);
                        f32x4_t cs[MT];
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            cs[mt] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int s = 0; s < SUB; ++s)
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) {
                                const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xv[d][mt][c][s]);
                                cs[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    av, __builtin_bit_cast(bf16x8_t, bh[s]), cs[mt], 0, 0, 0);
                                cs[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    av, __builtin_bit_cast(bf16x8_t, bl[s]), cs[mt], 0, 0, 0);
                            }
                        const float sc = (float)f16_from_bits((uint16_t)sv[d][c][t]);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                acc[t][mt][r] = fmaf(cs[mt][r], sc, acc[t][mt][r]);
                    }
            } else if (r0 + d < re) {
                f16x8_t av[MT][P][SUB];
                float bk[MT][4];  // the round's power of two of accumulator rows 16 mt + 4 q + r
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    if constexpr (XDT == EP_F16) {
#pragma unroll
                        for (int c = 0; c < P; ++c)
#pragma unroll
                            for (int s = 0; s < SUB; ++s)
                                av[mt][c][s] = __builtin_bit_cast(f16x8_t, xv[d][mt][c][s]);
                    } else {
                        // one exponent per row over the round's P pieces.
                        // D[m][n] of a 16x16 tile: lane n + 16 (m / 4),
                        // register m % 4; lane m holds row m's power of two
                        const float back = ldexpf(1.0f, bf16_operand<P * SUB>(&xv[d][mt][0][0], &av[mt][0][0]));
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            bk[mt][r] = __shfl(back, 4 * q + r, 64);
                    }
                }
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    f32x4_t cs[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        cs[mt] = XDT == EP_F16 ? acc[t][mt] : (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int c = 0; c < P; ++c) {
                        f16x8_t bv[SUB];
                        dequant_chunk<BITS>(tab, wv[d][c][t], sv[d][c][t], lane4, bv);
#pragma unroll
                        for (int s = 0; s < SUB; ++s)
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt)
                                cs[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[mt][c][s], bv[s], cs[mt], 0, 0, 0);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        if constexpr (XDT == EP_F16) {
                            acc[t][mt] = cs[mt];
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                acc[t][mt][r] += cs[mt][r] * bk[mt][r];
                        }
                    }
                }
            }
            issue(d, r0 + d + D);
        }
    }

    // the waves' sums, added in wave order, one tile at a time, in LDS over
    // the table (no longer needed once every wave has passed the barrier)
    float *red = (float *)tab;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        __syncthreads();
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[(wave * MT + mt) * 256 + (4 * q + r) * 16 + j] = acc[t][mt][r];
        __syncthreads();
        const int tile = (int)blockIdx.x + t * (int)gridDim.x;
        for (int i = tid; i < MT * 256; i += NT) {
            const int m = i >> 4, n = tile * 16 + (i & 15);  // i = (16 mt + row) * 16 + col
            if (tile < a.tiles && n < a.N && m < a.M) {
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < NW; ++w)
                    s += red[w * MT * 256 + i];
                const int64_t off = (int64_t)m * a.ldy + n;
                if (a.accumulate)
                    s += load_as_f32(a.y, a.y_dtype, off);
                store_from_f32(a.y, a.y_dtype, off, s);
            }
        }
    }
}

// Split-K with the activations held in registers: 8-bit indices, 17 <= M
// <= 64, fp16 activations, or bf16 ones with groups of a multiple of 64
// values (the bf16 path).  A workgroup's 8 waves split its K slice of 8 R
// values (R = 64 NC per wave).  Each wave takes its R columns of the MB
// 16-row activation blocks once (staged through LDS in rounds of whole
// rows), as MFMA operands, then streams its
// workgroup's row tiles (16 rows each: tiles blockIdx.x + it * gtiles)
// over those columns: lane (i, kq) loads 16 bytes of row i at k0 + 64 c +
// 16 kq, c < NC (a row's R bytes, contiguous, over the wave's NC loads), D
// tiles ahead of the MFMAs.  The MFMA k index 8 kq + j of sub-step (c, e)
// is the value k0 + 64 c + 16 kq + 8 e + j in both operands.  After each
// tile the waves' sums meet in LDS (two buffers, one barrier per tile) and
// are added in wave order: with one split into y, else into the f32
// partials [S][M][N] that sk_reduce_kernel adds in split order.  The
// activations are never converted: fp16 x is the B operand as it is,
// against fp16 weights (the tile of materialize(float16),
// runtime.py:78-89); bf16 x is the A operand of the bf16 MFMA against the
// codebook's exact bf16 hi + lo terms, each 64-value piece's f32 sums
// times its group scale (as sk1_kernel's bf16 path).  Against sk_kernel (K
// slices of 512 staged in LDS, the activations converted by every
// workgroup) the slices are 4-8x longer, so 4-8x fewer partials.  Where a
// time goes (14336 x 4096 at M = 64, seven tiles per workgroup): the table
// is built ~10 us after entry (the codebook and the 256 KiB of activations
// per CU arrive at ~28 GB/s per CU), then each tile takes ~2.7 us (~1.7 of
// lookups, MFMAs and VALU at two waves per SIMD, ~0.9 of barrier and wave
// sums).  Measured and not kept: bf16 x converted once per wave to fp16
// (exact power-of-two row rescale) for single fp16 MFMAs (4096 x 14336 at
// M = 64: 42.1 against 40.3 us); three tiles of loads in flight instead of
// two (no change).
template <int MB, int NC, int D, bool HL, bool G2>
__global__ void __launch_bounds__(kSkThreads) sk2_kernel(SkArgs a)
{
    constexpr int R = 64 * NC;          // K values of a wave
    constexpr int KW = kSkWaves * R;    // K values of a split
    static_assert(!G2 || (HL && NC % 2 == 0), "pairs of pieces per scale: the bf16 path");
    // one LDS block with the table first: at LDS address 0 a lookup's
    // address is the v_perm result itself (at 64 KiB it would take one
    // more add per lookup: the instruction's offset field is 16 bits)
    // activation staging: XR rows of the split's KW values per round (32 KiB)
    constexpr int XR = 16384 / KW, NR = MB * 16 / XR, WPR = kSkWaves / XR;
    constexpr int XS = KW * 2 + 16;  // staged row stride (bytes): conflict-free 16-byte reads
    struct Lds {
        uint32_t tab[kTabDwords];
        union {
            f32x4_t red[2][kSkWaves][MB][64];
            uint8_t xs[XR * XS];
        } u;
        uint32_t cbraw[kSkThreads];
        uint16_t cb[256];
    };
    __shared__ __align__(16) Lds sm;
    uint32_t *const tab = sm.tab;
    auto &red = sm.u.red;
    uint32_t *const s_cbraw = sm.cbraw;
    uint16_t *const s_cb = sm.cb;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, kq = lane >> 4;
    // workgroup L runs on XCD L % 8 (round-robin dispatch).  One split: XCD
    // x takes the consecutive tile groups x G / 8 .. (as near as G allows)
    // -- 14336 x 4096 at M = 17: 28.3 -> 27.0 us.  Several: the pair (split
    // L / gtiles, tile group L % gtiles), which puts the splits of a tile
    // group on one XCD when gtiles % 8 == 0; the per-XCD order there (an
    // XCD's L2 fetching one or two splits' activations, not every split's)
    // measured 33.8 -> 35.0 us at 14336 x 4096, M = 64.
    const int G = (int)gridDim.x, L = (int)blockIdx.x, xcd = L & 7;
    const int q = G == a.gtiles ? xcd * (G >> 3) + min(xcd, G & 7) + (L >> 3) : L;
    const int split = q / a.gtiles, tg = q - split * a.gtiles;
    const int k0 = split * KW + wave * R;
    const int nit = (a.tiles - tg + a.gtiles - 1) / a.gtiles;  // this workgroup's row tiles
    const auto rx = buffer_rsrc(a.x, a.xbytes), rw = buffer_rsrc(a.packed, a.wbytes);
    const auto rs = buffer_rsrc(a.scale, a.sbytes), rcb = buffer_rsrc(a.cb, a.cbbytes);

    // ---- loads in the order they are needed (results return in order):
    // codebook, the activations, the first D tiles' weights
    const uint32_t cbraw = __builtin_amdgcn_raw_buffer_load_b32(rcb, tid < 256 ? tid * 4 : kOut, 0, 0);
    // activations: round r stages rows r XR .. r XR + XR - 1 of the split as
    // whole contiguous rows (wave w loads 4 KiB of row w / WPR, 1 KiB per
    // instruction), then each lane reads its operand pieces of those rows.
    // Loaded straight into operand registers, every load instruction would
    // take 64 bytes from each of 16 rows (runs of 64 bytes), and the 256 KiB
    // per workgroup arrived at ~28 GB/s per CU (4096 x 4096 at M = 64: 18.9
    // -> 17.2 us staged).
    u32x4_t xraw[2][4];
    auto xload = [&](int slot, int r) {
        const int m = r * XR + wave / WPR;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int k = split * KW + ((wave % WPR) * 4096 + p * 1024 + lane * 16) / 2;
            const bool ok = r < NR && m < a.M && k < a.K;
            xraw[slot][p] = __builtin_amdgcn_raw_buffer_load_b128(
                rx, ok ? (int)(((int64_t)m * a.ldx + k) * 2) : (int)kOut, 0, 0);
        }
    };
    xload(0, 0);
    xload(1, 1);
    u32x4_t xv[MB][NC][2];
    // per piece, the same for every tile: whether it lies inside K and its
    // scale's group (the bf16 path scales the sums of the 64-value piece --
    // G2: of the pair of pieces c, c + 1 at a multiple of 128 -- by the
    // group of its first value, the same in the piece's four lanes)
    bool kin[NC], sin[NC];
    uint32_t sgrp[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int k = k0 + 64 * c + 16 * kq, ks = HL ? k0 + 64 * c : k;
        kin[c] = k < a.K;
        sin[c] = ks < a.K;
        sgrp[c] = (uint32_t)(ks / a.group);
    }
    u32x4_t wv[D][NC];
    uint32_t sv[D][NC];  // fp16 scale bits; 0 where masked
    auto issue = [&](int d, int it) {
        const int n = (tg + it * a.gtiles) * 16 + i;
        const bool live = it < nit && n < a.N;
        const uint32_t wrow = (uint32_t)n * a.row_bytes + (uint32_t)(k0 + 16 * kq);
        const uint32_t srow = (uint32_t)n * (uint32_t)a.lds;  // in range: sbytes fits 32 bits
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            wv[d][c] = __builtin_amdgcn_raw_buffer_load_b128(rw, live && kin[c] ? (int)(wrow + 64 * c) : (int)kOut,
                                                             0, 2);
            if (G2 && c % 2 == 1)
                continue;
            sv[d][c] = __builtin_amdgcn_raw_buffer_load_b16(
                rs, live && sin[c] ? (int)((srow + sgrp[c]) * 2) : (int)kOut, 0, 0);
        }
    };
    __builtin_amdgcn_sched_barrier(0);
    s_cbraw[tid] = cbraw;
    lds_barrier();
    if (tid < 256) {
        float c = 0.0f;
        if (tid < a.levels) {
            if (a.cb_dtype == EP_F32) {
                c = __uint_as_float(s_cbraw[tid]);
            } else {
                const uint16_t h = (uint16_t)(s_cbraw[tid >> 1] >> (16 * (tid & 1)));
                c = a.cb_dtype == EP_F16 ? (float)f16_from_bits(h) : bf16_to_f32(h);
            }
        }
        s_cb[tid] = f16_bits((f16_t)c);
    }
    lds_barrier();
    if constexpr (HL)
        build_table_hl(tab, s_cb);
    else
        build_table<8>(tab, s_cb);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        {
            const int row = wave / WPR;
#pragma unroll
            for (int p = 0; p < 4; ++p)
                *(u32x4_t *)(sm.u.xs + row * XS + (wave % WPR) * 4096 + p * 1024 + lane * 16) = xraw[r & 1][p];
        }
        lds_barrier();
        const int mb = r * XR / 16, i0 = (r * XR) % 16;
        if (i >= i0 && i < i0 + XR) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    xv[mb][c][e] = *(const u32x4_t *)(sm.u.xs + (i - i0) * XS + (wave * R + 64 * c + 16 * kq + 8 * e) * 2);
        }
        lds_barrier();
        xload(r & 1, r + 2);
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
        issue(d, d);

    const uint32_t lane4 = ((uint32_t)lane & 31) << 2;  // the lane's table copy
    for (int it0 = 0; it0 < nit; it0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int it = it0 + d;
            if (it >= nit)
                break;
            f32x4_t acc[MB], cs[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[mb] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                if constexpr (HL) {
                    u32x4_t bh[2], bl[2];
                    dequant_chunk_hl(tab, wv[d][c], lane4, bh, bl);
                    if (!G2 || c % 2 == 0)
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
                            cs[mb] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
                    // MB independent sums between two MFMAs on one sum
#pragma unroll
                    for (int e = 0; e < 2; ++e)
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int mb = 0; mb < MB; ++mb)
                                cs[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    __builtin_bit_cast(bf16x8_t, xv[mb][c][e]),
                                    __builtin_bit_cast(bf16x8_t, h ? bl[e] : bh[e]), cs[mb], 0, 0, 0);
                    if (!G2 || c % 2 == 1) {
                        const float sc = (float)f16_from_bits((uint16_t)sv[d][G2 ? c - 1 : c]);
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                acc[mb][r] = fmaf(cs[mb][r], sc, acc[mb][r]);
                    }
                } else {
                    // the weights are the A operand here: D[n][m]
                    f16x8_t bv[2];
                    dequant_chunk<8>(tab, wv[d][c], sv[d][c], lane4, bv);
#pragma unroll
                    for (int e = 0; e < 2; ++e)
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
                            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                bv[e], __builtin_bit_cast(f16x8_t, xv[mb][c][e]), acc[mb], 0, 0, 0);
                }
            }
            issue(d, it + D);
            // D[r][c] of a 16x16 block: lane c + 16 (r / 4), register r % 4
            // (rows m, columns n on the bf16 path; rows n, columns m else)
            const int buf = it & 1;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                red[buf][wave][mb][lane] = acc[mb];
            lds_barrier();
            if (tid < MB * 64) {
                const int mb = tid >> 6, l = tid & 63;
                f32x4_t s = red[buf][0][mb][l];
#pragma unroll
                for (int w = 1; w < kSkWaves; ++w)
                    s += red[buf][w][mb][l];
                // element r: row m0 + r dm, column n0 + r dn
                const int nt = (tg + it * a.gtiles) * 16;
                const int m0 = 16 * mb + (HL ? 4 * (l >> 4) : (l & 15)), dm = HL ? 1 : 0;
                const int n0 = nt + (HL ? (l & 15) : 4 * (l >> 4)), dn = HL ? 0 : 1;
                bool ok[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ok[r] = m0 + r * dm < a.M && n0 + r * dn < a.N;
                if (a.part) {
                    float *dst = a.part + ((int64_t)split * a.M + m0) * a.N + n0;
                    const int64_t step = (int64_t)dm * a.N + dn;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (ok[r])
                            dst[r * step] = s[r];
                } else if (a.y_dtype == EP_F32) {
                    float *y = (float *)a.y + (int64_t)m0 * a.ldy + n0;
                    const int64_t step = (int64_t)dm * a.ldy + dn;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (ok[r])
                            y[r * step] = a.accumulate ? y[r * step] + s[r] : s[r];
                } else {
                    uint16_t *y = (uint16_t *)a.y + (int64_t)m0 * a.ldy + n0;
                    const int64_t step = (int64_t)dm * a.ldy + dn;
                    const bool h = a.y_dtype == EP_F16;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (ok[r]) {
                            float t = s[r];
                            if (a.accumulate)
                                t += h ? (float)f16_from_bits(y[r * step]) : bf16_to_f32(y[r * step]);
                            y[r * step] = h ? f16_bits((f16_t)t) : f32_to_bf16(t);
                        }
                }
            }
        }
    }
}

// y[m, n] (=|+=) sum over splits s = 0 .. S-1 of part[s][m][n], in that
// order.  Four consecutive outputs per thread (N % 4 == 0: 16-byte loads),
// the loads of eight splits in flight at a time.
template <bool VEC>
__global__ void __launch_bounds__(256)
    sk_reduce_kernel(const float *part, int S, int M, int N, void *y, int y_dtype, int64_t ldy,
                     int accumulate)
{
    constexpr int V = VEC ? 4 : 1;
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
    const int64_t total = (int64_t)M * N;
    if (i >= total)
        return;
    float v[V];
#pragma unroll
    for (int t = 0; t < V; ++t)
        v[t] = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 8) {
        float p[8][V];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int s = s0 + u < S ? s0 + u : s0;  // in range; weighted out below
            const float *src = part + (int64_t)s * total + i;
            if constexpr (VEC) {
                const f32x4_t q = *(const f32x4_t *)src;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    p[u][t] = q[t];
            } else {
                p[u][0] = *src;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (s0 + u < S) {
#pragma unroll
                for (int t = 0; t < V; ++t)
                    v[t] += p[u][t];
            }
    }
    const int m = (int)(i / N), n = (int)(i % N);
#pragma unroll
    for (int t = 0; t < V; ++t) {
        const int64_t off = (int64_t)m * ldy + n + t;
        float r = v[t];
        if (accumulate)
            r += load_as_f32(y, y_dtype, off);
        store_from_f32(y, y_dtype, off, r);
    }
}

int sk_mt(int64_t M) { return M <= 16 ? 1 : (M <= 32 ? 2 : 4); }
int sk_split_k(int bits, int ld) { return ld * 4 * (bits == 4 ? sk_kpl<4>() : sk_kpl<8>()); }
int sk_splits_ld(int bits, int ld, int64_t K) { return (int)((K + sk_split_k(bits, ld) - 1) / sk_split_k(bits, ld)); }
// The longest split (most loads per tile) whose workgroups, one row tile
// each at most, still fill the CUs; 4 when none does.
int sk_choose_ld(int bits, int64_t M, int64_t N, int64_t K)
{
    const int64_t tiles = (N + kSkRows - 1) / kSkRows;
    for (int ld = sk_ld_max(bits, sk_mt(M)); ld > 4; ld /= 2)
        if (tiles * sk_splits_ld(bits, ld, K) >= device_cus())
            return ld;
    return 4;
}
int sk_splits(int bits, int64_t M, int64_t N, int64_t K) { return sk_splits_ld(bits, sk_choose_ld(bits, M, N, K), K); }

template <int BITS, int MT, int LD>
int sk_launch_x(const SkArgs &a, int S, int xdt, hipStream_t s)
{
    const dim3 grid((unsigned)a.gtiles, (unsigned)S);
    switch (xdt) {
    case EP_BF16:
        hipLaunchKernelGGL((sk_kernel<BITS, MT, EP_BF16, LD>), grid, dim3(kSkThreads), 0, s, a);
        break;
    case EP_F16:
        hipLaunchKernelGGL((sk_kernel<BITS, MT, EP_F16, LD>), grid, dim3(kSkThreads), 0, s, a);
        break;
    default:
        hipLaunchKernelGGL((sk_kernel<BITS, MT, EP_F32, LD>), grid, dim3(kSkThreads), 0, s, a);
        break;
    }
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

template <int BITS, int MT>
int sk_launch_ld(const SkArgs &a, int S, int ld, int xdt, hipStream_t s)
{
    if constexpr (sk_ld_max(BITS, MT) >= 16)
        if (ld == 16)
            return sk_launch_x<BITS, MT, 16>(a, S, xdt, s);
    if constexpr (sk_ld_max(BITS, MT) >= 8)
        if (ld == 8)
            return sk_launch_x<BITS, MT, 8>(a, S, xdt, s);
    return sk_launch_x<BITS, MT, 4>(a, S, xdt, s);
}

template <int BITS>
int sk_launch_bits(const SkArgs &a, int S, int ld, int xdt, hipStream_t s)
{
    if (a.M <= 16)
        return sk_launch_ld<BITS, 1>(a, S, ld, xdt, s);
    if (a.M <= 32)
        return sk_launch_ld<BITS, 2>(a, S, ld, xdt, s);
    return sk_launch_ld<BITS, 4>(a, S, ld, xdt, s);
}

// Row tiles per workgroup of the one-launch path: the fewest that keep the
// grid within one workgroup per CU; 0 when the path does not serve.  It
// serves 16-bit activations and enough 16-row tiles to fill 3/4 of the
// CUs, at most 4 per CU, at M <= 16 x the tiles per workgroup: a workgroup
// reads all M x K activations once from L2 (its waves split K) for all of
// its tiles, so fewer tiles per workgroup mean more activation bytes per
// weight byte, and past 16 M per tile the split-K kernel, which stages
// them once per split, is faster (4096 x 4096 at M = 64: 19.5 against 22.2
// us; 4096 x 14336: 53.6 against 67.7; 14336 x 4096 with four tiles per
// workgroup: 40.0 against 52.7 for split-K).  8-bit indices up to M = 64
// with fp16 activations or on the bf16 path (groups of a multiple of 64
// values), else up to M = 32; 4-bit indices up to M = 8.
int sk1_mt(int64_t M) { return M <= 16 ? 1 : (M <= 32 ? 2 : 4); }
bool sk1_hl(int bits, const ActDesc &x, int group) { return bits == 8 && x.dtype == EP_BF16 && group % 64 == 0; }
int sk1_tiles_per_wg(int bits, const ActDesc &x, int64_t M, int64_t N, int group)
{
    if (x.dtype == EP_F32)
        return 0;
    const bool wide = bits == 8 && (x.dtype == EP_F16 || sk1_hl(bits, x, group));
    if (M > (wide ? 64 : (bits == 8 ? 32 : 8)))
        return 0;
    const int64_t tiles = (N + 15) / 16, cus = device_cus();
    if (tiles * 4 < cus * 3)
        return 0;
    for (int t = 1; t <= 4; t *= 2)
        if (tiles <= t * cus)
            return M > 16 * t ? 0 : t;
    return 0;
}

// 16 waves with 8-bit indices, one 16-row activation block and one tile
// (four per SIMD hide the table lookups' latency), 8 otherwise (4-bit B
// operands and activations, more activation blocks, or the two or four
// tiles' weights at two pieces per round take the registers of two
// waves); two pieces per round (128 contiguous bytes of each row, whole
// 128-byte lines) for 8-bit indices and one activation block.  With one
// piece (64 bytes of a row per round) each line is read by two rounds:
// 8192 x 4096 at M = 4, two tiles on 16 waves, 17.3 -> 15.4 us on 8 waves
// with two pieces; 14336 x 4096 at M = 4, four tiles, 28.2 -> 27.2 us.
template <int BITS, int XDT, int T, int MT, bool HL>
void sk1_launch_t(const SkArgs &a, hipStream_t s)
{
    constexpr int NT = BITS == 8 && MT == 1 && T < 2 ? 1024 : 512;
    constexpr int P = BITS == 8 && MT == 1 ? 2 : 1;
    hipLaunchKernelGGL((sk1_kernel<BITS, XDT, T, 2, P, MT, NT, HL>), dim3((unsigned)a.gtiles), dim3(NT), 0, s, a);
}

template <int BITS, int XDT, int MT, bool HL>
void sk1_launch_m(const SkArgs &a, int tpw, hipStream_t s)
{
    if (tpw == 1)
        sk1_launch_t<BITS, XDT, 1, MT, HL>(a, s);
    else if (tpw == 2)
        sk1_launch_t<BITS, XDT, 2, MT, HL>(a, s);
    else
        sk1_launch_t<BITS, XDT, 4, MT, HL>(a, s);
}

template <int BITS, int XDT, bool HL>
void sk1_launch_x(const SkArgs &a, int tpw, hipStream_t s)
{
    const int mt = BITS == 4 ? 1 : sk1_mt(a.M);
    if (mt == 1)
        sk1_launch_m<BITS, XDT, 1, HL>(a, tpw, s);
    else if constexpr (BITS == 8) {
        if (mt == 2)
            sk1_launch_m<BITS, XDT, 2, HL>(a, tpw, s);
        else if constexpr (XDT == EP_F16 || HL)  // four blocks: fp16 or the bf16 path only
            sk1_launch_m<BITS, XDT, 4, HL>(a, tpw, s);
    }
}

// The register-resident split-K kernel: MB = ceil(M / 16) activation
// blocks, NC 64-value pieces per wave (the activations take 8 MB NC
// registers: 128 at most), loads D tiles ahead (one where the pieces are
// eight).  It serves 8-bit indices at 17 <= M <= 64 with fp16 activations,
// or bf16 ones with groups of a multiple of 64 values, at M > 32 and on
// layers of at least 2^25 weights: each workgroup takes its 64 x 8 R
// activations once and then costs ~2.7 us per tile on the bf16 path, so it
// pays where a workgroup streams several tiles or M is large (bf16 x,
// 4096 x 14336 at M = 64 / 48 / 32 / 17: 52.9 / 48.6 / 40.2 / 38.7 -> 36.2 /
// 31.3 / 29.5 / 30.8 us; 14336 x 4096: 42.5 / 40.3 / 34.0 / 32.0 -> 35.3 /
// 29.5 / 27.6 / 27.5; 4096 x 4096 at M = 64 / 48: 18.9 / 17.7 -> 17.2 /
// 16.0) and not at 4096 x 4096 below M = 33 (M = 17: 13.2 against 13.9).
int sk2_mb(int64_t M) { return (int)((M + 15) / 16); }
int sk2_split_k(int64_t M) { return kSkWaves * 64 * (sk2_mb(M) <= 2 ? 8 : 4); }
int sk2_splits(int64_t M, int64_t K) { return (int)((K + sk2_split_k(M) - 1) / sk2_split_k(M)); }
bool sk2_serves(int bits, const ActDesc &x, int64_t M, int64_t N, int64_t K, int group)
{
    return bits == 8 && M > 16 && M <= 64 && (M > 32 || N * K >= ((int64_t)1 << 25)) &&
           (x.dtype == EP_F16 || (x.dtype == EP_BF16 && group % 64 == 0));
}

template <int MB, bool HL>
void sk2_launch_m(const SkArgs &a, int S, hipStream_t s)
{
    constexpr int NC = MB <= 2 ? 8 : 4;
    constexpr int D = NC == 8 ? 1 : 2;
    const dim3 grid((unsigned)(a.gtiles * S));  // (split, tile group) pairs
    if (HL && a.group % 128 == 0)  // one scale per pair of 64-value pieces
        hipLaunchKernelGGL((sk2_kernel<MB, NC, D, HL, HL>), grid, dim3(kSkThreads), 0, s, a);
    else
        hipLaunchKernelGGL((sk2_kernel<MB, NC, D, HL, false>), grid, dim3(kSkThreads), 0, s, a);
}

template <bool HL>
void sk2_launch(const SkArgs &a, int S, hipStream_t s)
{
    const int mb = sk2_mb(a.M);
    if (mb == 2)
        sk2_launch_m<2, HL>(a, S, s);
    else if (mb == 3)
        sk2_launch_m<3, HL>(a, S, s);
    else
        sk2_launch_m<4, HL>(a, S, s);
}

}  // namespace

bool skinny_serves(const PackedDesc &w, const ActDesc &x, int64_t M)
{
    const int bits = w.bits();
    const int kpl = bits == 4 ? sk_kpl<4>() : sk_kpl<8>();
    if (M < 2 || M > 64 || w.N < 1 || w.K < kpl || w.K % kpl != 0 || w.group % kpl != 0)
        return false;
    if (w.scale_dtype != EP_F16)
        return false;  // fp16 group scales (the container's); f32 after make_trainable goes to the tiles
    // every buffer extent fits the 32-bit offsets of the buffer loads, below
    // the offset that masked lanes use
    const int esz = x.dtype == EP_F32 ? 4 : 2;
    const int64_t rb = bits == 4 ? w.K / 2 : w.K;
    const int64_t G = (w.K + w.group - 1) / w.group;
    if (w.N * rb > kOut || ((M - 1) * x.ld + w.K) * esz > kOut || ((w.N - 1) * w.ld_scale + G) * 2 > kOut)
        return false;
    if (((uintptr_t)w.packed & 15) != 0 || ((uintptr_t)x.ptr & 15) != 0)
        return false;
    return (x.ld * esz) % 16 == 0;
}

size_t skinny_workspace(int64_t M, int64_t N, int64_t K, int levels)
{
    // partial sums of every split (also with one split when accumulating);
    // the register-resident kernel's longer splits need no more
    const int bits = levels <= 16 ? 4 : 8;
    const int S = std::max(sk_splits(bits, M, N, K), M > 16 && M <= 64 ? sk2_splits(M, K) : 1);
    return (size_t)S * (size_t)M * (size_t)N * sizeof(float);
}

int launch_skinny(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y, void *ws,
                  size_t ws_bytes, hipStream_t stream)
{
    if (!skinny_serves(w, x, M))
        return EP_DECLINE_SHAPE;
    const int bits = w.bits();
    const bool reg = sk2_serves(bits, x, M, w.N, w.K, w.group);
    const int tpw1 = reg ? 0 : sk1_tiles_per_wg(bits, x, M, w.N, w.group);
    const int ld = sk_choose_ld(bits, M, w.N, w.K);
    const int S = reg ? sk2_splits(M, w.K) : sk_splits_ld(bits, ld, w.K);
    const bool partials = reg ? S > 1 : tpw1 == 0 && (S > 1 || y.accumulate);
    const size_t need = partials ? skinny_workspace(M, w.N, w.K, w.levels) : 0;
    if (need > 0 && (!ws || ws_bytes < need))
        return set_error(EP_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws_bytes);
    SkArgs a{};
    const int esz = x.dtype == EP_F32 ? 4 : 2;
    a.xbytes = (uint32_t)(((M - 1) * x.ld + w.K) * esz);
    a.wbytes = (uint32_t)(w.N * (bits == 4 ? w.K / 2 : w.K));
    a.sbytes = (uint32_t)(((w.N - 1) * w.ld_scale + (w.K + w.group - 1) / w.group) * 2);
    a.cbbytes = (uint32_t)(w.levels * (w.cb_dtype == EP_F32 ? 4 : 2));
    a.x = x.ptr;
    a.ldx = x.ld;
    a.M = (int)M;
    a.packed = w.packed;
    a.row_bytes = (uint32_t)(bits == 4 ? w.K / 2 : w.K);
    a.scale = w.scale;
    a.scale_dtype = w.scale_dtype;
    a.lds = w.ld_scale;
    a.cb = w.cb;
    a.cb_dtype = w.cb_dtype;
    a.levels = w.levels;
    a.N = (int)w.N;
    a.K = (int)w.K;
    a.group = w.group;
    a.y = y.ptr;
    a.y_dtype = y.dtype;
    a.ldy = y.ld;
    a.accumulate = y.accumulate;
    if (tpw1 > 0) {
        a.tiles = (int)((w.N + 15) / 16);
        a.gtiles = (a.tiles + tpw1 - 1) / tpw1;
        if (bits == 4)
            x.dtype == EP_F16 ? sk1_launch_x<4, EP_F16, false>(a, tpw1, stream)
                              : sk1_launch_x<4, EP_BF16, false>(a, tpw1, stream);
        else if (x.dtype == EP_F16)
            sk1_launch_x<8, EP_F16, false>(a, tpw1, stream);
        else if (sk1_hl(bits, x, w.group))
            sk1_launch_x<8, EP_BF16, true>(a, tpw1, stream);
        else
            sk1_launch_x<8, EP_BF16, false>(a, tpw1, stream);
        EP_HIP_CHECK(hipGetLastError());
        return EP_OK;
    }
    if (reg) {
        // one resident workgroup per CU (its LDS): S splits of gtiles
        // workgroups, each streaming every gtiles-th 16-row tile
        a.tiles = (int)((w.N + 15) / 16);
        a.gtiles = std::max(1, std::min(a.tiles, device_cus() / S));
        a.part = partials ? (float *)ws : nullptr;
        x.dtype == EP_F16 ? sk2_launch<false>(a, S, stream) : sk2_launch<true>(a, S, stream);
        EP_HIP_CHECK(hipGetLastError());
        return partials ? launch_split_reduce((const float *)ws, S, M, w.N, y, stream) : EP_OK;
    }
    a.tiles = (int)((w.N + kSkRows - 1) / kSkRows);
    // one resident workgroup per CU: enough row-tile groups that S of them
    // fill the device, at most sk_tpw tiles per workgroup
    const int cus = device_cus();
    const int tpw = 16 / ld;
    int g = (cus + S - 1) / S;
    const int gmin = (a.tiles + tpw - 1) / tpw;
    if (g < gmin)
        g = gmin;
    if (g > a.tiles)
        g = a.tiles;
    a.gtiles = g;
    a.part = partials ? (float *)ws : nullptr;
    const int rc = bits == 4 ? sk_launch_bits<4>(a, S, ld, x.dtype, stream) : sk_launch_bits<8>(a, S, ld, x.dtype, stream);
    if (rc != EP_OK || !partials)
        return rc;
    return launch_split_reduce((const float *)ws, S, M, w.N, y, stream);
}

int launch_split_reduce(const float *part, int S, int64_t M, int64_t N, const OutDesc &y, hipStream_t stream)
{
    const int64_t total = M * N;
    if (N % 4 == 0)
        hipLaunchKernelGGL(sk_reduce_kernel<true>, dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0,
                           stream, part, S, (int)M, (int)N, y.ptr, y.dtype, y.ld, y.accumulate);
    else
        hipLaunchKernelGGL(sk_reduce_kernel<false>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           stream, part, S, (int)M, (int)N, y.ptr, y.dtype, y.ld, y.accumulate);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

}  // namespace ep
