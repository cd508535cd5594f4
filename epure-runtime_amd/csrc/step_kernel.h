// Persistent batch-1 decode step for gfx950: one launch runs every layer of
// a decoder step (the caller side of the packed linears; the reference runs
// it through transformers with each q/k/v/o/gate/up/down a PackedLinear,
// epure/runtime.py:92-126, :373-415, one fused-kernel call per linear,
// epure/kernels/cuda.py:88-117).
//
// Why one launch: at batch 1 a layer moves ~112 MB of packed weights
// (Llama-3-8B shape), i.e. ~14 us at 8 TB/s, while a separate launch per
// linear pays its own ramp, prologue and drain (several us each).  Here one
// workgroup per CU stays resident for the whole step; the phases of a layer
//
//     qkv GEMV (RMSNorm in the activation load) -> attention ->
//     o GEMV (+= residual) -> gate|up GEMV (RMSNorm; SwiGLU at the output) ->
//     down GEMV (+= residual)
//
// follow each other without grid barriers: every workgroup issues the loads
// of its share of the NEXT phase's packed weights (which do not depend on
// activations) and builds that phase's LDS pair tables, then waits for the
// activations it needs, so HBM keeps streaming through each dependency.
//
// Cross-workgroup data (residual, q/k/v, attention output, SwiGLU output,
// split-KV partials) is tagged: each 32-bit value is stored together with a
// 32-bit tag (launch sequence, layer, phase) in one coherent 8-byte store,
// and a consumer re-reads (coherent sc1 loads) until every tag it needs is
// current.  A phase transition is then one memory round trip -- no store
// completion wait, counter or barrier -- and no device-scope fence is used
// (on gfx950 that writes back and invalidates the XCD's whole L2).  The
// phases' data dependencies are all-to-all, so a buffer is never rewritten
// while a consumer of its previous contents is still reading.  The launch
// sequence advances when the last workgroup finishes; every wait is bounded:
// a wait that outlasts ~0.1 s marks the step failed (sync[2]) and all
// waits then give up, so the grid always drains.
//
// GEMV arithmetic is a LUT dequant-GEMV (pair table per codebook in LDS:
// one lookup per packed byte gives two fp16 weights) whose dot products run
// on the matrix cores: v_mfma_f32_4x4x4_16b_f16 with a quad of rows as B
// and the activations as A, f32 accumulation, the group scale applied per
// 32 weights, permlane/DPP row sums and fixed-order cross-wave sums
// (deterministic).  The activations are compensated: after an exact
// power-of-two factor per 32 values each activation is split into two fp16
// terms, hi = fp16(x) and lo = fp16(x - hi) (~22 significant bits
// together), the A operand's rows 0 and 1, so every table lookup feeds two
// dot products.  The codebook entries are exact fp16 values, so
// the GEMV then agrees with float32 arithmetic to f32 accumulation order,
// which keeps bf16 storage roundings downstream (KV rows, attention output)
// on the same side as a float32 reference's.
#ifndef EP_STEP_KERNEL_H
#define EP_STEP_KERNEL_H

#include "ep_common.h"
#include "ep_internal.h"
#include "gemv_core.h"

namespace ep {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = 8;
// cache policy of the weight loads: nt (streamed, read once per step)
constexpr int kAuxStream = 2;
// Hand-over vectors every workgroup reads whole (the residual, the
// attention output, the SwiGLU output) are read through the L2 of each XCD
// first, which is only safe where no stale copy can be cached there -- so
// each rotates through kRing slots per layer (a slot comes back kRing
// layers later, long evicted by then); an entry whose tag is not current
// yet is re-read coherently (sc1).
constexpr int kRing = 32;
constexpr int kSpinLimit = 1 << 16;  // polls (~0.3-2 us each) before the step fails
constexpr int kD = 128;              // head_dim served
constexpr int kChunk = 64;           // KV positions per attention item (8 waves x 8)
constexpr int kEvents = 24;          // trace events per layer (debug)

// Geometry of a GEMV phase whose rows are S 256-byte slabs long: waves per
// row group (WPR), row groups per workgroup (RG) and slabs per wave (SPW).
// All 8 waves busy where possible, at most 4 slabs (64 activation VGPRs) per
// wave.
constexpr int geo_wpr(int S)
{
    return (S % 8 == 0 && S / 8 <= 4)   ? 8
           : (S <= 4 && 8 % S == 0)     ? S
           : (S % 4 == 0 && S / 4 <= 4) ? 4
           : (S % 7 == 0 && S / 7 <= 4) ? 7
                                        : 8;
}
constexpr int geo_rg(int S) { return 8 % geo_wpr(S) == 0 ? 8 / geo_wpr(S) : 1; }
constexpr int geo_spw(int S) { return (S + geo_wpr(S) - 1) / geo_wpr(S); }
constexpr int imax(int a, int b) { return a > b ? a : b; }
// First of N2 blocks issued after block bi of a loop of N1 blocks: block k
// goes out after block floor(k N1 / N2), spreading them evenly.
template <int N2, int N1>
EP_DEV constexpr int spread_lo(int bi)
{
    return (bi * N2 + N1 - 1) / N1;
}

// A decoder shape served by the persistent step.  RQ_* = row quads per row
// group per block of each GEMV phase (blocks are pipelined, the first ones
// issued before the phase's hand-over wait); MQ_* = the most row quads a
// workgroup's share of the phase may hold (the LDS accumulator is sized by
// it; the launch checks it against the grid).
template <int H_, int HQD_, int I_, int GQ_, int RQ_QKV_, int RQ_O_, int RQ_GU_, int RQ_D_,
          int MQ_QKV_, int MQ_O_, int MQ_GU_, int MQ_D_, int NB_QKV_ = 0, int NB_O_ = 0, int NB_GU_ = 0,
          int NB_D_ = 0, int GU_EARLY_ = 0, bool GEN_ = false, bool SF32_ = false>
struct Model {
    // GEN: H, HQD and I are maxima and the launch's own shape is read from
    // the arguments (the GEMV geometry is that of the maxima); SF32: f32
    // group scales (after make_trainable) instead of fp16
    static constexpr bool GEN = GEN_, SF32 = SF32_;
    // NB_* = block buffers of each phase (0: sized for the loads in flight)
    static constexpr int NB_QKV = NB_QKV_, NB_O = NB_O_, NB_GU = NB_GU_, NB_D = NB_D_;
    static constexpr int GU_EARLY = GU_EARLY_;
    static constexpr int H = H_, HQD = HQD_, I = I_, GQ = GQ_;
    static constexpr int SH = H / 512, SO = HQD / 512, SI = I / 512;
    static constexpr int RQ_QKV = RQ_QKV_, RQ_O = RQ_O_, RQ_GU = RQ_GU_, RQ_D = RQ_D_;
    static constexpr int MQ_QKV = MQ_QKV_, MQ_O = MQ_O_, MQ_GU = MQ_GU_, MQ_D = MQ_D_;
    // Per phase the region holds: activations as fp16 pairs (K / 2 dwords),
    // their lo terms (same size), one factor per 32 values, then the
    // accumulator [8 waves][rows].
    static constexpr int phase_bytes(int K, int red) { return K * 4 + K / 32 * 4 + red; }
    // attention scratch: q [GQ][D], k, v [D], per-wave max and sum [8][GQ],
    // per-wave P.V [8][GQ][D]
    static constexpr int ATT_BYTES = (GQ * kD + 2 * kD + 2 * kWaves * GQ + kWaves * GQ * kD) * 4;
    static constexpr int REGION =
        imax(imax(imax(phase_bytes(H, kWaves * 4 * MQ_QKV * 4),
                       phase_bytes(HQD, kWaves * 4 * MQ_O * 4)),
                  imax(phase_bytes(H, kWaves * 8 * MQ_GU * 4),
                       phase_bytes(I, kWaves * 4 * MQ_D * 4))),
             ATT_BYTES);
    static constexpr int LDS = kPairTabBytes + REGION + 32 * 2 + 16 * 4 + 64 * 4;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(H % 512 == 0 && HQD % 512 == 0 && I % 512 == 0, "rows of whole slabs");
};


// Where a phase of contraction length K keeps its activations, factors and
// accumulator inside the region.
struct PhaseLds {
    uint32_t *xs, *xl;  // hi and lo terms, fp16 pairs
    float *xf, *red;
};
EP_DEV PhaseLds phase_lds(char *region, int K)
{
    PhaseLds p;
    p.xs = (uint32_t *)region;
    p.xl = (uint32_t *)(region + K * 2);
    p.xf = (float *)(region + K * 4);
    p.red = (float *)(region + K * 4 + K / 32 * 4);
    return p;
}

// ---------------------------------------------------------------- barrier
// Workgroup barrier for LDS hand-offs: waits for this wave's LDS (and
// scalar) operations only.  __syncthreads() also fences global memory, i.e.
// waits for every global load and store of the wave still in flight -- the
// weight prefetch, the tagged stores -- which nothing here orders through a
// barrier (tagged data carries its own check).
EP_DEV void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------- memory
// Global-address-space accesses.  A generic (flat) access may complete out
// of order with other vector memory operations, so the compiler waits for
// ALL loads in flight (vmcnt(0)) before using any flat load's result -- which
// would drain the weight prefetch.  Every device-memory access here is
// therefore global (address space 1) or a buffer access.
template <class T>
EP_DEV T ldg(const T *p)
{
    return *(const __attribute__((address_space(1))) T *)p;
}
template <class T>
EP_DEV void stg(T *p, T v)
{
    *(__attribute__((address_space(1))) T *)p = v;
}
EP_DEV float ldg_as_f32(const void *p, int dt, int64_t i)
{
    if (dt == EP_F32)
        return ldg((const float *)p + i);
    if (dt == EP_F16)
        return (float)f16_from_bits(ldg((const uint16_t *)p + i));
    return bf16_to_f32(ldg((const uint16_t *)p + i));
}

// 16-byte load with sc1 (coherent at agent scope: sees other XCDs' sc1 stores).
EP_DEV u32x4_t ldc16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 16);
}
EP_DEV float ldc_f32(const float *p) { return ld_agent(const_cast<float *>(p)); }

// Tagged values: value bits in the low word, tag in the high word.
constexpr int PH_QKV = 0, PH_ATT = 1, PH_PART = 2, PH_O = 3, PH_ACT = 4, PH_DOWN = 5;
EP_DEV uint32_t tag_of(uint32_t seq, int layer, int phase)
{
    return (seq << 10) | (uint32_t)(layer * 8 + phase + 1);  // never 0 (zeroed buffers)
}
EP_DEV void st_tag(uint64_t *p, uint32_t bits, uint32_t tag)
{
    st_agent(p, (uint64_t)bits | ((uint64_t)tag << 32));
}
EP_DEV uint64_t ld_tag(const uint64_t *p) { return ld_agent(const_cast<uint64_t *>(p)); }

// Bounded wait: `again` sleeps briefly and returns true while the caller
// should keep polling.  After kSpinLimit polls it marks the step failed;
// any wait also gives up once the step is marked failed.
struct Spin {
    int it = 0;
    EP_DEV bool again(int *err)
    {
        if (++it > kSpinLimit) {
            st_agent(err, 1);
            return false;
        }
        if ((it & 31) == 0 && ld_agent(err) != 0)
            return false;
        // back off after the first polls: every poll of every thread is a
        // memory-side read that competes with the producers' traffic
        if (it < 4)
            __builtin_amdgcn_s_sleep(1);
        else
            __builtin_amdgcn_s_sleep(6);  // ~400 cycles
        return true;
    }
};

// f(std::integral_constant<int, 0>{}) .. f(..<N - 1>{}) in order, expanded at
// compile time.
template <int I, int N>
struct StaticFor {
    template <class F>
    static EP_DEV void run(F &f)
    {
        if constexpr (I < N) {
            f(std::integral_constant<int, I>{});
            StaticFor<I + 1, N>::run(f);
        }
    }
};
template <int N, class F>
EP_DEV void static_for(F &&f)
{
    StaticFor<0, N>::run(f);
}

// true when `p` holds on every active lane of the wave (a wave-uniform value)
EP_DEV bool wave_all(bool p) { return __builtin_amdgcn_ballot_w64(!p) == 0; }

// threadIdx.x through an opaque move: values derived from it are recomputed
// per phase instead of being hoisted out of the layer loop and kept live
// (registers) for the whole step.
EP_DEV int tid_fresh()
{
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
// Wave index in a scalar register (buffer descriptors built from it stay
// uniform).
EP_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(tid_fresh() >> 6); }

// 64 zero bytes in LDS (written once at kernel entry): rows 2 and 3 of the
// GEMV MFMAs' A operand.
EP_DEV uint32_t *lds_zeros()
{
    __shared__ __align__(16) uint32_t z[16];
    return z;
}

// ---------------------------------------------------------------- segments
// The virtual row-quad space of one GEMV phase of a layer: up to three
// weights stacked (q|k|v), or a gate/up pair sharing quad indices.
struct Segs {
    const uint8_t *pk0, *pk1, *pk2;
    const char *sc0, *sc1, *sc2;
    const void *cb0, *cb1, *cb2;
    uint64_t *y0, *y1, *y2;  // tagged outputs (q|k|v phase)
    int q1, q2;    // first virtual quad of segments 1 and 2 (INT_MAX: absent)
    int nq;        // virtual quads
    int qa, qb;    // this workgroup's share [qa, qb)
    int sfirst;    // segment of quad qa (LDS table slot 0)
    int ntab;      // tables the share needs (1 or 2)
    int ldsb;      // scale row bytes
    int ns, rb;    // 256-byte slabs and packed bytes of a row (K / 512, K / 2)
};

template <class T>
EP_DEV T sel3(int s, T a, T b, T c)
{
    return s == 0 ? a : (s == 1 ? b : c);
}

EP_DEV void share(Segs &g, int b, int G, bool paired)
{
    g.qa = (int)((int64_t)b * g.nq / G);
    g.qb = (int)((int64_t)(b + 1) * g.nq / G);
    if (paired) {
        g.sfirst = 0;
        g.ntab = 2;
    } else {
        g.sfirst = g.qa >= g.q2 ? 2 : (g.qa >= g.q1 ? 1 : 0);
        const int nxt = g.sfirst == 0 ? g.q1 : (g.sfirst == 1 ? g.q2 : 0x7fffffff);
        g.ntab = (g.qb > g.qa && g.qb - 1 >= nxt) ? 2 : 1;
    }
}

// ---------------------------------------------------------------- layer
struct StepLayer {
    const uint8_t *packed[7];  // q, k, v, o, gate, up, down
    const void *scale[7];      // fp16 [N][K / group]
    const void *cb[7];         // [levels] f32 or fp16
    const uint16_t *attn_norm, *mlp_norm, *q_norm, *k_norm;  // bf16 (q/k norm may be null)
    float *kcache, *vcache;  // [Hkv][max_pos][D] f32
};

// A layer descriptor as the kernel reads it: through the constant address
// space, so its pointers come in by scalar loads (waited for on their own
// counter; a vector load's wait would also wait for the weight prefetch).
using LayerC = const __attribute__((address_space(4))) StepLayer;

struct StepArgs {
    const StepLayer *layers;
    int n_layers;
    float *h0;          // [H] f32: the step's input embedding; the final residual on exit
    uint64_t *ht;       // [2 kRing][H] tagged residual: o and down outputs of each layer
    uint64_t *qt, *kt, *vt;  // [Hq * D], [Hkv * D], [Hkv * D] tagged f32
    uint64_t *at;       // [kRing][Hq * D] tagged f32: attention output
    uint64_t *actt;     // [kRing][I] tagged f32: silu(gate) * up
    uint64_t *part;     // [Hq][max_pos / kChunk + 1][D + 2] tagged split-KV partials
    int *sync;          // [0] finished workgroups, [1] launch sequence, [2] error flag
    const float *cos_t, *sin_t;  // [max_pos][D / 2]
    const int *state;            // [0] position
    int Hkv, max_pos, levels, group, cb_dtype;
    float eps, qk_eps, att_scale;
    long long *trace;  // optional [layers][kEvents][grid] wall-clock stamps
    int H, HQD, I;     // the shape (read by the generic variants)
};

// ---------------------------------------------------------------- GEMV phase
constexpr int MODE_STORE = 0;   // y_seg[row] = dot * rinv
constexpr int MODE_ACC = 1;     // h[row] += dot
constexpr int MODE_SWIGLU = 2;  // act[row] = silu(gate * rinv) * (up * rinv)

// One GEMV phase.  A workgroup's share [qa, qb) of virtual row quads (at
// most MAXQ) is cut into quad groups of QPB quads; lane (wave, lane) covers
// row 4 q + (lane >> 4) of each quad q of its row group, 16 bytes (32
// weights) of each of its SPW slabs.  A block is one slab of one quad group
// (NQ loads per lane), blocks run slab-major: a wave's activation chunk of
// a slab is read once for all the share's quads, and each row's partial sum
// stays in a register until the wave's last slab.  Blocks are pipelined
// NBUF deep: blocks 0 .. NBUF - 2 are issued by the caller (before the
// hand-over wait), block i + NBUF - 1 while block i is computed.  Waves run
// their blocks independently: each row's 16-lane sum goes to an LDS
// accumulator (one slot per wave and row), and the cross-wave sums and
// outputs are formed once, after the last block.
template <int S, int RQ, bool PAIRED, int MAXQ, int NBUF_SET = 0, bool SEG3 = false, bool SF32 = false,
          bool GEN = false>
struct Gemv {
    static constexpr int WPR = geo_wpr(S), RG = geo_rg(S), SPW = geo_spw(S);
    static constexpr int NQ = PAIRED ? 2 * RQ : RQ;  // loads (row quads) per lane per block
    static constexpr int QPB = RG * RQ;              // virtual quads per quad group
    static constexpr int QB = (MAXQ + QPB - 1) / QPB;  // quad groups of the largest share
    static constexpr int MAXB = SPW * QB;              // blocks of the largest share
    static constexpr bool XREG = SPW == 1;             // one activation chunk for the phase
    static constexpr int NPAIR = PAIRED ? 2 : 1;
    static constexpr int RED_ROWS = 4 * MAXQ * NPAIR;  // accumulator slots per wave
    static constexpr int RED_BYTES = kWaves * RED_ROWS * 4;
    // fp16 scales a wave needs per block: NQ quads x 4 rows x up to 4 groups
    // per slab (group >= 128) -- one 2-byte load per lane
    static_assert(NQ * 4 * 4 <= 64, "one scale load per wave and block");
    static_assert(RG * WPR <= kWaves, "waves");
    // Block buffers: enough blocks in flight to keep ~48 KiB of a CU's loads
    // requested (more than the CU's L1 holds in flight), the whole share at
    // most; NBUF - 1 of them are issued ahead of the phase's hand-over.
    static constexpr int BLOCK_BYTES = RG * WPR * 64 * 16 * NQ;
    static constexpr int NBUF_WANT = 1 + (49152 + BLOCK_BYTES - 1) / BLOCK_BYTES;
    static constexpr int NBUF_AUTO = NBUF_WANT < 2 ? 2 : (NBUF_WANT > MAXB + 1 ? MAXB + 1 : NBUF_WANT);
    // NBUF_SET < 0: the whole share in flight (every block issued ahead)
    static constexpr int NBUF = NBUF_SET > 0 ? NBUF_SET : (NBUF_SET < 0 ? MAXB + 1 : NBUF_AUTO);

    using SBits = typename std::conditional<SF32, uint32_t, uint16_t>::type;
    struct Blk {
        u32x4_t w[NQ];
        SBits s;     // one group scale (fp16 or f32 bits) per lane, spread to
                     // the lanes that use it at compute time; converted there
                     // (a conversion right after the load would wait for
                     // every load in flight)
    };

    // group scales: fp16 (the container's) or f32 (after make_trainable)
    static constexpr int kSEsz = SF32 ? 4 : 2;
    static EP_DEV SBits load_scale(const char *p) { return ldg((const SBits *)p); }
    static EP_DEV float scale_value(uint32_t bits)
    {
        if constexpr (SF32)
            return __uint_as_float(bits);
        else
            return (float)f16_from_bits((uint16_t)bits);
    }

    // This lane's place in the phase (cheap; recomputed where needed so it
    // holds no registers across phases).
    static EP_DEV bool wave_on(int wv) { return wv / WPR < RG; }
    // slabs and packed bytes of the phase's rows: S and S x 256 for the
    // tuned variants (compile-time, so the slab tests fold away); the
    // launch's own ns (at most S; S sets the geometry) for the generic ones
    static constexpr int RB = S * kSlabBytes;
    static EP_DEV int nslabs(int ns) { return GEN ? ns : S; }
    static EP_DEV int row_bytes(const Segs &sg) { return GEN ? sg.rb : RB; }
    static EP_DEV bool slab_on(int j, int wv, int ns)
    {
        return wave_on(wv) && (wv % WPR) + j * WPR < nslabs(ns);
    }
    static EP_DEV int slab(int j, int wv, int ns) { return slab_on(j, wv, ns) ? (wv % WPR) + j * WPR : 0; }
    // byte offset of the lane's 16-byte chunk of slab j within a row: lane
    // l covers chunk l >> 2 of row l & 3 of a quad (the 4x4x4 MFMA layout)
    static EP_DEV uint32_t chunk_byte(int j, int wv, int ns)
    {
        return (uint32_t)(slab(j, wv, ns) * kSlabBytes + ((tid_fresh() & 63) >> 2) * 16);
    }

    static EP_DEV int ngroups(const Segs &sg) { return (sg.qb - sg.qa + QPB - 1) / QPB; }

    // Virtual quad of slot i of quad group qg.
    static EP_DEV int vquad(const Segs &sg, int qg, int i, int wv)
    {
        return sg.qa + qg * QPB + (wv / WPR) * RQ + (PAIRED ? (i % RQ) : i);
    }
    static EP_DEV int seg_of(const Segs &sg, int vq, int i)
    {
        if constexpr (PAIRED)
            return i >= RQ ? 1 : 0;
        else
            return vq >= sg.q2 ? 2 : (vq >= sg.q1 ? 1 : 0);
    }
    static EP_DEV int first_quad(const Segs &sg, int s)
    {
        return PAIRED ? 0 : (s == 2 ? sg.q2 : (s == 1 ? sg.q1 : 0));
    }

    // Lane constants of the block scale loads (fixed for a phase): the lane
    // loads scale entry (i * 4 + r) * G + g of a block -- quad slot i, row
    // r of the quad, group g of the block's slab (G = 4, 2, 1 groups per
    // slab for groups of 128, 256, >= 512 weights; groups are powers of two).
    struct SLane {
        int i, r, g;  // quad slot (i < NQ: live), row, group within the slab
        int lgroup;   // log2(group)
    };
    static EP_DEV int lg_gps(int lgroup) { return lgroup <= 9 ? 9 - lgroup : 0; }
    static EP_DEV SLane slane(int group)
    {
        SLane sl;
        sl.lgroup = 31 - __builtin_clz((unsigned)group);
        const int lg = lg_gps(sl.lgroup);
        int n = tid_fresh() & 63;
        sl.g = n & ((1 << lg) - 1);
        n >>= lg;
        sl.r = n & 3;
        n >>= 2;
        sl.i = n < NQ ? n : NQ;
        return sl;
    }
    // first group of slab j in a scale row
    static EP_DEV int slab_group(int j, int wv, int lgroup, int ns)
    {
        const int sl = slab(j, wv, ns);
        return lgroup <= 9 ? sl << (9 - lgroup) : sl >> (lgroup - 9);
    }

    // Issues the packed-weight loads of block bi (non-temporal: every weight
    // byte is read once per step) and the wave's one scale load.  Buffer
    // loads for the weights: the quad's base is a scalar offset, the lane's
    // place a 32-bit vector offset.  The loads are issued for every block
    // index, also past the share or for an idle slab: there the descriptor
    // has no records, so they return zeros without touching memory -- a load
    // issued on one path only would make the compiler's wait counts after
    // the join assume the worst, and waits on in-order counters then drain
    // the whole pipeline.  A quad past the share reads the segment's first
    // quad, weighted 0 at use.  Idle waves never call it.
    static EP_DEV void issue(Blk &bk, const Segs &sg, int bi, const SLane &sl)
    {
        const int wv = wave_id();
        const int j = bi / QB, qg = bi % QB;
        const bool live = qg < ngroups(sg) && slab_on(j, wv, sg.ns);
        const int lane = tid_fresh() & 63;
        // the lane's row (lane & 3) and 16-byte chunk (lane >> 2) within a
        // quad's slab: the vector offset; the quad and slab offsets are
        // wave-uniform (scalar offset)
        const uint32_t woff = (uint32_t)(lane & 3) * row_bytes(sg) + (uint32_t)(lane >> 2) * 16u;
        const int sbyte = slab(j, wv, sg.ns) * kSlabBytes;
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int vq = vquad(sg, qg, i, wv);
            const bool ok = live && vq < sg.qb;
            const int s = seg_of(sg, ok ? vq : sg.qa, i);
            const int quad = ok ? vq - first_quad(sg, s) : 0;
            const auto rp = buffer_rsrc(sel3(s, sg.pk0, sg.pk1, sg.pk2), live ? 0x7fffffffu : 0u);
            bk.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rp, (int)woff, quad * 4 * row_bytes(sg) + sbyte, kAuxStream);
        }
        const bool sok = sl.i < NQ;
        if constexpr (!SEG3) {
            // one segment (or gate|up by quad slot): the lane's scale row is
            // the wave's first quad of the group (uniform) plus its own
            // quad slot and row; a quad past the share reads row 0
            const int li = PAIRED ? (sl.i >= RQ ? sl.i - RQ : sl.i) : sl.i;
            const int q0 = sg.qa + qg * QPB + (wv / WPR) * RQ;
            const bool ok = sok && live && li < sg.qb - q0;
            const uint32_t off = ok ? (uint32_t)((q0 * 4 + li * 4 + sl.r) * sg.ldsb +
                                                 (slab_group(j, wv, sl.lgroup, sg.ns) + sl.g) * kSEsz)
                                    : 0u;
            const char *base = PAIRED && sok && sl.i >= RQ ? sg.sc1 : sg.sc0;
            bk.s = load_scale(base + off);
        } else {
            const int vq = vquad(sg, qg, sok ? sl.i : 0, wv);
            const bool ok = sok && live && vq < sg.qb;
            const int s = seg_of(sg, ok ? vq : sg.qa, sok ? sl.i : 0);
            const int row = ok ? (vq - first_quad(sg, s)) * 4 + sl.r : 0;
            const int gi = ok ? slab_group(j, wv, sl.lgroup, sg.ns) + sl.g : 0;
            // one scale row may belong to another segment than the lane's
            // neighbours' (q|k|v): a per-lane address, row 0 of the segment
            // where the entry is not used
            const char *sc = sel3(s, sg.sc0, sg.sc1, sg.sc2) + (int64_t)row * sg.ldsb + gi * kSEsz;
            bk.s = load_scale(sc);
        }
    }

    // Blocks 0 .. NBUF - 2 of a phase, issued ahead of its hand-over wait.
    static EP_DEV void prefetch(Blk (&bb)[NBUF], const Segs &sg, int group)
    {
        if (!wave_on(wave_id()))
            return;
        const SLane sl = slane(group);
#pragma unroll
        for (int k = 0; k + 1 < NBUF; ++k)
            issue(bb[k], sg, k, sl);
    }

    // Blocks k0 .. k1 - 1 (below NBUF - 1), issued by every wave (an idle
    // wave's loads have no records): called from inside another phase's
    // straight-line block loop, where a load issued by some waves only
    // would make the compiler's wait counts after the join assume the worst.
    static EP_DEV void prefetch_range(Blk (&bb)[NBUF], const Segs &sg, int group, int k0, int k1)
    {
        const SLane sl = slane(group);
#pragma unroll
        for (int k = 0; k + 1 < NBUF; ++k)
            if (k >= k0 && k < k1)
                issue(bb[k], sg, k, sl);
    }

    // Runs the share; outputs are tagged (`tag`).
    //
    // Each wave first stages its own slabs of the activation vector
    // (`stage_fn()`, which waits only for the producers of those slabs and
    // returns the lane's sum of squares of the source values) and starts its
    // blocks right away: no workgroup barrier between staging and compute,
    // so a wave whose slabs are ready computes while the others still wait.
    // RMSNorm phases (MODE_STORE: q|k|v, MODE_SWIGLU: gate|up) put each
    // wave's sum of squares in part8; the factor 1/rms multiplies the
    // finished dot products.  MODE_ACC adds the share's residual rows
    // (`hv()`, one per output thread, taken before the blocks) and writes
    // the sum to ht (and to h0 when `last`).
    //
    // `nx(bi)` runs after block bi (every wave, every bi < MAXB, in order;
    // bi is a constant of the unrolled loop): the next phase's loads go out
    // there, into the registers the computed blocks left.
    template <int MODE, class STG, class HV, class NX>
    static EP_DEV void run(Blk (&bb)[NBUF], const Segs &sg, int group, const uint32_t *tab,
                           const PhaseLds &pl, float *part8, float *hrow, int K, float eps, STG &&stage_fn, HV &&hv,
                           uint64_t *ht, float *h0, bool last, uint64_t *act, uint32_t tag, NX &&nx)
    {
        constexpr bool RMS = MODE != MODE_ACC;
        const int wv = wave_id();
        // Straight-line over the most blocks a share can hold, NBUF buffers
        // rotated (a register copy of a block would wait for its loads):
        // block bi + NBUF - 1 is issued into the buffer block bi - 1 left.
        // Every block's loads are issued (zero-length where not live): with
        // no loop and no conditional loads the compiler's wait before each
        // block counts exactly the younger blocks still in flight.
        // (every wave stages: an idle wave's slabs read slab 0 and convert
        // nothing; staging outside the branch below keeps the register
        // allocation of its two sides alike)
        const float ssq = stage_fn();
        if constexpr (MODE == MODE_ACC) {
            // the share's residual rows (threads below nrow: wave 0), loaded
            // with the staging, into LDS for the output threads (a register
            // held across the blocks would take one from the prefetch)
            if (tid_fresh() < (sg.qb - sg.qa) * 4)
                hrow[tid_fresh()] = hv();
        }
        if constexpr (RMS) {
            // row groups past the first stage the same slabs again
            const float sw = wave_sum(ssq);
            if ((tid_fresh() & 63) == 0)
                part8[wv] = wave_on(wv) && wv < WPR ? sw : 0.0f;
        }
        // the wave's own staging stores are ordered before its reads (LDS
        // operations of one wave execute in order; this keeps the compiler
        // from moving a read above them)
        asm volatile("" ::: "memory");
        if (wave_on(wv)) {
            const SLane sl = slane(group);
            const LaneC lc = lane_consts(sl);
            if constexpr (GEN)
                stream_live(bb, sg, sl, lc, pl.xs, pl.xl, pl.xf, tab, pl.red, nx);
            else
                stream(bb, sg, sl, lc, pl.xs, pl.xl, pl.xf, tab, pl.red, nx);
        } else {
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi)
                nx(bi);
        }
        lds_sync();
        // cross-wave sums (fixed order) and outputs, one thread per row
        const int t = tid_fresh();
        const int nrow = (sg.qb - sg.qa) * 4;
        if (t < nrow) {
            float rinv = 1.0f;
            if constexpr (RMS) {
                float q2 = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < kWaves; ++w2)
                    q2 += part8[w2];
                rinv = rsqrtf(q2 / (float)K + eps);
            }
            const int q = t / 4;
            const int gg = (q % QPB) / RQ;  // row group that computed the row
            float v = 0.0f, u = 0.0f;
#pragma unroll
            for (int wr = 0; wr < WPR; ++wr) {
                v += pl.red[(gg * WPR + wr) * RED_ROWS + t];
                if constexpr (PAIRED)
                    u += pl.red[(gg * WPR + wr) * RED_ROWS + RED_ROWS / 2 + t];
            }
            const int row = sg.qa * 4 + t;
            if constexpr (MODE == MODE_STORE) {
                const int vq = sg.qa + q;
                const int s = vq >= sg.q2 ? 2 : (vq >= sg.q1 ? 1 : 0);
                st_tag(sel3(s, sg.y0, sg.y1, sg.y2) + (row - first_quad(sg, s) * 4),
                       __float_as_uint(v * rinv), tag);
            } else if constexpr (MODE == MODE_ACC) {
                const float hn = hrow[t] + v;
                st_tag(ht + row, __float_as_uint(hn), tag);
                if (last)
                    stg(h0 + row, hn);  // the lm_head's input (read by a later launch)
            } else {
                st_tag(act + row, __float_as_uint(silu_mul(v * rinv, u * rinv)), tag);
            }
        }
        lds_sync();  // LDS (tables, accumulator) free for the next phase
    }

    // The lane's A operand for slab j: lanes 4 b + 0 and 4 b + 1 hold the hi
    // and lo fp16 terms of the slab's activation chunk b (32 values as 16
    // pairs), lanes 4 b + 2 and 4 b + 3 zeros; and the chunk's factor.
    static EP_DEV float load_x(int j, int wv, int ns, const uint32_t *xs, const uint32_t *xlo, const float *xf,
                               f16x2_t (&xa)[16])
    {
        const int ai = tid_fresh() & 3;
        const uint32_t xo = chunk_byte(j, wv, ns);  // pair index = byte index
        // lanes 4 b + 2 and 4 b + 3 read the 64 zero bytes (no per-value select)
        const uint32_t *src = ai == 0 ? xs + xo : (ai == 1 ? xlo + xo : lds_zeros());
#pragma unroll
        for (int p = 0; p < 16; p += 4) {
            const u32x4_t q4 = *(const u32x4_t *)(src + p);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                xa[p + t] = as_f16x2(q4[t]);
        }
        return xf[xo / 16];
    }

    // Lane constants of a phase's block loop, computed once per phase (a
    // per-block recomputation from the thread index is VALU work on the
    // loop's critical resource): the lane's table copy, the ds_bpermute
    // addresses of its quads' scales, and where reduce() puts its row sum.
    struct LaneC {
        uint32_t lane4;     // (lane & 31) * 4: the lane's table copy
        uint32_t sidx[NQ];  // byte address of the lane holding quad i's scale
        int rvq;            // reduce: the row's quad within a quad group (large: no write)
        int raddr;          // reduce: accumulator slot of that row for quad group 0
    };
    static EP_DEV LaneC lane_consts(const SLane &sl)
    {
        LaneC lc;
        const int lane = tid_fresh() & 63, wave = wave_id();
        const int rq = lane & 3, c = lane >> 2;
        lc.lane4 = ((uint32_t)lane & 31) << 2;
        const int lg = lg_gps(sl.lgroup);
        const int gl = (c >> (4 - lg)) & ((1 << lg) - 1);
#pragma unroll
        for (int i = 0; i < NQ; ++i)
            lc.sidx[i] = (uint32_t)((((i * 4 + rq) << lg) | gl) << 2);
        const int row = lane >> 4;
        const int i = row == 1 ? 2 : (row == 2 ? 1 : row);  // rows 0..3 hold quads 0, 2, 1, 3
        const int rv = (wave / WPR) * RQ + (PAIRED ? (i % RQ) : i);
        lc.rvq = ((lane & 15) < 4 && i < NQ) ? rv : (1 << 20);
        lc.raddr = wave * RED_ROWS + (PAIRED && i >= RQ ? RED_ROWS / 2 : 0) + rv * 4 + rq;
        return lc;
    }

    // Dot products of the share's blocks into the rows' partial sums on the
    // matrix cores: v_mfma_f32_4x4x4_16b_f16 with block b = the lane's chunk,
    // A = activations (rows hi, lo, 0, 0), B = a quad's dequantized weights
    // (columns = its 4 rows); eight MFMAs take the chunk's 32 weights.  Lane
    // 4 b + r then holds the chunk's hi and lo dot products of row r (D rows
    // 0 and 1), scaled by the row's group scale and the chunk's factor.
    //
    // Schedule: the table lookups of all the phase's blocks form one stream
    // with kLookAhead reads in flight (two new reads per MFMA), across quad
    // and block boundaries: the next block's first lookups are already out
    // while a block's last MFMAs, its reduction and the next phase's loads
    // run, so the LDS never drains between blocks.  A block's set-up (the
    // loads of block bi + NBUF - 1 into the buffer block bi - 1 left, its
    // quads' table slots and scale shuffles) runs just before its first
    // lookup address is formed.  Scheduling fences hold the order.  Blocks past the share or
    // on an idle slab are streamed too (their loads are zero-length) and
    // contribute nothing.
    static constexpr int kLookAhead = 12;  // lgkmcnt counts at most 15
    template <class NX>
    static EP_DEV void stream(Blk (&bb)[NBUF], const Segs &sg, const SLane &sl, const LaneC &lc,
                              const uint32_t *xs, const uint32_t *xlo, const float *xf, const uint32_t *tab,
                              float *red, NX &nx)
    {
        const int wv = wave_id();
        const int ng = ngroups(sg);
        constexpr int NL = 16 * NQ;    // lookups per block
        constexpr int T = MAXB * NL;   // lookups of the phase
        uint32_t l4s[MAXB][NQ], sb[MAXB][NQ];
        bool qon[MAXB][NQ];
        auto start = [&](int bi) {
            if (bi + NBUF - 1 < MAXB)
                issue(bb[(bi + NBUF - 1) % NBUF], sg, bi + NBUF - 1, sl);
            const int j = bi / QB, qg = bi % QB;
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
                const int vq = vquad(sg, qg, i, wv);  // wave-uniform
                qon[bi][i] = vq < sg.qb && slab_on(j, wv, sg.ns);
                const int slot = PAIRED ? (i >= RQ ? 1 : 0) : (vq < sg.qb ? seg_of(sg, vq, i) - sg.sfirst : 0);
                l4s[bi][i] = lc.lane4 | ((uint32_t)slot << 7);
                sb[bi][i] = (uint32_t)__builtin_amdgcn_ds_bpermute((int)lc.sidx[i], (int)bb[bi % NBUF].s);
            }
        };
        // a lookup's table address (one v_perm of the weight byte), formed
        // one step ahead of its read so the read never waits on it
        auto addr = [&](int g) {
            const int bi = g / NL, m = g % NL, i = m >> 4, k = m & 15;
            return __builtin_amdgcn_perm(bb[bi % NBUF].w[i][k >> 2], l4s[bi][i], kSelByte[k & 3]);
        };
        constexpr int AHL = 2;  // addresses this many lookups ahead of the reads
        uint32_t ad[T + AHL];
        float acc[QB][NQ];
        f16x2_t xa[16];  // the slab's activations (MFMA A operand: hi, lo or 0)
        float fx = 0.0f;
        uint32_t tv[T];
        static_assert(kLookAhead + AHL <= NL, "the first window lies in block 0");
        start(0);
#pragma unroll
        for (int g = 0; g < kLookAhead + AHL; ++g)
            ad[g] = addr(g);
#pragma unroll
        for (int g = 0; g < kLookAhead; ++g)
            tv[g] = lds_read_u32(tab, ad[g]);
        f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) {
            const int j = bi / QB, qg = bi % QB;
#pragma unroll
            for (int n = 0; n < NL / 2; ++n) {
                const int g0 = kLookAhead + 2 * (bi * (NL / 2) + n);  // this step's two new lookups
                const int nb = (bi + 1) * NL;                         // the next block's first lookup
                const int ga = g0 + AHL;  // this step's two new addresses
                if (bi + 1 < MAXB && ga <= nb && nb < ga + 2)
                    start(bi + 1);
#pragma unroll
                for (int g = ga; g < ga + 2; ++g)
                    if (g < T)
                        ad[g] = addr(g);
#pragma unroll
                for (int g = g0; g < g0 + 2; ++g)
                    if (g < T)
                        tv[g] = lds_read_u32(tab, ad[g]);
                __builtin_amdgcn_sched_barrier(0);
                if (n == 0) {
                    if (qg == 0 && slab_on(j, wv, sg.ns))
                        fx = load_x(j, wv, sg.ns, xs, xlo, xf, xa);
                    if (j == 0) {
#pragma unroll
                        for (int i = 0; i < NQ; ++i)
                            acc[qg][i] = 0.0f;
                    }
                }
                const int i = n >> 3, nn = n & 7;
                const int st = bi * (NL / 2) + n;
                const f16x2_t a0 = xa[2 * nn], a1 = xa[2 * nn + 1];
                const f16x2_t b0 = as_f16x2(tv[2 * st]), b1 = as_f16x2(tv[2 * st + 1]);
                const f16x4_t av = {a0[0], a0[1], a1[0], a1[1]};
                const f16x4_t bv = {b0[0], b0[1], b1[0], b1[1]};
                d = __builtin_amdgcn_mfma_f32_4x4x4f16(av, bv, nn == 0 ? (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f} : d,
                                                       0, 0, 0);
                if (nn == 7) {
                    // a quad past the share or an idle slab adds nothing (a
                    // select: its A operand may never have been loaded)
                    const float sc = scale_value(sb[bi][i]);
                    const float upd = fmaf(d[0] + d[1], sc * fx, acc[qg][i]);
                    acc[qg][i] = qon[bi][i] ? upd : acc[qg][i];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if (j == SPW - 1 && qg < ng)
                reduce(sg, qg, lc, acc[qg], red);
            nx(bi);
        }
    }

    // The generic variants' block loop: their geometry is that of the
    // largest shape they serve, so a smaller shape leaves whole blocks past
    // its share or on idle slabs.  Those are skipped (a wave-uniform branch
    // around the block's lookups and dot products); every block's loads
    // are still issued, unconditionally, so the waits on them stay exact.
    // The table-lookup window restarts per block (it does not run ahead
    // into the next block as in stream()).
    template <class NX>
    static EP_DEV void stream_live(Blk (&bb)[NBUF], const Segs &sg, const SLane &sl, const LaneC &lc,
                                   const uint32_t *xs, const uint32_t *xlo, const float *xf, const uint32_t *tab,
                                   float *red, NX &nx)
    {
        const int wv = wave_id();
        const int ng = ngroups(sg);
        constexpr int NL = 16 * NQ;  // lookups per block
        float acc[QB][NQ];
        f16x2_t xa[16];
        float fx = 0.0f;
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) {
            const int j = bi / QB, qg = bi % QB;
            if (bi + NBUF - 1 < MAXB)
                issue(bb[(bi + NBUF - 1) % NBUF], sg, bi + NBUF - 1, sl);
            if (j == 0) {
#pragma unroll
                for (int i = 0; i < NQ; ++i)
                    acc[qg][i] = 0.0f;
            }
            if (qg < ng && slab_on(j, wv, sg.ns)) {  // wave-uniform
                uint32_t l4s[NQ], sb[NQ];
                bool qon[NQ];
#pragma unroll
                for (int i = 0; i < NQ; ++i) {
                    const int vq = vquad(sg, qg, i, wv);
                    qon[i] = vq < sg.qb;
                    const int slot = PAIRED ? (i >= RQ ? 1 : 0) : (vq < sg.qb ? seg_of(sg, vq, i) - sg.sfirst : 0);
                    l4s[i] = lc.lane4 | ((uint32_t)slot << 7);
                    sb[i] = (uint32_t)__builtin_amdgcn_ds_bpermute((int)lc.sidx[i], (int)bb[bi % NBUF].s);
                }
                if (qg == 0)
                    fx = load_x(j, wv, sg.ns, xs, xlo, xf, xa);
                auto addr = [&](int m) {
                    const int i = m >> 4, k = m & 15;
                    return __builtin_amdgcn_perm(bb[bi % NBUF].w[i][k >> 2], l4s[i], kSelByte[k & 3]);
                };
                uint32_t tv[NL];
#pragma unroll
                for (int m = 0; m < kLookAhead; ++m)
                    tv[m] = lds_read_u32(tab, addr(m));
                f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int n = 0; n < NL / 2; ++n) {
#pragma unroll
                    for (int m = kLookAhead + 2 * n; m < kLookAhead + 2 * n + 2; ++m)
                        if (m < NL)
                            tv[m] = lds_read_u32(tab, addr(m));
                    __builtin_amdgcn_sched_barrier(0);
                    const int i = n >> 3, nn = n & 7;
                    const f16x2_t a0 = xa[2 * nn], a1 = xa[2 * nn + 1];
                    const f16x2_t b0 = as_f16x2(tv[2 * n]), b1 = as_f16x2(tv[2 * n + 1]);
                    const f16x4_t av = {a0[0], a0[1], a1[0], a1[1]};
                    const f16x4_t bv = {b0[0], b0[1], b1[0], b1[1]};
                    d = __builtin_amdgcn_mfma_f32_4x4x4f16(av, bv, nn == 0 ? (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f} : d,
                                                           0, 0, 0);
                    if (nn == 7) {
                        const float sc = scale_value(sb[i]);
                        const float upd = fmaf(d[0] + d[1], sc * fx, acc[qg][i]);
                        acc[qg][i] = qon[i] ? upd : acc[qg][i];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (j == SPW - 1 && qg < ng)
                reduce(sg, qg, lc, acc[qg], red);
            nx(bi);
        }
    }

    // Each row's sum over the 16 chunks (lanes r, r + 4, .., r + 60) of quad
    // group qg into the LDS accumulator, the block's (up to) four quads
    // reduced together: v_permlane32_swap pairs quads 0|1 and 2|3 (lanes l
    // and l ^ 32 added, one quad per half), v_permlane16_swap pairs the two
    // results (lanes l and l ^ 16 added, one quad per 16-lane row: rows 0..3
    // hold quads 0, 2, 1, 3), then DPP row_ror 4 and 8 finish each row.
    static EP_DEV void reduce(const Segs &sg, int qg, const LaneC &lc, const float (&acc)[NQ], float *red)
    {
        float a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a[i] = i < NQ ? acc[i] : 0.0f;
        const auto s01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[0]), __float_as_uint(a[1]), false, false);
        const auto s23 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[2]), __float_as_uint(a[3]), false, false);
        const float u = __uint_as_float(s01[0]) + __uint_as_float(s01[1]);
        const float w = __uint_as_float(s23[0]) + __uint_as_float(s23[1]);
        const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(u), __float_as_uint(w), false, false);
        float v = __uint_as_float(t[0]) + __uint_as_float(t[1]);
        v += dpp_mov<0x124>(v);
        v += dpp_mov<0x128>(v);
        // the row's quad is qa + qg QPB + rvq; rows past the share are not written
        if (lc.rvq < sg.qb - sg.qa - qg * QPB)
            red[lc.raddr + qg * QPB * 4] = v;
    }
};

// ---------------------------------------------------------------- tables
// The 16 codebook entries of one table through the scalar cache (one
// 64-byte scalar load): the codebooks are constant during the launch, and a
// scalar load is waited for on its own counter (a vector load's wait could
// also wait for the weight prefetch issued around it).
EP_DEV float cb_pick(const void *cb, int dt, int l)
{
    float out = 0.0f;
    if (dt == EP_F32) {
        const __attribute__((address_space(4))) float *c =
            (const __attribute__((address_space(4))) float *)cb;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = c[i];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            out = l == i ? v[i] : out;
    } else {
        const __attribute__((address_space(4))) uint32_t *c =
            (const __attribute__((address_space(4))) uint32_t *)cb;
        uint32_t v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = c[i];
        uint32_t h = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            h = l == i ? (v[i / 2] >> (16 * (i & 1))) & 0xffffu : h;
        out = dt == EP_F16 ? (float)f16_from_bits((uint16_t)h) : bf16_to_f32((uint16_t)h);
    }
    return out;
}

// Thread t < 32 gets entry t & 15 of table slot t >> 4 of the phase (0 for
// entries >= levels and absent slots).  A codebook holds 16 entries
// (levels <= 16 is required).
EP_DEV float load_cb(const Segs &sg, int ntab, int levels, int cb_dtype)
{
    const int t = tid_fresh();
    const int slot = t >> 4, l = t & 15;
    const float v0 = cb_pick(sel3(sg.sfirst, sg.cb0, sg.cb1, sg.cb2), cb_dtype, l);
    float v1 = 0.0f;
    if (ntab > 1)
        v1 = cb_pick(sel3(sg.sfirst + 1, sg.cb0, sg.cb1, sg.cb2), cb_dtype, l);
    const float v = slot == 0 ? v0 : v1;
    return (t < 32 && l < levels && slot < ntab) ? v : 0.0f;
}

EP_DEV void build_tables(uint32_t *tab, uint16_t *cb16, float cbv, int ntab)
{
    if (tid_fresh() < 32)
        cb16[tid_fresh()] = f16_bits((f16_t)cbv);
    lds_sync();
    // Thread t writes dwords 4 e4 .. 4 e4 + 3, e4 = t + 512 it: entry
    // b = t / 16 + 32 it, slot (t / 8) & 1 -- so its low index is the same
    // for every it and its high index is t / 256 + 2 it: nine reads, all in
    // flight at once, then eight 16-byte writes.
    const int t = tid_fresh();
    const int slot = (t >> 3) & 1;
    if (slot < ntab) {
        const uint16_t *cb = cb16 + slot * 16;
        const uint32_t lo = cb[(t >> 4) & 15];
        uint32_t hi[8];
#pragma unroll
        for (int it = 0; it < 8; ++it)
            hi[it] = cb[(t >> 8) + 2 * it];
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const uint32_t v = lo | (hi[it] << 16);
            ((u32x4_t *)tab)[t + kThreads * it] = (u32x4_t){v, v, v, v};
        }
    }
    // the tables are complete before any wave (which stages its own slabs
    // and starts its blocks without a workgroup barrier) reads them
    lds_sync();
}

// ---------------------------------------------------------------- activations
constexpr int XS_RMS_H0 = 0;  // h0 (f32, untagged: written by an earlier launch) * norm weight
constexpr int XS_RMS = 1;     // tagged residual * norm weight (bf16); 1/rms returned
constexpr int XS_F32 = 3;     // tagged f32 (attention output, SwiGLU output)

// Stages this wave's slabs of a phase's K-vector into LDS as fp16 pairs
// with one exact power-of-two factor per 32 values (the 4 lanes of a
// 32-value chunk agree on it through a quad max), the same staging as
// gemv.hip's, split into hi and lo terms.  Slab s holds values 512 s ..
// 512 s + 511; lane l converts values 8 l .. 8 l + 7 of each of the wave's
// slabs (P::slab(j, wave) for the slabs the wave computes), one slab at a
// time, the next slab's first read (and its norm weights) issued before
// the current one is polled, so its round trip overlaps the current slab's
// wait and conversion (down phase of the 8B shapes, four slabs per wave:
// 1.129 -> 1.100 ms per Llama-3-8B step; two slabs' values in registers).
// Tagged groups whose tags are not all `tag` yet are re-read coherently,
// so a wave waits for its own slabs' producers only.  Returns the lane's
// sum of squares of the source values (RMS sources; the norm weight
// multiplies each value after it is squared).
template <class P, int XS>
EP_DEV float stage_wave(const void *x, const uint16_t *w, uint32_t tag, const PhaseLds &pl, int K, int ns, int *err)
{
    constexpr bool TAGGED = XS != XS_RMS_H0;
    constexpr bool RMS = XS == XS_RMS_H0 || XS == XS_RMS;
    constexpr int SPW = P::SPW;
    const int wv = wave_id();
    const int lane = tid_fresh() & 63;
    // exact extent: every group lies inside the vector
    const auto rs = buffer_rsrc(x, TAGGED ? (uint32_t)K * 8u : (uint32_t)K * 4u);
    u32x4_t q[2][4];
    u32x4_t wr[2];
    auto first = [&](int jj, u32x4_t (&qq)[4], u32x4_t &ww) {
        // group of 8 values (an idle slab reads slab 0: never used)
        const uint32_t e = (uint32_t)(P::slab(jj, wv, ns) * 64 + lane);
        if constexpr (TAGGED) {
#pragma unroll
            for (int h = 0; h < 4; ++h)  // a ring slot: first through the caches
                qq[h] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(e * 64 + 16 * h), 0, 0);
        } else {
            qq[0] = ldc16(rs, e * 32);
            qq[1] = ldc16(rs, e * 32 + 16);
        }
        if constexpr (RMS)
            ww = ldg((const u32x4_t *)(w + e * 8));
    };
    auto ready = [&](const u32x4_t (&g)[4]) {
        bool ok = true;
#pragma unroll
        for (int h = 0; h < 4; ++h)
            ok = ok && g[h][1] == tag && g[h][3] == tag;
        return ok;
    };
    first(0, q[0], wr[0]);
    float ssq = 0.0f;
    static_for<SPW>([&](auto jc) {
        constexpr int J = decltype(jc)::value;
        constexpr int B = J & 1;
        if constexpr (J + 1 < SPW)
            first(J + 1, q[B ^ 1], wr[B ^ 1]);
        if (!P::slab_on(J, wv, ns))  // wave-uniform
            return;
        const uint32_t e = (uint32_t)(P::slab(J, wv, ns) * 64 + lane);
        if constexpr (TAGGED) {
            Spin sp;
            while (!ready(q[B]) && sp.again(err)) {
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    q[B][h] = ldc16(rs, e * 64 + 16 * h);
            }
        }
        float v[8];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            if constexpr (TAGGED) {
                v[2 * h] = __uint_as_float(q[B][h][0]);
                v[2 * h + 1] = __uint_as_float(q[B][h][2]);
            } else {
                v[h] = __uint_as_float(q[B][0][h]);
                v[4 + h] = __uint_as_float(q[B][1][h]);
            }
        }
        if constexpr (RMS) {
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                float w0, w1;
                unpack_pair<EP_BF16>(wr[B][h], w0, w1);
                ssq = fmaf(v[2 * h], v[2 * h], fmaf(v[2 * h + 1], v[2 * h + 1], ssq));
                v[2 * h] *= w0;
                v[2 * h + 1] *= w1;
            }
        }
        float am = 0.0f;
#pragma unroll
        for (int h = 0; h < 8; ++h)
            am = fmaxf(am, fabsf(v[h]));
        am = fmaxf(am, dpp_mov<0xb1>(am));  // lanes ^ 1
        am = fmaxf(am, dpp_mov<0x4e>(am));  // lanes ^ 2
        const int ex = row_exponent(am);
        const float pw = ldexpf(1.0f, -ex);
        u32x4_t q4, l4;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float a0 = v[2 * p] * pw, a1 = v[2 * p + 1] * pw;
            const f16_t h0 = (f16_t)a0, h1 = (f16_t)a1;
            q4[p] = (uint32_t)f16_bits(h0) | ((uint32_t)f16_bits(h1) << 16);
            l4[p] = (uint32_t)f16_bits((f16_t)(a0 - (float)h0)) |
                    ((uint32_t)f16_bits((f16_t)(a1 - (float)h1)) << 16);
        }
        *(u32x4_t *)(pl.xs + e * 4) = q4;
        *(u32x4_t *)(pl.xl + e * 4) = l4;
        if ((e & 3) == 0)
            pl.xf[e >> 2] = ldexpf(1.0f, ex);
    });
    return ssq;
}

// ---------------------------------------------------------------- attention
EP_DEV void stamp(const StepArgs &a, int l, int ev, int thread = 0)
{
    if (a.trace && tid_fresh() == thread)
        a.trace[((int64_t)l * kEvents + ev) * gridDim.x + blockIdx.x] = (long long)wall_clock64();
}

// Item (kv head j, chunk c) covers positions [c * 64, c * 64 + 64) ∩
// [0, pos] for the GQ query heads of group j (short chunks spread the KV
// reads over many CUs: one CU streams only a few tens of GB/s).  Wave w
// owns the chunk's positions 8 w .. 8 w + 7; lane (r = lane >> 4,
// e = lane & 15) holds dims 8 e .. 8 e + 7 of rows 8 w + 4 k + r (k = 0, 1),
// as two 16-byte halves, so each pair of K or V load instructions reads
// four whole f32 rows (2 KB, contiguous).  Row pos is this step's k/v (from
// LDS), rows past pos are weighted 0.
constexpr int kRowsPerWave = kChunk / kWaves;  // 8
constexpr int kLoadsPerWave = kRowsPerWave / 4;  // 2
struct AttnRegs {
    f32x4_t k[kLoadsPerWave][2];  // K rows (f32), dims 8 e .. 8 e + 3 and 8 e + 4 .. 8 e + 7
    f32x4_t v[kLoadsPerWave][2];  // V rows (f32)
};

// K/V rows of item (j, c); a wave whose positions all lie past pos gets a
// zero-length descriptor (its loads return 0 and touch no memory).  The
// wave's rows pw0 .. pw0 + 7 exist when pw0 <= pos: pw0 is a multiple of 8,
// max_pos of 64.
EP_DEV f32x4_t ld_f4(__amdgpu_buffer_rsrc_t r, uint32_t off, int soff)
{
    const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, soff, 0);
    return (f32x4_t){__uint_as_float(q[0]), __uint_as_float(q[1]), __uint_as_float(q[2]),
                     __uint_as_float(q[3])};
}

EP_DEV void attn_load(AttnRegs &r, const float *kc, const float *vc, int j, int c, int pos,
                      int max_pos)
{
    const int lane = tid_fresh() & 63, wave = wave_id();
    const int pw0 = c * kChunk + wave * kRowsPerWave;
    const uint32_t bytes = pw0 <= pos ? kRowsPerWave * kD * 4u : 0u;
    const int64_t row0 = pw0 <= pos ? (int64_t)j * max_pos + pw0 : 0;
    const auto rk = buffer_rsrc(kc + row0 * kD, bytes);
    const auto rv = buffer_rsrc(vc + row0 * kD, bytes);
    const uint32_t off = (uint32_t)lane * 32;  // row lane >> 4, dims 8 (lane & 15)
#pragma unroll
    for (int k = 0; k < kLoadsPerWave; ++k)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            r.k[k][h] = ld_f4(rk, off + 16 * h, k * 4 * kD * 4);
#pragma unroll
    for (int k = 0; k < kLoadsPerWave; ++k)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            r.v[k][h] = ld_f4(rv, off + 16 * h, k * 4 * kD * 4);
}

// `done` runs once the item's partial or output is stored.
template <int GQ, class F>
EP_DEV void attn_item(const StepArgs &a, LayerC &L, int l, uint32_t seq, int j, int c,
                      int nchunk, int pos, char *scratch, uint64_t *at, const AttnRegs &r, F done)
{
    const int tid = tid_fresh(), lane = tid & 63, wave = wave_id();
    const int rr = lane >> 4, e16 = lane & 15;
    float *qs = (float *)scratch;        // [GQ][D]
    float *kn = qs + GQ * kD;            // [D]
    float *vn = kn + kD;                 // [D]
    float *mw = vn + kD;                 // [8][GQ] each wave's max score
    float *lw = mw + kWaves * GQ;        // [8][GQ] each wave's sum of exp(score - max)
    float *ow = lw + kWaves * GQ;        // [8][GQ][D] each wave's P.V (16-byte aligned)
    const int hq0 = j * GQ;
    int *err = a.sync + 2;


    // this step's q (GQ heads), k and v rows: per-head RMSNorm (Qwen3) and
    // rotate-half RoPE on q and k.  Lane l holds dims l and l + 64, the pair
    // RoPE rotates together.
    if (wave < GQ + 2) {
        const uint64_t *src = wave < GQ ? a.qt + (hq0 + wave) * kD
                                        : (wave == GQ ? a.kt + j * kD : a.vt + j * kD);
        const uint32_t tq = tag_of(seq, l, PH_QKV);
        uint64_t v0, v1;
        Spin sp;
        do {
            v0 = ld_tag(src + lane);
            v1 = ld_tag(src + lane + 64);
        } while (((uint32_t)(v0 >> 32) != tq || (uint32_t)(v1 >> 32) != tq) && sp.again(err));
        float x0 = __uint_as_float((uint32_t)v0), x1 = __uint_as_float((uint32_t)v1);
        if (wave <= GQ) {
            const uint16_t *nw = wave < GQ ? L.q_norm : L.k_norm;
            if (nw) {
                const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
                const float rn = rsqrtf(ss / (float)kD + a.qk_eps);
                x0 = x0 * rn * bf16_to_f32(ldg(nw + lane));
                x1 = x1 * rn * bf16_to_f32(ldg(nw + lane + 64));
            }
            const float cs = ldg(a.cos_t + (int64_t)pos * (kD / 2) + lane);
            const float sn = ldg(a.sin_t + (int64_t)pos * (kD / 2) + lane);
            float *dst = wave < GQ ? qs + wave * kD : kn;
            dst[lane] = x0 * cs - x1 * sn;
            dst[lane + 64] = x1 * cs + x0 * sn;
        } else {
            vn[lane] = x0;
            vn[lane + 64] = x1;
        }
    }
    lds_sync();
    stamp(a, l, 10);  // q/k/v received
    if (c == nchunk - 1 && tid < kD) {  // append this step's row (read by later steps only)
        const int64_t row = ((int64_t)j * a.max_pos + pos) * kD + tid;
        stg(L.kcache + row, kn[tid]);
        stg(L.vcache + row, vn[tid]);
    }

    // Each wave runs its 8 positions alone (online softmax): scores (8 dims
    // per lane, summed over the row's 16 lanes), the wave's max and sum of
    // exponentials over its rows (lanes l, l ^ 16, l ^ 32), its P.V, and one
    // LDS hand-off of (max, sum, P.V) per wave; the 8 waves are then
    // combined, rescaled to the item's max.
    const int pw0 = c * kChunk + wave * kRowsPerWave;
    const bool wave_live = pw0 <= pos;  // wave-uniform; then row pw0 is live
    float o[GQ][8];
#pragma unroll
    for (int g = 0; g < GQ; ++g)
#pragma unroll
        for (int t = 0; t < 8; ++t)
            o[g][t] = 0.0f;
    float osum[2 * GQ];  // the wave's P.V sums this lane stores (reduce-scattered)
#pragma unroll
    for (int m = 0; m < 2 * GQ; ++m)
        osum[m] = 0.0f;
    float mwv[GQ], lwv[GQ];
    if (wave_live) {
        float qv[GQ][8];
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            const f32x4_t a0 = *(const f32x4_t *)(qs + g * kD + e16 * 8);
            const f32x4_t a1 = *(const f32x4_t *)(qs + g * kD + e16 * 8 + 4);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                qv[g][t] = a0[t];
                qv[g][4 + t] = a1[t];
            }
        }
        // this step's k and v rows (the lane's 8 dims), read by every lane
        // and selected per row below (a read under the per-lane condition
        // would branch per value)
        float knl[8], vnl[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const f32x4_t k4 = *(const f32x4_t *)(kn + e16 * 8 + 4 * h);
            const f32x4_t v4 = *(const f32x4_t *)(vn + e16 * 8 + 4 * h);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                knl[4 * h + t] = k4[t];
                vnl[4 * h + t] = v4[t];
            }
        }
        float sc[GQ][kLoadsPerWave];
#pragma unroll
        for (int k = 0; k < kLoadsPerWave; ++k) {
            const int p = pw0 + 4 * k + rr;
            float kw[8];
#pragma unroll
            for (int t = 0; t < 8; ++t)  // row pos: this step's key
                kw[t] = p == pos ? knl[t] : r.k[k][t >> 2][t & 3];
#pragma unroll
            for (int g = 0; g < GQ; ++g) {
                float acc = 0.0f;
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    acc = fmaf(qv[g][t], kw[t], acc);
                const float sg = row16_sum(acc);
                sc[g][k] = p <= pos ? sg * a.att_scale : -INFINITY;
            }
        }
        float pe[GQ][kLoadsPerWave];
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            float m = sc[g][0];
#pragma unroll
            for (int k = 1; k < kLoadsPerWave; ++k)
                m = fmaxf(m, sc[g][k]);
            m = xor32_max(xor16_max(m));  // finite: row pw0 is live
            float ls = 0.0f;
#pragma unroll
            for (int k = 0; k < kLoadsPerWave; ++k) {
                pe[g][k] = sc[g][k] == -INFINITY ? 0.0f : __expf(sc[g][k] - m);
                ls += pe[g][k];
            }
            mwv[g] = m;
            lwv[g] = xor32_sum(xor16_sum(ls));
        }
#pragma unroll
        for (int k = 0; k < kLoadsPerWave; ++k) {
            const int p = pw0 + 4 * k + rr;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float vv = p == pos ? vnl[t] : (p < pos ? r.v[k][t >> 2][t & 3] : 0.0f);
#pragma unroll
                for (int g = 0; g < GQ; ++g)
                    o[g][t] = fmaf(pe[g][k], vv, o[g][t]);
            }
        }
        // the row sums (lanes l, l ^ 16, l ^ 32, l ^ 48) of the 8 GQ values,
        // reduce-scattered: permlane32 pairs values 2m, 2m + 1 (one per lane
        // half), permlane16 pairs those (one per 16-lane row); lane (row R,
        // e16) then holds value 4 m + q(R), q = 0, 2, 1, 3 for R = 0..3
        constexpr int NV = 8 * GQ;
        float u[NV / 2];
#pragma unroll
        for (int m = 0; m < NV / 2; ++m) {
            const int i0 = 2 * m, i1 = 2 * m + 1;
            const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(o[i0 / 8][i0 % 8]),
                                                            __float_as_uint(o[i1 / 8][i1 % 8]), false, false);
            u[m] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
        }
#pragma unroll
        for (int m = 0; m < NV / 4; ++m) {
            const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(u[2 * m]), __float_as_uint(u[2 * m + 1]),
                                                            false, false);
            osum[m] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
        }
    } else {
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            mwv[g] = -INFINITY;
            lwv[g] = 0.0f;
        }
    }
    stamp(a, l, 16);  // the wave's scores, softmax and P.V
    {
        const int q = 2 * (rr & 1) + (rr >> 1);  // the values this lane's row holds
#pragma unroll
        for (int m = 0; m < 2 * GQ; ++m) {
            const int g = m >> 1, t = 4 * (m & 1) + q;
            ow[(wave * GQ + g) * kD + e16 * 8 + t] = osum[m];
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            mw[wave * GQ + g] = mwv[g];
            lw[wave * GQ + g] = lwv[g];
        }
    }
    lds_sync();
    stamp(a, l, 11);  // scores, softmax, P.V done
    // the 8 waves rescaled to the item's max; thread (g, dims 2dd, 2dd + 1)
    const bool cth = tid < GQ * 64;
    const int g = tid / 64, dd = 2 * (tid % 64);
    float M = 0.0f, Ls = 0.0f, n0 = 0.0f, n1 = 0.0f;
    if (cth) {
        M = mw[g];  // wave 0 always holds a live row
#pragma unroll
        for (int w = 1; w < kWaves; ++w)
            M = fmaxf(M, mw[w * GQ + g]);
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mwg = mw[w * GQ + g];
            const float f = mwg == -INFINITY ? 0.0f : __expf(mwg - M);
            Ls = fmaf(lw[w * GQ + g], f, Ls);
            n0 = fmaf(ow[(w * GQ + g) * kD + dd], f, n0);
            n1 = fmaf(ow[(w * GQ + g) * kD + dd + 1], f, n1);
        }
    }
    uint64_t *outp = at + (hq0 + g) * kD + dd;
    const uint32_t tatt = tag_of(seq, l, PH_ATT), tpart = tag_of(seq, l, PH_PART);
    const int maxch = a.max_pos / kChunk + 1;
    if (nchunk > 1 && c > 0) {
        // publish the partial; chunk 0 of this kv head combines
        if (cth) {
            uint64_t *pp = a.part + ((int64_t)(hq0 + g) * maxch + c) * (kD + 2);
            st_tag(pp + 2 + dd, __float_as_uint(n0), tpart);
            st_tag(pp + 3 + dd, __float_as_uint(n1), tpart);
            if (dd == 0) {
                st_tag(pp, __float_as_uint(M), tpart);
                st_tag(pp + 1, __float_as_uint(Ls), tpart);
            }
        }
        done();
        return;
    }
    if (cth) {
        // running combine in chunk order over the partials of up to kCombine
        // chunks at once: per chunk two coherent 16-byte loads, (max, sum)
        // and the thread's two values.  Two polls are in flight, the next
        // one issued before the current one is checked, so a partial is
        // seen about one round trip after it lands rather than up to two.
        constexpr int kCombine = 6;
        const auto rp = buffer_rsrc(a.part + (int64_t)(hq0 + g) * maxch * (kD + 2),
                                    (uint32_t)maxch * (kD + 2) * 8u);
        using Poll = u32x4_t[2 * kCombine];
        auto fetch = [&](Poll &e, int c0) {
#pragma unroll
            for (int k = 0; k < kCombine; ++k) {
                const uint32_t off = (uint32_t)(c0 + k < nchunk ? c0 + k : c0) * (kD + 2) * 8u;
                e[2 * k] = ldc16(rp, off);
                e[2 * k + 1] = ldc16(rp, off + (uint32_t)(2 + dd) * 8u);
            }
        };
        auto ready = [&](const Poll &e, int c0) {
            bool ok = true;
#pragma unroll
            for (int k = 0; k < 2 * kCombine; ++k)
                ok = ok && (c0 + k / 2 >= nchunk || (e[k][1] == tpart && e[k][3] == tpart));
            return wave_all(ok);
        };
        auto merge = [&](const Poll &e, int c0) {
#pragma unroll
            for (int k = 0; k < kCombine; ++k) {
                if (c0 + k >= nchunk)
                    break;
                const float Mc = __uint_as_float(e[2 * k][0]);
                const float Mn = fmaxf(M, Mc);
                const float fa = __expf(M - Mn), fb = __expf(Mc - Mn);
                Ls = Ls * fa + __uint_as_float(e[2 * k][2]) * fb;
                n0 = n0 * fa + __uint_as_float(e[2 * k + 1][0]) * fb;
                n1 = n1 * fa + __uint_as_float(e[2 * k + 1][2]) * fb;
                M = Mn;
            }
        };
        for (int c0 = 1; c0 < nchunk; c0 += kCombine) {
            Poll pa, pb;
            fetch(pa, c0);
            Spin sp;
            for (;;) {
                sp.again(err);
                fetch(pb, c0);
                if (ready(pa, c0)) {
                    merge(pa, c0);
                    break;
                }
                if (!sp.again(err))
                    break;
                fetch(pa, c0);
                if (ready(pb, c0)) {
                    merge(pb, c0);
                    break;
                }
            }
        }
        st_tag(outp, __float_as_uint(n0 / Ls), tatt);
        st_tag(outp + 1, __float_as_uint(n1 / Ls), tatt);
    }
    stamp(a, l, 12);  // output written (combined)
    done();
}

// ---------------------------------------------------------------- kernel
// The residual rows an accumulating phase owns (one per output thread):
// the load is issued before the phase's activation staging
// (residual_issue), so it shares the staging's round trip, and checked at
// the phase's output (residual_take).  Layer
// 0's o reads the untagged input h0, later phases the tagged residual.
EP_DEV uint64_t residual_issue(const Segs &sg, const StepArgs &a, const uint64_t *hsrc)
{
    const int t = tid_fresh();
    const int n = (sg.qb - sg.qa) * 4;
    const int row = sg.qa * 4 + (t < n ? t : 0);
    return hsrc ? ld_tag(hsrc + row) : (uint64_t)__float_as_uint(ldg(a.h0 + row));
}
EP_DEV float residual_take(uint64_t v, const Segs &sg, const StepArgs &a, const uint64_t *hsrc,
                           uint32_t tag)
{
    const int t = tid_fresh();
    if (t >= (sg.qb - sg.qa) * 4)
        return 0.0f;
    if (!hsrc)
        return __uint_as_float((uint32_t)v);
    const uint64_t *p = hsrc + sg.qa * 4 + t;
    Spin sp;
    while ((uint32_t)(v >> 32) != tag && sp.again(a.sync + 2))
        v = ld_tag(p);
    return __uint_as_float((uint32_t)v);
}


// Segment tables of the four GEMV phases of a layer (scalar loads of the
// layer descriptor; recomputed where needed).
struct Shape {
    int Nq, Nkv, H, I, ldsb_h, ldsb_o, ldsb_i, b, G;
    int nsH, rbH, nsO, rbO, nsI, rbI;  // slabs and packed row bytes for K = H, Hq * D, I
    // this workgroup's shares of the four phases, fixed for the launch and
    // computed once (a share is a 64-bit division by the grid size, ~50
    // instructions per wave): q|k|v [qa, qb) with its first segment and
    // table count, o (after the attention workgroups), gate|up, down
    int q_qa, q_qb, q_sfirst, q_ntab, o_qa, o_qb, g_qa, g_qb, d_qa, d_qb;
};

EP_DEV Segs segs_qkv(LayerC &L, const StepArgs &a, const Shape &sh)
{
    Segs s;
    s.pk0 = L.packed[0];
    s.pk1 = L.packed[1];
    s.pk2 = L.packed[2];
    s.sc0 = (const char *)L.scale[0];
    s.sc1 = (const char *)L.scale[1];
    s.sc2 = (const char *)L.scale[2];
    s.cb0 = L.cb[0];
    s.cb1 = L.cb[1];
    s.cb2 = L.cb[2];
    s.y0 = a.qt;
    s.y1 = a.kt;
    s.y2 = a.vt;
    s.q1 = sh.Nq / 4;
    s.q2 = (sh.Nq + sh.Nkv) / 4;
    s.nq = (sh.Nq + 2 * sh.Nkv) / 4;
    s.ldsb = sh.ldsb_h;
    s.ns = sh.nsH;
    s.rb = sh.rbH;
    s.qa = sh.q_qa;
    s.qb = sh.q_qb;
    s.sfirst = sh.q_sfirst;
    s.ntab = sh.q_ntab;
    return s;
}

// One weight's rows: o (li 3; the workgroups below the attention ones hold
// an empty share) or down (li 6), the shares computed once per launch.
EP_DEV Segs segs_one(LayerC &L, int li, int N, int ldsb, const Shape &sh)
{
    Segs s;
    s.pk0 = s.pk1 = s.pk2 = L.packed[li];
    s.sc0 = s.sc1 = s.sc2 = (const char *)L.scale[li];
    s.cb0 = s.cb1 = s.cb2 = L.cb[li];
    s.y0 = s.y1 = s.y2 = nullptr;
    s.q1 = s.q2 = 0x7fffffff;
    s.nq = N / 4;
    s.ldsb = ldsb;
    s.ns = li == 3 ? sh.nsO : sh.nsI;
    s.rb = li == 3 ? sh.rbO : sh.rbI;
    s.qa = li == 3 ? sh.o_qa : sh.d_qa;  // a single segment: table slot 0 only
    s.qb = li == 3 ? sh.o_qb : sh.d_qb;
    s.sfirst = 0;
    s.ntab = 1;
    return s;
}

EP_DEV Segs segs_gu(LayerC &L, const Shape &sh)
{
    Segs s;
    s.pk0 = L.packed[4];
    s.pk1 = s.pk2 = L.packed[5];
    s.sc0 = (const char *)L.scale[4];
    s.sc1 = s.sc2 = (const char *)L.scale[5];
    s.cb0 = L.cb[4];
    s.cb1 = s.cb2 = L.cb[5];
    s.y0 = s.y1 = s.y2 = nullptr;
    s.q1 = s.q2 = 0x7fffffff;
    s.nq = sh.I / 4;
    s.ldsb = sh.ldsb_h;
    s.ns = sh.nsH;
    s.rb = sh.rbH;
    s.qa = sh.g_qa;
    s.qb = sh.g_qb;
    s.sfirst = 0;
    s.ntab = 2;
    return s;
}

template <class M>
__global__ void __launch_bounds__(kThreads) decode_step_kernel(StepArgs a)
{
    __shared__ __align__(16) char smem[M::LDS];
    uint32_t *tab = (uint32_t *)smem;
    char *region = smem + kPairTabBytes;
    uint16_t *cb16 = (uint16_t *)(region + M::REGION);
    float *part8 = (float *)(cb16 + 32);
    float *hrow = part8 + 16;
    // the shape: compile-time for the tuned variants, from the arguments
    // for the generic ones (whose template values are the maxima)
    const int H = M::GEN ? a.H : M::H, HQD = M::GEN ? a.HQD : M::HQD, I = M::GEN ? a.I : M::I;
    const PhaseLds lh = phase_lds(region, H), lo = phase_lds(region, HQD), li = phase_lds(region, I);

    using PQ = Gemv<M::SH, M::RQ_QKV, false, M::MQ_QKV, M::NB_QKV, true, M::SF32, M::GEN>;
    using PO = Gemv<M::SO, M::RQ_O, false, M::MQ_O, M::NB_O, false, M::SF32, M::GEN>;
    using PG = Gemv<M::SH, M::RQ_GU, true, M::MQ_GU, M::NB_GU, false, M::SF32, M::GEN>;
    using PD = Gemv<M::SI, M::RQ_D, false, M::MQ_D, M::NB_D, false, M::SF32, M::GEN>;
    // gate|up blocks issued during the attention window; the rest go out
    // during the o phase
    constexpr int kGuEarly = M::GU_EARLY < PG::NBUF - 1 ? M::GU_EARLY : PG::NBUF - 1;
    constexpr int kGuPace = 40;  // s_sleep units (64 cycles) between paced blocks
    constexpr int kGuLate = PG::NBUF - 1 - kGuEarly;

    if (tid_fresh() < 16)
        lds_zeros()[tid_fresh()] = 0u;  // read after the first table build's barrier
    LayerC *layers = (LayerC *)a.layers;
    const int pos = ldg(a.state);
    if (pos < 0 || pos >= a.max_pos)
        return;  // uniform: past the cache, nothing to do
    const int G = gridDim.x, b = blockIdx.x;
    const uint32_t seq = (uint32_t)ld_agent(a.sync + 1);
    int *err = a.sync + 2;

    Shape sh;
    sh.Nq = HQD;
    sh.Nkv = a.Hkv * kD;
    sh.H = H;
    sh.I = I;
    constexpr int kSEsz = M::SF32 ? 4 : 2;  // bytes of a group scale
    sh.ldsb_h = (H / a.group) * kSEsz;
    sh.ldsb_o = (HQD / a.group) * kSEsz;
    sh.ldsb_i = (I / a.group) * kSEsz;
    sh.nsH = H / (2 * kSlabBytes);
    sh.rbH = H / 2;
    sh.nsO = HQD / (2 * kSlabBytes);
    sh.rbO = HQD / 2;
    sh.nsI = I / (2 * kSlabBytes);
    sh.rbI = I / 2;
    sh.b = b;
    sh.G = G;

    const int nchunk = pos / kChunk + 1;
    const int nitems = a.Hkv * nchunk;
    // workgroups that run an attention item first hold no o rows (up to
    // half the grid): the o phase then never waits for its slowest members,
    // the combining attention workgroups
    const int xo = nitems < G / 2 ? nitems : G / 2;
    {
        Segs t;
        t.q1 = sh.Nq / 4;
        t.q2 = (sh.Nq + sh.Nkv) / 4;
        t.nq = (sh.Nq + 2 * sh.Nkv) / 4;
        share(t, b, G, false);
        sh.q_qa = t.qa;
        sh.q_qb = t.qb;
        sh.q_sfirst = t.sfirst;
        sh.q_ntab = t.ntab;
        t.q1 = t.q2 = 0x7fffffff;
        t.nq = H / 4;  // o: rows H, over the workgroups from xo
        if (b < xo) {
            sh.o_qa = sh.o_qb = 0;
        } else {
            share(t, b - xo, G - xo, false);
            sh.o_qa = t.qa;
            sh.o_qb = t.qb;
        }
        t.nq = I / 4;  // gate|up
        share(t, b, G, true);
        sh.g_qa = t.qa;
        sh.g_qb = t.qb;
        t.nq = H / 4;  // down: rows H
        share(t, b, G, false);
        sh.d_qa = t.qa;
        sh.d_qb = t.qb;
    }

    typename PQ::Blk qb[PQ::NBUF];
    typename PO::Blk ob[PO::NBUF];
    typename PG::Blk gb[PG::NBUF];
    typename PD::Blk db[PD::NBUF];

    // Each phase's codebooks are loaded one phase ahead (a wait on a load
    // issued after the weight prefetch would wait for the whole prefetch).
    float cbv;
    {
        const Segs sq = segs_qkv(layers[0], a, sh);
        cbv = load_cb(sq, sq.ntab, a.levels, a.cb_dtype);
        __builtin_amdgcn_sched_barrier(0);
        PQ::prefetch(qb, sq, a.group);
        build_tables(tab, cb16, cbv, sq.ntab);
        const Segs so = segs_one(layers[0], 3, H, sh.ldsb_o, sh);
        cbv = load_cb(so, so.ntab, a.levels, a.cb_dtype);
    }

    for (int l = 0; l < a.n_layers; ++l) {
        LayerC &L = layers[l];
        // this layer's ring slots: residual after o and after down, the
        // attention output, the SwiGLU output; the previous layer's residual
        const uint32_t gl = seq * (uint32_t)a.n_layers + (uint32_t)l;
        uint64_t *h_o = a.ht + (size_t)((2 * gl) % (2 * kRing)) * H;
        uint64_t *h_d = a.ht + (size_t)((2 * gl + 1) % (2 * kRing)) * H;
        const uint64_t *h_prev = l == 0 ? nullptr : a.ht + (size_t)((2 * gl - 1) % (2 * kRing)) * H;
        uint64_t *at_l = a.at + (size_t)(gl % kRing) * HQD;
        uint64_t *actl = a.actt + (size_t)(gl % kRing) * I;
        const bool last = l + 1 == a.n_layers;
        stamp(a, l, 0);
        // ---- q|k|v (RMSNorm of the residual in the activation load)
        {
            const Segs sq = segs_qkv(L, a, sh);
            const uint32_t tprev = tag_of(seq, l - 1, PH_DOWN);
            PQ::template run<MODE_STORE>(
                qb, sq, a.group, tab, lh, part8, hrow, H, a.eps,
                [&] {
                    return l == 0 ? stage_wave<PQ, XS_RMS_H0>(a.h0, L.attn_norm, 0, lh, H, sh.nsH, err)
                                  : stage_wave<PQ, XS_RMS>(h_prev, L.attn_norm, tprev, lh, H, sh.nsH, err);
                },
                [] { return 0.0f; }, nullptr, a.h0, false, nullptr, tag_of(seq, l, PH_QKV), [](int) {});
        }
        stamp(a, l, 1);
        // Attention workgroups issue their first item's K/V rows (cached by
        // earlier steps) and wait for q|k|v at once; their o weights go out
        // once the item's result is stored (loads issued before a wait
        // would delay it: results return in order) and the o table is built
        // after the attention.  The other workgroups prefetch o and build
        // its table now.
        const Segs so = segs_one(L, 3, H, sh.ldsb_o, sh);
        if (b < nitems) {
            AttnRegs ar;
            attn_load(ar, L.kcache, L.vcache, b % a.Hkv, b / a.Hkv, pos, a.max_pos);
            stamp(a, l, 9);
            // (the first item apart: a loop-carried merge of its preloaded
            // rows with a later item's loads would wait for every load in
            // flight)
            attn_item<M::GQ>(a, L, l, seq, b % a.Hkv, b / a.Hkv, nchunk, pos, region, at_l, ar,
                             [&] { PO::prefetch(ob, so, a.group); });
            lds_sync();
            for (int it = b + G; it < nitems; it += G) {
                AttnRegs r2;
                attn_load(r2, L.kcache, L.vcache, it % a.Hkv, it / a.Hkv, pos, a.max_pos);
                attn_item<M::GQ>(a, L, l, seq, it % a.Hkv, it / a.Hkv, nchunk, pos, region, at_l, r2,
                                 [] {});
                lds_sync();
            }
            PG::prefetch_range(gb, segs_gu(L, sh), a.group, 0, kGuEarly);
            if (so.qb > so.qa)
                build_tables(tab, cb16, cbv, so.ntab);
        } else {
            PO::prefetch(ob, so, a.group);
            build_tables(tab, cb16, cbv, so.ntab);
            // the early gate|up blocks paced (~1.1 us apart): a burst of
            // every block at once fills the memory queues that the
            // attention chain's hand-overs and K/V reads go through
            {
                const Segs sgu = segs_gu(L, sh);
#pragma unroll
                for (int k = 0; k < kGuEarly; ++k) {
                    if (k > 0)
                        __builtin_amdgcn_s_sleep(kGuPace);
                    PG::prefetch_range(gb, sgu, a.group, k, k + 1);
                }
            }
            stamp(a, l, 9);
        }
        {
            const Segs sg = segs_gu(L, sh);
            cbv = load_cb(sg, sg.ntab, a.levels, a.cb_dtype);
        }
        stamp(a, l, 2);
        // ---- o (+= residual); attention workgroups below xo hold no o rows
        // and go straight on to gate|up (no wait for the attention output)
        {
            const Segs so = segs_one(L, 3, H, sh.ldsb_o, sh);
            if (so.qb > so.qa) {
                const uint64_t hraw = residual_issue(so, a, h_prev);
                const uint32_t tatt = tag_of(seq, l, PH_ATT), tprev = tag_of(seq, l - 1, PH_DOWN);
                PO::template run<MODE_ACC>(
                    ob, so, a.group, tab, lo, part8, hrow, HQD, 0.0f,
                    [&] {
                        const float r = stage_wave<PO, XS_F32>(at_l, nullptr, tatt, lo, HQD, sh.nsO, err);
                        stamp(a, l, 3);
                        return r;
                    },
                    [&] { return residual_take(hraw, so, a, h_prev, tprev); }, h_o, a.h0, false, nullptr,
                    tag_of(seq, l, PH_O), [&](int bi) {
                        const Segs sgu = segs_gu(L, sh);  // (formed where used: scalar registers)
                        PG::prefetch_range(gb, sgu, a.group, kGuEarly + spread_lo<kGuLate, PO::MAXB>(bi),
                                           kGuEarly + spread_lo<kGuLate, PO::MAXB>(bi + 1));
                    });
            } else {
                PG::prefetch_range(gb, segs_gu(L, sh), a.group, kGuEarly, PG::NBUF - 1);
            }
        }
        stamp(a, l, 4);
        {
            const Segs sg = segs_gu(L, sh);
            stamp(a, l, 13);
            stamp(a, l, 14, 448);
            build_tables(tab, cb16, cbv, sg.ntab);
            stamp(a, l, 15);
            const Segs sd = segs_one(L, 6, H, sh.ldsb_i, sh);
            cbv = load_cb(sd, sd.ntab, a.levels, a.cb_dtype);
        }
        // ---- gate|up -> silu(gate) * up
        {
            const Segs sg = segs_gu(L, sh);
            const uint32_t to = tag_of(seq, l, PH_O);
            PG::template run<MODE_SWIGLU>(
                gb, sg, a.group, tab, lh, part8, hrow, H, a.eps,
                [&] {
                    const float r = stage_wave<PG, XS_RMS>(h_o, L.mlp_norm, to, lh, H, sh.nsH, err);
                    stamp(a, l, 5);
                    return r;
                },
                [] { return 0.0f; }, nullptr, a.h0, false, actl, tag_of(seq, l, PH_ACT), [&](int bi) {
                    const Segs sd = segs_one(L, 6, H, sh.ldsb_i, sh);
                    PD::prefetch_range(db, sd, a.group, spread_lo<PD::NBUF - 1, PG::MAXB>(bi),
                                       spread_lo<PD::NBUF - 1, PG::MAXB>(bi + 1));
                });
        }
        stamp(a, l, 6);
        {
            const Segs sd = segs_one(L, 6, H, sh.ldsb_i, sh);
            build_tables(tab, cb16, cbv, sd.ntab);
            if (!last) {
                const Segs sq = segs_qkv(layers[l + 1], a, sh);
                cbv = load_cb(sq, sq.ntab, a.levels, a.cb_dtype);
            }
        }
        // ---- down (+= residual)
        {
            const Segs sd = segs_one(L, 6, H, sh.ldsb_i, sh);
            const uint64_t hraw = residual_issue(sd, a, h_o);
            const uint32_t tact = tag_of(seq, l, PH_ACT), to = tag_of(seq, l, PH_O);
            PD::template run<MODE_ACC>(
                db, sd, a.group, tab, li, part8, hrow, I, 0.0f,
                [&] {
                    const float r = stage_wave<PD, XS_F32>(actl, nullptr, tact, li, I, sh.nsI, err);
                    stamp(a, l, 7);
                    return r;
                },
                [&] { return residual_take(hraw, sd, a, h_o, to); }, h_d, a.h0, last, nullptr,
                tag_of(seq, l, PH_DOWN), [&](int bi) {
                    // the next layer's q|k|v (an empty share after the last layer)
                    Segs sqn = segs_qkv(layers[last ? l : l + 1], a, sh);
                    if (last)
                        sqn.qb = sqn.qa;
                    PQ::prefetch_range(qb, sqn, a.group, spread_lo<PQ::NBUF - 1, PD::MAXB>(bi),
                                       spread_lo<PQ::NBUF - 1, PD::MAXB>(bi + 1));
                });
        }
        stamp(a, l, 8);
        if (!last) {
            const Segs sq = segs_qkv(layers[l + 1], a, sh);
            build_tables(tab, cb16, cbv, sq.ntab);
            const Segs so = segs_one(layers[l + 1], 3, H, sh.ldsb_o, sh);
            cbv = load_cb(so, so.ntab, a.levels, a.cb_dtype);
        }
    }
    // the last workgroup to finish advances the launch sequence (every
    // workgroup has read it by then)
    __syncthreads();  // the step's stores complete before the count
    if (tid_fresh() == 0 && counter_add(a.sync, 1) == G - 1) {
        st_agent(a.sync, 0);
        st_agent(a.sync + 1, (int)(seq + 1));
    }
}

template <class M>
int launch_model(const StepArgs &a, hipStream_t stream)
{
    static int grid = 0;
    if (grid == 0) {
        int per_cu = 0;
        EP_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<M>,
                                                                  kThreads, 0));
        if (per_cu < 1)
            return set_error(EP_DECLINE_SHAPE, "decode step: kernel does not fit a CU");
        grid = device_cus();  // one resident workgroup per CU (LDS > half a CU's)
    }
    const int H = M::GEN ? a.H : M::H, HQD = M::GEN ? a.HQD : M::HQD, I = M::GEN ? a.I : M::I;
    if (H > M::H || HQD > M::HQD || I > M::I)
        return set_error(EP_DECLINE_SHAPE, "decode step: shape beyond the variant's maxima");
    // every qkv share must touch at most two of q, k, v (two LDS tables)
    const int Nkv = a.Hkv * kD;
    const int maxshare = ((HQD + 2 * Nkv) / 4 + grid - 1) / grid;
    if (maxshare >= Nkv / 4)
        return set_error(EP_DECLINE_SHAPE, "decode step: qkv share spans three weights");
    // every share must fit its LDS accumulator (and an accumulating share
    // the 64 residual slots)
    auto quads = [&](int rows) { return (rows / 4 + grid - 1) / grid; };
    const int ogrid = grid - grid / 2;  // workgroups left for o when attention takes half
    if (quads(HQD + 2 * Nkv) > M::MQ_QKV || (H / 4 + ogrid - 1) / ogrid > M::MQ_O || quads(I) > M::MQ_GU ||
        quads(H) > M::MQ_D || quads(H) * 4 > 64)
        return set_error(EP_DECLINE_SHAPE, "decode step: %d workgroups too few for the shape",
                         grid);
    hipLaunchKernelGGL(decode_step_kernel<M>, dim3(grid), dim3(kThreads), 0, stream, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

// Workspace: sync words, then the tagged buffers (8 bytes per value).
struct StepWs {
    size_t sync, ht, qt, kt, vt, at, actt, part, total;
};
StepWs step_ws(int H, int I, int Hq, int Hkv, int D, int max_pos)
{
    StepWs w;
    size_t o = 0;
    auto take = [&](size_t n) {
        const size_t at = o;
        o += (n * 8 + 255) / 256 * 256;
        return at;
    };
    w.sync = take(8);
    w.ht = take((size_t)2 * kRing * H);
    w.qt = take((size_t)Hq * D);
    w.kt = take((size_t)Hkv * D);
    w.vt = take((size_t)Hkv * D);
    w.at = take((size_t)kRing * Hq * D);
    w.actt = take((size_t)kRing * I);
    w.part = take((size_t)Hq * (max_pos / kChunk + 1) * (D + 2));
    w.total = o;
    return w;
}

// The kernel arguments of a launch (the workspace already checked).
StepArgs make_step_args(const StepDesc &d)
{
    const StepWs w = step_ws(d.H, d.I, d.Hq, d.Hkv, d.D, d.max_pos);
    char *ws = (char *)d.ws;
    StepArgs a{};
    a.layers = (const StepLayer *)d.layers;
    a.n_layers = d.n_layers;
    a.h0 = d.h;
    a.ht = (uint64_t *)(ws + w.ht);
    a.qt = (uint64_t *)(ws + w.qt);
    a.kt = (uint64_t *)(ws + w.kt);
    a.vt = (uint64_t *)(ws + w.vt);
    a.at = (uint64_t *)(ws + w.at);
    a.actt = (uint64_t *)(ws + w.actt);
    a.part = (uint64_t *)(ws + w.part);
    a.sync = (int *)(ws + w.sync);
    a.cos_t = d.cos_t;
    a.sin_t = d.sin_t;
    a.state = d.state;
    a.Hkv = d.Hkv;
    a.max_pos = d.max_pos;
    a.levels = d.levels;
    a.group = d.group;
    a.cb_dtype = d.cb_dtype;
    a.H = d.H;
    a.HQD = d.Hq * d.D;
    a.I = d.I;
    a.eps = d.eps;
    a.qk_eps = d.qk_eps;
    a.att_scale = d.att_scale;
    a.trace = d.trace;
    return a;
}

}  // namespace

// Generic variants (step_gen_*.hip): H, Hq * D <= 4096 and I <= 16384, each a
// multiple of 512, GQ = Hq / Hkv in 1..8, fp16 or f32 group scales.
constexpr int kGenH = 4096, kGenI = 16384;
int launch_decode_step_gen_a(const StepDesc &d, int gq, bool sf32, hipStream_t stream);  // GQ 1..4
int launch_decode_step_gen_b(const StepDesc &d, int gq, bool sf32, hipStream_t stream);  // GQ 5..8

}  // namespace ep

#endif  // EP_STEP_KERNEL_H
