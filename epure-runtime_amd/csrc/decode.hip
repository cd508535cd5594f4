// Decode-step kernels around the packed GEMV: attention over the KV cache
// and the bf16 lm_head with greedy selection.
//
// These are the caller side of the packed linears (the reference leaves
// them to transformers: runtime.py:389-415 loads a LlamaForCausalLM /
// Qwen3ForCausalLM whose q/k/v/o/gate/up/down are PackedLinear).  The math
// follows those modules: per-head RMSNorm on q/k (Qwen3 only), rotate-half
// RoPE, grouped-query causal softmax attention, RMSNorm before the lm_head,
// greedy argmax (lowest index on ties, as torch.argmax).
//
// Every kernel reads the decode position from device memory (state[0]), so
// one captured HIP graph replays every step unchanged.  Split-work kernels
// combine in the workgroup that arrives last on a per-item counter, which
// that workgroup resets to 0 for the next replay (no memset in the graph);
// the partials go through coherent agent-scope stores/loads rather than
// device-scope fences (which would flush the XCD's L2).
#include "ep_common.h"
#include "ep_internal.h"

namespace ep {
namespace {


constexpr int kChunk = 64;  // KV positions per attention workgroup
constexpr int kMaxD = 128;  // head_dim served


// Sum of a value held by every thread of a 256-thread workgroup.
EP_DEV float block_sum256(float v, float *scratch)
{
    v = wave_sum_bfly(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0)
        scratch[wave] = v;
    __syncthreads();
    return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

// In-place per-head RMSNorm (optional) and rotate-half RoPE of one head
// vector held in LDS (D floats), by threads 0..D-1 of the workgroup.
EP_DEV void norm_rope(float *vec, const uint16_t *nw, float eps, const float *cs, const float *sn,
                      int D, float *scratch)
{
    const int t = threadIdx.x;
    if (nw) {
        const float x = t < D ? vec[t] : 0.0f;
        const float ss = block_sum256(x * x, scratch);
        const float r = rsqrtf(ss / (float)D + eps);
        __syncthreads();
        if (t < D)
            vec[t] = x * r * bf16_to_f32(nw[t]);
    }
    __syncthreads();
    const int half = D / 2;
    float out = 0.0f;
    if (t < D) {
        const int i = t < half ? t : t - half;
        const float c = cs[i], s = sn[i];
        out = t < half ? vec[t] * c - vec[t + half] * s : vec[t] * c + vec[t - half] * s;
    }
    __syncthreads();
    if (t < D)
        vec[t] = out;
    __syncthreads();
}

struct AttnArgs {
    const float *q;        // [Hq * D] this step's query (GEMV output)
    const float *k;        // [Hkv * D] this step's key
    const float *v;        // [Hkv * D] this step's value
    const uint16_t *qn_w;  // [D] bf16 q RMSNorm weight, or null
    const uint16_t *kn_w;  // [D] bf16 k RMSNorm weight, or null
    float qk_eps;
    float *kcache;         // [Hkv][max_pos][D] f32
    float *vcache;         // [Hkv][max_pos][D] f32
    const float *cos_t;    // [max_pos][D / 2]
    const float *sin_t;
    const int *state;      // state[0] = position of this step's token
    float *part;           // [Hq][max_chunks][D + 2]
    int *counters;         // [Hq], zero between launches
    float *out;            // [Hq * D] f32
    int Hq, Hkv, D, max_pos;
    float scale;
};

// Grid (Hq, max_pos / kChunk); 256 threads.  Workgroup (h, c) attends query
// head h over positions [c * 64, c * 64 + 64) ∩ [0, pos]; the last chunk
// also holds this step's key/value, which the first query head of the
// group writes to the cache.  Other workgroups never read cache row `pos`,
// so there is no write/read race on it.  Cache rows, scores, softmax and
// the output are float32 (the precision of the reference model's float32
// forward, runtime.py:_runtime_dtype on CPU).
__global__ void __launch_bounds__(256) attention_kernel(AttnArgs a)
{
    __shared__ float qs[kMaxD], kn[kMaxD], vn[kMaxD];
    __shared__ float sc[kChunk];
    __shared__ float scratch[8];
    __shared__ float opart[16][kMaxD];
    __shared__ int s_last;

    const int h = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
    const int D = a.D, pos = a.state[0];
    if (pos < 0 || pos >= a.max_pos)  // past the cache: nothing to do
        return;
    const int nact = pos / kChunk + 1;
    if (c >= nact)
        return;
    const int group = a.Hq / a.Hkv;
    const int kvh = h / group;
    const int t0 = c * kChunk;
    const int t1 = min(t0 + kChunk, pos + 1);
    const float *cs = a.cos_t + (int64_t)pos * (D / 2);
    const float *sn = a.sin_t + (int64_t)pos * (D / 2);
    const float *kbase = a.kcache + (int64_t)kvh * a.max_pos * D;
    const float *vbase = a.vcache + (int64_t)kvh * a.max_pos * D;

    // K and V tiles go out first: they depend only on the position.
    // K: thread -> (position t/4, D/4-dim quarter t%4, 4 dims per load);
    // V: thread -> (8-dim slice t%16, positions t/16 + 16 i).  Cache row
    // `pos` is not read (this step's k/v come from the projections below).
    const int ktl = t >> 2, kq = t & 3, kdn = D / 4;
    const bool kok = t0 + ktl < t1 && t0 + ktl != pos;
    f32x4_t kr[kMaxD / 16];
#pragma unroll
    for (int i = 0; i < kMaxD / 16; ++i) {
        const int d = kq * kdn + i * 4;
        kr[i] = (kok && i * 4 < kdn) ? *(const f32x4_t *)(kbase + (int64_t)(t0 + ktl) * D + d)
                                     : (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
    }
    const int vdc = t & 15, vpg = t >> 4;
    f32x4_t vr[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tl = vpg + 16 * i;
        const bool ok = t0 + tl < t1 && t0 + tl != pos && vdc * 8 < D;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
            vr[i][hh] = ok ? *(const f32x4_t *)(vbase + (int64_t)(t0 + tl) * D + vdc * 8 + 4 * hh)
                           : (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
    }

    if (t < D)
        qs[t] = a.q[h * D + t];
    const bool has_new = (c == nact - 1);
    if (has_new && t < D) {
        kn[t] = a.k[kvh * D + t];
        vn[t] = a.v[kvh * D + t];
    }
    norm_rope(qs, a.qn_w, a.qk_eps, cs, sn, D, scratch);
    if (has_new) {
        norm_rope(kn, a.kn_w, a.qk_eps, cs, sn, D, scratch);
        if (t < D && h % group == 0) {
            const int64_t row = ((int64_t)kvh * a.max_pos + pos) * D + t;
            a.kcache[row] = kn[t];
            a.vcache[row] = vn[t];
        }
        __syncthreads();
    }

    // scores
    {
        const int tp = t0 + ktl;
        float s = 0.0f;
        if (tp < t1) {
            const int d0 = kq * kdn;
            if (tp == pos) {
                for (int d = d0; d < d0 + kdn; ++d)
                    s = fmaf(qs[d], kn[d], s);
            } else {
#pragma unroll
                for (int i = 0; i < kMaxD / 16; ++i)
                    if (i * 4 < kdn) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            s = fmaf(qs[d0 + i * 4 + e], kr[i][e], s);
                    }
            }
        }
        s += __shfl_xor(s, 1, 4);
        s += __shfl_xor(s, 2, 4);
        if (kq == 0)
            sc[ktl] = tp < t1 ? s * a.scale : -INFINITY;
    }
    __syncthreads();
    // chunk max / exp / sum (wave 0)
    if (t < 64) {
        const float s = sc[t];
        const float m = wave_max_bfly(s);
        const float p = t0 + t < t1 ? __expf(s - m) : 0.0f;
        const float l = wave_sum_bfly(p);
        sc[t] = p;
        if (t == 0) {
            scratch[4] = m;
            scratch[5] = l;
        }
    }
    __syncthreads();
    // o[d] = sum_t p[t] v[t][d] from the V registers, then a fixed-order sum
    // over the 16 position groups
    if (vdc * 8 < D) {
        float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tl = vpg + 16 * i;
            const int tp = t0 + tl;
            if (tp < t1) {
                const float p = sc[tl];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    o[e] = fmaf(p, tp == pos ? vn[vdc * 8 + e] : vr[i][e >> 2][e & 3], o[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
            opart[vpg][vdc * 8 + e] = o[e];
    }
    __syncthreads();
    if (t < D) {
        float acc = 0.0f;
        for (int g = 0; g < 16; ++g)
            acc += opart[g][t];
        opart[0][t] = acc;
    }
    __syncthreads();
    float *pp = a.part + ((int64_t)h * (a.max_pos / kChunk) + c) * (D + 2);
    if (t < D)
        st_agent(pp + 2 + t, opart[0][t]);
    if (t == 0) {
        st_agent(pp, scratch[4]);
        st_agent(pp + 1, scratch[5]);
    }
    // publish, then the last chunk to arrive combines
    wait_stores();
    __syncthreads();
    if (t == 0)
        s_last = counter_add(&a.counters[h], 1) == nact - 1;
    __syncthreads();
    if (!s_last)
        return;
    float *base = a.part + (int64_t)h * (a.max_pos / kChunk) * (D + 2);
    float M = -INFINITY;
    for (int j = 0; j < nact; ++j)
        M = fmaxf(M, ld_agent(base + (int64_t)j * (D + 2)));
    float L = 0.0f, o = 0.0f;
    for (int j = 0; j < nact; ++j) {
        float *pj = base + (int64_t)j * (D + 2);
        const float w = __expf(ld_agent(pj) - M);
        L = fmaf(ld_agent(pj + 1), w, L);
        if (t < D)
            o = fmaf(ld_agent(pj + 2 + t), w, o);
    }
    if (t < D)
        a.out[h * D + t] = o / L;
    if (t == 0)
        st_agent(&a.counters[h], 0);
}

struct HeadArgs {
    float *h;                // [H] residual (read: final norm input; written: next embedding)
    const uint16_t *norm_w;  // [H] bf16
    float eps;
    const uint16_t *W;       // [V][H] bf16 lm_head
    float *logits;           // [V] or null
    int V, H;
    float *part_val;         // [grid]
    int *part_idx;           // [grid]
    int *counter;            // [1], zero between launches
    int *state;              // [0] pos, [1] token
    const int *prompt;       // [n_prompt]
    int n_prompt;
    int *tokens;             // [max_pos + 1]: tokens[p] = token at position p
    int *argmax_out;         // [max_pos]: greedy choice after position p
    const uint16_t *embed;   // [V][H] bf16
    int max_pos;
};

constexpr int kHeadPerLane = 64;  // activations per lane: H <= 4096
// two waves per SIMD: each wave keeps two rows' loads in flight while it
// computes, so a CU holds 128 KB of requests (one wave per SIMD left the
// stream latency-bound at ~5.8 TB/s)
constexpr int kHeadWaves = 8;

template <int CTRL>
EP_DEV float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes of each DPP row, in every lane of the row.
EP_DEV float row16_sum_dpp(float v)
{
    v += dpp_f<0x128>(v);  // row_ror 8
    v += dpp_f<0x124>(v);  // row_ror 4
    v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
    return v;
}

// lm_head GEMV with the final RMSNorm fused in front and greedy selection
// behind.  The workgroup normalizes the residual once into LDS (float32: the
// reference model's float32 forward); each wave keeps its 64 values in
// registers and streams whole bf16 rows with 16-byte loads, two rows in
// flight, every product an exact f32 FMA of the widened bf16 weight; row
// sums use DPP within 16-lane rows and readlane across them.
__global__ void __launch_bounds__(64 * kHeadWaves) lm_head_kernel(HeadArgs a)
{
    __shared__ float wv[kHeadWaves];
    __shared__ int wi[kHeadWaves];
    __shared__ float ssq_s[kHeadWaves];
    __shared__ int s_last;
    __shared__ __align__(16) float xs[64 * kHeadPerLane];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.H;
    const int nld = H / 512;  // 16-byte loads per lane per row

    const int gw = blockIdx.x * kHeadWaves + wave, nw = gridDim.x * kHeadWaves;
    // first rows' loads go out before the normalization
    u32x4_t w[2][kHeadPerLane / 8];
    auto load_rows = [&](int r0) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int r = r0 + q * nw;
            const int rs = r < a.V ? r : (r0 < a.V ? r0 : 0);
#pragma unroll
            for (int i = 0; i < kHeadPerLane / 8; ++i)
                if (i < nld)
                    w[q][i] = __builtin_nontemporal_load(
                        (const u32x4_t *)(a.W + (int64_t)rs * H + (lane + 64 * i) * 8));
        }
    };
    if (gw < a.V)
        load_rows(gw);

    float ss = 0.0f;
    for (int k = threadIdx.x * 4; k < H; k += 4 * 64 * kHeadWaves) {
        const f32x4_t v = *(const f32x4_t *)(a.h + k);
        ss = fmaf(v[0], v[0], fmaf(v[1], v[1], fmaf(v[2], v[2], fmaf(v[3], v[3], ss))));
    }
    ss = wave_sum_bfly(ss);
    if (lane == 0)
        ssq_s[wave] = ss;
    __syncthreads();
    float sst = 0.0f;
#pragma unroll
    for (int w = 0; w < kHeadWaves; ++w)
        sst += ssq_s[w];
    const float rinv = rsqrtf(sst / (float)H + a.eps);
    for (int k = threadIdx.x; k < H; k += 64 * kHeadWaves)
        xs[k] = a.h[k] * rinv * bf16_to_f32(a.norm_w[k]);
    __syncthreads();
    // lane's values: dims (lane + 64 i) * 8 .. + 7 of load i
    float x[kHeadPerLane];
#pragma unroll
    for (int i = 0; i < kHeadPerLane / 8; ++i) {
        f32x4_t a0 = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
        if (i < nld) {
            a0 = *(const f32x4_t *)(xs + (lane + 64 * i) * 8);
            a1 = *(const f32x4_t *)(xs + (lane + 64 * i) * 8 + 4);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[8 * i + e] = a0[e];
            x[8 * i + 4 + e] = a1[e];
        }
    }

    float best = -INFINITY;
    int besti = 0x7fffffff;
    for (int rb = gw; rb < a.V; rb += 2 * nw) {
        float sacc[2] = {0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int i = 0; i < kHeadPerLane / 8; ++i)
                if (i < nld) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t wp = w[q][i][e];
                        sacc[q] = fmaf(__uint_as_float(wp << 16), x[8 * i + 2 * e], sacc[q]);
                        sacc[q] = fmaf(__uint_as_float(wp & 0xffff0000u), x[8 * i + 2 * e + 1],
                                       sacc[q]);
                    }
                }
        if (rb + 2 * nw < a.V)
            load_rows(rb + 2 * nw);  // next rows in flight during the reduction
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float v = row16_sum_dpp(sacc[q]);
            const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
                              __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)) +
                              __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
                              __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
            const int r = rb + q * nw;
            if (r < a.V) {
                if (a.logits && lane == 0)
                    a.logits[r] = tot;
                if (tot > best || (tot == best && r < besti)) {
                    best = tot;
                    besti = r;
                }
            }
        }
    }
    if (lane == 0) {
        wv[wave] = best;
        wi[wave] = besti;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = wv[0];
        int bi = wi[0];
        for (int w = 1; w < kHeadWaves; ++w)
            if (wv[w] > b || (wv[w] == b && wi[w] < bi)) {
                b = wv[w];
                bi = wi[w];
            }
        st_agent(a.part_val + blockIdx.x, b);
        st_agent(a.part_idx + blockIdx.x, bi);
        wait_stores();
        s_last = counter_add(a.counter, 1) == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last)
        return;
    // last workgroup: global argmax, next token, next embedding
    float b = -INFINITY;
    int bi = 0x7fffffff;
    for (int j = threadIdx.x; j < (int)gridDim.x; j += 64 * kHeadWaves) {
        const float v = ld_agent(a.part_val + j);
        const int i = ld_agent(a.part_idx + j);
        if (v > b || (v == b && i < bi)) {
            b = v;
            bi = i;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(b, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > b || (ov == b && oi < bi)) {
            b = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        wv[wave] = b;
        wi[wave] = bi;
    }
    __syncthreads();
    __shared__ int s_next;
    if (threadIdx.x == 0) {
        float bb = wv[0];
        int bbi = wi[0];
        for (int w = 1; w < kHeadWaves; ++w)
            if (wv[w] > bb || (wv[w] == bb && wi[w] < bbi)) {
                bb = wv[w];
                bbi = wi[w];
            }
        // no logit compares (all NaN): argmax -1, and token 0 feeds the next
        // step so every later access stays inside the tables
        const bool valid = bbi >= 0 && bbi < a.V;
        const int pos = a.state[0];
        const int next = pos + 1 < a.n_prompt ? a.prompt[pos + 1] : (valid ? bbi : 0);
        if (pos < a.max_pos) {
            a.argmax_out[pos] = valid ? bbi : -1;
            a.tokens[pos + 1] = next;
        }
        a.state[0] = pos + 1;
        a.state[1] = next;
        s_next = next;
        st_agent(a.counter, 0);
    }
    __syncthreads();
    const int next = s_next;
    for (int k = threadIdx.x; k < H; k += 64 * kHeadWaves)
        a.h[k] = bf16_to_f32(a.embed[(int64_t)next * H + k]);
}

// h = embed[state[1]] (the first step's input).
__global__ void __launch_bounds__(256) embed_kernel(const uint16_t *embed, const int *state,
                                                   float *h, int H)
{
    const int tok = state[1];
    for (int k = threadIdx.x; k < H; k += 256)
        h[k] = bf16_to_f32(embed[(int64_t)tok * H + k]);
}

}  // namespace

int launch_attention(const AttnDesc &d, hipStream_t stream)
{
    if (d.D > kMaxD || d.D % 8 != 0 || d.Hq % d.Hkv != 0 || d.max_pos % kChunk != 0)
        return set_error(EP_DECLINE_SHAPE, "attention: head_dim %d / heads %d,%d / max_pos %d",
                         d.D, d.Hq, d.Hkv, d.max_pos);
    AttnArgs a{d.q, d.k, d.v, d.qn_w, d.kn_w, d.qk_eps, d.kcache, d.vcache, d.cos_t, d.sin_t,
               d.state, d.part, d.counters, d.out, d.Hq, d.Hkv, d.D, d.max_pos, d.scale};
    hipLaunchKernelGGL(attention_kernel, dim3(d.Hq, d.max_pos / kChunk), dim3(256), 0, stream, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

size_t attention_workspace(int Hq, int D, int max_pos)
{
    return (size_t)Hq * (max_pos / kChunk) * (D + 2) * sizeof(float);
}

int launch_lm_head(const HeadDesc &d, hipStream_t stream)
{
    if (d.H % 512 != 0 || d.H > 64 * kHeadPerLane)
        return set_error(EP_DECLINE_SHAPE, "lm_head: hidden %d must be a multiple of 512, <= %d",
                         d.H, 64 * kHeadPerLane);
    if (d.grid < 1 || d.grid > 65535)
        return set_error(EP_ERR_ARG, "lm_head: grid %d", d.grid);
    HeadArgs a{d.h, d.norm_w, d.eps, d.W, d.logits, d.V, d.H, d.part_val, d.part_idx,
               d.counter, d.state, d.prompt, d.n_prompt, d.tokens, d.argmax_out, d.embed,
               d.max_pos};
    hipLaunchKernelGGL(lm_head_kernel, dim3(d.grid), dim3(64 * kHeadWaves), 0, stream, a);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

int launch_embed(const uint16_t *embed, const int *state, float *h, int H, hipStream_t stream)
{
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(256), 0, stream, embed, state, h, H);
    EP_HIP_CHECK(hipGetLastError());
    return EP_OK;
}

}  // namespace ep
