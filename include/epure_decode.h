/*
 * epure_decode.h -- C ABI of the batch-1 decode step built around the fused
 * packed GEMV (include/epure_hip.h).
 *
 * The reference runs decode through transformers with every q/k/v/o/
 * gate/up/down linear replaced by a PackedLinear (epure/runtime.py:261-262,
 * :373-415) and calls the fused kernel once per linear per token
 * (epure/kernels/cuda.py:88-117).  These entry points are the MI355X form
 * of that step: the packed GEMVs with the RMSNorm / SwiGLU of the decoder
 * fused into their activation load, grouped-query attention over a float32
 * KV cache (the decoder computes in float32 semantics: residual, attention
 * and the lm_head input are f32), and the bf16 lm_head with greedy
 * selection.
 *
 * All entry points follow include/epure_hip.h conventions (device pointers,
 * caller-owned buffers, return codes, no host synchronisation).  The token
 * position is read from device memory (`state[0]`), so a captured HIP graph
 * of one step replays for every token.
 */
#ifndef EPURE_DECODE_H
#define EPURE_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* activation sources for ep_fused_gemv */
#define EP_XSRC_PLAIN 0   /* x[K] in x_dtype */
#define EP_XSRC_RMSNORM 1 /* x = rmsnorm(h) * w: h f32 [K] (x), w bf16 [K] (x_aux), eps */
#define EP_XSRC_SWIGLU 2  /* x = silu(g) * u: g f32 [K] (x), u f32 [K] (x_aux) */

/*
 * y_i[N_i] (=|+=) W_i[N_i, K] . x for nseg (1..3) packed weights sharing K,
 * group, levels and element types (q/k/v of one layer, or gate/up), with x
 * built by the fused activation source.  Same arithmetic as
 * ep_dequant_matmul at M = 1.  Replaces, per segment, one call of
 * epure/kernels/cuda.py:88-117 linear(x, store) at batch 1.
 * Scale rows are dense: ld_scale = ceil(K / group).
 */
int ep_fused_gemv(int xsrc, const void *x, int x_dtype, const void *x_aux, float eps,
                  int64_t K, int group, int levels, int scale_dtype, int cb_dtype, int nseg,
                  const uint8_t *const *packed, const void *const *scale, const void *const *cb,
                  void *const *y, const int64_t *N, int y_dtype, int accumulate, void *stream);

/*
 * Grouped-query decode attention for one layer at position p = state[0]:
 * optional per-head RMSNorm of q and k (weights qn_w / kn_w, bf16, NULL =
 * none), rotate-half RoPE with cos/sin rows p of [max_pos][D/2] f32
 * tables, append of this step's k/v at row p of the [Hkv][max_pos][D] f32
 * caches, causal softmax over rows 0..p scaled by `scale`, output
 * [Hq * D] f32 (float32 throughout, the precision of the reference
 * model's float32 forward).  `part` needs ep_attention_workspace()
 * bytes; `counters` holds Hq ints that are zero before the first call and
 * are left zero by every call.  head_dim <= 128, max_pos % 64 == 0.
 */
size_t ep_attention_workspace(int Hq, int D, int max_pos);
int ep_decode_attention(const float *q, const float *k, const float *v, const uint16_t *qn_w,
                        const uint16_t *kn_w, float qk_eps, float *kcache, float *vcache,
                        const float *cos_t, const float *sin_t, const int *state, float *part,
                        int *counters, float *out, int Hq, int Hkv, int D, int max_pos,
                        float scale, void *stream);

/*
 * logits = W[V, H] (bf16) . (rmsnorm(h) * norm_w) in f32, then greedy
 * selection: with p = state[0], argmax_out[p] = argmax (lowest index on
 * ties), the next token is prompt[p + 1] while p + 1 < n_prompt, else the
 * argmax; tokens[p + 1] = next; state = {p + 1, next}; h = embed[next]
 * (f32).  `logits` may be NULL.  part_val / part_idx hold `grid` entries;
 * `counter` is one int, zero before the first call and left zero.
 * H % 512 == 0, H <= 4096.
 */
int ep_lm_head_argmax(float *h, const uint16_t *norm_w, float eps, const uint16_t *W,
                      float *logits, int V, int H, float *part_val, int *part_idx, int *counter,
                      int *state, const int *prompt, int n_prompt, int *tokens, int *argmax_out,
                      const uint16_t *embed, int max_pos, int grid, void *stream);

/*
 * Persistent decode step: every layer of one batch-1 step in ONE launch (one
 * resident workgroup per CU).  Phases hand over through tagged data in the
 * workspace: each value a workgroup produces for others is stored with the
 * (launch, layer, phase) tag, and consumers poll the values until every tag
 * is current -- no grid barrier; the next phase's packed weights are in
 * flight across each hand-over.  Same math as the per-layer sequence
 * ep_fused_gemv(q|k|v, RMSNorm)
 * -> ep_decode_attention -> ep_fused_gemv(o, +=) -> ep_fused_gemv(gate|up,
 * RMSNorm) -> ep_fused_gemv(down, SwiGLU, +=), i.e. the transformers
 * decoder layer whose linears the reference replaces with PackedLinear
 * (epure/runtime.py:261-262, :373-415), at batch 1.  Follow it with
 * ep_lm_head_argmax on the same h.
 *
 * `layers` (device memory) holds n_layers (<= 100) descriptors of
 * ep_decode_step_layer_bytes() bytes: 27 device pointers in this order --
 * packed[7], scale[7] (fp16 [N][K/group]), cb[7] (16 entries f32 or fp16,
 * entries >= levels ignored) for
 * q, k, v, o, gate, up, down; attn_norm, mlp_norm, q_norm, k_norm (bf16
 * [H], [H], [D], [D]; q/k norm NULL for Llama); kcache, vcache (f32
 * [Hkv][max_pos][D]).  h [H] f32 holds the step's input embedding and
 * receives the final residual (the lm_head's input).  `workspace`
 * (ep_decode_step_workspace bytes: the tagged hand-over buffers) must be
 * zeroed before the first call and is left valid for the next; its int
 * word 2 becomes nonzero if a hand-over wait timed out (the step's results
 * are then garbage).  `trace`, when not NULL, receives wall-clock stamps
 * [n_layers][24][grid] (debug).  Served (ep_decode_step_serves): D = 128,
 * 4-bit indices, groups a power of two >= 128, fp16 or f32 group scales,
 * and either a tuned shape (Llama-3-8B, Qwen3-8B, Qwen3-4B, Llama-3.2-3B,
 * Qwen3-1.7B, with fp16 scales) or the generic variants: H and Hq * D up
 * to 4096, I up to 16384, each a multiple of 512, Hq / Hkv in 1..8 (the
 * geometry of the largest such shape, blocks past a smaller shape's share
 * skipped).  Other shapes decline (> 0).  Position = state[0].  Launches
 * that share a workspace must be stream-ordered (two in flight on one
 * workspace race).
 */
size_t ep_decode_step_layer_bytes(void);
size_t ep_decode_step_workspace(int H, int I, int Hq, int Hkv, int D, int max_pos);
int ep_decode_step_serves(int H, int I, int Hq, int Hkv, int D, int max_pos, int levels,
                          int group, int scale_dtype, int cb_dtype);
int ep_decode_step(const void *layers, int n_layers, float *h, void *workspace,
                   size_t workspace_bytes, const float *cos_t, const float *sin_t,
                   const int *state, int H, int I, int Hq, int Hkv, int D, int max_pos,
                   int levels, int group, int scale_dtype, int cb_dtype, float eps,
                   float qk_eps, float att_scale, long long *trace, void *stream);

/* h[H] = embed[state[1]] as f32 (the first step's input). */
int ep_embed_token(const uint16_t *embed, const int *state, float *h, int H, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* EPURE_DECODE_H */
