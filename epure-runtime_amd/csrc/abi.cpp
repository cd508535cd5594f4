// extern "C" entry points of libepure_hip.so (declared in include/epure_hip.h).
//
// Validation, kernel selection and error reporting live here; kernels live
// in gemv.hip (small M), mfma.hip (large M), backward.hip and tile.hip.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "epure_decode.h"
#include "epure_hip.h"
#include "ep_internal.h"

namespace ep {

static thread_local char g_err[512];

int set_error(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

static int g_cus = 0;

int device_cus()
{
    if (g_cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            g_cus = n;
        else
            g_cus = 256;
    }
    return g_cus;
}

static bool valid_dtype(int dt) { return dt == EP_F32 || dt == EP_F16 || dt == EP_BF16; }

static int check_weight(const PackedDesc &w)
{
    if (w.levels < 1 || w.levels > 256)
        return set_error(EP_DECLINE_LEVELS, "levels=%d outside 1..256", w.levels);
    if (!valid_dtype(w.scale_dtype) || !valid_dtype(w.cb_dtype))
        return set_error(EP_DECLINE_DTYPE, "scale/cb dtype not served (scale %d, cb %d)",
                         w.scale_dtype, w.cb_dtype);
    if (w.group < 1)
        return set_error(EP_ERR_ARG, "group=%d must be >= 1", w.group);
    if (w.N < 0 || w.K < 0)
        return set_error(EP_ERR_ARG, "negative shape N=%lld K=%lld", (long long)w.N,
                         (long long)w.K);
    const int64_t G = (w.K + w.group - 1) / w.group;
    if (w.K > 0 && w.ld_scale < G)
        return set_error(EP_ERR_ARG, "ld_scale=%lld < ceil(K/group)=%lld", (long long)w.ld_scale,
                         (long long)G);
    if (w.N > 0 && w.K > 0 && (!w.packed || !w.scale || !w.cb))
        return set_error(EP_ERR_ARG, "null weight pointer");
    return EP_OK;
}

}  // namespace ep

using namespace ep;

extern "C" {

int ep_abi_version(void) { return EP_ABI_VERSION; }

const char *ep_last_error(void) { return g_err; }

int ep_hip_available(void)
{
    static int cached = -1;
    if (cached >= 0)
        return cached;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        cached = 0;
        return cached;
    }
    int found = 0;
    for (int d = 0; d < n && !found; ++d) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, d) == hipSuccess &&
            strncmp(prop.gcnArchName, "gfx950", 6) == 0)
            found = 1;
    }
    cached = found;
    if (found)
        (void)device_cus();
    return cached;
}

size_t ep_dequant_matmul_workspace(int64_t M, int64_t N, int64_t K, int levels, int group)
{
    (void)group;
    // Any M may land on the MFMA path (shapes the GEMV does not serve), so
    // the per-row exponent buffer is always requested; 2..64 rows may take
    // the split-K path and its partial sums.
    size_t need = mfma_workspace(M);
    const size_t b = (M >= 2 && M <= 64) ? skinny_workspace(M, N, K, levels) : 0;
    const size_t c = M > 64 ? prefill_workspace(M, N, K, levels) : 0;
    need = need > b ? need : b;
    return need > c ? need : c;
}

int ep_dequant_matmul(const void *x, int x_dtype, int64_t ldx, const uint8_t *packed,
                      const void *scale, int scale_dtype, int64_t ld_scale, const void *cb,
                      int cb_dtype, int levels, int group, int64_t M, int64_t N, int64_t K,
                      void *y, int y_dtype, int64_t ldy, int flags, void *workspace,
                      size_t workspace_bytes, void *stream)
{
    g_err[0] = 0;
    PackedDesc w{packed, scale, scale_dtype, ld_scale, cb, cb_dtype, levels, group, N, K};
    int rc = check_weight(w);
    if (rc != EP_OK)
        return rc;
    if (!valid_dtype(x_dtype) || !valid_dtype(y_dtype))
        return set_error(EP_DECLINE_DTYPE, "x/y dtype not served (x %d, y %d)", x_dtype, y_dtype);
    if (M < 0)
        return set_error(EP_ERR_ARG, "negative M");
    if (M == 0 || N == 0)
        return EP_OK;
    if (!x || !y)
        return set_error(EP_ERR_ARG, "null x or y");
    if ((M > 1 && ldx < K) || (M > 1 && ldy < N))
        return set_error(EP_ERR_ARG, "ldx/ldy smaller than the row length");
    ActDesc xa{x, x_dtype, M > 1 ? ldx : K};
    OutDesc ya{y, y_dtype, M > 1 ? ldy : N, (flags & EP_FLAG_ACCUMULATE) ? 1 : 0};
    hipStream_t s = (hipStream_t)stream;
    // 1..4 rows: the LUT GEMV (one launch) where it serves; 2..64 rows: the
    // split-K MFMA path; more: the MFMA tiles
    if (gemv_serves(w, xa, M))
        return launch_gemv(w, xa, M, ya, s);
    if (skinny_serves(w, xa, M))
        return launch_skinny(w, xa, M, ya, workspace, workspace_bytes, s);
    if (M > 64 && prefill_serves(w, xa, M))
        return launch_prefill(w, xa, M, ya, workspace, workspace_bytes, s);
    if (mfma_serves(w, xa, M))
        return launch_mfma(w, xa, M, ya, workspace, workspace_bytes, s);
    if (M <= 64)
        return launch_gemv_generic(w, xa, M, ya, s);
    return set_error(EP_DECLINE_SHAPE,
                     "no kernel serves M=%lld N=%lld K=%lld group=%d levels=%d with these strides",
                     (long long)M, (long long)N, (long long)K, group, levels);
}

int ep_expert_matmul(const void *x, int x_dtype, int64_t ldx, const int32_t *expert_ids, int64_t T,
                     const uint8_t *packed, const void *scale, int scale_dtype, int64_t ld_scale,
                     const void *cb, int cb_dtype, int levels, int group, int64_t E, int64_t N,
                     int64_t K, void *y, int y_dtype, int64_t ldy, void *stream)
{
    g_err[0] = 0;
    PackedDesc w{packed, scale, scale_dtype, ld_scale, cb, cb_dtype, levels, group, N, K};
    int rc = check_weight(w);
    if (rc != EP_OK)
        return rc;
    if (!valid_dtype(x_dtype) || !valid_dtype(y_dtype))
        return set_error(EP_DECLINE_DTYPE, "x/y dtype not served (x %d, y %d)", x_dtype, y_dtype);
    if (T < 0 || E < 1 || E > INT32_MAX)
        return set_error(EP_ERR_ARG, "T=%lld E=%lld", (long long)T, (long long)E);
    if (T == 0 || N == 0)
        return EP_OK;
    if (!x || !y || !expert_ids)
        return set_error(EP_ERR_ARG, "null x, y or expert_ids");
    if ((T > 1 && ldx < K) || (T > 1 && ldy < N))
        return set_error(EP_ERR_ARG, "ldx/ldy smaller than the row length");
    const int64_t rb = levels <= 16 ? K / 2 : K;
    if (E * N * rb >= ((int64_t)1 << 40))
        return set_error(EP_DECLINE_SHAPE, "expert stack too large");
    ActDesc xa{x, x_dtype, ldx};
    OutDesc ya{y, y_dtype, ldy, 0};
    return launch_gemv_gather(w, xa, T, expert_ids, (int)E, ya, (hipStream_t)stream);
}

size_t ep_expert_matmul_grouped_workspace(int64_t T, int64_t E, int64_t K)
{
    return expert_grouped_workspace(T, E, K);
}

int ep_expert_matmul_grouped(const void *x, int x_dtype, int64_t ldx, const int32_t *expert_ids, int64_t T,
                             const uint8_t *packed, const void *scale, int scale_dtype, int64_t ld_scale,
                             const void *cb, int cb_dtype, int levels, int group, int64_t E, int64_t N,
                             int64_t K, void *y, int y_dtype, int64_t ldy, void *workspace,
                             size_t workspace_bytes, void *stream)
{
    g_err[0] = 0;
    PackedDesc w{packed, scale, scale_dtype, ld_scale, cb, cb_dtype, levels, group, N, K};
    int rc = check_weight(w);
    if (rc != EP_OK)
        return rc;
    if (!valid_dtype(x_dtype) || !valid_dtype(y_dtype))
        return set_error(EP_DECLINE_DTYPE, "x/y dtype not served (x %d, y %d)", x_dtype, y_dtype);
    if (T < 0 || E < 1 || E > INT32_MAX)
        return set_error(EP_ERR_ARG, "T=%lld E=%lld", (long long)T, (long long)E);
    if (T == 0 || N == 0)
        return EP_OK;
    if (!x || !y || !expert_ids)
        return set_error(EP_ERR_ARG, "null x, y or expert_ids");
    if ((T > 1 && ldx < K) || (T > 1 && ldy < N))
        return set_error(EP_ERR_ARG, "ldx/ldy smaller than the row length");
    const int64_t rb = levels <= 16 ? K / 2 : K;
    if (E * N * rb >= ((int64_t)1 << 40))
        return set_error(EP_DECLINE_SHAPE, "expert stack too large");
    ActDesc xa{x, x_dtype, ldx};
    OutDesc ya{y, y_dtype, ldy, 0};
    return launch_expert_grouped(w, xa, T, expert_ids, (int)E, ya, workspace, workspace_bytes,
                                 (hipStream_t)stream);
}

size_t ep_dequant_matmul_bwd_workspace(int64_t M, int64_t N, int64_t K, int levels, int group)
{
    return backward_workspace(M, N, K, levels, group);
}

int ep_dequant_matmul_bwd(const void *gy, int gy_dtype, int64_t ldgy, const void *x, int x_dtype,
                          int64_t ldx, const uint8_t *packed, const void *scale, int scale_dtype,
                          int64_t ld_scale, const void *cb, int cb_dtype, int levels, int group,
                          int64_t M, int64_t N, int64_t K, void *grad_x, int gx_dtype,
                          int64_t ldgx, float *grad_cb, float *grad_scale, int64_t ld_gscale,
                          void *workspace, size_t workspace_bytes, void *stream)
{
    g_err[0] = 0;
    PackedDesc w{packed, scale, scale_dtype, ld_scale, cb, cb_dtype, levels, group, N, K};
    int rc = check_weight(w);
    if (rc != EP_OK)
        return rc;
    if (!valid_dtype(gy_dtype) || !valid_dtype(x_dtype) || (grad_x && !valid_dtype(gx_dtype)))
        return set_error(EP_DECLINE_DTYPE, "gy/x/grad_x dtype not served");
    if (M < 0)
        return set_error(EP_ERR_ARG, "negative M");
    // activation strides only matter where there are rows to read
    if ((M > 0 && (ldgy < N || ldx < K || (grad_x && ldgx < K))) ||
        (grad_scale && ld_gscale < (K + group - 1) / group))
        return set_error(EP_ERR_ARG, "leading dimension smaller than the row length");
    ActDesc gya{gy, gy_dtype, ldgy};
    ActDesc xa{x, x_dtype, ldx};
    OutDesc gxa{grad_x, gx_dtype, ldgx, 0};
    return launch_backward(w, gya, xa, M, gxa, grad_cb, grad_scale, ld_gscale, workspace,
                           workspace_bytes, (hipStream_t)stream);
}

int ep_unpack_indices(const uint8_t *packed, int64_t n, int levels, uint8_t *idx, void *stream)
{
    g_err[0] = 0;
    if (levels < 1 || levels > 256)
        return set_error(EP_DECLINE_LEVELS, "levels=%d outside 1..256", levels);
    if (n < 0 || (n > 0 && (!packed || !idx)))
        return set_error(EP_ERR_ARG, "bad unpack arguments");
    return launch_unpack(packed, n, levels, idx, (hipStream_t)stream);
}

int ep_dequant_tile(const uint8_t *packed, const void *scale, int scale_dtype, int64_t ld_scale,
                    const void *cb, int cb_dtype, int levels, int group, int64_t N, int64_t K,
                    void *out, int out_dtype, int64_t ldo, void *stream)
{
    g_err[0] = 0;
    PackedDesc w{packed, scale, scale_dtype, ld_scale, cb, cb_dtype, levels, group, N, K};
    int rc = check_weight(w);
    if (rc != EP_OK)
        return rc;
    if (!valid_dtype(out_dtype))
        return set_error(EP_DECLINE_DTYPE, "out dtype %d not served", out_dtype);
    if (N > 0 && K > 0 && (!out || ldo < K))
        return set_error(EP_ERR_ARG, "bad output buffer");
    return launch_dequant_tile(w, out, out_dtype, ldo, (hipStream_t)stream);
}

int ep_embedding_rows(const uint8_t *packed, const void *scale, int scale_dtype, int64_t ld_scale,
                      const void *cb, int cb_dtype, int levels, int group, int64_t N, int64_t K,
                      const int64_t *ids, int64_t n_ids, void *out, int out_dtype, int64_t ldo,
                      void *stream)
{
    g_err[0] = 0;
    PackedDesc w{packed, scale, scale_dtype, ld_scale, cb, cb_dtype, levels, group, N, K};
    int rc = check_weight(w);
    if (rc != EP_OK)
        return rc;
    if (!valid_dtype(out_dtype))
        return set_error(EP_DECLINE_DTYPE, "out dtype %d not served", out_dtype);
    if (n_ids < 0 || (n_ids > 0 && K > 0 && (!ids || !out || ldo < K)))
        return set_error(EP_ERR_ARG, "bad embedding arguments");
    return launch_embedding_rows(w, ids, n_ids, out, out_dtype, ldo, (hipStream_t)stream);
}

int ep_fused_gemv(int xsrc, const void *x, int x_dtype, const void *x_aux, float eps, int64_t K,
                  int group, int levels, int scale_dtype, int cb_dtype, int nseg,
                  const uint8_t *const *packed, const void *const *scale, const void *const *cb,
                  void *const *y, const int64_t *N, int y_dtype, int accumulate, void *stream)
{
    g_err[0] = 0;
    if (nseg < 1 || nseg > 3 || !packed || !scale || !cb || !y || !N || !x)
        return set_error(EP_ERR_ARG, "fused GEMV: bad segment arguments");
    if ((xsrc != EP_XSRC_PLAIN && !x_aux) || !valid_dtype(y_dtype) ||
        (xsrc == EP_XSRC_PLAIN && !valid_dtype(x_dtype)))
        return set_error(EP_ERR_ARG, "fused GEMV: bad activation arguments");
    FusedGemv f{};
    f.xsrc = xsrc;
    f.x = x;
    f.x_dtype = x_dtype;
    f.x2 = x_aux;
    f.eps = eps;
    f.K = K;
    f.group = group;
    f.levels = levels;
    f.scale_dtype = scale_dtype;
    f.cb_dtype = cb_dtype;
    f.y_dtype = y_dtype;
    f.accumulate = accumulate ? 1 : 0;
    f.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        PackedDesc w{packed[i], scale[i], scale_dtype, (K + group - 1) / group, cb[i], cb_dtype,
                     levels, group, N[i], K};
        int rc = check_weight(w);
        if (rc != EP_OK)
            return rc;
        if (!y[i])
            return set_error(EP_ERR_ARG, "fused GEMV: null output %d", i);
        f.seg[i] = FusedSeg{packed[i], scale[i], cb[i], y[i], N[i]};
    }
    return launch_gemv_fused(f, (hipStream_t)stream);
}

size_t ep_attention_workspace(int Hq, int D, int max_pos)
{
    return attention_workspace(Hq, D, max_pos);
}

int ep_decode_attention(const float *q, const float *k, const float *v, const uint16_t *qn_w,
                        const uint16_t *kn_w, float qk_eps, float *kcache, float *vcache,
                        const float *cos_t, const float *sin_t, const int *state, float *part,
                        int *counters, float *out, int Hq, int Hkv, int D, int max_pos,
                        float scale, void *stream)
{
    g_err[0] = 0;
    if (!q || !k || !v || !kcache || !vcache || !cos_t || !sin_t || !state || !part ||
        !counters || !out || Hq < 1 || Hkv < 1 || D < 2 || max_pos < 1)
        return set_error(EP_ERR_ARG, "attention: bad arguments");
    AttnDesc d{q, k, v, qn_w, kn_w, qk_eps, kcache, vcache, cos_t, sin_t, state, part, counters,
               out, Hq, Hkv, D, max_pos, scale};
    return launch_attention(d, (hipStream_t)stream);
}

int ep_lm_head_argmax(float *h, const uint16_t *norm_w, float eps, const uint16_t *W, float *logits,
                      int V, int H, float *part_val, int *part_idx, int *counter, int *state,
                      const int *prompt, int n_prompt, int *tokens, int *argmax_out,
                      const uint16_t *embed, int max_pos, int grid, void *stream)
{
    g_err[0] = 0;
    if (!h || !norm_w || !W || !part_val || !part_idx || !counter || !state || !tokens ||
        !argmax_out || !embed || V < 1 || H < 1 || (n_prompt > 0 && !prompt))
        return set_error(EP_ERR_ARG, "lm_head: bad arguments");
    HeadDesc d{h, norm_w, eps, W, logits, V, H, part_val, part_idx, counter, state, prompt,
               n_prompt, tokens, argmax_out, embed, max_pos, grid};
    return launch_lm_head(d, (hipStream_t)stream);
}

int ep_embed_token(const uint16_t *embed, const int *state, float *h, int H, void *stream)
{
    g_err[0] = 0;
    if (!embed || !state || !h || H < 1)
        return set_error(EP_ERR_ARG, "embed: bad arguments");
    return launch_embed(embed, state, h, H, (hipStream_t)stream);
}

size_t ep_decode_step_layer_bytes(void) { return decode_step_layer_bytes(); }

size_t ep_decode_step_workspace(int H, int I, int Hq, int Hkv, int D, int max_pos)
{
    if (H < 1 || I < 1 || Hq < 1 || Hkv < 1 || D < 1 || max_pos < 1)
        return 0;
    return decode_step_workspace(H, I, Hq, Hkv, D, max_pos);
}

static StepDesc step_desc(int H, int I, int Hq, int Hkv, int D, int max_pos, int levels, int group,
                          int scale_dtype, int cb_dtype)
{
    StepDesc d{};
    d.H = H;
    d.I = I;
    d.Hq = Hq;
    d.Hkv = Hkv;
    d.D = D;
    d.max_pos = max_pos;
    d.levels = levels;
    d.group = group;
    d.scale_dtype = scale_dtype;
    d.cb_dtype = cb_dtype;
    return d;
}

int ep_decode_step_serves(int H, int I, int Hq, int Hkv, int D, int max_pos, int levels, int group,
                          int scale_dtype, int cb_dtype)
{
    g_err[0] = 0;
    if (H < 1 || I < 1 || Hq < 1 || Hkv < 1 || D < 1 || max_pos < 1 || group < 1)
        return 0;
    return decode_step_serves(step_desc(H, I, Hq, Hkv, D, max_pos, levels, group, scale_dtype,
                                        cb_dtype)) == EP_OK;
}

int ep_decode_step(const void *layers, int n_layers, float *h, void *workspace,
                   size_t workspace_bytes, const float *cos_t, const float *sin_t, const int *state,
                   int H, int I, int Hq, int Hkv, int D, int max_pos, int levels, int group,
                   int scale_dtype, int cb_dtype, float eps, float qk_eps, float att_scale,
                   long long *trace, void *stream)
{
    g_err[0] = 0;
    if (!layers || n_layers < 1 || !h || !workspace || !cos_t || !sin_t || !state || H < 1 ||
        I < 1 || Hq < 1 || Hkv < 1 || D < 1 || max_pos < 1 || group < 1)
        return set_error(EP_ERR_ARG, "decode step: bad arguments");
    if (((uintptr_t)h | (uintptr_t)workspace) & 15)
        return set_error(EP_ERR_ARG, "decode step: h/workspace not 16-byte aligned");
    StepDesc d = step_desc(H, I, Hq, Hkv, D, max_pos, levels, group, scale_dtype, cb_dtype);
    d.layers = layers;
    d.n_layers = n_layers;
    d.h = h;
    d.ws = workspace;
    d.ws_bytes = workspace_bytes;
    d.cos_t = cos_t;
    d.sin_t = sin_t;
    d.state = state;
    d.eps = eps;
    d.qk_eps = qk_eps;
    d.att_scale = att_scale;
    d.trace = trace;
    return launch_decode_step(d, (hipStream_t)stream);
}

}  // extern "C"
