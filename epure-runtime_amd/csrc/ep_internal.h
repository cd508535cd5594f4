// Internal launch interface between the C ABI (abi.cpp) and the kernel
// translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ep {

// Everything that describes one packed weight W[N, K].
struct PackedDesc {
    const uint8_t *packed;
    const void *scale;
    int scale_dtype;
    int64_t ld_scale;
    const void *cb;
    int cb_dtype;
    int levels;
    int group;
    int64_t N, K;
    int bits() const { return levels <= 16 ? 4 : 8; }
};

struct ActDesc {
    const void *ptr;
    int dtype;
    int64_t ld;
};

struct OutDesc {
    void *ptr;
    int dtype;
    int64_t ld;
    int accumulate;
};

// Compute units of the current device (queried once, at library load or
// first use; never inside a stream capture after ep_hip_available()).
int device_cus();

// Sets the calling thread's error message; returns `code`.
int set_error(int code, const char *fmt, ...);

// All launchers return EP_OK / a decline code (> 0) / an error (< 0).
int launch_gemv(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                hipStream_t stream);
int launch_gemv_generic(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                        hipStream_t stream);
// One GEMV per token over a stack of E weights shaped as w (w.packed and
// w.scale point at expert 0): y[t] = x[t] . W[ids[t]]^T, ids on the device.
int launch_gemv_gather(const PackedDesc &w, const ActDesc &x, int64_t T, const int *ids, int E,
                       const OutDesc &y, hipStream_t stream);
bool gemv_serves(const PackedDesc &w, const ActDesc &x, int64_t M);

// Decode-step GEMV: M = 1, up to three weights sharing K (fused q/k/v or
// gate/up), activation taken from a fused prologue.
struct FusedSeg {
    const uint8_t *packed;
    const void *scale;
    const void *cb;
    void *y;
    int64_t N;
};
struct FusedGemv {
    int xsrc;  // 0 plain x (x_dtype), 1 rmsnorm(h f32, w bf16), 2 silu(g) * u (f32)
    const void *x;
    int x_dtype;
    const void *x2;
    float eps;
    int64_t K;
    int group, levels, scale_dtype, cb_dtype, y_dtype, accumulate;
    int nseg;
    FusedSeg seg[3];
};
int launch_gemv_fused(const FusedGemv &f, hipStream_t stream);

// Decode attention over an f32 KV cache (decode.hip).
struct AttnDesc {
    const float *q, *k, *v;
    const uint16_t *qn_w, *kn_w;
    float qk_eps;
    float *kcache, *vcache;  // [Hkv][max_pos][D]
    const float *cos_t, *sin_t;
    const int *state;
    float *part;
    int *counters;
    float *out;  // [Hq * D]
    int Hq, Hkv, D, max_pos;
    float scale;
};
int launch_attention(const AttnDesc &d, hipStream_t stream);
size_t attention_workspace(int Hq, int D, int max_pos);

// lm_head + final norm + greedy selection + next embedding (decode.hip).
struct HeadDesc {
    float *h;
    const uint16_t *norm_w;
    float eps;
    const uint16_t *W;
    float *logits;
    int V, H;
    float *part_val;
    int *part_idx;
    int *counter;
    int *state;
    const int *prompt;
    int n_prompt;
    int *tokens;
    int *argmax_out;
    const uint16_t *embed;
    int max_pos;
    int grid;
};
int launch_lm_head(const HeadDesc &d, hipStream_t stream);
int launch_embed(const uint16_t *embed, const int *state, float *h, int H, hipStream_t stream);

// Persistent decode step (step.hip): every layer of one batch-1 step in one
// launch.  `layers` points to n_layers device-side descriptors of
// decode_step_layer_bytes() each.
struct StepDesc {
    const void *layers;
    int n_layers;
    float *h;   // [H] f32 in (embedding) / out (final residual)
    void *ws;   // decode_step_workspace() bytes, zeroed before the first launch
    size_t ws_bytes;
    const float *cos_t, *sin_t;
    const int *state;
    int H, I, Hq, Hkv, D, max_pos, levels, group, scale_dtype, cb_dtype;
    float eps, qk_eps, att_scale;
    long long *trace;
};
int launch_decode_step(const StepDesc &d, hipStream_t stream);
int decode_step_serves(const StepDesc &d);
size_t decode_step_workspace(int H, int I, int Hq, int Hkv, int D, int max_pos);
size_t decode_step_layer_bytes();

int launch_mfma(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                void *ws, size_t ws_bytes, hipStream_t stream);
bool mfma_serves(const PackedDesc &w, const ActDesc &x, int64_t M);
size_t mfma_workspace(int64_t M);
// Stacked experts grouped on the device (mfma.hip): a stable sort of the
// tokens by expert, then one MFMA launch over each expert's row tiles.
size_t expert_grouped_workspace(int64_t T, int64_t E, int64_t K);
bool expert_grouped_serves(const PackedDesc &w, const ActDesc &x, int64_t T, int64_t E);
int launch_expert_grouped(const PackedDesc &w, const ActDesc &x, int64_t T, const int *ids, int E,
                          const OutDesc &y, void *ws, size_t ws_bytes, hipStream_t stream);
// The prefill kernel over tiles of expert-sorted token rows (prefill.hip).
bool prefill_grouped_serves(const PackedDesc &w, const ActDesc &x, int64_t T);
size_t prefill_grouped_workspace(int64_t T, int64_t K);
int launch_prefill_grouped(const PackedDesc &w, const ActDesc &x, int64_t T, const int *perm,
                           const int *tiles, const int *ntiles, int bm, unsigned tiles_y, const OutDesc &y,
                           void *ws, hipStream_t stream);

// Small-M (2..64 rows) split-K dequant-matmul on MFMA (skinny.hip).
int launch_skinny(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y, void *ws,
                  size_t ws_bytes, hipStream_t stream);
bool skinny_serves(const PackedDesc &w, const ActDesc &x, int64_t M);
size_t skinny_workspace(int64_t M, int64_t N, int64_t K, int levels);
// y (=|+=) sum over s < S of part[s][M][N], in split order (skinny.hip).
int launch_split_reduce(const float *part, int S, int64_t M, int64_t N, const OutDesc &y,
                        hipStream_t stream);

// Prefill (more than 64 rows) dequant-matmul on 32x32x16 MFMA (prefill.hip).
int launch_prefill(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y, void *ws,
                   size_t ws_bytes, hipStream_t stream);
bool prefill_serves(const PackedDesc &w, const ActDesc &x, int64_t M);
size_t prefill_workspace(int64_t M, int64_t N, int64_t K, int levels);

int launch_backward(const PackedDesc &w, const ActDesc &gy, const ActDesc &x, int64_t M,
                    const OutDesc &gx, float *grad_cb, float *grad_scale, int64_t ld_gscale,
                    void *ws, size_t ws_bytes, hipStream_t stream);
size_t backward_workspace(int64_t M, int64_t N, int64_t K, int levels, int group);

int launch_unpack(const uint8_t *packed, int64_t n, int levels, uint8_t *idx, hipStream_t stream);
int launch_read_probe(const void *buf, int64_t bytes, uint32_t *sink, int grid, hipStream_t stream);
int launch_embedding_rows(const PackedDesc &w, const int64_t *ids, int64_t n_ids, void *out,
                          int out_dtype, int64_t ldo, hipStream_t stream);
int launch_dequant_tile(const PackedDesc &w, void *out, int out_dtype, int64_t ldo,
                        hipStream_t stream);

// Library GEMM (blas.cpp, hipBLASLt): D[m x n] (f32, column-major) = alpha *
// op(A) . op(B), fp16 or bf16 operands, f32 accumulation.
size_t blas_workspace_bytes();
// true once device `dev` has a hipBLASLt handle (created by a call outside
// stream capture); a caller under capture without one takes another route
bool blas_ready(int dev);
int blas_gemm_f32out(int ta, int tb, int64_t m, int64_t n, int64_t k, int ab_dtype, const void *A,
                     int64_t lda, const void *B, int64_t ldb, float *D, int64_t ldd, float alpha,
                     void *ws, size_t ws_bytes, hipStream_t stream);

// Checks a HIP call; on failure records the error and returns EP_ERR_HIP.
#define EP_HIP_CHECK(expr)                                                                 \
    do {                                                                                   \
        hipError_t _e = (expr);                                                            \
        if (_e != hipSuccess)                                                              \
            return ::ep::set_error(EP_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
    } while (0)

}  // namespace ep
