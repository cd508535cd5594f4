/*
 * epure_hip.h -- C ABI of the MI355X (gfx950) fused codebook dequant-matmul.
 *
 * A packed weight W[N, K] is stored the way the reference keeps it resident
 * (epure/runtime.py:57-89):
 *   packed  uint8, the FLAT index stream of N*K indices; 4-bit when
 *           levels <= 16 (two per byte, even position in the low nibble,
 *           runtime.py:34-45), else one uint8 index per byte;
 *   scale   [N, ceil(K/group)] fp16 (container) or fp32 (after
 *           finetune.make_trainable, finetune.py:78), row stride ld_scale;
 *   cb      [levels] fp32 (container, runtime.py:243) or fp16.
 *   W[n,k] = cb[idx[n,k]] * scale[n, k / group]; an index >= levels reads 0
 *   (the Rust LUT, kernel/src/lib.rs:58-59).
 *
 * Conventions (all entry points):
 *   - plain device pointers and sizes; the caller owns every buffer,
 *     including workspaces; nothing here allocates or frees device memory,
 *     with one exception: the backward's library route (512 tokens and
 *     more) creates a hipBLASLt handle per device on its first call, and a
 *     side stream with two events per caller stream on a later call, both
 *     kept for the process (never under stream capture);
 *   - work is enqueued on `stream` (a hipStream_t; NULL = the null stream);
 *     no host synchronisation, with one exception: the first library-route
 *     backward call of a shape bucket (every dimension rounded up to a
 *     power of two) outside capture times its GEMM candidates and waits for
 *     them on the host.  Every call is capture-safe (under capture the
 *     backward takes no timing and, before a handle exists, the fused
 *     kernels instead of the library);
 *   - return 0 on success; > 0 = DECLINE (the caller falls back to
 *     materialize, the `None` of epure/kernels/__init__.py:5-11);
 *     < 0 = error, with a message from ep_last_error().
 *
 * Element type codes are the EP_* values below.
 */
#ifndef EPURE_HIP_H
#define EPURE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EP_ABI_VERSION 1

/* element types */
#define EP_F32 0
#define EP_F16 1
#define EP_BF16 2

/* flags for ep_dequant_matmul */
#define EP_FLAG_ACCUMULATE 1 /* y += x.W^T instead of y = x.W^T */

/* return codes */
#define EP_OK 0
#define EP_DECLINE_DTYPE 1  /* unsupported element type combination */
#define EP_DECLINE_SHAPE 2  /* shape/stride the kernels do not serve */
#define EP_DECLINE_LEVELS 3 /* levels outside 1..256 */
#define EP_ERR_ARG (-1)
#define EP_ERR_HIP (-2)
#define EP_ERR_WORKSPACE (-3)

/* Version of this ABI (EP_ABI_VERSION). */
int ep_abi_version(void);

/*
 * 1 if a gfx950 device is visible, else 0.  Cheap and side-effect free
 * after the first call.  Replaces epure/kernels/cuda.py:49-50 available().
 */
int ep_hip_available(void);

/* Last error message of the calling thread ("" if none). */
const char *ep_last_error(void);

/*
 * Workspace bytes ep_dequant_matmul needs for this shape (a few bytes per
 * activation row).  The caller passes at least this much.
 */
size_t ep_dequant_matmul_workspace(int64_t M, int64_t N, int64_t K, int levels, int group);

/*
 * y[M, N] (=|+=) x[M, K] . W[N, K]^T
 *
 * Replaces the reference's per-packed-linear kernel entry:
 *   epure/kernels/_triton.py:477-512  dequant_matmul(x, packed, scale, cb,
 *                                     group, bits, n_out, k_in)
 *   kernel/src/lib.rs:94-151          epure_kernel.dequant_matmul(x, packed,
 *                                     scales, cb, group, four_bit)
 * x: x_dtype (EP_BF16 / EP_F16 / EP_F32), row stride ldx elements.
 * y: y_dtype, row stride ldy elements.  Accumulation is fp32; weights enter
 * the products as fp16(cb[idx]) (the dot-product path) or
 * fp16(cb[idx]*scale) (the MFMA path); x enters as fp16 after an exact
 * per-row power-of-two rescale, so it cannot overflow fp16.
 * The kernel is chosen from M: the LUT GEMV at M = 1 (up to 4 where its
 * activations fit), register-dequant MFMA kernels up to M = 64 (one launch
 * per linear for 8-bit indices at M <= 16 and wide N; for 8-bit indices at
 * 33 <= M <= 64, and at 17 <= M <= 32 on layers of at least 2^25 weights,
 * split-K over slices of 2048 or 4096 values with each wave's activations
 * held in registers;
 * split-K over slices of at most 1024 otherwise; the splits' f32 partials
 * summed in split order), dequant-to-LDS + MFMA above.  Each reads the
 * packed bytes exactly once per launch.
 */
int ep_dequant_matmul(const void *x, int x_dtype, int64_t ldx,
                      const uint8_t *packed, const void *scale, int scale_dtype,
                      int64_t ld_scale, const void *cb, int cb_dtype, int levels,
                      int group, int64_t M, int64_t N, int64_t K,
                      void *y, int y_dtype, int64_t ldy, int flags,
                      void *workspace, size_t workspace_bytes, void *stream);

/*
 * Expert-indexed packed linear for a few tokens: y[t, :] = x[t, :] . W[e_t]^T
 * with e_t = expert_ids[t] (int32, device memory) and W[e] the rows
 * e*N .. e*N + N - 1 of a stack of E weights folded as (E*N, K) with one
 * codebook (`packed`, `scale` point at expert 0; ld_scale = K / group).
 * Replaces the per-expert loop of the stacked-expert forward (the
 * reference's expert holder materializes the whole slab per call,
 * epure/runtime.py:163-186): one launch, the ids read on the device, so the
 * call has no host synchronization and can be captured in a HIP graph.
 * The batch-1 LUT GEMV runs once per token (weights re-read per token: meant
 * for decode-sized T). Ids outside [0, E) are clamped on the device; callers
 * that can synchronize check them first. Returns EP_DECLINE_SHAPE where the
 * GEMV does not serve the shape (the caller then groups tokens per expert).
 */
int ep_expert_matmul(const void *x, int x_dtype, int64_t ldx, const int32_t *expert_ids, int64_t T,
                     const uint8_t *packed, const void *scale, int scale_dtype, int64_t ld_scale,
                     const void *cb, int cb_dtype, int levels, int group, int64_t E, int64_t N,
                     int64_t K, void *y, int y_dtype, int64_t ldy, void *stream);

/*
 * The same product for any token count, grouped by expert on the device:
 * a stable sort of the tokens by id (clamped into [0, E)), then one MFMA
 * launch whose workgroups take row tiles of one expert's tokens, each
 * reading that expert's weight rows once per tile and storing at the
 * tokens' own rows of y: the prefill MFMA kernel (32-, 64- or 128-row
 * tiles) where its shape rules hold (fp16 scales), else the generic MFMA
 * kernel (32- or 64-row tiles).
 * Replaces the reference's per-call slab materialization
 * (epure/runtime.py:163-186) and the caller's host-side grouping of tokens
 * per expert: no host synchronization, capturable in a HIP graph,
 * deterministic (no atomics in the product).  E <= 1024,
 * T <= 2^24, K % 64 == 0, 16-byte aligned rows (else EP_DECLINE_SHAPE).
 * Workspace: ep_expert_matmul_grouped_workspace(T, E, K) bytes.
 */
size_t ep_expert_matmul_grouped_workspace(int64_t T, int64_t E, int64_t K);
int ep_expert_matmul_grouped(const void *x, int x_dtype, int64_t ldx, const int32_t *expert_ids, int64_t T,
                             const uint8_t *packed, const void *scale, int scale_dtype, int64_t ld_scale,
                             const void *cb, int cb_dtype, int levels, int group, int64_t E, int64_t N,
                             int64_t K, void *y, int y_dtype, int64_t ldy, void *workspace,
                             size_t workspace_bytes, void *stream);

/*
 * Compressed-state backward of y = x . W^T with frozen indices
 * (fine-tuning/README.md:62-68; autograd through runtime.py:84-88):
 *   grad_x[M, K]            = gy[M, N] . W                (gx_dtype; NULL = skip)
 *   grad_cb[levels]   (f32) = sum_{idx==l} (gy^T x)[n,k] * scale[n, k/group]
 *   grad_scale[N, G]  (f32) = sum_{k in g} (gy^T x)[n,k] * cb[idx[n,k]]
 * (grad_cb / grad_scale NULL = skip).  grad_cb and grad_scale are
 * overwritten, not accumulated, and are deterministic (fixed-order
 * reductions).  `packed` is only read.
 * Two routes, chosen by shape:
 *   M < 512 (or N, K < 256): the fused kernels.  Each grad_W tile stays in
 *     registers and is reduced against the codebook in place: neither W nor
 *     grad_W is written to memory; the workspace holds per-row exponents,
 *     an fp16 copy of gy and grad_x split partials.
 *   M >= 512: library GEMMs.  The workspace receives W materialized as fp16
 *     [N, K] and grad_W = gy^T . x as f32 [N, K] (written once, read once by
 *     the epilogue that forms grad_scale and grad_cb), plus the fp16 gy, an
 *     f32 [M, K] grad_x product and two 32 MiB hipBLASLt workspaces.
 *     EPURE_BWD_FUSED=1 in the environment (read on the first call) keeps
 *     every M on the fused kernels instead.
 * ep_dequant_matmul_bwd_workspace() returns the larger of the two needs.
 */
size_t ep_dequant_matmul_bwd_workspace(int64_t M, int64_t N, int64_t K, int levels, int group);
int ep_dequant_matmul_bwd(const void *gy, int gy_dtype, int64_t ldgy,
                          const void *x, int x_dtype, int64_t ldx,
                          const uint8_t *packed, const void *scale, int scale_dtype,
                          int64_t ld_scale, const void *cb, int cb_dtype, int levels,
                          int group, int64_t M, int64_t N, int64_t K,
                          void *grad_x, int gx_dtype, int64_t ldgx,
                          float *grad_cb, float *grad_scale, int64_t ld_gscale,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * idx[0..n) = the unpacked index stream (epure/runtime.py:48-54 _unpack4),
 * run by the same device decode the GEMV uses.
 */
int ep_unpack_indices(const uint8_t *packed, int64_t n, int levels, uint8_t *idx, void *stream);

/*
 * out[N, K] (out_dtype, row stride ldo) = dequantized weight, with the
 * rounding of epure/runtime.py:78-89 materialize(dtype):
 *   EP_F32: f32(cb[idx]) * f32(scale)  (== container.dequantize,
 *           epure/container.py:70-88; exact for fp16-valued cb/scale)
 *   EP_F16 / EP_BF16: dtype(dtype(cb[idx]) * dtype(scale)).
 */
int ep_dequant_tile(const uint8_t *packed, const void *scale, int scale_dtype,
                    int64_t ld_scale, const void *cb, int cb_dtype, int levels,
                    int group, int64_t N, int64_t K, void *out, int out_dtype,
                    int64_t ldo, void *stream);

/*
 * out[i, 0..K) = row ids[i] of the dequantized weight (same rounding as
 * ep_dequant_tile), for i < n_ids: the packed embedding lookup that expands
 * only the rows a batch asks for (epure/runtime.py:129-156,
 * PackedEmbedding.forward; the reference gathers, unpacks and multiplies
 * with torch ops).  An id outside [0, N) gives a row of zeros (the caller
 * checks ranges where it can raise, as torch indexing does).
 */
int ep_embedding_rows(const uint8_t *packed, const void *scale, int scale_dtype,
                      int64_t ld_scale, const void *cb, int cb_dtype, int levels,
                      int group, int64_t N, int64_t K, const int64_t *ids, int64_t n_ids,
                      void *out, int out_dtype, int64_t ldo, void *stream);

/*
 * Streaming-read probe: reads bytes (a multiple of 16, 16-byte aligned) of
 * buf once with the dequant kernels' load shape (16-byte non-temporal loads,
 * 8 in flight per lane, 512-thread workgroups, `grid` of them) and writes
 * one XOR word per workgroup to sink[grid] (the XOR of all sink words is the
 * XOR of the buffer's 32-bit words).  The practical HBM read ceiling the
 * kernels are measured against; the reference's counterpart is its
 * same-traffic diagnostic kernel, epure/kernels/_triton.py:188-236
 * (dequant_nolut).
 */
int ep_read_probe(const void *buf, int64_t bytes, uint32_t *sink, int grid, void *stream);

/*
 * ep_dequant_matmul without a workspace argument, for callers that cannot
 * allocate device memory (code being captured into a HIP graph, serving
 * loops that forbid allocation).  No counterpart in the reference: its
 * kernels allocate their outputs per call.  Same arguments, semantics and
 * return codes as ep_dequant_matmul; the workspace is a static device array
 * of ep_noalloc_scratch_bytes() bytes (32 MiB) per GPU, kept until the
 * process ends.  Shapes whose ep_dequant_matmul_workspace exceeds it are
 * rejected with EP_ERR_WORKSPACE before any launch.  Nothing is allocated
 * and nothing in the scratch must start at zero; calls that overlap on one
 * GPU (two streams or threads at once) race on the shared scratch.
 */
size_t ep_noalloc_scratch_bytes(void);
int ep_dequant_matmul_noalloc(const void *x, int x_dtype, int64_t ldx,
                              const uint8_t *packed, const void *scale, int scale_dtype,
                              int64_t ld_scale, const void *cb, int cb_dtype, int levels,
                              int group, int64_t M, int64_t N, int64_t K,
                              void *y, int y_dtype, int64_t ldy, int flags, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* EPURE_HIP_H */
