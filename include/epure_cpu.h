/*
 * libepure_cpu.so: the fused dequant-matmul on host cores (the CPU half of
 * the drop-in boundary; epure/kernels/cpu.py binds it with ctypes).
 */
#ifndef EPURE_CPU_H
#define EPURE_CPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * out[m, n] = x[m, k] . dequant(packed)[n, k]^T in float32, bit-identical to
 * the reference's Rust kernel.  Replaces the PyO3 entry
 *   kernel/src/lib.rs:94-151  epure_kernel.dequant_matmul(x, packed, scales,
 *                             cb, group, four_bit)
 * called from epure/kernels/cpu.py:69.  x holds x_len floats, m = x_len / k
 * (truncating, lib.rs:113) with k = 2 * row_bytes (four_bit) or row_bytes;
 * packed [n][row_bytes] u8 (low nibble = even k); scales [n][n_groups] f32;
 * cb [levels] f32 (an index >= levels contributes 0).  nthreads <= 0: the
 * default pool (ep_cpu_threads).  Returns 0, or -1 (levels > 256), -2 (fewer
 * than ceil(k / group) scale columns), -3 (bad pointer / size / group),
 * -4 (out of memory): the cases where the Rust code raises.
 */
int ep_cpu_dequant_matmul_f32(const float *x, int64_t x_len, const uint8_t *packed, int64_t n,
                              int64_t row_bytes, const float *scales, int64_t n_groups,
                              const float *cb, int64_t levels, int64_t group, int four_bit,
                              float *out, int nthreads);

/* Default worker threads (EPURE_CPU_THREADS, else the online logical CPUs);
 * replaces kernel/src/lib.rs:155-157 threads(). */
size_t ep_cpu_threads(void);

/*
 * Chunked rANS decode of an .ebin index stream, replacing the reference's
 * epure/container.py:40-51 rans_decode (constriction's stack AnsCoder, one
 * coder per chunk).  words: the concatenated chunks as 32-bit words (chunk c
 * holds chunk_words[c] words and decodes to chunk_symbols[c] symbols);
 * cdf[0..nlevels]: the model's left-sided cumulative table at 24-bit
 * precision (cdf[0] = 0, cdf[nlevels] = 2^24, strictly increasing).  out
 * receives the sum of chunk_symbols bytes.  Chunks decode in parallel
 * (nthreads <= 0: ep_cpu_threads()).  Returns 0, -3 (bad argument), -4 (out
 * of memory) or -5 (malformed cdf).
 */
int ep_rans_decode(const uint32_t *words, const int64_t *chunk_words, const int64_t *chunk_symbols,
                   int nchunks, const uint32_t *cdf, int nlevels, uint8_t *out, int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* EPURE_CPU_H */
