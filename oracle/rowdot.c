/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle, never the product.
 *
 * Plain-C restatement of the reference's Rust fused CPU kernel
 * (kernel/src/lib.rs).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker or
 * the timed CPU baseline.
 *
 * Semantics kept identical to the Rust code so the result is bit-for-bit the
 * same IEEE-754 float32 computation:
 *   - build_lut (lib.rs:36-40): lut[l] = cb[l] * scale, rounded to f32; the
 *     table is 256 zeros first, so an index >= levels contributes 0
 *     (lib.rs:58-59, :63).
 *   - row_dot (lib.rs:47-88): per group (step_by(group), lib.rs:61-62), per
 *     activation row m: acc = 0; k ascending; acc += x[m,k] * lut[idx]
 *     (product rounded, then sum rounded -- Rust never contracts to FMA, so
 *     this file is compiled with -ffp-contract=off); 4-bit: low nibble is the
 *     even k, the high nibble is skipped when k+1 == chunk_end
 *     (lib.rs:69-79); 8-bit: one byte per k (lib.rs:80-84); then
 *     out[m] += acc (lib.rs:85).
 *   - dequant_matmul (lib.rs:94-151): k = row_bytes*2 for 4-bit
 *     (lib.rs:112); m = len(x) / k, truncating (lib.rs:113); rows are
 *     independent and split across threads (lib.rs:121-136, rayon); the
 *     [n, m] accumulator is transposed to [m, n] on the way out
 *     (lib.rs:141-146).
 *   - threads (lib.rs:155-157): number of worker threads used.
 *
 * Errors that the Rust code raises (slice index panics when `scales` has
 * too few columns, levels > 256) are returned as negative codes here.
 */
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static void build_lut(const float *cb, size_t levels, float scale, float *lut)
{
    for (size_t i = 0; i < levels; i++)
        lut[i] = cb[i] * scale;
}

static void row_dot(const float *x, size_t m, size_t k, const uint8_t *packed_row,
                    const float *scales_row, const float *cb, size_t levels,
                    size_t group, int four_bit, float *out /* [m] */)
{
    float lut[256];
    memset(lut, 0, sizeof(lut));
    size_t gi = 0;
    for (size_t chunk_start = 0; chunk_start < k; chunk_start += group, gi++) {
        size_t chunk_end = chunk_start + group < k ? chunk_start + group : k;
        build_lut(cb, levels, scales_row[gi], lut);
        for (size_t mi = 0; mi < m; mi++) {
            const float *xrow = x + mi * k;
            float acc = 0.0f;
            if (four_bit) {
                size_t kk = chunk_start;
                while (kk < chunk_end) {
                    uint8_t byte = packed_row[kk >> 1];
                    float p = xrow[kk] * lut[byte & 0x0F];
                    acc = acc + p;
                    if (kk + 1 < chunk_end) {
                        float q = xrow[kk + 1] * lut[byte >> 4];
                        acc = acc + q;
                    }
                    kk += 2;
                }
            } else {
                for (size_t kk = chunk_start; kk < chunk_end; kk++) {
                    float p = xrow[kk] * lut[packed_row[kk]];
                    acc = acc + p;
                }
            }
            out[mi] = out[mi] + acc;
        }
    }
}

typedef struct {
    const float *x;
    size_t m, k, row_bytes, n_groups, levels, group;
    const uint8_t *packed;
    const float *scales, *cb;
    int four_bit;
    float *acc; /* [n, m] */
    size_t row_lo, row_hi;
} job_t;

static void *worker(void *arg)
{
    job_t *j = (job_t *)arg;
    for (size_t row = j->row_lo; row < j->row_hi; row++)
        row_dot(j->x, j->m, j->k, j->packed + row * j->row_bytes,
                j->scales + row * j->n_groups, j->cb, j->levels, j->group,
                j->four_bit, j->acc + row * j->m);
    return NULL;
}

size_t oracle_threads(void)
{
    const char *env = getenv("RAYON_NUM_THREADS");
    if (env && atoi(env) > 0)
        return (size_t)atoi(env);
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (size_t)n : 1;
}

/*
 * out must hold m*n floats where m = x_len / k.  Returns m (>= 0) or a
 * negative error: -1 levels > 256, -2 scales too narrow for ceil(k/group),
 * -3 group == 0, -4 allocation failure.
 */
long long oracle_dequant_matmul_f32(const float *x, size_t x_len, const uint8_t *packed,
                                    size_t n, size_t row_bytes, const float *scales,
                                    size_t n_groups, const float *cb, size_t levels,
                                    size_t group, int four_bit, float *out, int nthreads)
{
    if (levels > 256)
        return -1;
    if (group == 0)
        return -3;
    size_t k = four_bit ? row_bytes * 2 : row_bytes;
    size_t m = k ? x_len / k : 0;
    if (k && (k + group - 1) / group > n_groups)
        return -2;
    size_t cells = m * n;
    float *acc = (float *)calloc(cells ? cells : 1, sizeof(float));
    if (!acc)
        return -4;
    size_t nt = nthreads > 0 ? (size_t)nthreads : oracle_threads();
    if (nt > n)
        nt = n ? n : 1;
    job_t *jobs = (job_t *)calloc(nt, sizeof(job_t));
    pthread_t *tids = (pthread_t *)calloc(nt, sizeof(pthread_t));
    if (!jobs || !tids) {
        free(acc);
        free(jobs);
        free(tids);
        return -4;
    }
    size_t per = nt ? (n + nt - 1) / nt : 0;
    for (size_t t = 0; t < nt; t++) {
        job_t j = {x, m, k, row_bytes, n_groups, levels, group, packed, scales, cb, four_bit,
                   acc, t * per, (t + 1) * per < n ? (t + 1) * per : n};
        if (j.row_lo > n)
            j.row_lo = n;
        jobs[t] = j;
    }
    if (nt <= 1) {
        if (nt == 1)
            worker(&jobs[0]);
    } else {
        for (size_t t = 0; t < nt; t++)
            pthread_create(&tids[t], NULL, worker, &jobs[t]);
        for (size_t t = 0; t < nt; t++)
            pthread_join(tids[t], NULL);
    }
    /* lib.rs:141-146: single-threaded transpose [n, m] -> [m, n] */
    for (size_t row = 0; row < n; row++)
        for (size_t mi = 0; mi < m; mi++)
            out[mi * n + row] = acc[row * m + mi];
    free(acc);
    free(jobs);
    free(tids);
    return (long long)m;
}
