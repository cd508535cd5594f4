/*
 * libepure_cpu.so: the fused dequant-matmul on host cores, behind
 * epure/kernels/cpu.py (the reference's CPU backend, epure/kernels/cpu.py:
 * 37-70, which calls the Rust epure_kernel.dequant_matmul,
 * kernel/src/lib.rs:94-151).
 *
 * Result contract: bit-identical to the Rust kernel.  Per output row and per
 * group of `group` k values, the Rust code builds lut[l] = cb[l] * scale
 * (f32, lib.rs:36-40; entries past `levels` stay 0, lib.rs:58-59), sums
 * acc += x[m][k] * lut[idx] for k ascending with every product rounded and
 * then added (no FMA contraction: this file is built with
 * -ffp-contract=off), and adds the group's acc into out[m] (lib.rs:61-87).
 * Each row's operation sequence here is exactly that one.
 *
 * Speed: the Rust loop runs one row's dependent add chain at a time, so it
 * is bound by the FP-add latency.  Here a thread takes a block of 8 rows and
 * advances their 8 independent chains together, k by k: the same additions
 * in the same order per row, with 8x the instruction-level parallelism.
 * Rows are split over threads in contiguous blocks (pthreads; the reference
 * uses rayon over rows, lib.rs:121-136).
 */
#include <errno.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define EP_CPU_ROWS 8 /* rows advanced together */

typedef struct {
    const float *x;
    int64_t m, k;
    const uint8_t *packed;
    int64_t n, row_bytes;
    const float *scales;
    int64_t n_groups;
    const float *cb;
    int64_t levels, group;
    int four_bit;
    float *out; /* [m][n] */
    int64_t row0, row1;
} Job;

/* Rows [r0, r0 + NR) of every activation row.  NR is a compile-time
 * constant so the NR accumulators stay in registers. */
#define DEFINE_ROWS_BLOCK(NAME, NR)                                                           \
    static void NAME(const Job *j, int64_t r0)                                                \
    {                                                                                         \
        float lut[NR][256];                                                                   \
        memset(lut, 0, sizeof(lut)); /* entries >= levels read 0 (lib.rs:58-59) */          \
        const uint8_t *rowp[NR];                                                              \
        for (int r = 0; r < NR; ++r)                                                          \
            rowp[r] = j->packed + (r0 + r) * j->row_bytes;                                    \
        for (int64_t mi = 0; mi < j->m; ++mi) {                                               \
            const float *xr = j->x + mi * j->k;                                               \
            float sum[NR];                                                                    \
            for (int r = 0; r < NR; ++r)                                                      \
                sum[r] = 0.0f;                                                                \
            int64_t gi = 0;                                                                   \
            for (int64_t cs = 0; cs < j->k; cs += j->group, ++gi) {                           \
                const int64_t ce = cs + j->group < j->k ? cs + j->group : j->k;               \
                float acc[NR];                                                                \
                for (int r = 0; r < NR; ++r) {                                                \
                    const float s = j->scales[(r0 + r) * j->n_groups + gi];                   \
                    for (int64_t l = 0; l < j->levels; ++l)                                   \
                        lut[r][l] = j->cb[l] * s;                                             \
                    acc[r] = 0.0f;                                                            \
                }                                                                             \
                if (j->four_bit) {                                                            \
                    /* the high nibble only while kk + 1 < chunk_end (lib.rs:69-79) */        \
                    int64_t kk = cs;                                                          \
                    for (; kk + 1 < ce; kk += 2) {                                            \
                        const float x0 = xr[kk], x1 = xr[kk + 1];                             \
                        for (int r = 0; r < NR; ++r) {                                        \
                            const uint8_t b = rowp[r][kk >> 1];                               \
                            const float p = x0 * lut[r][b & 0x0F];                            \
                            acc[r] = acc[r] + p;                                              \
                            const float q = x1 * lut[r][b >> 4];                              \
                            acc[r] = acc[r] + q;                                              \
                        }                                                                     \
                    }                                                                         \
                    if (kk < ce) {                                                            \
                        const float x0 = xr[kk];                                              \
                        for (int r = 0; r < NR; ++r) {                                        \
                            const float p = x0 * lut[r][rowp[r][kk >> 1] & 0x0F];             \
                            acc[r] = acc[r] + p;                                              \
                        }                                                                     \
                    }                                                                         \
                } else {                                                                      \
                    for (int64_t kk = cs; kk < ce; ++kk) {                                    \
                        const float x0 = xr[kk];                                              \
                        for (int r = 0; r < NR; ++r) {                                        \
                            const float p = x0 * lut[r][rowp[r][kk]];                         \
                            acc[r] = acc[r] + p;                                              \
                        }                                                                     \
                    }                                                                         \
                }                                                                             \
                for (int r = 0; r < NR; ++r)                                                  \
                    sum[r] = sum[r] + acc[r]; /* out[m] += acc (lib.rs:85) */                 \
            }                                                                                 \
            for (int r = 0; r < NR; ++r)                                                      \
                j->out[mi * j->n + r0 + r] = sum[r];                                          \
        }                                                                                     \
    }

DEFINE_ROWS_BLOCK(rows_block8, EP_CPU_ROWS)
DEFINE_ROWS_BLOCK(rows_block1, 1)

static void *run_job(void *arg)
{
    const Job *j = (const Job *)arg;
    int64_t r = j->row0;
    for (; r + EP_CPU_ROWS <= j->row1; r += EP_CPU_ROWS)
        rows_block8(j, r);
    for (; r < j->row1; ++r)
        rows_block1(j, r);
    return NULL;
}

/* Worker threads used by default: EPURE_CPU_THREADS if set, else the online
 * logical CPUs (rayon's default pool size, lib.rs:155-157). */
size_t ep_cpu_threads(void)
{
    const char *env = getenv("EPURE_CPU_THREADS");
    if (env && *env) {
        char *end = NULL;
        errno = 0;
        const long v = strtol(env, &end, 10);
        if (errno == 0 && end && *end == '\0' && v > 0 && v <= 4096)
            return (size_t)v;
    }
    const long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (size_t)n : 1;
}

/*
 * out[m][n] = x[m][k] . dequant(packed)[n][k]^T, f32.
 *
 * Arguments as the PyO3 function receives them (lib.rs:94-117): x holds
 * x_len floats (C order), m = x_len / k truncating (lib.rs:113); packed is
 * [n][row_bytes] bytes with k = 2 * row_bytes (four_bit) or row_bytes;
 * scales [n][n_groups] f32; cb [levels] f32.  nthreads <= 0 uses
 * ep_cpu_threads().  Returns 0, or a negative code where the Rust code
 * raises: -1 levels > 256 (lut[..levels], lib.rs:58-63), -2 too few scale
 * columns for ceil(k / group) groups (scales_row[gi], lib.rs:63), -3 a null
 * pointer, zero group or negative size, -4 no memory for the thread table.
 * A worker thread that cannot be started leaves its rows to the caller's
 * thread.
 */
int ep_cpu_dequant_matmul_f32(const float *x, int64_t x_len, const uint8_t *packed, int64_t n,
                              int64_t row_bytes, const float *scales, int64_t n_groups,
                              const float *cb, int64_t levels, int64_t group, int four_bit,
                              float *out, int nthreads)
{
    if (x_len < 0 || n < 0 || row_bytes < 0 || n_groups < 0 || levels < 0 || group <= 0)
        return -3;
    if (levels > 256)
        return -1;
    const int64_t k = four_bit ? row_bytes * 2 : row_bytes;
    const int64_t m = k > 0 ? x_len / k : 0;
    if (m == 0 || n == 0)
        return 0;
    if ((k + group - 1) / group > n_groups)
        return -2;
    if (!x || !packed || !scales || (levels > 0 && !cb) || !out)
        return -3;

    int nt = nthreads > 0 ? nthreads : (int)ep_cpu_threads();
    const int64_t blocks = (n + EP_CPU_ROWS - 1) / EP_CPU_ROWS;
    if (nt > blocks)
        nt = (int)blocks;
    if (nt < 1)
        nt = 1;

    const Job base = {x, m, k, packed, n, row_bytes, scales, n_groups, cb, levels, group,
                      four_bit, out, 0, 0};
    Job *jobs = (Job *)malloc(sizeof(Job) * (size_t)nt);
    pthread_t *tids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nt);
    if (!jobs || !tids) {
        free(jobs);
        free(tids);
        return -4;
    }
    for (int t = 0; t < nt; ++t) {
        jobs[t] = base;
        jobs[t].row0 = blocks * t / nt * EP_CPU_ROWS;
        jobs[t].row1 = blocks * (t + 1) / nt * EP_CPU_ROWS;
        if (jobs[t].row1 > n)
            jobs[t].row1 = n;
    }
    int started = 0;
    for (int t = 1; t < nt; ++t) {
        if (pthread_create(&tids[t], NULL, run_job, &jobs[t]) != 0)
            break;
        ++started;
    }
    run_job(&jobs[0]);
    for (int t = started + 1; t < nt; ++t)
        run_job(&jobs[t]);
    for (int t = 1; t <= started; ++t)
        pthread_join(tids[t], NULL);
    free(jobs);
    free(tids);
    return 0;
}
