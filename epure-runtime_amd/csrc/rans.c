/*
 * Chunked rANS decode of .ebin index streams (part of libepure_cpu.so).
 *
 * The reference decodes each chunk with the `constriction` library
 * (epure/container.py:28-51: stream.stack.AnsCoder over u32 words,
 * stream.model.Categorical built from the stored symbol counts).  That
 * library is not available to this build, so this is a restatement of its
 * published stack-ANS algorithm:
 *
 *   coder state: 64 bits; compressed data: a stack of 32-bit words; model:
 *   a categorical distribution quantized to PRECISION = 24 bits, given as
 *   its left-sided cumulative table cdf[0..n] (cdf[0] = 0, cdf[n] = 2^24,
 *   every symbol a nonzero probability).
 *   start:  the state is popped from the top of the stack: the last word is
 *           the state's high half, the word below it its low half (a stack
 *           holding one word gives a state of that word).
 *   decode: q = state mod 2^24; find s with cdf[s] <= q < cdf[s + 1];
 *           state = (state >> 24) * (cdf[s + 1] - cdf[s]) + (q - cdf[s]);
 *           then, while the state's high half is 0 and words remain, shift
 *           the next popped word into its low half.
 *
 * Chunks are independent coders, so they are decoded in parallel.  Parity
 * with constriction's own output is unpinned (no .ebin fixture exists to
 * check against); the tests pin the decoder against an encoder that
 * inverts exactly these steps.
 */
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#include "../../include/epure_cpu.h"

#define RANS_PRECISION 24

typedef struct {
    const uint32_t *words;
    const int64_t *word_off, *nwords, *sym_off, *nsym;
    int nchunks;
    const uint32_t *cdf;
    int nlevels;
    uint8_t *out;
    int t, nt;
    int err;
} RansJob;

static int find_symbol(const uint32_t *cdf, int n, uint32_t q)
{
    int lo = 0, hi = n;  /* cdf[lo] <= q < cdf[hi] */
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cdf[mid] <= q)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

static int decode_chunk(const uint32_t *w, int64_t nw, int64_t nsym, const uint32_t *cdf, int n,
                        uint8_t *out)
{
    int64_t top = nw;  /* words [0, top) remain on the stack */
    uint64_t state = 0;
    if (top > 0)
        state = w[--top];
    if (top > 0)
        state = (state << 32) | w[--top];
    const uint32_t mask = (1u << RANS_PRECISION) - 1u;
    for (int64_t i = 0; i < nsym; ++i) {
        const uint32_t q = (uint32_t)(state & mask);
        const int s = find_symbol(cdf, n, q);
        const uint64_t p = (uint64_t)(cdf[s + 1] - cdf[s]);
        state = (state >> RANS_PRECISION) * p + (uint64_t)(q - cdf[s]);
        while ((state >> 32) == 0 && top > 0)
            state = (state << 32) | w[--top];
        out[i] = (uint8_t)s;
    }
    return 0;
}

static void *run_rans(void *arg)
{
    RansJob *j = (RansJob *)arg;
    for (int c = j->t; c < j->nchunks; c += j->nt)
        decode_chunk(j->words + j->word_off[c], j->nwords[c], j->nsym[c], j->cdf, j->nlevels,
                     j->out + j->sym_off[c]);
    return NULL;
}

int ep_rans_decode(const uint32_t *words, const int64_t *chunk_words, const int64_t *chunk_symbols,
                   int nchunks, const uint32_t *cdf, int nlevels, uint8_t *out, int nthreads)
{
    if (nchunks < 0 || nlevels < 1 || nlevels > 256 || !cdf || (nchunks > 0 && (!chunk_words ||
                                                                                 !chunk_symbols)))
        return -3;
    if (cdf[0] != 0 || cdf[nlevels] != (1u << RANS_PRECISION))
        return -5;
    for (int s = 0; s < nlevels; ++s)
        if (cdf[s + 1] <= cdf[s])
            return -5;  /* every symbol needs a nonzero probability */
    int64_t *offs = (int64_t *)malloc(sizeof(int64_t) * 2 * (size_t)(nchunks + 1));
    if (!offs)
        return -4;
    int64_t *word_off = offs, *sym_off = offs + nchunks + 1;
    word_off[0] = sym_off[0] = 0;
    for (int c = 0; c < nchunks; ++c) {
        if (chunk_words[c] < 0 || chunk_symbols[c] < 0) {
            free(offs);
            return -3;
        }
        word_off[c + 1] = word_off[c] + chunk_words[c];
        sym_off[c + 1] = sym_off[c] + chunk_symbols[c];
    }
    if ((word_off[nchunks] > 0 && !words) || (sym_off[nchunks] > 0 && !out)) {
        free(offs);
        return -3;
    }
    int nt = nthreads > 0 ? nthreads : (int)ep_cpu_threads();
    if (nt > nchunks)
        nt = nchunks;
    if (nt < 1)
        nt = 1;
    RansJob *jobs = (RansJob *)malloc(sizeof(RansJob) * (size_t)nt);
    pthread_t *tids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nt);
    if (!jobs || !tids) {
        free(jobs);
        free(tids);
        free(offs);
        return -4;
    }
    for (int t = 0; t < nt; ++t)
        jobs[t] = (RansJob){words, word_off, chunk_words, sym_off, chunk_symbols, nchunks, cdf,
                            nlevels, out, t, nt, 0};
    int started = 0;
    for (int t = 1; t < nt; ++t) {
        if (pthread_create(&tids[t], NULL, run_rans, &jobs[t]) != 0)
            break;
        ++started;
    }
    run_rans(&jobs[0]);
    for (int t = started + 1; t < nt; ++t)
        run_rans(&jobs[t]);
    for (int t = 1; t <= started; ++t)
        pthread_join(tids[t], NULL);
    free(jobs);
    free(tids);
    free(offs);
    return 0;
}
