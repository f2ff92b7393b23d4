/*
 * expf_check.c -- pins the decode kernels' expf restatement (csrc/libm_expf.h)
 * against the host C library: the count of float inputs in a range of bit
 * patterns whose results differ in any bit (NaN against NaN counts as
 * equal). Host only; built into libsllm_synth.so for the tests.
 */
#define _POSIX_C_SOURCE 200809L

#include "../csrc/libm_expf.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

static const uint64_t k_tab[32] = SLLM_EXPF_TAB_INIT;

typedef struct span {
    uint64_t lo, hi, bad;
    uint32_t first;
} span;

static void *check_span(void *arg) {
    span *s = arg;
    s->bad = 0;
    s->first = 0;
    for (uint64_t u = s->lo; u < s->hi; ++u) {
        const uint32_t b = (uint32_t) u;
        float x;
        memcpy(&x, &b, 4);
        const float want = expf(x), got = sllm_libm_expf(x, k_tab);
        uint32_t bw, bg;
        memcpy(&bw, &want, 4);
        memcpy(&bg, &got, 4);
        if (bw != bg && !(want != want && got != got)) {
            if (s->bad == 0) s->first = b;
            s->bad++;
        }
    }
    return NULL;
}

/* mismatches over bit patterns [lo, hi) (hi <= 2^32), split over `threads`;
 * *first (if not NULL) receives the lowest mismatching pattern found by the
 * first thread that found one */
uint64_t sllm_expf_mismatches(uint64_t lo, uint64_t hi, int threads, uint32_t *first) {
    if (hi > (1ull << 32)) hi = 1ull << 32;
    if (lo >= hi) return 0;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    span sp[64];
    pthread_t tid[64];
    int made[64] = { 0 };
    for (int t = 0; t < threads; ++t) {
        sp[t].lo = lo + (hi - lo) * (uint64_t) t / (uint64_t) threads;
        sp[t].hi = lo + (hi - lo) * (uint64_t) (t + 1) / (uint64_t) threads;
        if (t > 0) made[t] = pthread_create(&tid[t], NULL, check_span, &sp[t]) == 0;
    }
    check_span(&sp[0]);
    uint64_t bad = 0;
    int have_first = 0;
    for (int t = 0; t < threads; ++t) {
        if (t > 0) {
            if (made[t]) pthread_join(tid[t], NULL);
            else check_span(&sp[t]);
        }
        bad += sp[t].bad;
        if (sp[t].bad && !have_first) {
            have_first = 1;
            if (first) *first = sp[t].first;
        }
    }
    return bad;
}

typedef struct strided {
    uint32_t first, stride;
    uint64_t lo, hi;
    float   *out;
} strided;

static void *expf_strided(void *arg) {
    strided *s = arg;
    for (uint64_t i = s->lo; i < s->hi; ++i) {
        const uint32_t b = s->first + (uint32_t) i * s->stride;
        float x;
        memcpy(&x, &b, 4);
        s->out[i] = expf(x);
    }
    return NULL;
}

/* the host C library's expf of the floats whose bit patterns are
 * first + i * stride (mod 2^32), i < n, into out, over `threads` threads:
 * the reference values for the device build's expf */
void sllm_expf_strided(uint32_t first, uint32_t stride, uint64_t n, float *out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    strided sp[64];
    pthread_t tid[64];
    int made[64] = { 0 };
    for (int t = 0; t < threads; ++t) {
        sp[t] = (strided) { first, stride, n * (uint64_t) t / (uint64_t) threads,
                            n * (uint64_t) (t + 1) / (uint64_t) threads, out };
        if (t > 0) made[t] = pthread_create(&tid[t], NULL, expf_strided, &sp[t]) == 0;
    }
    expf_strided(&sp[0]);
    for (int t = 1; t < threads; ++t) {
        if (made[t]) pthread_join(tid[t], NULL);
        else expf_strided(&sp[t]);
    }
}
