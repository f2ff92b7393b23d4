/*
 * synth.c -- seeded synthetic I2_S workloads (libsllm_synth.so).
 *
 * The reference has no public weights in this image, so every workload is
 * synthetic, generated on the host so that the CPU and GPU see identical
 * bytes:
 *
 *   - ternary codes i.i.d. uniform over {0,1,2} (ternary -1/0/+1, p = 1/3),
 *     packed in the I2_S transposed tile layout (src/quant.c:72-100): element
 *     k of row r goes to byte r*K/4 + (k/128)*32 + k%32 at shift
 *     6 - 2*((k%128)/32); the 32-byte tail holds the f32 scale then zeros
 *     (src/quant.c:102-106, src/gguf.c:268-282);
 *   - one per-tensor scale w_scale = 0.5 + 1.5*u, u uniform on [0,1);
 *   - activations ~ N(0,1) by Box-Muller in double, rounded to f32.
 *
 * Random numbers are SplitMix64 outputs indexed by position (output i of a
 * stream seeded s is mix(s + (i+1)*0x9E3779B97F4A7C15)), so any slice can be
 * generated independently and the work splits across threads without
 * changing a single byte.
 */
#define _POSIX_C_SOURCE 200809L

#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ull
#define SCALE_SALT 0x5CA1E5CA1E5CA1E5ull

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* output i (0-based) of the SplitMix64 stream seeded `seed` */
static inline uint64_t splitmix_at(uint64_t seed, uint64_t i) {
    return mix64(seed + (i + 1) * GOLDEN);
}

/* code of element idx = r*K + k of tensor `seed` */
static inline unsigned code_at(uint64_t seed, uint64_t idx) {
    return (unsigned) ((splitmix_at(seed, idx) >> 32) % 3u);
}

uint64_t sllm_synth_seed(unsigned cfg, unsigned set, unsigned layer, unsigned matrix) {
    return 0x5A9F1A00ull ^ ((uint64_t) cfg << 40) ^ ((uint64_t) set << 24) ^
           ((uint64_t) layer << 8) ^ (uint64_t) matrix;
}

float sllm_synth_scale(uint64_t seed) {
    const double u = (double) (splitmix_at(seed ^ SCALE_SALT, 0) >> 40) * 0x1p-24;
    return (float) (0.5 + 1.5 * u);
}

/* unpacked codes, n_rows x n, row-major (for tests and small cases) */
void sllm_synth_codes(uint64_t seed, size_t n_rows, size_t n, uint8_t *codes) {
    for (size_t i = 0; i < n_rows * n; ++i) codes[i] = (uint8_t) code_at(seed, i);
}

typedef struct {
    uint64_t seed;
    size_t n, r0, r1;
    uint8_t *out;
} pack_job;

static void pack_rows(const pack_job *j) {
    const size_t row_bytes = j->n / 4;
    for (size_t r = j->r0; r < j->r1; ++r) {
        uint8_t *row = j->out + r * row_bytes;
        const uint64_t base = (uint64_t) r * j->n;
        for (size_t b = 0; b < j->n / 128; ++b) {
            for (unsigned l = 0; l < 32; ++l) {
                unsigned byte = 0;
                for (unsigned f = 0; f < 4; ++f) {
                    byte |= code_at(j->seed, base + 128 * b + 32 * f + l) << (6 - 2 * f);
                }
                row[32 * b + l] = (uint8_t) byte;
            }
        }
    }
}

static void *pack_thread(void *arg) {
    pack_rows(arg);
    return NULL;
}

/*
 * Fill `packed` (n_rows*n/4 + 32 bytes) with tensor `seed`. n must be a
 * multiple of 128. Returns 0, or -1 on a bad argument.
 */
int sllm_synth_i2s(uint64_t seed, size_t n_rows, size_t n, uint8_t *packed, int threads) {
    if (packed == NULL || n == 0 || n % 128 != 0) return -1;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if ((size_t) threads > n_rows) threads = n_rows ? (int) n_rows : 1;
    pack_job jobs[64];
    pthread_t tid[64];
    int started[64] = { 0 };
    for (int t = 0; t < threads; ++t) {
        jobs[t] = (pack_job) { seed, n, n_rows * (size_t) t / (size_t) threads,
                               n_rows * (size_t) (t + 1) / (size_t) threads, packed };
        if (t > 0) started[t] = pthread_create(&tid[t], NULL, pack_thread, &jobs[t]) == 0;
    }
    pack_rows(&jobs[0]);
    for (int t = 1; t < threads; ++t) {
        if (started[t]) pthread_join(tid[t], NULL);
        else pack_rows(&jobs[t]);
    }
    uint8_t *tail = packed + n_rows * (n / 4);
    memset(tail, 0, 32);
    const float s = sllm_synth_scale(seed);
    memcpy(tail, &s, sizeof s);
    return 0;
}

/* count values ~ N(0,1), Box-Muller in double, one pair per two outputs */
void sllm_synth_normal(uint64_t seed, size_t count, float *out) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < count; i += 2) {
        const uint64_t a = splitmix_at(seed, i), b = splitmix_at(seed, i + 1);
        const double u1 = ((double) (a >> 11) + 1.0) * 0x1p-53;   /* (0, 1] */
        const double u2 = (double) (b >> 11) * 0x1p-53;           /* [0, 1) */
        const double rad = sqrt(-2.0 * log(u1));
        out[i] = (float) (rad * cos(two_pi * u2));
        if (i + 1 < count) out[i + 1] = (float) (rad * sin(two_pi * u2));
    }
}

/* IEEE binary32 -> binary16, round to nearest even (overflow to infinity,
 * gradual underflow to subnormals) */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t) (sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t) (sign | 0x7C00u);          /* >= 65520: infinity */
    if (ax < 0x38800000u) {                                               /* below 2^-14: subnormal */
        float a;
        memcpy(&a, &ax, sizeof a);
        return (uint16_t) (sign | (uint32_t) nearbyintf(a * 0x1p24f));   /* exact scaling, RNE */
    }
    uint32_t h = ((ax >> 23) - 112u) << 10 | ((ax >> 13) & 0x3FFu);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;           /* may carry into the exponent */
    return (uint16_t) (sign | h);
}

typedef struct {
    uint64_t seed;
    size_t i0, i1;
    uint16_t *out;
} f16_job;

static void normal_f16_range(const f16_job *j) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = j->i0; i < j->i1; i += 2) {
        const uint64_t a = splitmix_at(j->seed, i), b = splitmix_at(j->seed, i + 1);
        const double u1 = ((double) (a >> 11) + 1.0) * 0x1p-53;
        const double u2 = (double) (b >> 11) * 0x1p-53;
        const double rad = sqrt(-2.0 * log(u1));
        j->out[i] = f32_to_f16((float) (rad * cos(two_pi * u2)));
        if (i + 1 < j->i1) j->out[i + 1] = f32_to_f16((float) (rad * sin(two_pi * u2)));
    }
}

static void *f16_thread(void *arg) {
    normal_f16_range(arg);
    return NULL;
}

/* The values of sllm_synth_normal(seed, count, .) rounded to binary16 (round
 * to nearest even), split over threads on even indices. */
void sllm_synth_normal_f16(uint64_t seed, size_t count, uint16_t *out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    f16_job jobs[64];
    pthread_t tid[64];
    int started[64] = { 0 };
    const size_t pairs = (count + 1) / 2;
    for (int t = 0; t < threads; ++t) {
        size_t i0 = 2 * (pairs * (size_t) t / (size_t) threads);
        size_t i1 = 2 * (pairs * (size_t) (t + 1) / (size_t) threads);
        if (i1 > count) i1 = count;
        jobs[t] = (f16_job) { seed, i0, i1, out };
        if (t > 0) started[t] = pthread_create(&tid[t], NULL, f16_thread, &jobs[t]) == 0;
    }
    normal_f16_range(&jobs[0]);
    for (int t = 1; t < threads; ++t) {
        if (started[t]) pthread_join(tid[t], NULL);
        else normal_f16_range(&jobs[t]);
    }
}
