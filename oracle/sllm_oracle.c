/*
 * sllm_oracle.c -- CPU restatement of saphira-llm's I2_S ternary path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT: see sllm_oracle.h for who may use it and
 * how each function is pinned. Built -O2 -std=c11 -march=x86-64-v3
 * -ffp-contract=off, the reference's own arithmetic contract (Makefile:34-41).
 */
#define _POSIX_C_SOURCE 200809L

#include "sllm_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* activation quantiser: src/i2s_gemm.c:45-83                          */
/* ------------------------------------------------------------------ */

void orc_quant_act(const float *x, size_t n, int8_t *q, orc_act *act) {
    /* pass 1: absolute maximum, no epsilon floor (i2s_gemm.c:63-69) */
    float amax = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    /* reciprocal scale, 0 for an all-zero row (i2s_gemm.c:70) */
    const float s = amax > 0.0f ? 127.0f / amax : 0.0f;
    /* pass 2: round half away from zero, clamp, running sum (:73-82) */
    int32_t sum = 0;
    for (size_t i = 0; i < n; ++i) {
        int v = (int) roundf(x[i] * s);
        if (v > 127) v = 127;
        if (v < -128) v = -128;
        q[i] = (int8_t) v;
        sum += v;
    }
    act->scale = s;
    act->sum = sum;
}

void orc_quant_act_rows(const float *x, size_t n, size_t m, int8_t *q, orc_act *act) {
    for (size_t t = 0; t < m; ++t) {
        orc_quant_act(x + t * n, n, q + t * n, act + t);
    }
}

/* ------------------------------------------------------------------ */
/* dot products                                                        */
/* ------------------------------------------------------------------ */

/* src/i2s_gemm.c:89-112: element 32*field + lane of each 128-block lives in
 * byte `lane` of the block's 32 bytes, at bit shift 6 - 2*field. */
int32_t orc_dot_scalar(const uint8_t *w, const int8_t *q, size_t n) {
    int32_t acc = 0;
    for (size_t b = 0; b < n / ORC_I2S_QK; ++b) {
        const uint8_t *blk = w + 32 * b;
        const int8_t *qb = q + ORC_I2S_QK * b;
        for (unsigned lane = 0; lane < 32; ++lane) {
            for (unsigned f = 0; f < 4; ++f) {
                const int32_t c = (blk[lane] >> (6 - 2 * f)) & 3;
                acc += c * (int32_t) qb[32 * f + lane];
            }
        }
    }
    return acc;
}

static inline int32_t hadd8_epi32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_unpackhi_epi64(s, s));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

/* src/i2s_gemm.c:143-185: one 32-byte load gives the four code vectors of a
 * block; maddubs (codes unsigned x activations signed) into int16, the four
 * products summed in int16 (at most 4*2*254 in magnitude, exact), then madd
 * by one into int32. */
int32_t orc_dot_v3(const uint8_t *w, const int8_t *q, size_t n) {
    const __m256i m3 = _mm256_set1_epi8(3);
    const __m256i ones = _mm256_set1_epi16(1);
    __m256i acc = _mm256_setzero_si256();
    for (size_t b = 0; b < n / ORC_I2S_QK; ++b) {
        const __m256i p = _mm256_loadu_si256((const __m256i *) (w + 32 * b));
        const int8_t *qb = q + ORC_I2S_QK * b;
        __m256i s16 = _mm256_setzero_si256();
        for (int f = 0; f < 4; ++f) {
            const __m256i c = _mm256_and_si256(_mm256_srli_epi16(p, 6 - 2 * f), m3);
            const __m256i a = _mm256_loadu_si256((const __m256i *) (qb + 32 * f));
            s16 = _mm256_add_epi16(s16, _mm256_maddubs_epi16(c, a));
        }
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(s16, ones));
    }
    return hadd8_epi32(acc);
}

/* src/i2s_gemm.c:189-237: dpbusd straight into four int32 accumulators, one
 * per field, summed at the end. */
__attribute__((target("avx2,avxvnni")))
int32_t orc_dot_vnni(const uint8_t *w, const int8_t *q, size_t n) {
    const __m256i m3 = _mm256_set1_epi8(3);
    __m256i acc[4] = { _mm256_setzero_si256(), _mm256_setzero_si256(),
                       _mm256_setzero_si256(), _mm256_setzero_si256() };
    for (size_t b = 0; b < n / ORC_I2S_QK; ++b) {
        const __m256i p = _mm256_loadu_si256((const __m256i *) (w + 32 * b));
        const int8_t *qb = q + ORC_I2S_QK * b;
        for (int f = 0; f < 4; ++f) {
            const __m256i c = _mm256_and_si256(_mm256_srli_epi16(p, 6 - 2 * f), m3);
            const __m256i a = _mm256_loadu_si256((const __m256i *) (qb + 32 * f));
            acc[f] = _mm256_dpbusd_avx_epi32(acc[f], c, a);
        }
    }
    return hadd8_epi32(_mm256_add_epi32(_mm256_add_epi32(acc[0], acc[1]),
                                        _mm256_add_epi32(acc[2], acc[3])));
}

int orc_vnni_supported(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avxvnni") ? 1 : 0;
}

typedef int32_t (*orc_dot_fn)(const uint8_t *, const int8_t *, size_t);

static orc_dot_fn dot_for(int path) {
    if (path == ORC_DOT_VNNI && orc_vnni_supported()) return orc_dot_vnni;
    if (path == ORC_DOT_SCALAR) return orc_dot_scalar;
    return orc_dot_v3;
}

/* src/i2s_gemm.c:246-269. A NULL pointer or n < 128 gives dot 0 / no write,
 * as the reference does. */
void orc_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
              int32_t *rows_out, int path) {
    if (w == NULL || q == NULL || rows_out == NULL) return;
    const orc_dot_fn dot = dot_for(path);
    for (size_t r = 0; r < n_rows; ++r) {
        rows_out[r] = n < ORC_I2S_QK ? 0 : dot(w + r * (n / 4), q, n);
    }
}

/* src/i2s_gemm.c:271-290: one division per activation column, then a
 * subtraction and one multiply per element. */
float orc_epilogue(int32_t dot, int32_t act_sum, float act_scale, float w_scale) {
    const float post = w_scale / act_scale;
    return (float) (dot - act_sum) * post;
}

/* ------------------------------------------------------------------ */
/* format helpers: src/quant.c:72-146                                  */
/* ------------------------------------------------------------------ */

/* src/quant.c:77-100. Written in the per-4096-block form the reference uses:
 * block of 1024 bytes, 32 chunks of 32 bytes, four 2-bit fields per byte with
 * field 0 at the top. */
uint8_t orc_code(const uint8_t *packed, size_t k) {
    const size_t block = k / 4096, in = k % 4096;
    const size_t chunk = (in / 128) % 32;
    const unsigned field = (unsigned) ((in % 128) / 32);
    const uint8_t byte = packed[block * 1024 + chunk * 32 + in % 32];
    return (uint8_t) ((byte >> (6 - 2 * field)) & 3);
}

/* src/quant.c:102-106: the f32 scale at byte n_elements/4 */
float orc_scale(const void *packed, size_t n_elements) {
    float s;
    memcpy(&s, (const uint8_t *) packed + n_elements / 4, sizeof s);
    return s;
}

/* src/quant.c:126-146: code -> {-1, 0, +1, 0} times the scale */
void orc_dequant(const void *packed, float *dst, size_t n) {
    static const float map[4] = { -1.0f, 0.0f, 1.0f, 0.0f };
    const float s = orc_scale(packed, n);
    for (size_t k = 0; k < n; ++k) {
        dst[k] = s * map[orc_code((const uint8_t *) packed, k)];
    }
}

/* tests/harness.h:105-126: the converter reshapes each 128-block to (4, 32)
 * and ORs (q[a][b] << (6 - 2a)) into byte b. Independent of orc_code. */
void orc_pack_converter(uint8_t *dst, const uint8_t *codes, size_t n) {
    memset(dst, 0, n / 4 + 32);
    for (size_t blk = 0; blk * 128 < n; ++blk) {
        for (size_t j = 0; j < 128 && blk * 128 + j < n; ++j) {
            dst[blk * 32 + j % 32] |= (uint8_t) (codes[blk * 128 + j] << (6 - 2 * (j / 32)));
        }
    }
}

/* ------------------------------------------------------------------ */
/* one projection: src/forward.c:651-655                                */
/* ------------------------------------------------------------------ */

void orc_linear(const uint8_t *w, size_t n_rows, size_t n, const float *x,
                float *y, int8_t *q_out, int32_t *dots_out, orc_act *act_out,
                int path) {
    int8_t *q = q_out ? q_out : malloc(n);
    int32_t *d = dots_out ? dots_out : malloc(n_rows * sizeof(int32_t));
    orc_act act;
    orc_quant_act(x, n, q, &act);
    orc_gemv(w, n_rows, n, q, d, path);
    const float ws = orc_scale(w, n_rows * n);
    for (size_t r = 0; r < n_rows; ++r) {
        y[r] = orc_epilogue(d[r], act.sum, act.scale, ws);
    }
    if (act_out) *act_out = act;
    if (!q_out) free(q);
    if (!dots_out) free(d);
}

/* ------------------------------------------------------------------ */
/* row-parallel CPU timing path                                        */
/* ------------------------------------------------------------------ */

#define ORC_ROW_GRAIN 64u          /* src/forward.c:145-147 */
#define ORC_ROWS_PER_THREAD 512u   /* src/forward.c:171-173 */
#define ORC_CHUNKS_PER_THREAD 16u  /* src/thread.c:42 */

struct orc_pool {
    int total;                     /* workers + the calling thread */
    pthread_t *tid;
    pthread_mutex_t mtx;
    pthread_cond_t go, done;
    unsigned long gen;
    int pending;
    int quit;
    /* current region */
    const uint8_t *w;
    size_t row_bytes, n, n_rows, chunk;
    const int8_t *q;
    int32_t *out;
    orc_dot_fn dot;
    atomic_size_t cursor;
};

static void run_chunks(orc_pool *p) {
    for (;;) {
        const size_t b = atomic_fetch_add(&p->cursor, p->chunk);
        if (b >= p->n_rows) break;
        const size_t e = b + p->chunk < p->n_rows ? b + p->chunk : p->n_rows;
        for (size_t r = b; r < e; ++r) {
            p->out[r] = p->dot(p->w + r * p->row_bytes, p->q, p->n);
        }
    }
}

static void *worker(void *arg) {
    orc_pool *p = arg;
    unsigned long seen = 0;
    pthread_mutex_lock(&p->mtx);
    for (;;) {
        while (!p->quit && p->gen == seen) pthread_cond_wait(&p->go, &p->mtx);
        if (p->quit) break;
        seen = p->gen;
        pthread_mutex_unlock(&p->mtx);
        run_chunks(p);
        pthread_mutex_lock(&p->mtx);
        if (--p->pending == 0) pthread_cond_signal(&p->done);
    }
    pthread_mutex_unlock(&p->mtx);
    return NULL;
}

orc_pool *orc_pool_create(int threads) {
    orc_pool *p = calloc(1, sizeof *p);
    if (p == NULL) return NULL;
    p->total = threads < 1 ? 1 : threads;
    pthread_mutex_init(&p->mtx, NULL);
    pthread_cond_init(&p->go, NULL);
    pthread_cond_init(&p->done, NULL);
    p->tid = calloc((size_t) p->total, sizeof(pthread_t));
    int started = 1;
    for (int i = 1; i < p->total; ++i) {
        if (pthread_create(&p->tid[i], NULL, worker, p) != 0) break;
        ++started;
    }
    p->total = started;   /* degrade to what started, as src/thread.c:326-338 */
    return p;
}

int orc_pool_threads(const orc_pool *p) { return p ? p->total : 1; }

void orc_pool_destroy(orc_pool *p) {
    if (p == NULL) return;
    pthread_mutex_lock(&p->mtx);
    p->quit = 1;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mtx);
    for (int i = 1; i < p->total; ++i) pthread_join(p->tid[i], NULL);
    free(p->tid);
    pthread_cond_destroy(&p->go);
    pthread_cond_destroy(&p->done);
    pthread_mutex_destroy(&p->mtx);
    free(p);
}

/* src/forward.c:196-205 split policy over src/thread.c:389-465 chunking */
void orc_gemv_parallel(orc_pool *p, const uint8_t *w, size_t n_rows, size_t n,
                       const int8_t *q, int32_t *rows_out, int path) {
    const int t = orc_pool_threads(p);
    if (t < 2 || n_rows < (size_t) ORC_ROWS_PER_THREAD * (size_t) t ||
        n_rows < 2u * ORC_ROW_GRAIN) {
        orc_gemv(w, n_rows, n, q, rows_out, path);
        return;
    }
    size_t chunk = n_rows / ((size_t) t * ORC_CHUNKS_PER_THREAD);
    if (chunk < ORC_ROW_GRAIN) chunk = ORC_ROW_GRAIN;
    pthread_mutex_lock(&p->mtx);
    p->w = w; p->row_bytes = n / 4; p->n = n; p->n_rows = n_rows; p->chunk = chunk;
    p->q = q; p->out = rows_out; p->dot = dot_for(path);
    atomic_store(&p->cursor, 0);
    p->pending = t - 1;
    p->gen++;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mtx);
    run_chunks(p);   /* the caller works too */
    pthread_mutex_lock(&p->mtx);
    while (p->pending > 0) pthread_cond_wait(&p->done, &p->mtx);
    pthread_mutex_unlock(&p->mtx);
}

void orc_gemv_epilogue_parallel(orc_pool *p, const uint8_t *w, size_t n_rows, size_t n,
                                const int8_t *q, const orc_act *act, int32_t *dots, float *y,
                                int path) {
    orc_gemv_parallel(p, w, n_rows, n, q, dots, path);
    const float ws = orc_scale(w, n_rows * n);
    for (size_t r = 0; r < n_rows; ++r) y[r] = orc_epilogue(dots[r], act->sum, act->scale, ws);
}

uint64_t orc_fnv1a64(const void *data, size_t n) {
    const unsigned char *b = data;
    uint64_t h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; ++i) {
        h ^= b[i];
        h *= 1099511628211ULL;
    }
    return h;
}
