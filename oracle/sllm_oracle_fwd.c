/*
 * sllm_oracle_fwd.c -- CPU restatement of saphira-llm's decode step.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT (see sllm_oracle.h). Built like the rest
 * of the oracle: -O2 -std=c11 -march=x86-64-v3 -ffp-contract=off, the
 * reference's arithmetic contract (Makefile:34-41). The float operations are
 * written out one lane at a time in the order the reference's AVX2 code
 * performs them, so every result carries the same bits; explicit fmaf()
 * stands where the reference calls an FMA intrinsic, and nothing else fuses.
 *
 * Pinning (tests/test_oracle_fwd.py): each op against the reference's own
 * src/ops.c compiled into oracle/_ref, bit for bit, on random and edge inputs;
 * the whole token against the reference's own sllm_forward (src/forward.c,
 * src/gguf.c in oracle/_ref) on synthetic GGUF models, logits bit for bit.
 */
#define _POSIX_C_SOURCE 200809L

#include "sllm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float f_from(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 -> binary32, exact (src/quant.c:24-45; the lm_head's
 * _mm256_cvtph_ps in src/ops.c:106-154 converts the same way) */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1Fu) return f_from(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return f_from(sign);
        /* subnormal: normalise */
        int e = -1;
        do { ++e; man <<= 1; } while ((man & 0x400u) == 0);
        return f_from(sign | ((uint32_t) (112 - e) << 23) | ((man & 0x3FFu) << 13));
    }
    return f_from(sign | ((exp + 112u) << 23) | (man << 13));
}

/* The token-embedding lookup's own conversion (src/forward.c:239-262, used at
 * :624). It agrees with IEEE for zeros, normals, infinities and NaNs, but
 * rebuilds a subnormal with an exponent field one lower than the value
 * needs (112 - shifts where 113 - shifts is exact), so every binary16
 * subnormal enters the residual stream at exactly half its value. The
 * decode step reproduces that, since the logits follow from it. */
float orc_f16_to_f32_embd(uint16_t h) {
    const float f = orc_f16_to_f32(h);
    if ((h & 0x7C00u) != 0 || (h & 0x3FFu) == 0) return f;
    return f_from(f_bits(f) - (1u << 23));
}

/* ------------------------------------------------------------------ */
/* RMSNorm: src/ops.c:254-322                                           */
/* ------------------------------------------------------------------ */

/* Squares in f32, widened to double into four lanes -- lane k takes the
 * square of x[8i+k], then of x[8i+4+k] -- the lanes folded 0..3, a scalar
 * tail, the mean narrowed to f32, scale = 1/sqrtf(mean + eps), dst = scale *
 * x, then dst * weight. dst may alias x. */
void orc_rms_norm(float *dst, const float *x, const float *weight, size_t n, float eps) {
    double lane[4] = { 0.0, 0.0, 0.0, 0.0 };
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        float sq[8];
        for (int j = 0; j < 8; ++j) sq[j] = x[i + j] * x[i + j];
        for (int k = 0; k < 4; ++k) lane[k] += (double) sq[k];
        for (int k = 0; k < 4; ++k) lane[k] += (double) sq[k + 4];
    }
    double ss = 0.0;
    for (int k = 0; k < 4; ++k) ss += lane[k];
    for (; i < n; ++i) ss += (double) x[i] * (double) x[i];
    const float mean = (float) (ss / (double) n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (size_t j = 0; j < n; ++j) dst[j] = scale * x[j];
    if (weight != NULL) {
        for (size_t j = 0; j < n; ++j) dst[j] = dst[j] * weight[j];
    }
}

/* ------------------------------------------------------------------ */
/* ggml_v_expf, one lane: src/ops.c:342-379                             */
/* ------------------------------------------------------------------ */

/* The lane's value does not depend on its neighbours: the vector code's
 * early exit (no lane out of range) returns fma(j, k, k), which is what the
 * full blend gives such a lane too. */
float orc_v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = f_bits(z) << 23;
    const float k = f_from(e + f_bits(1.0f));
    const int c = fabsf(n) > 126.0f;
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                              fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                         u, 0x1.ffffecp-1f * b);
    if (!c) return fmaf(j, k, k);
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = f_from(g + 0x7f000000u);
    const float s2 = f_from(e - g);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

/* ------------------------------------------------------------------ */
/* softmax and SiLU: src/ops.c:386-440                                  */
/* ------------------------------------------------------------------ */

void orc_softmax(float *x, size_t n) {
    if (n == 0) return;
    float max = x[0];
    for (size_t i = 1; i < n; ++i) {
        if (x[i] > max) max = x[i];
    }
    double sum = 0.0;
    size_t i = 0;
    for (; i + 7 < n; i += 8) {
        float v[8];
        for (int j = 0; j < 8; ++j) {
            v[j] = orc_v_expf(x[i + j] - max);
            x[i + j] = v[j];
        }
        double t[4];
        for (int j = 0; j < 4; ++j) t[j] = (double) v[j] + (double) v[j + 4];
        sum += t[0] + t[1] + t[2] + t[3];
    }
    for (; i < n; ++i) {
        const float e = expf(x[i] - max);     /* the scalar tail is libm's expf */
        x[i] = e;
        sum += (double) e;
    }
    const float inv = (float) (1.0 / sum);
    for (size_t j = 0; j < n; ++j) x[j] *= inv;
}

void orc_silu(float *x, size_t n) {
    size_t i = 0;
    for (; i + 7 < n; i += 8) {
        for (int j = 0; j < 8; ++j) {
            const float v = x[i + j];
            const float e = orc_v_expf(0.0f - v);
            x[i + j] = v / (1.0f + e);
        }
    }
    for (; i < n; ++i) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* ------------------------------------------------------------------ */
/* RoPE, NeoX pairing: src/ops.c:467-549                                */
/* ------------------------------------------------------------------ */

/* cos / sin of pair k at `pos`: the angle built by repeated f32
 * multiplication from (float) pos, libm powf / cosf / sinf. */
void orc_rope_cos_sin(size_t n_rot, int32_t pos, float theta, float freq_scale, float *cs, float *sn) {
    if (n_rot % 2 != 0) n_rot -= 1;
    const size_t half = n_rot / 2;
    const float theta_scale = powf(theta, -2.0f / (float) n_rot);
    float theta_k = (float) pos;
    for (size_t k = 0; k < half; ++k) {
        const float f = freq_scale * theta_k;
        cs[k] = cosf(f);
        sn[k] = sinf(f);
        theta_k *= theta_scale;
    }
}

void orc_rope_neox(float *x, size_t n_rot, int32_t pos, float theta, float freq_scale) {
    if (n_rot < 2) return;
    if (n_rot % 2 != 0) n_rot -= 1;
    const size_t half = n_rot / 2;
    const float theta_scale = powf(theta, -2.0f / (float) n_rot);
    float theta_k = (float) pos;
    for (size_t k = 0; k < half; ++k) {
        const float f = freq_scale * theta_k;
        const float c = cosf(f);
        const float s = sinf(f);
        theta_k *= theta_scale;
        const float xa = x[k], xb = x[k + half];
        x[k] = xa * c - xb * s;
        x[k + half] = xa * s + xb * c;
    }
}

/* ------------------------------------------------------------------ */
/* F16 row . f32 vector: src/ops.c:106-154                              */
/* ------------------------------------------------------------------ */

/* Four accumulators of eight lanes: element d + 8j + l of each 32-element
 * step goes into acc[j][l] with an FMA; then acc0 += acc2, acc1 += acc3,
 * acc0 += acc1; lanes l and l+4 added; then (t0 + t1) + (t2 + t3); then a
 * scalar tail (multiply, add). */
float orc_dot_f16(const uint16_t *row, const float *x, size_t n) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    size_t d = 0;
    if (n >= 32) {
        const size_t np = n & ~(size_t) 31;
        for (; d < np; d += 32) {
            for (int j = 0; j < 4; ++j) {
                for (int l = 0; l < 8; ++l) {
                    const size_t k = d + 8 * (size_t) j + (size_t) l;
                    acc[j][l] = fmaf(orc_f16_to_f32(row[k]), x[k], acc[j][l]);
                }
            }
        }
    }
    for (int off = 2; off >= 1; off >>= 1) {
        for (int i = 0; i < off; ++i) {
            for (int l = 0; l < 8; ++l) acc[i][l] = acc[i][l] + acc[off + i][l];
        }
    }
    float t0[4];
    for (int l = 0; l < 4; ++l) t0[l] = acc[0][l] + acc[0][l + 4];
    const float h01 = t0[0] + t0[1], h23 = t0[2] + t0[3];
    float s = h01 + h23;
    for (; d < n; ++d) s += orc_f16_to_f32(row[d]) * x[d];
    return s;
}

/* src/forward.c:876-883: first strictly greater value wins */
int32_t orc_argmax(const float *logits, int32_t n) {
    int32_t best = 0;
    float bv = logits[0];
    for (int32_t i = 1; i < n; ++i) {
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    }
    return best;
}

/* ------------------------------------------------------------------ */
/* one decode token: src/forward.c:589-835 with n = 1                   */
/* ------------------------------------------------------------------ */

struct orc_ctx {
    int32_t n_ctx;
    size_t  kv_per_layer;
    float  *k_cache, *v_cache;     /* [layer][head_kv][pos][head_dim] */
    float  *x, *xn, *ffn_inp, *cq, *ck, *cv, *cattn, *cproj, *g, *u, *h, *scores;
    int8_t *q;
    int32_t *dots;
};

static size_t big_of(const orc_model *m) { return (size_t) (m->n_embd > m->n_ff ? m->n_embd : m->n_ff); }

orc_ctx *orc_ctx_new(const orc_model *m, int32_t n_ctx) {
    orc_ctx *c = calloc(1, sizeof *c);
    if (c == NULL) return NULL;
    const size_t hd = (size_t) (m->n_embd / m->n_head);
    const size_t gqa = hd * (size_t) m->n_head_kv;
    c->n_ctx = n_ctx;
    c->kv_per_layer = (size_t) m->n_head_kv * (size_t) n_ctx * hd;
    c->k_cache = calloc(c->kv_per_layer * (size_t) m->n_layer, sizeof(float));
    c->v_cache = calloc(c->kv_per_layer * (size_t) m->n_layer, sizeof(float));
    const size_t e = (size_t) m->n_embd, f = (size_t) m->n_ff;
    c->x = malloc(e * 4); c->xn = malloc(e * 4); c->ffn_inp = malloc(e * 4);
    c->cq = malloc(e * 4); c->ck = malloc(gqa * 4); c->cv = malloc(gqa * 4);
    c->cattn = malloc(e * 4); c->cproj = malloc(e * 4);
    c->g = malloc(f * 4); c->u = malloc(f * 4); c->h = malloc(f * 4);
    c->scores = malloc((size_t) n_ctx * 4);
    c->q = malloc(big_of(m));
    c->dots = malloc(big_of(m) * 4);
    if (!c->k_cache || !c->v_cache || !c->x || !c->xn || !c->ffn_inp || !c->cq || !c->ck || !c->cv ||
        !c->cattn || !c->cproj || !c->g || !c->u || !c->h || !c->scores || !c->q || !c->dots) {
        orc_ctx_free(c);
        return NULL;
    }
    return c;
}

void orc_ctx_free(orc_ctx *c) {
    if (c == NULL) return;
    free(c->k_cache); free(c->v_cache);
    free(c->x); free(c->xn); free(c->ffn_inp); free(c->cq); free(c->ck); free(c->cv);
    free(c->cattn); free(c->cproj); free(c->g); free(c->u); free(c->h); free(c->scores);
    free(c->q); free(c->dots);
    free(c);
}

float *orc_ctx_k_cache(orc_ctx *c) { return c->k_cache; }
float *orc_ctx_v_cache(orc_ctx *c) { return c->v_cache; }

/* One projection as src/forward.c:651-655 runs it, with the activation
 * already quantised: GEMV, then (float)(dot - sum) * (w_scale / act_scale).
 * The raw dots are appended to *trace when it is not NULL. */
static void project(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q, const orc_act *act,
                    int32_t *dots, float *out, int32_t **trace) {
    orc_gemv(w, n_rows, n, q, dots, ORC_DOT_V3);
    const float post = orc_scale(w, n_rows * n) / act->scale;
    for (size_t r = 0; r < n_rows; ++r) out[r] = ((float) (dots[r] - act->sum)) * post;
    if (trace != NULL && *trace != NULL) {
        memcpy(*trace, dots, n_rows * sizeof(int32_t));
        *trace += n_rows;
    }
}

static void quant(const float *x, size_t n, int8_t *q, orc_act *act, orc_act **acts) {
    orc_quant_act(x, n, q, act);
    if (acts != NULL && *acts != NULL) *(*acts)++ = *act;
}

typedef struct lm_job {
    const uint16_t *embd;
    const float *xn;
    float *out;
    size_t n_embd, begin, end;
} lm_job;

static void *lm_rows(void *arg) {
    const lm_job *j = arg;
    for (size_t v = j->begin; v < j->end; ++v) j->out[v] = orc_dot_f16(j->embd + v * j->n_embd, j->xn, j->n_embd);
    return NULL;
}

int orc_forward_token(const orc_model *m, orc_ctx *c, int32_t token, int32_t pos, float *logits,
                      int lm_threads, int32_t *dots_trace, orc_act *act_trace) {
    if (token < 0 || token >= m->n_vocab || pos < 0 || pos >= c->n_ctx) return -1;
    const size_t n_embd = (size_t) m->n_embd, n_ff = (size_t) m->n_ff;
    const size_t hd = n_embd / (size_t) m->n_head;
    const size_t hkv = (size_t) m->n_head_kv, gqa = hd * hkv;
    const size_t grp = (size_t) (m->n_head / m->n_head_kv);
    const float attn_scale = 1.0f / sqrtf((float) hd);
    int32_t *trace = dots_trace;
    orc_act *acts = act_trace;
    orc_act act;

    for (size_t d = 0; d < n_embd; ++d) c->x[d] = orc_f16_to_f32_embd(m->tok_embd[(size_t) token * n_embd + d]);

    for (int32_t il = 0; il < m->n_layer; ++il) {
        const orc_layer *L = &m->layers[il];
        orc_rms_norm(c->xn, c->x, L->attn_norm, n_embd, m->eps);
        /* Q, K, V share one quantised activation */
        quant(c->xn, n_embd, c->q, &act, &acts);
        project(L->wq, n_embd, n_embd, c->q, &act, c->dots, c->cq, &trace);
        project(L->wk, gqa, n_embd, c->q, &act, c->dots, c->ck, &trace);
        project(L->wv, gqa, n_embd, c->q, &act, c->dots, c->cv, &trace);
        for (int32_t h = 0; h < m->n_head; ++h) orc_rope_neox(c->cq + (size_t) h * hd, (size_t) m->n_rot, pos, m->rope_base, 1.0f);
        for (size_t h = 0; h < hkv; ++h) orc_rope_neox(c->ck + h * hd, (size_t) m->n_rot, pos, m->rope_base, 1.0f);
        float *kbase = c->k_cache + (size_t) il * c->kv_per_layer;
        float *vbase = c->v_cache + (size_t) il * c->kv_per_layer;
        for (size_t h = 0; h < hkv; ++h) {
            memcpy(kbase + (h * (size_t) c->n_ctx + (size_t) pos) * hd, c->ck + h * hd, hd * sizeof(float));
            memcpy(vbase + (h * (size_t) c->n_ctx + (size_t) pos) * hd, c->cv + h * hd, hd * sizeof(float));
        }
        const size_t npast = (size_t) pos + 1;
        for (int32_t h = 0; h < m->n_head; ++h) {
            const size_t kvh = (size_t) h / grp;
            const float *qh = c->cq + (size_t) h * hd;
            const float *kc = kbase + kvh * (size_t) c->n_ctx * hd;
            const float *vc = vbase + kvh * (size_t) c->n_ctx * hd;
            for (size_t s = 0; s < npast; ++s) {
                float acc = 0.0f;
                for (size_t d = 0; d < hd; ++d) acc += qh[d] * kc[s * hd + d];
                c->scores[s] = acc * attn_scale;
            }
            orc_softmax(c->scores, npast);
            float *oh = c->cattn + (size_t) h * hd;
            for (size_t d = 0; d < hd; ++d) oh[d] = 0.0f;
            for (size_t s = 0; s < npast; ++s) {
                const float w = c->scores[s];
                for (size_t d = 0; d < hd; ++d) oh[d] += w * vc[s * hd + d];
            }
        }
        orc_rms_norm(c->xn, c->cattn, L->attn_sub_norm, n_embd, m->eps);
        quant(c->xn, n_embd, c->q, &act, &acts);
        project(L->wo, n_embd, n_embd, c->q, &act, c->dots, c->cproj, &trace);
        for (size_t d = 0; d < n_embd; ++d) c->ffn_inp[d] = c->cproj[d] + c->x[d];
        orc_rms_norm(c->xn, c->ffn_inp, L->ffn_norm, n_embd, m->eps);
        /* gate and up share one quantised activation */
        quant(c->xn, n_embd, c->q, &act, &acts);
        project(L->w_gate, n_ff, n_embd, c->q, &act, c->dots, c->g, &trace);
        project(L->w_up, n_ff, n_embd, c->q, &act, c->dots, c->u, &trace);
        orc_silu(c->g, n_ff);
        for (size_t r = 0; r < n_ff; ++r) c->h[r] = c->g[r] * c->u[r];
        orc_rms_norm(c->h, c->h, L->ffn_sub_norm, n_ff, m->eps);
        quant(c->h, n_ff, c->q, &act, &acts);
        project(L->w_down, n_embd, n_ff, c->q, &act, c->dots, c->cproj, &trace);
        for (size_t d = 0; d < n_embd; ++d) c->x[d] = c->cproj[d] + c->ffn_inp[d];
    }

    orc_rms_norm(c->xn, c->x, m->output_norm, n_embd, m->eps);
    const size_t nv = (size_t) m->n_vocab;
    /* rows are independent, so splitting them over threads changes no bit */
    const int nt = lm_threads < 1 ? 1 : (lm_threads > 64 ? 64 : lm_threads);
    pthread_t tid[64];
    int created[64] = { 0 };
    lm_job jobs[64];
    for (int t = 0; t < nt; ++t) {
        jobs[t] = (lm_job) { m->tok_embd, c->xn, logits, n_embd, nv * (size_t) t / (size_t) nt,
                             nv * (size_t) (t + 1) / (size_t) nt };
    }
    for (int t = 1; t < nt; ++t) created[t] = pthread_create(&tid[t], NULL, lm_rows, &jobs[t]) == 0;
    lm_rows(&jobs[0]);
    for (int t = 1; t < nt; ++t) {
        if (created[t]) pthread_join(tid[t], NULL);
        else lm_rows(&jobs[t]);
    }
    return 0;
}
