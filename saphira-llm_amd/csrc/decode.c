/*
 * decode.c -- the BitNet-b1.58 decode step on gfx950 (sllm_gfx950_decode.h).
 *
 * Host side of decode_kernels.hip: uploads a model, lays a context out in one
 * device allocation, and enqueues one token as a fixed sequence of launches
 * that read the token and position from a device-resident step record, so
 * the same sequence (or a HIP graph of it) serves every position and the
 * output kernel can feed the next token itself.
 *
 * Argument structs mirror decode_kernels.hip field for field (sizes asserted).
 */
#define _POSIX_C_SOURCE 200809L

#include "shim_internal.h"

#include <saphira_amd/sllm_gfx950_decode.h>

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* every entry point that reaches the device: -60 while the library is closed */
#define DEC_NEED_OPEN()                                                                  \
    do {                                                                                 \
        if (!sllm_shim_is_open()) return sllm_shim_fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open"); \
    } while (0)

/* ------------------------------------------------------------------ */
/* device-side layouts                                                 */
/* ------------------------------------------------------------------ */

typedef struct k_dec_step {
    int32_t        token, pos, next, advance;
    uint64_t       reserved0;
    uint32_t       reserved1, err;
    const int32_t *feed;
    int32_t       *gen;
    int32_t        n_feed, i_feed, n_gen, cap_gen;
} k_dec_step;

typedef struct k_dec_stage {
    const void       *a;
    const float      *b;
    float            *v_out;
    const float      *norm_w;
    const k_dec_step *step;
    int8_t           *q_out;
    sllm_gfx950_act  *act_out;
    float             eps;
    uint32_t          k, mode, pad;
} k_dec_stage;

typedef struct k_dec_attn {
    const float      *q, *k, *v;
    float            *k_cache, *v_cache;
    const float      *rope;
    float            *scores;
    float            *out;
    const k_dec_step *step;
    float             attn_scale;
    uint32_t          n_head, n_kv, hd, half, n_ctx, sc_stride;
    uint32_t          chunk_base;
    const uint8_t    *ahead;
    uint64_t          ahead_bytes;
} k_dec_attn;

typedef struct k_dec_lm {
    const float    *a, *b;
    const float    *norm_w;
    const uint16_t *embd;
    float          *logits;
    uint64_t       *partial;
    k_dec_step     *step;
    float           eps;
    uint32_t        n_embd, n_vocab, pad;
} k_dec_lm;

typedef struct k_chk_prep {
    const void      *a;
    const float     *b;
    const int32_t   *tokens;
    float           *v_out;
    const float     *norm_w;
    int8_t          *q_out;
    sllm_gfx950_act *act_out;
    float           *xn_out;
    float            eps;
    uint32_t         k, mode, pad;
} k_chk_prep;

typedef struct k_chk_lm {
    const float    *xn;
    const uint16_t *embd;
    float          *logits;
    uint32_t        n_embd, n_vocab, n_tok, n_wg;
} k_chk_lm;

/* one GEMV stage's kernel arguments (dec_gemv_args) */
typedef struct k_dec_gemv_args {
    k_dec_stage st;
    k_gemv_job  job[3];
    uint32_t    n_slabs[3];
    uint32_t    n_wg;
    uint32_t    pair;
    uint32_t    pad[3];
} k_dec_gemv_args;

_Static_assert(sizeof(k_dec_step) == 64, "k_dec_step must match dec_step");
_Static_assert(sizeof(k_dec_gemv_args) == 296, "k_dec_gemv_args must match dec_gemv_args");
_Static_assert(sizeof(k_dec_stage) == 72, "k_dec_stage must match dec_stage");
_Static_assert(sizeof(k_dec_attn) == 120, "k_dec_attn must match dec_attn");
_Static_assert(sizeof(k_dec_lm) == 72, "k_dec_lm must match dec_lm");
_Static_assert(sizeof(k_chk_prep) == 80, "k_chk_prep must match chk_prep");
_Static_assert(sizeof(k_chk_lm) == 40, "k_chk_lm must match chk_lm");

enum { IN_PLAIN = 0, IN_RESID = 1, IN_EMBED = 2, IN_SILU = 3 };

/* kernel constants (decode_kernels.hip) */
#define ATT_THREADS 256
#define PV_THREADS  512
#define PV_HPW      2
#define ATT_POS     64
#define PV_SLICE    8
#define LM_THREADS  256
#define LM_ROWS     32
#define LM_MAX_E    8192
#define LM_WG_PER_CU 2    /* output workgroups per CU (LDS: 32 KiB each); 2 ran 4 us per token faster than 4 */
#define CHK_THREADS  512
#define CLM_THREADS  256
#define CLM_TOK      4    /* tokens per chunk output-head workgroup */
#define CS_TOK       8    /* tokens per chunk scores workgroup (half that up to CS_SMALL tokens) */
#define CS_SMALL     128
#define CSW_THREADS  1024 /* the one-wave-unit scores kernel: sixteen waves per CU */
#define CSW_LDS_PAD  98304u   /* its (unused) LDS: more than half a CU's, one workgroup per CU */
#define CP_TOK       4    /* tokens per chunk p.V workgroup */
#define CP_THREADS   1024 /* threads per chunk p.V workgroup: sixteen waves, one workgroup per CU */
#define CSM_WAVES    4    /* waves per chunk softmax workgroup */
#define CSM_HALF     256  /* rows of at most this many positions take half a wave */
/* sllm_k_chk_kv_store stages a token's query row (n_head * hd = n_embd floats) in 7168 floats of LDS */
_Static_assert(SLLM_GFX950_DEC_MAX_WIDTH <= 7168, "query row of the chunk KV store");

/* projections of a block, in the reference's order (src/forward.c:642-793) */
enum { P_Q, P_K, P_V, P_O, P_GATE, P_UP, P_DOWN, N_PROJ };
/* GEMV stages of a block */
enum { S_QKV, S_O, S_FFN, S_DOWN, N_STAGE };

#define BOS_TOKEN 128000   /* src/forward.c:909 */

/* ------------------------------------------------------------------ */
/* model                                                               */
/* ------------------------------------------------------------------ */

typedef struct dev_layer {
    uint8_t *w[N_PROJ];
    float   *attn_norm, *attn_sub_norm, *ffn_norm, *ffn_sub_norm;
} dev_layer;

struct sllm_gfx950_model {
    int32_t    n_layer, n_embd, n_ff, n_head, n_head_kv, n_rot, n_vocab, hd, gqa;
    float      eps, rope_base;
    void      *blob;
    uint16_t  *tok_embd;
    float     *output_norm;
    dev_layer *layers;
};

static size_t align256(size_t v) { return (v + 255u) & ~(size_t) 255u; }
static size_t i2s_bytes(size_t rows, size_t k) { return rows * k / 4 + 32; }

/* (rows, K) of each projection */
static void proj_shape(const struct sllm_gfx950_model *m, int p, size_t *rows, size_t *k) {
    const size_t e = (size_t) m->n_embd, f = (size_t) m->n_ff, g = (size_t) m->gqa;
    static const int kind[N_PROJ] = { 0, 1, 1, 0, 2, 2, 3 };
    switch (kind[p]) {
    case 0:  *rows = e; *k = e; break;
    case 1:  *rows = g; *k = e; break;
    case 2:  *rows = f; *k = e; break;
    default: *rows = e; *k = f; break;
    }
}

static int check_desc(const sllm_gfx950_model_desc *d) {
    if (d->n_layer < 1 || d->n_embd < 1 || d->n_ff < 1 || d->n_head < 1 || d->n_head_kv < 1 ||
        d->n_vocab < 1 || d->n_rot < 0 || d->tok_embd == NULL || d->output_norm == NULL || d->layers == NULL) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "model: missing tensors or non-positive sizes");
    }
    for (int32_t il = 0; il < d->n_layer; ++il) {
        const sllm_gfx950_layer_desc *L = &d->layers[il];
        if (!L->wq || !L->wk || !L->wv || !L->wo || !L->w_gate || !L->w_up || !L->w_down ||
            !L->attn_norm || !L->attn_sub_norm || !L->ffn_norm || !L->ffn_sub_norm) {
            return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "model: layer %d lacks a tensor", il);
        }
    }
    /* need_i2s (src/forward.c:306-316): every I2_S width a multiple of 128 */
    if (d->n_embd % 128 || d->n_ff % 128) {
        return sllm_shim_fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "model: n_embd %d / n_ff %d not multiples of 128",
                              d->n_embd, d->n_ff);
    }
    if (d->n_embd % d->n_head || d->n_head % d->n_head_kv) {
        return sllm_shim_fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "model: heads do not divide n_embd / n_head");
    }
    const int32_t hd = d->n_embd / d->n_head, grp = d->n_head / d->n_head_kv;
    if (d->n_rot > hd) return sllm_shim_fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "model: n_rot %d > head dim %d", d->n_rot, hd);
    if (hd > SLLM_GFX950_DEC_MAX_HEAD_DIM || hd % PV_SLICE || grp > SLLM_GFX950_DEC_MAX_GQA ||
        d->n_embd > SLLM_GFX950_DEC_MAX_WIDTH || d->n_ff > SLLM_GFX950_DEC_MAX_WIDTH) {
        return sllm_shim_fail(SLLM_GFX950_ERR_TOO_LARGE,
                              "model: head dim %d (<= %d, multiple of %d), %d query heads per KV head (<= %d), "
                              "widths %d / %d (<= %d)", hd, SLLM_GFX950_DEC_MAX_HEAD_DIM, PV_SLICE, grp,
                              SLLM_GFX950_DEC_MAX_GQA, d->n_embd, d->n_ff, SLLM_GFX950_DEC_MAX_WIDTH);
    }
    return SLLM_GFX950_OK;
}

int sllm_gfx950_model_upload(const sllm_gfx950_model_desc *d, sllm_gfx950_model **out) {
    DEC_NEED_OPEN();
    if (!sllm_shim_is_open()) return sllm_shim_fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open");
    if (d == NULL || out == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "model_upload: NULL argument");
    *out = NULL;
    int st = check_desc(d);
    if (st != SLLM_GFX950_OK) return st;
    struct sllm_gfx950_model *m = calloc(1, sizeof *m);
    if (m == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_NOMEM, "model_upload: host");
    m->n_layer = d->n_layer; m->n_embd = d->n_embd; m->n_ff = d->n_ff; m->n_head = d->n_head;
    m->n_head_kv = d->n_head_kv; m->n_rot = d->n_rot; m->n_vocab = d->n_vocab;
    m->hd = d->n_embd / d->n_head;
    m->gqa = m->hd * d->n_head_kv;
    m->eps = d->eps;
    m->rope_base = d->rope_base;
    m->layers = calloc((size_t) d->n_layer, sizeof *m->layers);
    if (m->layers == NULL) { free(m); return sllm_shim_fail(SLLM_GFX950_ERR_NOMEM, "model_upload: host"); }

    const size_t e = (size_t) m->n_embd, f = (size_t) m->n_ff;
    size_t total = align256((size_t) m->n_vocab * e * 2) + align256(e * 4);
    for (int32_t il = 0; il < m->n_layer; ++il) {
        for (int p = 0; p < N_PROJ; ++p) {
            size_t rows, k;
            proj_shape(m, p, &rows, &k);
            total += align256(i2s_bytes(rows, k));
        }
        total += 3 * align256(e * 4) + align256(f * 4);
    }
    hipError_t he = hipMalloc(&m->blob, total);
    if (he != hipSuccess) {
        free(m->layers);
        free(m);
        return sllm_shim_hip_fail(he, "model_upload: hipMalloc");
    }
    uint8_t *at = m->blob;
#define PUT(dst, src, bytes)                                                                   \
    do {                                                                                       \
        (dst) = (void *) at;                                                                   \
        if (he == hipSuccess) he = hipMemcpy(at, (src), (bytes), hipMemcpyHostToDevice);       \
        at += align256(bytes);                                                                 \
    } while (0)
    PUT(m->tok_embd, d->tok_embd, (size_t) m->n_vocab * e * 2);
    PUT(m->output_norm, d->output_norm, e * 4);
    for (int32_t il = 0; il < m->n_layer; ++il) {
        const sllm_gfx950_layer_desc *L = &d->layers[il];
        dev_layer *D = &m->layers[il];
        const uint8_t *src[N_PROJ] = { L->wq, L->wk, L->wv, L->wo, L->w_gate, L->w_up, L->w_down };
        for (int p = 0; p < N_PROJ; ++p) {
            size_t rows, k;
            proj_shape(m, p, &rows, &k);
            PUT(D->w[p], src[p], i2s_bytes(rows, k));
        }
        PUT(D->attn_norm, L->attn_norm, e * 4);
        PUT(D->attn_sub_norm, L->attn_sub_norm, e * 4);
        PUT(D->ffn_norm, L->ffn_norm, e * 4);
        PUT(D->ffn_sub_norm, L->ffn_sub_norm, f * 4);
    }
#undef PUT
    if (he != hipSuccess) {
        hipFree(m->blob);
        free(m->layers);
        free(m);
        return sllm_shim_hip_fail(he, "model_upload: hipMemcpy");
    }
    *out = m;
    return SLLM_GFX950_OK;
}

void sllm_gfx950_model_free(sllm_gfx950_model *m) {
    if (m == NULL) return;
    if (sllm_shim_is_open()) hipFree(m->blob);
    free(m->layers);
    free(m);
}

size_t sllm_gfx950_trace_dots(const sllm_gfx950_model *m) {
    if (m == NULL) return 0;
    return (size_t) m->n_layer * (3 * (size_t) m->n_embd + 2 * (size_t) m->gqa + 2 * (size_t) m->n_ff);
}

/* ------------------------------------------------------------------ */
/* context                                                             */
/* ------------------------------------------------------------------ */

/* Device buffers of a chunk of up to `cap` tokens, each [token][width]
 * (src/forward.c:489-504 holds the same columns on the host). */
typedef struct chunk_bufs {
    void            *dev;
    int32_t          cap;
    int32_t         *tokens;
    float           *x, *fi, *q, *k, *v, *attn, *proj, *g, *u, *xn, *scores, *logits;
    int8_t          *q8;
    sllm_gfx950_act *act;
} chunk_bufs;

struct sllm_gfx950_ctx {
    const struct sllm_gfx950_model *m;
    int32_t       n_ctx, n_past;
    void         *dev;
    float        *k_cache, *v_cache, *rope, *scores, *logits;
    float        *x, *ffn_inp, *qkv, *attn, *o, *h, *down;
    k_dec_step   *step;
    int32_t      *feed, *gen;
    uint64_t     *lm_partial;      /* one argmax key per output workgroup */
    uint32_t      lm_wg;
    k_dec_gemv_args *gargs;        /* n_layer * N_STAGE kernel argument blocks */
    k_dec_attn   *attn_args;       /* n_layer */
    k_dec_lm      lm_args;
    size_t        kv_per_layer;    /* floats */
    hipFunction_t f_gemv, f_scores, f_pv, f_lm, f_argmax;
    hipFunction_t f_prep, f_kvs, f_cscores, f_cscores4, f_cscores_w, f_csoft, f_cpv, f_clm, f_keys;
    uint32_t      sc_stride;
    chunk_bufs    chk;
    int           graph_on, graph_ready;
    hipGraph_t    graph;
    hipGraphExec_t graph_exec;
    int           have_logits;     /* c->logits hold the last position's logits */
    /* generate_greedy keeps at most `inflight` tokens enqueued ahead of the
     * host: an event recorded after each token, waited on `inflight` tokens
     * later */
    int32_t       inflight;
    hipEvent_t    inflight_ev[SLLM_GFX950_DEC_MAX_INFLIGHT];
    int           n_inflight_ev;
};

/* Workgroups of a projection's GEMV: one row group each (decode GEMVs are a
 * few MB, and latency, not bandwidth per workgroup, bounds them). */
static uint32_t proj_slabs(const struct sllm_gfx950_model *m, int p, int *variant) {
    size_t rows, k;
    proj_shape(m, p, &rows, &k);
    *variant = sllm_shim_slab_variant((uint32_t) k);
    const uint32_t g = sllm_shim_slab_group_rows(*variant);
    return (uint32_t) ((rows + g - 1) / g);
}

static uint32_t pad8(uint32_t v) { return (v + 7u) & ~7u; }

static void fill_args(sllm_gfx950_ctx *c, int32_t *trace_dots, sllm_gfx950_act *trace_acts) {
    const struct sllm_gfx950_model *m = c->m;
    const size_t e = (size_t) m->n_embd, f = (size_t) m->n_ff, g = (size_t) m->gqa;
    int32_t *tr = trace_dots;
    for (int32_t il = 0; il < m->n_layer; ++il) {
        const dev_layer *L = &m->layers[il];
        k_gemv_job J[N_PROJ];
        uint32_t slabs[N_PROJ];
        float *out_f[N_PROJ] = { c->qkv, c->qkv + e, c->qkv + e + g, c->o, c->h, NULL, c->down };
        for (int p = 0; p < N_PROJ; ++p) {
            size_t rows, k;
            proj_shape(m, p, &rows, &k);
            int variant;
            slabs[p] = proj_slabs(m, p, &variant);
            J[p] = (k_gemv_job) { L->w[p], NULL, NULL, NULL, out_f[p], tr, (uint32_t) rows, (uint32_t) k,
                                  (uint32_t) variant, 0 };
            if (tr != NULL) tr += rows;
        }
        sllm_gfx950_act *ta = trace_acts != NULL ? trace_acts + (size_t) il * 4 : NULL;
        k_dec_gemv_args *A = c->gargs + (size_t) il * N_STAGE;
        memset(A, 0, N_STAGE * sizeof *A);
        A[S_QKV].st = (k_dec_stage) {
            il == 0 ? (const void *) m->tok_embd : (const void *) c->down, il == 0 ? NULL : c->ffn_inp,
            c->x, L->attn_norm, c->step, NULL, ta ? ta + 0 : NULL, m->eps, (uint32_t) e,
            il == 0 ? IN_EMBED : IN_RESID, 0 };
        A[S_O].st = (k_dec_stage) { c->attn, NULL, NULL, L->attn_sub_norm, c->step, NULL, ta ? ta + 1 : NULL,
                                    m->eps, (uint32_t) e, IN_PLAIN, 0 };
        A[S_FFN].st = (k_dec_stage) { c->o, c->x, c->ffn_inp, L->ffn_norm, c->step, NULL, ta ? ta + 2 : NULL,
                                      m->eps, (uint32_t) e, IN_RESID, 0 };
        A[S_DOWN].st = (k_dec_stage) { c->h, NULL, NULL, L->ffn_sub_norm, c->step, NULL, ta ? ta + 3 : NULL,
                                       m->eps, (uint32_t) f, IN_PLAIN, 0 };
        /* Q, K, V share the attention input; gate and up are one pair whose
         * slabs cover both (up has none of its own) */
        A[S_QKV].job[0] = J[P_Q]; A[S_QKV].job[1] = J[P_K]; A[S_QKV].job[2] = J[P_V];
        A[S_QKV].n_slabs[0] = slabs[P_Q]; A[S_QKV].n_slabs[1] = slabs[P_K]; A[S_QKV].n_slabs[2] = slabs[P_V];
        A[S_O].job[0] = J[P_O]; A[S_O].job[1] = J[P_O]; A[S_O].job[2] = J[P_O];
        A[S_O].n_slabs[0] = slabs[P_O];
        A[S_FFN].job[0] = J[P_GATE]; A[S_FFN].job[1] = J[P_UP]; A[S_FFN].job[2] = J[P_GATE];
        A[S_FFN].n_slabs[0] = slabs[P_GATE];
        A[S_FFN].pair = 1;
        A[S_DOWN].job[0] = J[P_DOWN]; A[S_DOWN].job[1] = J[P_DOWN]; A[S_DOWN].job[2] = J[P_DOWN];
        A[S_DOWN].n_slabs[0] = slabs[P_DOWN];
        for (int st = 0; st < N_STAGE; ++st) {
            A[st].n_wg = pad8(A[st].n_slabs[0] + A[st].n_slabs[1] + A[st].n_slabs[2]);
        }
    }
}

/* cos / sin of every (position, pair) as the reference computes them per
 * token (src/ops.c:467-549): theta_scale = powf(base, -2/n_rot) with n_rot
 * made even, the angle of pair k at pos is (float)pos times theta_scale k
 * times over (one f32 product per step), through the C library's cosf / sinf */
static void rope_table(const struct sllm_gfx950_model *m, int32_t n_ctx, float *out) {
    const int32_t n_rot = m->n_rot - (m->n_rot % 2);
    const int32_t half = n_rot / 2;
    if (half == 0) return;
    const float theta_scale = powf(m->rope_base, -2.0f / (float) n_rot);
    for (int32_t pos = 0; pos < n_ctx; ++pos) {
        float theta = (float) pos;
        float *row = out + (size_t) pos * (size_t) half * 2;
        for (int32_t k = 0; k < half; ++k) {
            const float ang = 1.0f * theta;
            row[2 * k] = cosf(ang);
            row[2 * k + 1] = sinf(ang);
            theta *= theta_scale;
        }
    }
}

static int set_args(sllm_gfx950_ctx *c, int32_t *trace_dots, sllm_gfx950_act *trace_acts) {
    fill_args(c, trace_dots, trace_acts);
    c->graph_ready = 0;
    return SLLM_GFX950_OK;
}

static int drop_graph(sllm_gfx950_ctx *c) {
    if (c->graph_exec) hipGraphExecDestroy(c->graph_exec);
    if (c->graph) hipGraphDestroy(c->graph);
    c->graph_exec = NULL;
    c->graph = NULL;
    c->graph_ready = 0;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_ctx_new(const sllm_gfx950_model *m, int32_t n_ctx, sllm_gfx950_ctx **out) {
    DEC_NEED_OPEN();
    if (!sllm_shim_is_open()) return sllm_shim_fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open");
    if (m == NULL || out == NULL || n_ctx < 1) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "ctx_new: bad arguments");
    *out = NULL;
    const int32_t grp = m->n_head / m->n_head_kv;
    if ((int64_t) grp * n_ctx > SLLM_GFX950_DEC_MAX_GQA_CTX) {
        return sllm_shim_fail(SLLM_GFX950_ERR_TOO_LARGE, "ctx_new: %d query heads per KV head x n_ctx %d > %d",
                              grp, n_ctx, SLLM_GFX950_DEC_MAX_GQA_CTX);
    }
    sllm_gfx950_ctx *c = calloc(1, sizeof *c);
    if (c == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_NOMEM, "ctx_new: host");
    c->m = m;
    c->n_ctx = n_ctx;
    c->inflight = SLLM_GFX950_DEC_DEFAULT_INFLIGHT;
    const size_t e = (size_t) m->n_embd, f = (size_t) m->n_ff, g = (size_t) m->gqa;
    const int32_t half = (m->n_rot - m->n_rot % 2) / 2;
    c->kv_per_layer = (size_t) m->n_head_kv * (size_t) n_ctx * (size_t) m->hd;
    const uint32_t sc_stride = (uint32_t) ((n_ctx + 7) & ~7);
    c->sc_stride = sc_stride;
    const uint32_t n_pass = (uint32_t) ((m->n_vocab + LM_ROWS - 1) / LM_ROWS);
    const uint32_t lm_cap = (uint32_t) (sllm_shim_cu() > 0 ? sllm_shim_cu() : 256) * LM_WG_PER_CU;
    /* passes dealt round-robin: as many workgroups as give every one the
     * same number of passes (but the last few, one fewer) */
    const uint32_t lm_per = (n_pass + lm_cap - 1) / lm_cap, lm_wg = (n_pass + lm_per - 1) / lm_per;
    const size_t sizes[] = {
        c->kv_per_layer * (size_t) m->n_layer * 4,          /* k cache */
        c->kv_per_layer * (size_t) m->n_layer * 4,          /* v cache */
        (size_t) n_ctx * (size_t) (half > 0 ? half : 1) * 8, /* rope */
        (size_t) m->n_head * (size_t) sc_stride * 4,        /* scores */
        (size_t) m->n_vocab * 4,                            /* logits */
        e * 4, e * 4, (e + 2 * g) * 4, e * 4, e * 4, f * 4, e * 4,   /* x ffn_inp qkv attn o h down */
        sizeof(k_dec_step),
        (size_t) n_ctx * 4, (size_t) n_ctx * 4,             /* feed, gen */
        (size_t) lm_wg * 8,                                 /* output argmax keys */
    };
    enum { N_BUF = sizeof sizes / sizeof sizes[0] };
    size_t total = 0;
    for (int i = 0; i < N_BUF; ++i) total += align256(sizes[i]);
    c->gargs = calloc((size_t) m->n_layer * N_STAGE, sizeof *c->gargs);
    c->attn_args = calloc((size_t) m->n_layer, sizeof *c->attn_args);
    float *rope_host = malloc(sizes[2]);
    int st = SLLM_GFX950_OK;
    if (!c->gargs || !c->attn_args || !rope_host) {
        st = sllm_shim_fail(SLLM_GFX950_ERR_NOMEM, "ctx_new: host");
    }
    hipError_t he = hipSuccess;
    if (st == SLLM_GFX950_OK) {
        he = hipMalloc(&c->dev, total);
        /* cleared on the library stream, which does not order against the
         * null stream */
        if (he == hipSuccess) he = hipMemsetAsync(c->dev, 0, total, sllm_shim_stream());
        if (he == hipSuccess) he = hipStreamSynchronize(sllm_shim_stream());
        if (he != hipSuccess) st = sllm_shim_hip_fail(he, "ctx_new: device memory");
    }
    if (st == SLLM_GFX950_OK) {
        void *p[N_BUF];
        uint8_t *at = c->dev;
        for (int i = 0; i < N_BUF; ++i) { p[i] = at; at += align256(sizes[i]); }
        c->k_cache = p[0]; c->v_cache = p[1]; c->rope = p[2]; c->scores = p[3]; c->logits = p[4];
        c->x = p[5]; c->ffn_inp = p[6]; c->qkv = p[7]; c->attn = p[8]; c->o = p[9]; c->h = p[10];
        c->down = p[11]; c->step = p[12]; c->feed = p[13]; c->gen = p[14]; c->lm_partial = p[15];
        c->lm_wg = lm_wg;
        rope_table(m, n_ctx, rope_host);
        he = hipMemcpy(c->rope, rope_host, sizes[2], hipMemcpyHostToDevice);
        if (he != hipSuccess) st = sllm_shim_hip_fail(he, "ctx_new: rope table");
    }
    free(rope_host);
    if (st == SLLM_GFX950_OK) st = set_args(c, NULL, NULL);
    if (st == SLLM_GFX950_OK) {
        const float attn_scale = 1.0f / sqrtf((float) m->hd);      /* src/forward.c:616 */
        for (int32_t il = 0; il < m->n_layer; ++il) {
            c->attn_args[il] = (k_dec_attn) {
                c->qkv, c->qkv + e, c->qkv + e + g,
                c->k_cache + (size_t) il * c->kv_per_layer, c->v_cache + (size_t) il * c->kv_per_layer,
                c->rope, c->scores, c->attn, c->step, attn_scale,
                (uint32_t) m->n_head, (uint32_t) m->n_head_kv, (uint32_t) m->hd, (uint32_t) half,
                (uint32_t) n_ctx, sc_stride, 0, NULL, 0 };
            /* what the chunk's scores kernel reads ahead: this layer's O,
             * gate, up and down weights and the next layer's Q, K and V (one
             * run of the model allocation, in that order) */
            const dev_layer *D = &m->layers[il];
            const int more = il + 1 < m->n_layer;
            size_t rows, k;
            proj_shape(m, more ? P_V : P_DOWN, &rows, &k);
            const uint8_t *from = (const uint8_t *) D->w[P_O];
            const uint8_t *to = (const uint8_t *) (more ? m->layers[il + 1].w[P_V] : D->w[P_DOWN]) + i2s_bytes(rows, k);
            c->attn_args[il].ahead = from;
            c->attn_args[il].ahead_bytes = (uint64_t) (to - from) & ~(uint64_t) 15;
        }
        c->lm_args = (k_dec_lm) { c->down, c->ffn_inp, m->output_norm, m->tok_embd, c->logits, c->lm_partial,
                                  c->step, m->eps, (uint32_t) m->n_embd, (uint32_t) m->n_vocab, 0 };
        if ((st = sllm_shim_decode_function("sllm_k_dec_gemv", &c->f_gemv)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_dec_scores", &c->f_scores)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_dec_pv", &c->f_pv)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_dec_lm_head", &c->f_lm)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_prep", &c->f_prep)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_kv_store", &c->f_kvs)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_scores", &c->f_cscores)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_scores4", &c->f_cscores4)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_scores_w", &c->f_cscores_w)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_softmax", &c->f_csoft)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_pv", &c->f_cpv)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_lm_head", &c->f_clm)) == SLLM_GFX950_OK &&
            (st = sllm_shim_decode_function("sllm_k_chk_keys", &c->f_keys)) == SLLM_GFX950_OK) {
            st = sllm_shim_decode_function("sllm_k_dec_argmax", &c->f_argmax);
        }
    }
    if (st != SLLM_GFX950_OK) {
        sllm_gfx950_ctx_free(c);
        return st;
    }
    *out = c;
    return SLLM_GFX950_OK;
}

void sllm_gfx950_ctx_free(sllm_gfx950_ctx *c) {
    if (c == NULL) return;
    if (sllm_shim_is_open()) {
        hipStreamSynchronize(sllm_shim_stream());
        drop_graph(c);
        if (c->dev) hipFree(c->dev);
        if (c->chk.dev) hipFree(c->chk.dev);
    }
    if (sllm_shim_is_open()) {
        for (int i = 0; i < c->n_inflight_ev; ++i) hipEventDestroy(c->inflight_ev[i]);
    }
    free(c->gargs);
    free(c->attn_args);
    free(c);
}

int32_t sllm_gfx950_ctx_n_past(const sllm_gfx950_ctx *c) { return c ? c->n_past : 0; }

const float *sllm_gfx950_ctx_logits(const sllm_gfx950_ctx *c) { return c ? c->logits : NULL; }

int sllm_gfx950_ctx_reset(sllm_gfx950_ctx *c) {
    DEC_NEED_OPEN();
    if (c == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "ctx_reset: NULL");
    const hipStream_t s = sllm_shim_stream();
    hipError_t he = hipSuccess;
    if (c->n_past > 0) {
        /* the live prefix of every (layer, KV head): n_past positions of
         * every 8-dimension key and value slice */
        const size_t hd = (size_t) c->m->hd, rows = (size_t) c->m->n_layer * (size_t) c->m->n_head_kv;
        he = hipMemset2DAsync(c->k_cache, (size_t) c->n_ctx * PV_SLICE * 4, 0, (size_t) c->n_past * PV_SLICE * 4,
                              rows * (hd / PV_SLICE), s);
        if (he == hipSuccess) {
            he = hipMemset2DAsync(c->v_cache, (size_t) c->n_ctx * PV_SLICE * 4, 0, (size_t) c->n_past * PV_SLICE * 4,
                                  rows * (hd / PV_SLICE), s);
        }
    }
    if (he == hipSuccess) he = hipMemsetAsync(c->step, 0, sizeof(k_dec_step), s);
    if (he == hipSuccess) he = hipStreamSynchronize(s);
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "ctx_reset");
    c->n_past = 0;
    c->have_logits = 0;
    return SLLM_GFX950_OK;
}

/* ------------------------------------------------------------------ */
/* one token                                                           */
/* ------------------------------------------------------------------ */

static int launch_token(sllm_gfx950_ctx *c) {
    const struct sllm_gfx950_model *m = c->m;
    int st = SLLM_GFX950_OK;
    const uint32_t kv_chunks = (uint32_t) ((c->n_ctx + ATT_POS - 1) / ATT_POS);
    const uint32_t slices = (uint32_t) (m->hd / PV_SLICE);
    /* p.V workgroups per (KV head, slice): two query heads each */
    const uint32_t pv_wpk = (uint32_t) ((m->n_head / m->n_head_kv + PV_HPW - 1) / PV_HPW);
    for (int32_t il = 0; il < m->n_layer && st == SLLM_GFX950_OK; ++il) {
        for (int s = 0; s < N_STAGE && st == SLLM_GFX950_OK; ++s) {
            k_dec_gemv_args *A = &c->gargs[(size_t) il * N_STAGE + s];
            void *args[] = { A };
            st = sllm_shim_launch(c->f_gemv, A->n_wg, 1, SLLM_SLAB_THREADS, 0, args);
            if (s == S_QKV && st == SLLM_GFX950_OK) {
                void *aargs[] = { &c->attn_args[il] };
                /* at most eight KV heads: eight columns of workgroups, KV head h
                 * in column h (XCD h) for both kernels (decode_kernels.hip) */
                const int cols = m->n_head_kv <= 8;
                if (cols) st = sllm_shim_launch(c->f_scores, 8u * kv_chunks, 1, ATT_THREADS, 0, aargs);
                else st = sllm_shim_launch(c->f_scores, (uint32_t) m->n_head_kv, kv_chunks, ATT_THREADS, 0, aargs);
                if (st == SLLM_GFX950_OK) {
                    const uint32_t n_pv = (cols ? 8u : (uint32_t) m->n_head_kv) * slices * pv_wpk;
                    st = sllm_shim_launch(c->f_pv, n_pv, 1, PV_THREADS, 0, aargs);
                }
            }
        }
    }
    if (st == SLLM_GFX950_OK) {
        void *largs[] = { &c->lm_args };
        st = sllm_shim_launch(c->f_lm, c->lm_wg, 1, LM_THREADS, 0, largs);
    }
    if (st == SLLM_GFX950_OK) {
        const uint64_t *partial = c->lm_partial;
        const float *logits = c->logits;
        k_dec_step *step = c->step;
        uint32_t n = c->lm_wg;
        void *aargs[] = { (void *) &partial, &n, (void *) &logits, (void *) &step };
        st = sllm_shim_launch(c->f_argmax, 1, 1, 256, 0, aargs);
    }
    return st;
}

static int enqueue_token(sllm_gfx950_ctx *c) {
    if (!c->graph_on) return launch_token(c);
    const hipStream_t s = sllm_shim_stream();
    if (!c->graph_ready) {
        drop_graph(c);
        hipError_t he = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (he != hipSuccess) return sllm_shim_hip_fail(he, "graph: begin capture");
        const int st = launch_token(c);
        hipGraph_t graph = NULL;
        he = hipStreamEndCapture(s, &graph);
        if (st != SLLM_GFX950_OK) { if (graph) hipGraphDestroy(graph); return st; }
        if (he != hipSuccess) return sllm_shim_hip_fail(he, "graph: end capture");
        c->graph = graph;
        he = hipGraphInstantiate(&c->graph_exec, graph, NULL, NULL, 0);
        if (he != hipSuccess) { drop_graph(c); return sllm_shim_hip_fail(he, "graph: instantiate"); }
        c->graph_ready = 1;
    }
    hipError_t he = hipGraphLaunch(c->graph_exec, s);
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "graph: launch");
    return SLLM_GFX950_OK;
}

int sllm_gfx950_ctx_set_graph(sllm_gfx950_ctx *c, int on) {
    DEC_NEED_OPEN();
    if (c == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "ctx_set_graph: NULL");
    c->graph_on = on != 0;
    if (!c->graph_on) {
        hipStreamSynchronize(sllm_shim_stream());
        drop_graph(c);
    }
    return SLLM_GFX950_OK;
}

/* write the step record: token at pos, then the given feed / gen state */
static int set_step(sllm_gfx950_ctx *c, const k_dec_step *hs) {
    hipError_t he = hipMemcpyAsync(c->step, hs, sizeof *hs, hipMemcpyHostToDevice, sllm_shim_stream());
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "step record");
    return SLLM_GFX950_OK;
}

int sllm_gfx950_forward(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, int32_t token, int32_t pos,
                        float *logits) {
    DEC_NEED_OPEN();
    if (m == NULL || c == NULL || c->m != m) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward: model / context");
    if (pos < c->n_past || pos >= c->n_ctx) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward: pos %d outside [n_past %d, n_ctx %d)", pos, c->n_past, c->n_ctx);
    }
    if (token < 0 || token >= m->n_vocab) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward: token %d out of range", token);
    k_dec_step hs;
    memset(&hs, 0, sizeof hs);
    hs.token = token;
    hs.pos = pos;
    int st = set_step(c, &hs);
    if (st == SLLM_GFX950_OK) st = enqueue_token(c);
    if (st != SLLM_GFX950_OK) return st;
    c->n_past = pos + 1;
    c->have_logits = 1;
    if (logits != NULL) {
        const hipStream_t s = sllm_shim_stream();
        hipError_t he = hipMemcpyAsync(logits, c->logits, (size_t) m->n_vocab * 4, hipMemcpyDeviceToHost, s);
        if (he == hipSuccess) he = hipStreamSynchronize(s);
        if (he != hipSuccess) return sllm_shim_hip_fail(he, "forward: logits");
    }
    return SLLM_GFX950_OK;
}

int sllm_gfx950_ctx_argmax(sllm_gfx950_ctx *c, int32_t *token) {
    DEC_NEED_OPEN();
    if (c == NULL || token == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "ctx_argmax: NULL");
    k_dec_step hs;
    hipError_t he = hipMemcpyAsync(&hs, c->step, sizeof hs, hipMemcpyDeviceToHost, sllm_shim_stream());
    if (he == hipSuccess) he = hipStreamSynchronize(sllm_shim_stream());
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "ctx_argmax");
    *token = hs.next;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_generate_greedy(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, const int32_t *prompt,
                                int32_t n_prompt, int32_t n_new, int32_t *out) {
    DEC_NEED_OPEN();
    if (m == NULL || c == NULL || c->m != m || out == NULL || n_prompt < 0 || n_new < 0 ||
        (n_prompt > 0 && prompt == NULL)) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "generate_greedy: bad arguments");
    }
    if ((int64_t) n_prompt + n_new + c->n_past > c->n_ctx) {
        return sllm_shim_fail(SLLM_GFX950_ERR_TOO_LARGE, "generate_greedy: %d + %d + %d positions > n_ctx %d",
                              n_prompt, n_new, c->n_past, c->n_ctx);
    }
    for (int32_t i = 0; i < n_prompt; ++i) {
        if (prompt[i] < 0 || prompt[i] >= m->n_vocab) {
            return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "generate_greedy: prompt token %d out of range", prompt[i]);
        }
    }
    const int32_t base = c->n_past;
    const hipStream_t s = sllm_shim_stream();
    while (c->n_inflight_ev < c->inflight) {
        const hipError_t he = hipEventCreateWithFlags(&c->inflight_ev[c->n_inflight_ev], hipEventDisableTiming);
        if (he != hipSuccess) return sllm_shim_hip_fail(he, "generate_greedy: events");
        c->n_inflight_ev++;
    }
    k_dec_step hs;
    memset(&hs, 0, sizeof hs);
    hs.pos = base;
    hs.advance = 1;
    int32_t steps;
    int32_t gen_at = 0;
    if (n_prompt > 0) {
        /* the prompt, then n_new tokens; the argmax after the last prompt
         * token is out[0] (src/forward.c:921-934) */
        hs.token = prompt[0];
        hs.feed = c->feed;
        hs.n_feed = n_prompt;
        hs.i_feed = 1;
        hs.gen = c->gen;
        hs.cap_gen = n_new;
        steps = n_prompt + n_new;
        hipError_t he = hipMemcpyAsync(c->feed, prompt, (size_t) n_prompt * 4, hipMemcpyHostToDevice, s);
        if (he != hipSuccess) return sllm_shim_hip_fail(he, "generate_greedy: prompt");
    } else {
        /* no prompt: start from the last logits' argmax, or BOS in a fresh
         * context (src/forward.c:909-920); out[0] is that token */
        if (n_new == 0) return SLLM_GFX950_OK;
        int32_t first = BOS_TOKEN;
        if (base > 0 && !c->have_logits) {
            return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "generate_greedy: no prompt and no last logits "
                                  "(restore them with ctx_kv_load, or give a prompt)");
        }
        if (base > 0) {
            const int st = sllm_gfx950_ctx_argmax(c, &first);
            if (st != SLLM_GFX950_OK) return st;
        }
        if (first < 0 || first >= m->n_vocab) {
            return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "generate_greedy: first token %d out of range", first);
        }
        out[0] = first;
        hs.token = first;
        hs.gen = c->gen;
        hs.cap_gen = n_new - 1;
        gen_at = 1;
        steps = n_new;
    }
    int st = set_step(c, &hs);
    for (int32_t i = 0; i < steps && st == SLLM_GFX950_OK; ++i) {
        /* at most c->inflight tokens enqueued ahead: wait for token i - inflight */
        hipEvent_t ev = c->inflight_ev[i % c->inflight];
        if (i >= c->inflight) {
            const hipError_t he = hipEventSynchronize(ev);
            if (he != hipSuccess) return sllm_shim_hip_fail(he, "generate_greedy: in-flight wait");
        }
        st = enqueue_token(c);
        if (st == SLLM_GFX950_OK) {
            const hipError_t he = hipEventRecord(ev, s);
            if (he != hipSuccess) return sllm_shim_hip_fail(he, "generate_greedy: in-flight event");
        }
    }
    if (st != SLLM_GFX950_OK) return st;
    c->n_past = base + steps;
    c->have_logits = 1;
    const int32_t n_copy = n_new - gen_at;
    hipError_t he = hipSuccess;
    if (n_copy > 0) he = hipMemcpyAsync(out + gen_at, c->gen, (size_t) n_copy * 4, hipMemcpyDeviceToHost, s);
    if (he == hipSuccess) he = hipStreamSynchronize(s);
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "generate_greedy: tokens");
    return SLLM_GFX950_OK;
}

int sllm_gfx950_ctx_kv_load(sllm_gfx950_ctx *c, const float *k, const float *v, int32_t n_pos,
                            const float *logits) {
    DEC_NEED_OPEN();
    if (c == NULL || k == NULL || v == NULL || n_pos < 0 || n_pos > c->n_ctx) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "ctx_kv_load: bad arguments");
    }
    const struct sllm_gfx950_model *m = c->m;
    const size_t hd = (size_t) m->hd, rows = (size_t) m->n_layer * (size_t) m->n_head_kv;
    const size_t n_sl = hd / PV_SLICE, np = (size_t) n_pos;
    const size_t pitch = (size_t) c->n_ctx * PV_SLICE * 4;
    const hipStream_t s = sllm_shim_stream();
    /* both caches are slice-major, [layer][KV head][dimension / 8][position][8]:
     * the [layer][KV head][position][hd] rows are rearranged on the host first */
    float *ks = NULL, *vs = NULL;
    if (n_pos > 0) {
        ks = malloc(2 * rows * np * hd * sizeof *ks);
        if (ks == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_NOMEM, "ctx_kv_load: host staging");
        vs = ks + rows * np * hd;
        for (size_t r = 0; r < rows; ++r) {
            for (size_t sl = 0; sl < n_sl; ++sl) {
                float *kd = ks + (r * n_sl + sl) * np * PV_SLICE, *vd = vs + (r * n_sl + sl) * np * PV_SLICE;
                for (size_t p = 0; p < np; ++p) {
                    memcpy(kd + p * PV_SLICE, k + (r * np + p) * hd + sl * PV_SLICE, PV_SLICE * 4);
                    memcpy(vd + p * PV_SLICE, v + (r * np + p) * hd + sl * PV_SLICE, PV_SLICE * 4);
                }
            }
        }
    }
    hipError_t he = hipSuccess;
    if (n_pos > 0) {
        const size_t w = np * PV_SLICE * 4;
        he = hipMemcpy2DAsync(c->k_cache, pitch, ks, w, w, rows * n_sl, hipMemcpyHostToDevice, s);
        if (he == hipSuccess) he = hipMemcpy2DAsync(c->v_cache, pitch, vs, w, w, rows * n_sl, hipMemcpyHostToDevice, s);
    }
    /* positions past the restored prefix read as absent (zero) in every
     * (layer, KV head), as src/forward.c:1098-1118 clears them */
    if (he == hipSuccess && n_pos < c->n_ctx) {
        const size_t from = np * PV_SLICE * 4;
        he = hipMemset2DAsync((uint8_t *) c->k_cache + from, pitch, 0, pitch - from, rows * n_sl, s);
        if (he == hipSuccess) he = hipMemset2DAsync((uint8_t *) c->v_cache + from, pitch, 0, pitch - from, rows * n_sl, s);
    }
    if (he == hipSuccess && logits != NULL) {
        he = hipMemcpyAsync(c->logits, logits, (size_t) m->n_vocab * 4, hipMemcpyHostToDevice, s);
    }
    if (he != hipSuccess) {
        hipStreamSynchronize(s);               /* the staging buffer may still be read */
        free(ks);
        return sllm_shim_hip_fail(he, "ctx_kv_load");
    }
    int st = SLLM_GFX950_OK;
    if (logits != NULL) {
        /* the restored logits' argmax becomes the step record's next token,
         * what an empty-prompt generate continues from (src/forward.c:909-912) */
        k_dec_step hs;
        memset(&hs, 0, sizeof hs);
        st = set_step(c, &hs);
        uint64_t *partial = c->lm_partial;
        const uint64_t *cpartial = c->lm_partial;
        const float *lg = c->logits;
        k_dec_step *step = c->step;
        uint32_t nv = (uint32_t) m->n_vocab, nw = c->lm_wg;
        void *kargs[] = { (void *) &lg, &nv, (void *) &partial };
        void *aargs[] = { (void *) &cpartial, &nw, (void *) &lg, (void *) &step };
        if (st == SLLM_GFX950_OK) st = sllm_shim_launch(c->f_keys, c->lm_wg, 1, 256, 0, kargs);
        if (st == SLLM_GFX950_OK) st = sllm_shim_launch(c->f_argmax, 1, 1, 256, 0, aargs);
    }
    he = hipStreamSynchronize(s);
    free(ks);
    if (st != SLLM_GFX950_OK) return st;
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "ctx_kv_load");
    c->n_past = n_pos;
    c->have_logits = logits != NULL;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_ctx_set_inflight(sllm_gfx950_ctx *c, int32_t tokens) {
    DEC_NEED_OPEN();
    if (c == NULL || tokens < 1 || tokens > SLLM_GFX950_DEC_MAX_INFLIGHT) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "ctx_set_inflight: tokens must be 1..%d",
                              SLLM_GFX950_DEC_MAX_INFLIGHT);
    }
    c->inflight = tokens;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_ctx_trace(sllm_gfx950_ctx *c, int32_t *dots, sllm_gfx950_act *acts) {
    DEC_NEED_OPEN();
    if (c == NULL || (dots == NULL) != (acts == NULL)) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "ctx_trace: give both buffers or neither");
    }
    hipError_t he = hipStreamSynchronize(sllm_shim_stream());
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "ctx_trace");
    drop_graph(c);
    return set_args(c, dots, acts);
}

/* ------------------------------------------------------------------ */
/* chunks of tokens                                                    */
/* ------------------------------------------------------------------ */

static uint32_t cu_count(void) {
    const int cu = sllm_shim_cu();
    return (uint32_t) (cu > 0 ? cu : 256);
}

/* the chunk buffers for at least n tokens (kept, grown on demand) */
static int chunk_reserve(sllm_gfx950_ctx *c, int32_t n) {
    if (n <= c->chk.cap) return SLLM_GFX950_OK;
    const struct sllm_gfx950_model *m = c->m;
    const int32_t cap = (n + 15) & ~15;
    const size_t t = (size_t) cap, e = (size_t) m->n_embd, f = (size_t) m->n_ff, g = (size_t) m->gqa;
    const size_t big = e > f ? e : f;
    const size_t sizes[] = {
        t * 4,                                              /* tokens */
        t * e * 4, t * e * 4, t * e * 4, t * g * 4, t * g * 4,   /* x fi q k v */
        t * e * 4, t * e * 4, t * f * 4, t * f * 4, t * e * 4,   /* attn proj g u xn */
        t * (size_t) m->n_head * c->sc_stride * 4,          /* scores */
        t * (size_t) m->n_vocab * 4,                        /* logits */
        t * big,                                            /* q8 */
        t * sizeof(sllm_gfx950_act),                        /* act */
    };
    enum { N_BUF = sizeof sizes / sizeof sizes[0] };
    size_t total = 0;
    for (int i = 0; i < N_BUF; ++i) total += align256(sizes[i]);
    hipError_t he = hipStreamSynchronize(sllm_shim_stream());
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "chunk buffers");
    if (c->chk.dev) hipFree(c->chk.dev);
    memset(&c->chk, 0, sizeof c->chk);
    void *dev = NULL;
    he = hipMalloc(&dev, total);
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "chunk buffers: hipMalloc");
    void *p[N_BUF];
    uint8_t *at = dev;
    for (int i = 0; i < N_BUF; ++i) { p[i] = at; at += align256(sizes[i]); }
    chunk_bufs *B = &c->chk;
    B->dev = dev; B->cap = cap;
    B->tokens = p[0]; B->x = p[1]; B->fi = p[2]; B->q = p[3]; B->k = p[4]; B->v = p[5];
    B->attn = p[6]; B->proj = p[7]; B->g = p[8]; B->u = p[9]; B->xn = p[10]; B->scores = p[11];
    B->logits = p[12]; B->q8 = p[13]; B->act = p[14];
    return SLLM_GFX950_OK;
}

static int prep(sllm_gfx950_ctx *c, int32_t n, uint32_t mode, const void *a, const float *b, float *v_out,
                const float *norm_w, uint32_t k, int quantise, float *xn_out) {
    k_chk_prep P = { a, b, c->chk.tokens, v_out, norm_w, quantise ? c->chk.q8 : NULL,
                     quantise ? c->chk.act : NULL, xn_out, c->m->eps, k, mode, 0 };
    void *args[] = { &P };
    return sllm_shim_launch(c->f_prep, (uint32_t) n, 1, CHK_THREADS, 0, args);
}

/* One chunk of n tokens at positions base .. base + n - 1, the chunk's tokens
 * already in chk.tokens: src/forward.c:589-835 layer by layer, every
 * projection one MFMA GEMM over the n quantised rows. all_logits: the output
 * head for every token into chk.logits (and the last row into c->logits);
 * otherwise for the last token only, straight into c->logits. Either way the
 * last row's argmax lands in the step record. Q, K and V are one launch,
 * gate and up another. */
static int launch_chunk(sllm_gfx950_ctx *c, int32_t n, int32_t base, int all_logits) {
    const struct sllm_gfx950_model *m = c->m;
    const chunk_bufs *B = &c->chk;
    const size_t e = (size_t) m->n_embd, f = (size_t) m->n_ff, g = (size_t) m->gqa;
    const uint32_t pos_blocks = (uint32_t) ((base + n + ATT_POS - 1) / ATT_POS);
    int st = SLLM_GFX950_OK;
    int l_out_in_x = 0;                 /* the layer below's down GEMM left l_out in x */
    for (int32_t il = 0; il < m->n_layer && st == SLLM_GFX950_OK; ++il) {
        const dev_layer *L = &m->layers[il];
        /* l_out of the layer below (cproj + cffn_inp), or the embedding; attn_norm */
        if (il == 0) st = prep(c, n, IN_EMBED, m->tok_embd, NULL, B->x, L->attn_norm, (uint32_t) e, 1, NULL);
        else if (l_out_in_x) st = prep(c, n, IN_PLAIN, B->x, NULL, NULL, L->attn_norm, (uint32_t) e, 1, NULL);
        else st = prep(c, n, IN_RESID, B->proj, B->fi, B->x, L->attn_norm, (uint32_t) e, 1, NULL);
        k_dec_attn A = c->attn_args[il];
        A.q = B->q; A.k = B->k; A.v = B->v; A.scores = B->scores; A.out = B->attn;
        A.chunk_base = (uint32_t) base;
        /* Q, K, V; where the GEMM's row tiles hold whole heads its epilogue
         * also ropes the queries and stores the keys and values, else
         * sllm_k_chk_kv_store does */
        int store = 1;
        if (st == SLLM_GFX950_OK) {
            const sllm_gfx950_gemm_job qkv[3] = { { L->w[P_Q], e, B->q, NULL }, { L->w[P_K], g, B->k, NULL },
                                                  { L->w[P_V], g, B->v, NULL } };
            const k_gemm_rope R = { A.rope, A.k_cache, A.v_cache, A.n_ctx, A.hd, A.half, (uint32_t) base };
            st = sllm_shim_gemm_qkv_rope(qkv, e, B->q8, B->act, (size_t) n, &R);
            if (st == SLLM_SHIM_NOT_FUSED) st = sllm_gfx950_gemm_multi(qkv, 3, e, B->q8, B->act, (size_t) n);
            else store = 0;
        }
        void *aargs[] = { &A };
        if (st == SLLM_GFX950_OK && store) st = sllm_shim_launch(c->f_kvs, (uint32_t) n, 1, ATT_THREADS, 0, aargs);
        if (st == SLLM_GFX950_OK) {
            uint32_t n_tok = (uint32_t) n;
            void *sargs[] = { &A, &n_tok };
            if (n > CS_SMALL && m->hd % 32 == 0) {
                /* units of one wave dealt evenly over one workgroup per CU
                 * (measured: the workgroups of 8 tokens x 64 positions take
                 * 1.4 rounds of the CUs at 512 tokens, and the dispatcher
                 * leaves some CUs with twice the others' share) */
                st = sllm_shim_launch(c->f_cscores_w, cu_count(), 1, CSW_THREADS, CSW_LDS_PAD, sargs);
            } else {
                /* eight tokens per workgroup, four for small chunks (measured:
                 * the grid of a 64-token chunk is too small at eight) */
                const int tok = n > CS_SMALL ? CS_TOK : CS_TOK / 2;
                st = sllm_shim_launch_3d(tok == CS_TOK ? c->f_cscores : c->f_cscores4, (uint32_t) m->n_head_kv, pos_blocks,
                                         (uint32_t) ((n + tok - 1) / tok), ATT_THREADS, 0, sargs);
            }
        }
        if (st == SLLM_GFX950_OK) {
            uint32_t n_tok = (uint32_t) n;
            void *margs[] = { &A, &n_tok };
            /* the rows of at most CSM_HALF positions two to a wave,
             * the others one (decode_kernels.hip: csm_short_rows) */
            const uint32_t n_short = (uint32_t) (base >= CSM_HALF ? 0 : (n < CSM_HALF - base ? n : CSM_HALF - base)) *
                                     (uint32_t) m->n_head;
            const uint32_t waves = (n_short + 1) / 2 + (uint32_t) n * (uint32_t) m->n_head - n_short;
            st = sllm_shim_launch(c->f_csoft, (waves + CSM_WAVES - 1) / CSM_WAVES, 1, CSM_WAVES * 64, 0,
                                  margs);
        }
        if (st == SLLM_GFX950_OK) {
            uint32_t n_tok = (uint32_t) n;
            void *pargs[] = { &A, &n_tok };
            /* one workgroup per CU, the units dealt over its SIMDs */
            st = sllm_shim_launch(c->f_cpv, cu_count(), 1, CP_THREADS, CSW_LDS_PAD, pargs);
        }
        /* attn_sub_norm, O; where the tile has the form, its epilogue also
         * forms ffn_inp = attn_out + inpSA (into fi) */
        if (st == SLLM_GFX950_OK) st = prep(c, n, IN_PLAIN, B->attn, NULL, NULL, L->attn_sub_norm, (uint32_t) e, 1, NULL);
        int fi_done = 0;
        if (st == SLLM_GFX950_OK) {
            st = sllm_shim_gemm_res(L->w[P_O], e, e, B->q8, B->act, (size_t) n, B->fi, B->x);
            if (st == SLLM_GFX950_OK) fi_done = 1;
            else if (st == SLLM_SHIM_NOT_FUSED) st = sllm_gfx950_gemm(L->w[P_O], e, e, B->q8, B->act, (size_t) n, B->proj, NULL);
        }
        /* ffn_inp (unless done); ffn_norm; gate, up */
        if (st == SLLM_GFX950_OK)
            st = fi_done ? prep(c, n, IN_PLAIN, B->fi, NULL, NULL, L->ffn_norm, (uint32_t) e, 1, NULL)
                         : prep(c, n, IN_RESID, B->proj, B->x, B->fi, L->ffn_norm, (uint32_t) e, 1, NULL);
        int glu = 1;
        if (st == SLLM_GFX950_OK) {
            /* where the token count's tile has a gate + up form, its
             * epilogue makes h = silu(gate) * up (into g) */
            st = sllm_shim_gemm_glu(L->w[P_GATE], L->w[P_UP], f, e, B->q8, B->act, (size_t) n, B->g);
            if (st == SLLM_SHIM_NOT_FUSED) {
                const sllm_gfx950_gemm_job gu[2] = { { L->w[P_GATE], f, B->g, NULL }, { L->w[P_UP], f, B->u, NULL } };
                glu = 0;
                st = sllm_gfx950_gemm_multi(gu, 2, e, B->q8, B->act, (size_t) n);
            }
        }
        /* silu(gate) * up (unless done), ffn_sub_norm, down */
        if (st == SLLM_GFX950_OK)
            st = glu ? prep(c, n, IN_PLAIN, B->g, NULL, NULL, L->ffn_sub_norm, (uint32_t) f, 1, NULL)
                     : prep(c, n, IN_SILU, B->g, B->u, NULL, L->ffn_sub_norm, (uint32_t) f, 1, NULL);
        /* down; below the last layer, where the tile has the form, its
         * epilogue also forms l_out = ffn_out + ffn_inp (into x: its inpSA
         * is consumed by now; the last layer's parts stay apart for the
         * output head's residual sum) */
        l_out_in_x = 0;
        if (st == SLLM_GFX950_OK && il + 1 < m->n_layer) {
            st = sllm_shim_gemm_res(L->w[P_DOWN], e, f, B->q8, B->act, (size_t) n, B->x, B->fi);
            if (st == SLLM_GFX950_OK) l_out_in_x = 1;
            else if (st == SLLM_SHIM_NOT_FUSED) st = SLLM_GFX950_OK;
        }
        if (st == SLLM_GFX950_OK && !l_out_in_x)
            st = sllm_gfx950_gemm(L->w[P_DOWN], e, f, B->q8, B->act, (size_t) n, B->proj, NULL);
    }
    if (st != SLLM_GFX950_OK) return st;
    const hipStream_t s = sllm_shim_stream();
    const float *last = c->logits;
    if (all_logits) {
        /* l_out, output_norm per token, every token's row of logits */
        st = prep(c, n, IN_RESID, B->proj, B->fi, NULL, m->output_norm, (uint32_t) e, 0, B->xn);
        const uint32_t n_tb = (uint32_t) ((n + CLM_TOK - 1) / CLM_TOK);
        const uint32_t n_rb = (uint32_t) ((m->n_vocab + CLM_THREADS - 1) / CLM_THREADS);
        k_chk_lm L = { B->xn, m->tok_embd, B->logits, (uint32_t) e, (uint32_t) m->n_vocab, (uint32_t) n,
                       pad8(n_tb * n_rb) };
        void *largs[] = { &L };
        if (st == SLLM_GFX950_OK) st = sllm_shim_launch(c->f_clm, L.n_wg, 1, CLM_THREADS, 0, largs);
        if (st == SLLM_GFX950_OK) {
            hipError_t he = hipMemcpyAsync(c->logits, B->logits + (size_t) (n - 1) * (size_t) m->n_vocab,
                                           (size_t) m->n_vocab * 4, hipMemcpyDeviceToDevice, s);
            if (he != hipSuccess) st = sllm_shim_hip_fail(he, "chunk: last logits");
        }
        uint64_t *partial = c->lm_partial;
        uint32_t nv = (uint32_t) m->n_vocab;
        void *kargs[] = { (void *) &last, &nv, (void *) &partial };
        if (st == SLLM_GFX950_OK) st = sllm_shim_launch(c->f_keys, c->lm_wg, 1, 256, 0, kargs);
    } else {
        /* the last token alone, through the decode step's output kernel */
        k_dec_lm L = c->lm_args;
        L.a = B->proj + (size_t) (n - 1) * e;
        L.b = B->fi + (size_t) (n - 1) * e;
        void *largs[] = { &L };
        st = sllm_shim_launch(c->f_lm, c->lm_wg, 1, LM_THREADS, 0, largs);
    }
    if (st == SLLM_GFX950_OK) {
        const uint64_t *partial = c->lm_partial;
        k_dec_step *step = c->step;
        uint32_t nw = c->lm_wg;
        void *aargs[] = { (void *) &partial, &nw, (void *) &last, (void *) &step };
        st = sllm_shim_launch(c->f_argmax, 1, 1, 256, 0, aargs);
    }
    return st;
}

int sllm_gfx950_forward_chunk(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, const int32_t *tokens, int32_t n,
                              int32_t base, float *logits) {
    DEC_NEED_OPEN();
    if (m == NULL || c == NULL || c->m != m || tokens == NULL) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward_chunk: model / context / tokens");
    }
    if (n < 1 || n > SLLM_GFX950_DEC_MAX_CHUNK) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward_chunk: n = %d outside [1, %d]", n, SLLM_GFX950_DEC_MAX_CHUNK);
    }
    if (base < c->n_past || (int64_t) base + n > c->n_ctx) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward_chunk: positions [%d, %d) outside [n_past %d, n_ctx %d)",
                              base, base + n, c->n_past, c->n_ctx);
    }
    for (int32_t t = 0; t < n; ++t) {
        if (tokens[t] < 0 || tokens[t] >= m->n_vocab) {
            return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward_chunk: token %d out of range", tokens[t]);
        }
    }
    if (n == 1) return sllm_gfx950_forward(m, c, tokens[0], base, logits);
    int st = chunk_reserve(c, n);
    if (st != SLLM_GFX950_OK) return st;
    const hipStream_t s = sllm_shim_stream();
    hipError_t he = hipMemcpyAsync(c->chk.tokens, tokens, (size_t) n * 4, hipMemcpyHostToDevice, s);
    if (he != hipSuccess) return sllm_shim_hip_fail(he, "forward_chunk: tokens");
    k_dec_step hs;
    memset(&hs, 0, sizeof hs);
    hs.token = tokens[n - 1];
    hs.pos = base + n - 1;
    st = set_step(c, &hs);
    if (st == SLLM_GFX950_OK) st = launch_chunk(c, n, base, logits != NULL);
    if (st != SLLM_GFX950_OK) return st;
    c->n_past = base + n;
    c->have_logits = 1;
    if (logits != NULL) {
        he = hipMemcpyAsync(logits, c->chk.logits, (size_t) n * (size_t) m->n_vocab * 4, hipMemcpyDeviceToHost, s);
        if (he == hipSuccess) he = hipStreamSynchronize(s);
        if (he != hipSuccess) return sllm_shim_hip_fail(he, "forward_chunk: logits");
    }
    return SLLM_GFX950_OK;
}

int sllm_gfx950_forward_prefill_chunked(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, const int32_t *tokens,
                                        int32_t n, int32_t chunk, float *logits) {
    DEC_NEED_OPEN();
    if (m == NULL || c == NULL || c->m != m || (tokens == NULL && n > 0) || n < 0) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward_prefill_chunked: bad arguments");
    }
    if (chunk < 1 || chunk > SLLM_GFX950_DEC_MAX_CHUNK) {
        return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "forward_prefill_chunked: chunk %d outside [1, %d]", chunk,
                              SLLM_GFX950_DEC_MAX_CHUNK);
    }
    if (n > c->n_ctx) {
        return sllm_shim_fail(SLLM_GFX950_ERR_TOO_LARGE, "forward_prefill_chunked: %d tokens > n_ctx %d", n, c->n_ctx);
    }
    for (int32_t done = 0; done < n;) {
        const int32_t take = n - done < chunk ? n - done : chunk;
        const int st = sllm_gfx950_forward_chunk(m, c, tokens + done, take, done,
                                                 logits != NULL ? logits + (size_t) done * (size_t) m->n_vocab : NULL);
        if (st != SLLM_GFX950_OK) return st;
        done += take;
    }
    return SLLM_GFX950_OK;
}
