/*
 * ref_driver.c -- glue compiled WITH the reference's own sources into
 * oracle/_ref/libsllm_ref.so (test infrastructure, see sllm_oracle.h).
 *
 * The reference's row-parallel GEMV (sllm_gemv, src/forward.c:145-205) is a
 * static function inside forward.c, which pulls in the whole model. These few
 * lines restate its split policy over the reference's own pool and kernels,
 * so the CPU figure beside the GPU is the reference's code doing the work.
 */
#include <saphira_llm/i2s_gemm.h>
#include <saphira_llm/quant.h>
#include <saphira_llm/thread.h>

#include <stddef.h>
#include <stdint.h>

#define REF_ROW_GRAIN 64u          /* src/forward.c:145-147 */
#define REF_ROWS_PER_THREAD 512u   /* src/forward.c:171-173 */

sllm_pool *ref_pool_create(int threads) {
    sllm_pool_config cfg = { threads, NULL, 0, NULL };
    return sllm_pool_create(&cfg);
}

typedef struct {
    const uint8_t *w;
    size_t row_bytes, n;
    const int8_t *q;
    int32_t *out;
} ref_gemv_job;

static void ref_gemv_rows(void *vctx, size_t begin, size_t end) {
    const ref_gemv_job *j = vctx;
    sllm_i2s_gemv(j->w + begin * j->row_bytes, end - begin, j->n, j->q, j->out + begin);
}

/* src/forward.c:196-205 */
void ref_gemv(sllm_pool *pool, const uint8_t *w, size_t n_rows, size_t n,
              const int8_t *q, int32_t *out) {
    const int t = pool ? sllm_pool_threads(pool) : 1;
    const size_t min_rows = t < 2 ? (size_t) -1 : (size_t) REF_ROWS_PER_THREAD * (size_t) t;
    if (n_rows < min_rows || n_rows < 2u * REF_ROW_GRAIN) {
        sllm_i2s_gemv(w, n_rows, n, q, out);
        return;
    }
    ref_gemv_job j = { w, n / 4u, n, q, out };
    sllm_parallel_rows(pool, ref_gemv_rows, &j, n_rows, REF_ROW_GRAIN);
}

/* The same row split without the distribution threshold: every GEMV goes
 * to the pool in grain-64 chunks (the reference's policy keeps GEMVs below
 * 512 rows per thread on the calling thread). */
void ref_gemv_all(sllm_pool *pool, const uint8_t *w, size_t n_rows, size_t n,
                  const int8_t *q, int32_t *out) {
    ref_gemv_job j = { w, n / 4u, n, q, out };
    sllm_parallel_rows(pool, ref_gemv_rows, &j, n_rows, REF_ROW_GRAIN);
}

/* One projection after quantisation, as src/forward.c:652-655 does it:
 * the GEMV, then the epilogue with the tensor's trailing scale. With
 * `distribute_all` the GEMV ignores the distribution threshold. */
void ref_gemv_epilogue(sllm_pool *pool, const uint8_t *w, size_t n_rows, size_t n,
                       const int8_t *q, const sllm_i2s_act *act, int32_t *dots, float *y,
                       int distribute_all) {
    if (distribute_all) ref_gemv_all(pool, w, n_rows, n, q, dots);
    else ref_gemv(pool, w, n_rows, n, q, dots);
    const float ws = sllm_i2s_scale(w, n_rows * n);
    for (size_t r = 0; r < n_rows; ++r) {
        y[r] = sllm_i2s_epilogue(dots[r], act->sum, act->scale, ws);
    }
}

/* ------------------------------------------------------------------ */
/* the reference's own decode step, on a model held in memory          */
/* ------------------------------------------------------------------ */

#include <saphira_llm/forward.h>
#include <saphira_llm/gguf.h>

#include <stdlib.h>

/* A GGUF image parsed in place (src/gguf.c sllm_gguf_open_memory) and the
 * model loaded from it (src/forward.c:318-455). The image must outlive it. */
typedef struct ref_model {
    sllm_gguf   gguf;
    sllm_model *model;
} ref_model;

ref_model *ref_model_open(const void *image, size_t size, int *status) {
    ref_model *r = calloc(1, sizeof *r);
    if (r == NULL) { *status = SLLM_ERR_NOMEM; return NULL; }
    char err[256];
    sllm_status st = sllm_gguf_open_memory(image, size, &r->gguf, err, sizeof err);
    if (st == SLLM_OK) {
        st = sllm_model_load(&r->gguf, &r->model);
        if (st != SLLM_OK) sllm_gguf_close(&r->gguf);
    }
    *status = (int) st;
    if (st != SLLM_OK) { free(r); return NULL; }
    return r;
}

void ref_model_close(ref_model *r) {
    if (r == NULL) return;
    sllm_model_free(r->model);
    sllm_gguf_close(&r->gguf);
    free(r);
}

sllm_ctx *ref_ctx_new(ref_model *r, int32_t n_ctx) {
    sllm_ctx *c = NULL;
    return sllm_ctx_new(r->model, n_ctx, &c) == SLLM_OK ? c : NULL;
}

void ref_ctx_free(sllm_ctx *c) { sllm_ctx_free(c); }

void ref_ctx_set_pool(sllm_ctx *c, sllm_pool *pool) { sllm_ctx_set_pool(c, pool); }

/* src/forward.c:846-849 */
int ref_forward(ref_model *r, sllm_ctx *c, int32_t token, int32_t pos, float *logits) {
    return (int) sllm_forward(r->model, c, token, pos, logits);
}

/* defined in src/forward.c:876-883 without a header declaration */
int32_t sllm_argmax(const float *logits, int32_t n);
int32_t ref_argmax(const float *logits, int32_t n) { return sllm_argmax(logits, n); }

/* src/forward.c:1038-1100: restore a saved cache and the last logits */
int ref_state_load(ref_model *r, sllm_ctx *c, const char *path) {
    return (int) sllm_state_load(r->model, c, path);
}

/* src/forward.c:589-835 (n tokens as one chunk) and :846-868 */
int ref_forward_chunk(ref_model *r, sllm_ctx *c, const int32_t *tokens, int32_t n, int32_t base, float *logits) {
    return (int) sllm_forward_chunk(r->model, c, tokens, n, base, logits);
}

int ref_prefill_chunked(ref_model *r, sllm_ctx *c, const int32_t *tokens, int32_t n, int32_t chunk, float *logits) {
    return (int) sllm_forward_prefill_chunked(r->model, c, tokens, n, chunk, logits);
}
