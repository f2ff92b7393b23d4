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
