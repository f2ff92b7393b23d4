/*
 * sllm_oracle.h -- CPU restatement of saphira-llm's I2_S ternary path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT. Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load this library, and only to check
 * GPU results (or, for bench.py, for the CPU figure reported beside the GPU). The
 * product path (saphira-llm_amd/) never links, loads or calls it.
 *
 * Every function restates the reference behaviour at the file:line given
 * beside it (paths relative to the saphira-llm source tree). The restatement
 * is written from the documented algorithm, not copied; where the order of
 * operations fixes the bits (quantiser, epilogue) the order is kept.
 *
 * Pinning (how each function is checked against something other than
 * itself; the tests named live in tests/test_oracle.py):
 *   orc_code / orc_dequant / orc_scale  -- upstream converter vectors
 *       (i2s-converter.txt: packed bytes + independently decoded values),
 *       the converter-definition packer, and the scale-offset KAT.
 *   orc_quant_act   -- the upstream-held LCG activation (act_scale/act_sum
 *       recorded in i2s-reference.txt at n=2560 and n=6912) and the
 *       zero-row / max-2 KATs.
 *   orc_dot_*       -- brute force over decoded codes, the identity
 *       sum(c*q) - sum(q) == sum((c-1)*q), and agreement of the scalar, AVX2
 *       and AVX-VNNI forms; plus the compiled reference where it is built.
 *   orc_epilogue    -- the upstream (dot, epilogue) value pairs recorded in
 *       i2s-reference.txt, and the grouping KAT.
 */
#ifndef SLLM_ORACLE_H
#define SLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_I2S_QK 128

typedef struct orc_act {
    float   scale;   /* 127 / amax, or 0 for an all-zero row */
    int32_t sum;     /* sum of the quantised values          */
} orc_act;

/* dot kernels the oracle can run (mirrors the reference's v3 / VNNI levels) */
enum { ORC_DOT_SCALAR = 0, ORC_DOT_V3 = 1, ORC_DOT_VNNI = 2 };

/* src/i2s_gemm.c:45-83 */
void    orc_quant_act(const float *x, size_t n, int8_t *q, orc_act *act);
/* the same, over m consecutive rows of n values (one act per row) */
void    orc_quant_act_rows(const float *x, size_t n, size_t m, int8_t *q, orc_act *act);

/* src/i2s_gemm.c:89-112 */
int32_t orc_dot_scalar(const uint8_t *w, const int8_t *q, size_t n);
/* src/i2s_gemm.c:143-185 (AVX2 maddubs form) */
int32_t orc_dot_v3(const uint8_t *w, const int8_t *q, size_t n);
/* src/i2s_gemm.c:189-237 (AVX-VNNI, four accumulators) */
int32_t orc_dot_vnni(const uint8_t *w, const int8_t *q, size_t n);
int     orc_vnni_supported(void);

/* src/i2s_gemm.c:246-269: rows_out[r] = dot(w + r*n/4, q, n) */
void    orc_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                 int32_t *rows_out, int path);

/* src/i2s_gemm.c:271-290 */
float   orc_epilogue(int32_t dot, int32_t act_sum, float act_scale, float w_scale);

/* src/quant.c:77-100, :102-106, :140-146 */
uint8_t orc_code(const uint8_t *packed, size_t k);
float   orc_scale(const void *packed, size_t n_elements);
void    orc_dequant(const void *packed, float *dst, size_t n);

/* tests/harness.h:105-126: pack codes {0,1,2} by the converter's definition */
void    orc_pack_converter(uint8_t *dst, const uint8_t *codes, size_t n);

/*
 * One projection as src/forward.c:651-655 runs it: quantise x (one row of n),
 * GEMV against n_rows rows, epilogue with the tensor's trailing scale.
 * q_out / dots_out / act_out may be NULL.
 */
void    orc_linear(const uint8_t *w, size_t n_rows, size_t n, const float *x,
                   float *y, int8_t *q_out, int32_t *dots_out, orc_act *act_out,
                   int path);

/*
 * Row-parallel GEMV for CPU timing: the split policy of src/forward.c:145-205
 * (serial below 512 rows per thread or 2*64 rows; else grain-64 chunks)
 * over a pthread pool with an atomic cursor (src/thread.c:389-465 semantics).
 */
typedef struct orc_pool orc_pool;
orc_pool *orc_pool_create(int threads);
void      orc_pool_destroy(orc_pool *p);
int       orc_pool_threads(const orc_pool *p);
void      orc_gemv_parallel(orc_pool *p, const uint8_t *w, size_t n_rows, size_t n,
                            const int8_t *q, int32_t *rows_out, int path);
/* the parallel GEMV followed by the epilogue (src/forward.c:652-655) */
void      orc_gemv_epilogue_parallel(orc_pool *p, const uint8_t *w, size_t n_rows, size_t n,
                                     const int8_t *q, const orc_act *act, int32_t *dots,
                                     float *y, int path);

/* FNV-1a 64 as tests/test_i2s.c:42-50 hashes fixtures */
uint64_t  orc_fnv1a64(const void *data, size_t n);

/*
 * The decode step (sllm_oracle_fwd.c): the float operations of
 * src/ops.c and the token loop of src/forward.c:589-835, in the reference's
 * order, lane by lane. Pinned against the reference's ops.c / forward.c
 * compiled into oracle/_ref (tests/test_oracle_fwd.py).
 */
float    orc_f16_to_f32(uint16_t h);
float    orc_f16_to_f32_embd(uint16_t h);                                                  /* src/forward.c:239-262 */
void     orc_rms_norm(float *dst, const float *x, const float *weight, size_t n, float eps); /* src/ops.c:254-322 */
float    orc_v_expf(float x);                                                              /* src/ops.c:342-379 */
void     orc_softmax(float *x, size_t n);                                                  /* src/ops.c:386-422 */
void     orc_silu(float *x, size_t n);                                                     /* src/ops.c:428-440 */
void     orc_rope_neox(float *x, size_t n_rot, int32_t pos, float theta, float freq_scale); /* src/ops.c:467-549 */
void     orc_rope_cos_sin(size_t n_rot, int32_t pos, float theta, float freq_scale, float *cs, float *sn);
float    orc_dot_f16(const uint16_t *row, const float *x, size_t n);                       /* src/ops.c:106-154 */
int32_t  orc_argmax(const float *logits, int32_t n);                                       /* src/forward.c:876-883 */

/* A BitNet-b1.58 model held in host memory (the fields of sllm_model that
 * the decode step reads, src/forward.c:318-455). I2_S tensors include their
 * 32-byte tails. */
typedef struct orc_layer {
    const uint8_t *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    const float   *attn_norm, *attn_sub_norm, *ffn_norm, *ffn_sub_norm;
} orc_layer;

typedef struct orc_model {
    int32_t          n_layer, n_embd, n_ff, n_head, n_head_kv, n_rot, n_vocab;
    float            eps, rope_base;
    const uint16_t  *tok_embd;       /* n_vocab x n_embd f16, also the lm_head */
    const float     *output_norm;
    const orc_layer *layers;
} orc_model;

typedef struct orc_ctx orc_ctx;
orc_ctx *orc_ctx_new(const orc_model *m, int32_t n_ctx);
void     orc_ctx_free(orc_ctx *c);
/* [layer][head_kv][pos][head_dim] f32 caches (src/forward.c:466-518) */
float   *orc_ctx_k_cache(orc_ctx *c);
float   *orc_ctx_v_cache(orc_ctx *c);
/*
 * One token at position pos (src/forward.c:589-835, n = 1): logits of every
 * vocabulary row. dots_trace, when not NULL, receives every projection's raw
 * int32 dots in order (per layer q, k, v, o, gate, up, down); act_trace, when
 * not NULL, every activation's scale/sum (per layer: attn, o, ffn, down).
 * lm_threads splits the lm_head rows (results do not depend on it).
 */
int      orc_forward_token(const orc_model *m, orc_ctx *c, int32_t token, int32_t pos, float *logits,
                           int lm_threads, int32_t *dots_trace, orc_act *act_trace);

#ifdef __cplusplus
}
#endif

#endif /* SLLM_ORACLE_H */
