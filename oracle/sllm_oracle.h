/*
 * sllm_oracle.h -- CPU restatement of saphira-llm's I2_S ternary path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT. Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or, for bench.py, as the CPU figure reported beside the GPU). The
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

#ifdef __cplusplus
}
#endif

#endif /* SLLM_ORACLE_H */
