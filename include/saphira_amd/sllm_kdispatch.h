/*
 * sllm_kdispatch.h -- kernel dispatch for the I2_S ternary path.
 *
 * The reference selects its ternary kernel through one function pointer,
 * g_dot, installed once at model load before any worker exists
 * (src/i2s_gemm.c:239-258, :315-363; src/forward.c:334), and its op executor
 * reaches the kernels through sllm_gemv / sllm_i2s_quant_act
 * (src/forward.c:190-205, :651-793). This header widens that pointer into a
 * table of rows, one per kernel family, each carrying the full kernel-layer
 * signature set of include/saphira_llm/i2s_gemm.h:57-82. The op executor
 * calls sllm_kdispatch_*; which silicon answers is decided once, at load.
 *
 * This library ships exactly one row, "gfx950" (libsllm_gfx950). A host that
 * also has CPU kernels (the reference's scalar / v3 / vnni) registers them as
 * further rows with sllm_kdispatch_register. There is no silent fallback
 * between rows: selecting an unavailable row fails, and calling through the
 * table with no row installed aborts with a message.
 */
#ifndef SAPHIRA_AMD_SLLM_KDISPATCH_H
#define SAPHIRA_AMD_SLLM_KDISPATCH_H

#include <stddef.h>
#include <stdint.h>

#include <saphira_amd/sllm_gfx950.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sllm_kernel_row {
    const char *name;                    /* "gfx950", "vnni", ...                 */
    int         priority;                /* higher wins under "auto"              */
    /* Bring the row up (open the device, ...). Returns 0 when usable. */
    int     (*open)(void);
    /* include/saphira_llm/i2s_gemm.h:57-58 */
    void    (*quant_act)(const float *x, size_t n, int8_t *q_out, sllm_gfx950_act *out);
    /* include/saphira_llm/i2s_gemm.h:72 */
    int32_t (*dot)(const uint8_t *w, const int8_t *q, size_t n);
    /* include/saphira_llm/i2s_gemm.h:81-82 */
    void    (*gemv)(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q, int32_t *rows_out);
    /* Drop what the row holds for freed models (the gfx950 row: the device
     * copies its GEMVs uploaded), or NULL. No counterpart in the reference,
     * whose CPU rows hold nothing: sllm_model_free (src/forward.c:457)
     * calls it through sllm_kdispatch_release. */
    void    (*release)(void);
} sllm_kernel_row;

#define SLLM_KDISPATCH_MAX_ROWS 8

/* Add a row (copied). Returns SLLM_GFX950_ERR_ARG on a bad or duplicate row
 * or a full table. Must happen before select, like the reference's rule that
 * the kernel is chosen before any worker exists (src/forward.c:324-334). */
int  sllm_kdispatch_register(const sllm_kernel_row *row);
/* Rows in the table, in registration order (the built-in gfx950 row first). */
size_t                 sllm_kdispatch_count(void);
const sllm_kernel_row *sllm_kdispatch_row(size_t i);

/* Install the row called `name`, or under "auto" the highest-priority row
 * whose open() succeeds. Returns the row's open() status on failure, in
 * which case nothing is installed. */
int  sllm_kdispatch_select(const char *name);
/* The installed row, or NULL. */
const sllm_kernel_row *sllm_kdispatch_installed(void);
/* The installed row's name, "none" before any select. The diagnostic the
 * reference reads as sllm_i2s_dot_isa / sllm_i2s_installed_isa
 * (include/saphira_llm/i2s_gemm.h:113, :137; printed by bench/tg_bench.c:231
 * and checked after model load by tests/test_i2s.c:500-537). Pinning one row
 * without "auto", the reference's sllm_i2s_select_level (i2s_gemm.h:134), is
 * sllm_kdispatch_select with that row's name. */
const char            *sllm_kdispatch_installed_name(void);
/* Forget the installed row (tests). */
void sllm_kdispatch_reset(void);

/* The op executor's calls. Abort with a message when no row is installed. */
void    sllm_kdispatch_quant_act(const float *x, size_t n, int8_t *q_out, sllm_gfx950_act *out);
int32_t sllm_kdispatch_dot(const uint8_t *w, const int8_t *q, size_t n);
/* src/forward.c:196-205's sllm_gemv with the row chosen at load: a GPU row
 * takes the whole matrix in one call; there is no CPU row split here. */
void    sllm_kdispatch_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                            int32_t *rows_out);
/* The installed row's release hook, where it has one (sllm_model_free,
 * src/forward.c:457); nothing before any select. */
void    sllm_kdispatch_release(void);

#ifdef __cplusplus
}
#endif

#endif /* SAPHIRA_AMD_SLLM_KDISPATCH_H */
