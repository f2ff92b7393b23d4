/*
 * sllm_gfx950.h -- C ABI of the MI355X (gfx950) I2_S ternary kernel row.
 *
 * libsllm_gfx950.so is C11 host code that reaches HIP only through a thin
 * shim (hipModuleLoadData / hipModuleLaunchKernel on an embedded gfx950 code
 * object, plus device buffers). No torch, no C++ types cross this boundary:
 * plain pointers, sizes and int status codes.
 *
 * Two layers:
 *
 *  1. The kernel-row functions sllm_gfx950_i2s_* keep the exact signatures
 *     and semantics of the reference's kernel layer
 *     (include/saphira_llm/i2s_gemm.h:57-95) on HOST pointers, so the row can
 *     be installed behind the reference's kernel dispatch without touching its
 *     callers (src/forward.c:190-205, :651-793). Weights are looked up in a
 *     registry of tensors uploaded byte-for-byte at load time.
 *
 *  2. The device functions sllm_gfx950_* (no i2s_ infix) take DEVICE pointers,
 *     enqueue on the library's stream and return a status. This is the path a
 *     device-resident forward pass uses; the quantiser, GEMV and epilogue can
 *     be fused and several independent GEMVs share one launch.
 *
 * Packed I2_S tensors are the on-disk bytes unchanged: N rows of K/4 bytes in
 * the transposed 128-element tile layout, then a 32-byte tail whose first
 * four bytes are the f32 per-tensor scale (src/quant.c:72-106,
 * src/gguf.c:268-282). K must be a multiple of 128 (src/forward.c:306-316).
 *
 * Errors: functions returning int return SLLM_GFX950_OK (0) or a negative
 * status; sllm_gfx950_last_error() has the message. The void/int32 kernel-row
 * functions mirror reference signatures that cannot return a status; on any
 * failure (no device opened, unregistered weights, a HIP error) they print the
 * reason to stderr and abort(). They never fall back to a CPU computation.
 */
#ifndef SAPHIRA_AMD_SLLM_GFX950_H
#define SAPHIRA_AMD_SLLM_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. Codes the reference also has keep its sllm_status numbers
 * (include/saphira_llm/status.h:26-56); the device codes are new. */
enum {
    SLLM_GFX950_OK                 = 0,
    SLLM_GFX950_ERR_ARG            = -1,   /* SLLM_ERR_ARG                          */
    SLLM_GFX950_ERR_NOMEM          = -2,   /* SLLM_ERR_NOMEM (host or device)       */
    SLLM_GFX950_ERR_IO             = -3,   /* SLLM_ERR_IO: a model file unreadable  */
    SLLM_GFX950_ERR_UNSUPPORTED    = -4,   /* SLLM_ERR_UNSUPPORTED                  */
    SLLM_GFX950_ERR_GGUF_MAGIC     = -10,  /* SLLM_ERR_GGUF_MAGIC: not a GGUF file  */
    SLLM_GFX950_ERR_GGUF_VERSION   = -11,  /* SLLM_ERR_GGUF_VERSION: not version 3  */
    SLLM_GFX950_ERR_GGUF_TRUNCATED = -12,  /* SLLM_ERR_GGUF_TRUNCATED               */
    SLLM_GFX950_ERR_GGUF_TYPE      = -14,  /* SLLM_ERR_GGUF_TYPE: bad value type    */
    SLLM_GFX950_ERR_GGUF_TENSOR    = -15,  /* SLLM_ERR_GGUF_TENSOR: bad descriptor  */
    SLLM_GFX950_ERR_GGUF_ALIGNMENT = -16,  /* SLLM_ERR_GGUF_ALIGNMENT               */
    SLLM_GFX950_ERR_GGUF_LAYOUT    = -17,  /* SLLM_ERR_GGUF_LAYOUT: extent / overlap */
    SLLM_GFX950_ERR_GGUF_KEYDUP    = -18,  /* SLLM_ERR_GGUF_KEYDUP                  */
    SLLM_GFX950_ERR_ARCH           = -30,  /* SLLM_ERR_ARCH_UNSUPPORTED             */
    SLLM_GFX950_ERR_KV_MISSING     = -31,  /* SLLM_ERR_KV_MISSING (or mistyped)     */
    SLLM_GFX950_ERR_TENSOR_SHAPE   = -34,  /* SLLM_ERR_TENSOR_SHAPE: K % 128 != 0   */
    SLLM_GFX950_ERR_TOO_LARGE      = -36,  /* SLLM_ERR_TOO_LARGE: K above the limit */
    SLLM_GFX950_ERR_NO_DEVICE      = -60,  /* no gfx950 device, or library not open */
    SLLM_GFX950_ERR_HIP            = -61,  /* a HIP runtime call failed             */
    SLLM_GFX950_ERR_NOT_REGISTERED = -62   /* host weights not in any registered tensor */
};

/* Elements per I2_S block (include/saphira_llm/i2s_gemm.h:25). */
#define SLLM_GFX950_QK    128
/* Largest K the GEMV stages in LDS (one int8 activation row). */
#define SLLM_GFX950_MAX_K 65536

/* Per-row activation metadata. Same layout as sllm_i2s_act
 * (include/saphira_llm/i2s_gemm.h:37-40): 8 bytes, scale then sum. */
typedef struct sllm_gfx950_act {
    float   scale;   /* 127 / amax, or 0 for an all-zero row */
    int32_t sum;     /* sum of the quantised values          */
} sllm_gfx950_act;

/* ------------------------------------------------------------------ */
/* lifecycle                                                           */
/* ------------------------------------------------------------------ */

/* Open HIP device `device`, check it is gfx950, load the code object and
 * create the library stream. Called once at model load, as the reference
 * selects its kernel in sllm_model_load (src/forward.c:334). Idempotent. */
int         sllm_gfx950_open(int device);
void        sllm_gfx950_close(void);
int         sllm_gfx950_is_open(void);
const char *sllm_gfx950_status_string(int status);
const char *sllm_gfx950_last_error(void);
/* name: device marketing/arch name; cu: compute units; hbm: bytes of HBM */
int         sllm_gfx950_device_info(char *name, size_t name_len, int *cu, size_t *hbm);

/* ------------------------------------------------------------------ */
/* device memory and the library stream                                */
/* ------------------------------------------------------------------ */

int   sllm_gfx950_malloc(void **dptr, size_t bytes);
int   sllm_gfx950_free(void *dptr);
int   sllm_gfx950_h2d(void *dst_dev, const void *src_host, size_t bytes);   /* synchronous */
int   sllm_gfx950_d2h(void *dst_host, const void *src_dev, size_t bytes);   /* synchronous */
int   sllm_gfx950_sync(void);           /* wait for the library stream */
void *sllm_gfx950_stream(void);         /* the hipStream_t everything is enqueued on */
/* Events recorded on the library stream around enqueued work. */
int   sllm_gfx950_timer_start(void);
int   sllm_gfx950_timer_stop(float *ms);   /* waits for the stop event */
/* A numbered set of events on the library stream, for timing individual
 * launches inside a longer run: reserve n, record any of them between
 * launches, read the elapsed time between two (waits for the later one). */
int   sllm_gfx950_events_reserve(int n);
int   sllm_gfx950_event_record(int i);
int   sllm_gfx950_event_elapsed(int i, int j, float *ms);

/* Calibration kernels (no counterpart in the reference). A plain device
 * copy and a read-only XOR checksum (n_partials workgroup partials) of known
 * size: they measure the achievable HBM bandwidth beside the GEMV and scale
 * the HBM byte counters. bytes must be a multiple of 16, pointers 16-byte
 * aligned. */
int   sllm_gfx950_copy(void *dst, const void *src, size_t bytes);
int   sllm_gfx950_checksum(const void *src, size_t bytes, uint32_t *partials, uint32_t n_partials);

/* Diagnostic (no counterpart in the reference): the decode step's expf --
 * the restatement of the C library's expf that the softmax's scalar tail
 * runs on the device -- for the floats whose bit patterns are
 * first + i * stride (mod 2^32), i < n, into out (device memory, n floats),
 * so that a test can hold the device build against the host library. */
int   sllm_gfx950_diag_expf(uint32_t first, uint32_t stride, uint32_t n, float *out);

/* ------------------------------------------------------------------ */
/* device-pointer kernels (asynchronous, library stream)               */
/* ------------------------------------------------------------------ */

/* Replaces sllm_i2s_quant_act (include/saphira_llm/i2s_gemm.h:57-58,
 * src/i2s_gemm.c:45-83) for n_tok consecutive rows of n floats:
 * q[t*n + i], act[t]. Bit-exact with the reference. */
int sllm_gfx950_quant_act(const float *x, size_t n, size_t n_tok,
                          int8_t *q, sllm_gfx950_act *act);

/* Replaces sllm_i2s_gemv (include/saphira_llm/i2s_gemm.h:81-82,
 * src/i2s_gemm.c:260-269): rows_out[r] = sum_k code(r,k) * q[k], int32, for
 * r < n_rows, where w points at row 0 of a packed tensor (or at any row
 * boundary inside one). */
int sllm_gfx950_gemv(const uint8_t *w, size_t n_rows, size_t n,
                     const int8_t *q, int32_t *rows_out);

/* The GEMV with the epilogue fused: out[r] = (float)(dot_r - act->sum) *
 * (w_scale / act->scale), the grouping of src/i2s_gemm.c:271-290 as inlined at
 * src/forward.c:653-655. w must be the whole tensor: w_scale is read from its
 * tail at w + n_rows*n/4. */
int sllm_gfx950_gemv_epilogue(const uint8_t *w, size_t n_rows, size_t n,
                              const int8_t *q, const sllm_gfx950_act *act,
                              float *out);

/* One projection as src/forward.c:651-655 performs it: quantise x (n
 * floats), GEMV, epilogue into out (n_rows floats). q / act, when not NULL,
 * receive the quantised row and its scale/sum (give both or neither). For
 * K <= 7168 this is one launch: the slab kernel quantises x in LDS itself
 * (the quantiser's operations, so the same bits); larger K (or the
 * streaming path forced with sllm_gfx950_set_tuning) runs a quantiser
 * launch first. */
int sllm_gfx950_linear(const uint8_t *w, size_t n_rows, size_t n, const float *x,
                       int8_t *q, sllm_gfx950_act *act, float *out);

/* One independent GEMV of a batch.
 *   x != NULL: x is quantised per token (as sllm_gfx950_linear); q / act
 *              are optional outputs (both or neither), written once per
 *              job. Every job quantises its own x, with identical bits for
 *              jobs sharing one x (Q/K/V, gate/up).
 *   x == NULL: q / act are inputs (act only needed for out).
 * out and/or rows_out may be NULL, not both. Device pointers, 16-byte
 * aligned. */
typedef struct sllm_gfx950_gemv_job {
    const uint8_t   *w;         /* whole packed tensor (codes + tail)    */
    size_t           n_rows;    /* N                                     */
    size_t           n;         /* K, multiple of 128                    */
    const float     *x;         /* K f32, or NULL                        */
    int8_t          *q;         /* K int8                                */
    sllm_gfx950_act *act;       /* scale / sum                           */
    float           *out;       /* N f32 epilogue output, or NULL        */
    int32_t         *rows_out;  /* N int32 raw dots, or NULL             */
} sllm_gfx950_gemv_job;

/* Run independent GEMVs (Q, K and V against one activation, gate and up,
 * or many layers' matrices) in one launch when every K <= 7168 (else also a
 * quantiser and a streaming launch). The job tables are built and uploaded
 * on each call, and the call waits for the stream before freeing them; a
 * plan uploads them once. */
int sllm_gfx950_gemv_batch(const sllm_gfx950_gemv_job *jobs, size_t n_jobs);

/* Device memory of sllm_gfx950_gemv_batch_noalloc: a static array on each
 * device, held until the process ends. */
#define SLLM_GFX950_NOALLOC_SCRATCH_BYTES (1u << 20)
/* Most jobs one sllm_gfx950_gemv_batch_noalloc call takes. */
#define SLLM_GFX950_NOALLOC_MAX_JOBS      1024

/* sllm_gfx950_gemv_batch that allocates nothing. No counterpart in the
 * reference (whose kernels allocate nothing per call either): it is for
 * callers that cannot allocate device memory -- tight serving loops and
 * harnesses that forbid hipMalloc. The job table, the per-workgroup
 * descriptors and the quantised rows of streaming jobs that give no q / act
 * go into a static device array of SLLM_GFX950_NOALLOC_SCRATCH_BYTES instead
 * of per-call buffers; the results are sllm_gfx950_gemv_batch's, bit for
 * bit. A batch whose tables and rows exceed the array, or more than
 * SLLM_GFX950_NOALLOC_MAX_JOBS jobs, is refused with
 * SLLM_GFX950_ERR_TOO_LARGE before anything is enqueued. Every call on one
 * device shares that device's array: calls are serialised by a library lock
 * and each waits for its launches before returning, so the array is free
 * again when a call returns (nothing in it needs to start at zero). Like
 * sllm_gfx950_gemv_batch, the call synchronises the library stream. */
int sllm_gfx950_gemv_batch_noalloc(const sllm_gfx950_gemv_job *jobs, size_t n_jobs);

typedef struct sllm_gfx950_plan sllm_gfx950_plan;
int  sllm_gfx950_plan_create(const sllm_gfx950_gemv_job *jobs, size_t n_jobs,
                             sllm_gfx950_plan **plan);
int  sllm_gfx950_plan_run(const sllm_gfx950_plan *plan);
/* plan_run that also records numbered event `event` (see
 * sllm_gfx950_event_record) between the quantiser launch (present only for
 * streaming jobs carrying x) and the GEMV launches, so each can be timed on
 * the stream it runs on. */
int  sllm_gfx950_plan_run_marked(const sllm_gfx950_plan *plan, int event);
void sllm_gfx950_plan_destroy(sllm_gfx950_plan *plan);

/* ------------------------------------------------------------------ */
/* several tokens against one tensor (int8 MFMA)                       */
/* ------------------------------------------------------------------ */

/* The projections of a chunk of m tokens (src/forward.c:589-793 with
 * n = m > 1, where each token is quantised on its own and runs its own
 * GEMV and epilogue against the same tensor) as one int8-MFMA GEMM:
 *   rows_out[t][r] = sum_k code(r,k) * q[t][k]            (int32, exact)
 *   out[t][r]      = (float)(rows_out[t][r] - act[t].sum) * (w_scale / act[t].scale)
 * for t < m, r < n_rows; q is m rows of n int8 (n a multiple of 128), act m
 * scale/sum pairs, out / rows_out m rows of n_rows (either may be NULL, not
 * both; act is read only for out). w is the whole packed tensor (codes and
 * tail). Device pointers, 16-byte aligned. The results are the reference's
 * token by token, bit for bit. */
int sllm_gfx950_gemm(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                     const sllm_gfx950_act *act, size_t m, float *out, int32_t *rows_out);

/* One tensor of sllm_gfx950_gemm_multi: its packed weights and outputs, as
 * the arguments of sllm_gfx950_gemm. */
typedef struct sllm_gfx950_gemm_job {
    const uint8_t *w;
    size_t         n_rows;
    float         *out;        /* [m][n_rows] epilogue, or NULL */
    int32_t       *rows_out;   /* [m][n_rows] raw dots, or NULL (not both) */
} sllm_gfx950_gemm_job;

/* Up to three tensors of width n against the same m quantised rows in one
 * launch -- the reference's Q / K / V, or gate / up, of every token of a
 * chunk over one quantised activation (src/forward.c:645-665, :756-773).
 * Each job's outputs are what sllm_gfx950_gemm writes for it. */
int sllm_gfx950_gemm_multi(const sllm_gfx950_gemm_job *jobs, size_t n_jobs, size_t n, const int8_t *q,
                           const sllm_gfx950_act *act, size_t m);

/* Quantise m rows of x (m x n f32, one scale/sum per row, as
 * sllm_gfx950_quant_act) into q / act, then sllm_gfx950_gemm: two launches. */
int sllm_gfx950_linear_batch(const uint8_t *w, size_t n_rows, size_t n, const float *x, size_t m,
                             int8_t *q, sllm_gfx950_act *act, float *out, int32_t *rows_out);

/* A plan of GEMMs over many tensors in one launch (no counterpart in the
 * reference, whose chunk path runs each tensor of each token on its own):
 * every job is one sllm_gfx950_gemm -- its own packed tensor, K, m token
 * rows q / act and outputs -- and all jobs share m. The tables are uploaded
 * once, at creation; each run is one launch on the library stream. K must
 * be a multiple of 256 (every BitNet-2B projection); at most 2^31 row tiles.
 * Outputs are sllm_gfx950_gemm's, bit for bit. */
typedef struct sllm_gfx950_gemm_plan_job {
    const uint8_t         *w;
    size_t                 n_rows;
    size_t                 n;          /* K */
    const int8_t          *q;          /* [m][n] int8 */
    const sllm_gfx950_act *act;        /* [m]; NULL only without out */
    float                 *out;        /* [m][n_rows] epilogue, or NULL */
    int32_t               *rows_out;   /* [m][n_rows] raw dots, or NULL (not both) */
} sllm_gfx950_gemm_plan_job;

typedef struct sllm_gfx950_gemm_plan sllm_gfx950_gemm_plan;
int  sllm_gfx950_gemm_plan_create(const sllm_gfx950_gemm_plan_job *jobs, size_t n_jobs, size_t m,
                                  sllm_gfx950_gemm_plan **plan);
int  sllm_gfx950_gemm_plan_run(const sllm_gfx950_gemm_plan *plan);
void sllm_gfx950_gemm_plan_destroy(sllm_gfx950_gemm_plan *plan);

/* GEMM tile override for tuning and tests: 0 automatic (by m and the grid),
 * 1: 16 tokens x 16 rows per workgroup (K split over its waves), 2: 32 x 128,
 * 3: 64 x 128, 4: 128 x 128 staged through two LDS buffers, 5: the same
 * through one buffer, 6..9: 16 x 64, 32 x 64, 32 x 128 and 64 x 256 copied
 * straight into a ring of LDS stages, 10..13: 64 x 256, 64 x 128, 32 x 256
 * and 32 x 128 the same way with eight waves in two K groups, 14 and 15:
 * 16 x 64 and 32 x 64 with sixteen waves in four K groups (4 and up need
 * K % 256 == 0; tile 3 otherwise). A plan takes the override when it is
 * one of 6, 7, 10, 11 or 13, else its own choice. */
int sllm_gfx950_set_gemm_tile(int tile);

/* Launch-geometry override for tuning sweeps and tests; affects launches
 * and plans created afterwards. All zero (variant -1) is automatic.
 *   path           0 auto and 2: slab kernel for K <= 7168, streaming kernel
 *                  above; 1: streaming kernel for every K
 *   variant        slab geometry: 0 (8 lanes x 5 chunks per row) or 1
 *                  (16 x 7), used when it covers K; -1 auto
 *   lanes_per_row  streaming kernel: 4, 8 or 16
 *   waves          streaming kernel: waves per workgroup, 1..16
 *   rows_per_wg    streaming kernel: rows per workgroup
 *   slab_kib       slab kernel: KiB of packed weights per workgroup (0: 136) */
int sllm_gfx950_set_tuning(int path, int variant, int lanes_per_row, int waves, int rows_per_wg,
                           int slab_kib);

/* ------------------------------------------------------------------ */
/* host-pointer kernel row (the reference's signatures)                */
/* ------------------------------------------------------------------ */

/* Upload a packed I2_S tensor (n_rows*n/4 code bytes + 32-byte tail)
 * byte-for-byte and remember it under its host address, so the kernel-row
 * functions below can be handed the same borrowed pointers the reference's
 * model holds (include/saphira_llm/forward.h:27-31). Registering the same
 * range again (a second model over one image) shares the device copy and
 * counts a reference; unregister drops one and frees the copy with the last.
 * A range that overlaps a registered one otherwise is refused (-1). */
int sllm_gfx950_tensor_register(const void *packed, size_t n_rows, size_t n);
int sllm_gfx950_tensor_unregister(const void *packed);
/* The kernel row's own upload on first use, standing in for a registration
 * at load: the first sllm_gemv of a whole matrix (src/forward.c:196-205)
 * acquires it -- uploaded as register does, unless a registered or acquired
 * tensor already covers its n_rows*n/4 + 32 bytes (then nothing happens).
 * A range that overlaps one otherwise is refused (-1). Acquired copies are
 * not counted per model: release_acquired drops them all (a model still in
 * use acquires its tensors again on its next GEMV), which the row does when
 * a model is freed (sllm_model_free, src/forward.c:457). Registered ranges
 * are left as they are. */
int sllm_gfx950_tensor_acquire(const void *packed, size_t n_rows, size_t n);
int sllm_gfx950_tensor_release_acquired(void);
/* The device copy of a registered host address (inside any tensor), or NULL. */
const void *sllm_gfx950_tensor_device(const void *host);

/* src/i2s_gemm.c:45-83 on the GPU. */
void    sllm_gfx950_i2s_quant_act(const float *x, size_t n, int8_t *q_out,
                                  sllm_gfx950_act *out);
/* src/i2s_gemm.c:246-258: one row; 0 when w or q is NULL or n < 128. */
int32_t sllm_gfx950_i2s_dot(const uint8_t *w, const int8_t *q, size_t n);
/* src/i2s_gemm.c:260-269: w may be any row boundary inside a registered
 * tensor (src/forward.c:190-194 passes w + begin*row_bytes). Returns without
 * writing when w, q or rows_out is NULL. */
void    sllm_gfx950_i2s_gemv(const uint8_t *w, size_t n_rows, size_t n,
                             const int8_t *q, int32_t *rows_out);

#ifdef __cplusplus
}
#endif

#endif /* SAPHIRA_AMD_SLLM_GFX950_H */
