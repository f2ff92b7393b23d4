/*
 * shim_internal.h -- what the library's C files share and do not export.
 *
 * gfx950_shim.c owns the device, the stream and the loaded code objects;
 * decode.c builds on them. Everything here has hidden visibility: the
 * exported interface is the headers under include/saphira_amd.
 */
#ifndef SLLM_SHIM_INTERNAL_H
#define SLLM_SHIM_INTERNAL_H

#include <saphira_amd/sllm_gfx950.h>

#include <hip/hip_runtime_api.h>

#include <stdint.h>

#define SLLM_HIDDEN __attribute__((visibility("hidden")))

/* device-side argument layouts, mirrors of i2s_device.h */
typedef struct k_gemv_job {
    const uint8_t         *w;
    const float           *x;
    int8_t                *q;
    sllm_gfx950_act       *act;
    float                 *out_f;
    int32_t               *out_i;
    uint32_t               n_rows;
    uint32_t               k;
    uint32_t               variant;
    uint32_t               pad;
} k_gemv_job;

/* One workgroup's share of a job (mirror of wg_desc): slab a of b slabs for
 * the slab kernels, rows [a, b) for the streaming kernel. */
typedef struct k_wg_desc {
    uint32_t job;
    uint32_t a;
    uint32_t b;
    uint32_t flags;
} k_wg_desc;

enum { WG_PUBLISH = 1, WG_PAIR = 2 };

_Static_assert(sizeof(k_gemv_job) == 64, "k_gemv_job must match gemv_job in i2s_device.h");
_Static_assert(sizeof(k_wg_desc) == 16, "k_wg_desc must match wg_desc in i2s_device.h");

/* slab geometry of the device code: variant 0 (K <= 2560) puts 8 lanes on a
 * row, variant 1 (K <= 7168) 16; a workgroup of four waves covers one group
 * of 4 * 64 / lanes rows per pass */
#define SLLM_SLAB_THREADS 256
#define SLLM_SLAB_MAX_K   7168u
#define SLLM_SLAB_MAX_ROWS 1024u
SLLM_HIDDEN int      sllm_shim_slab_variant(uint32_t k);
SLLM_HIDDEN uint32_t sllm_shim_slab_group_rows(int variant);

SLLM_HIDDEN int         sllm_shim_is_open(void);
SLLM_HIDDEN hipStream_t sllm_shim_stream(void);
SLLM_HIDDEN int         sllm_shim_cu(void);
SLLM_HIDDEN int         sllm_shim_fail(int status, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
SLLM_HIDDEN int         sllm_shim_hip_fail(hipError_t e, const char *what);
/* an entry point of the decode code object */
SLLM_HIDDEN int         sllm_shim_decode_function(const char *name, hipFunction_t *f);
/* grid gx x gy of `block` threads on the library stream */
SLLM_HIDDEN int         sllm_shim_launch(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t block,
                                         uint32_t lds, void **args);
SLLM_HIDDEN int         sllm_shim_launch_3d(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz,
                                            uint32_t block, uint32_t lds, void **args);

/* A chunk's Q + K + V GEMM (jobs 0, 1, 2, each with an f32 output) with the
 * attention's cache store in its epilogue (mirror of gemm_rope in
 * i2s_kernels.hip): queries roped in place in jobs[0].out, keys roped into
 * k_cache and values into v_cache (both slice-major), token t at position
 * pos0 + t; jobs[1].out and jobs[2].out are not written.
 * SLLM_SHIM_NOT_FUSED (nothing launched) where the chosen tile does not
 * hold whole heads: the caller then runs the plain GEMM and its own store. */
typedef struct k_gemm_rope {
    const float *rope;
    float       *k_cache, *v_cache;
    uint32_t     n_ctx, hd, half, pos0;
} k_gemm_rope;
_Static_assert(sizeof(k_gemm_rope) == 40, "k_gemm_rope must match gemm_rope in i2s_kernels.hip");
#define SLLM_SHIM_NOT_FUSED 1
SLLM_HIDDEN int         sllm_shim_gemm_qkv_rope(const sllm_gfx950_gemm_job jobs[3], size_t n, const int8_t *q,
                                                const sllm_gfx950_act *act, size_t m, const k_gemm_rope *r);

/* A chunk's gate + up GEMM (two tensors of n_rows x n) whose epilogue writes
 * h = silu(gate) * up into out ([m][n_rows] f32) in place of the two
 * products. SLLM_SHIM_NOT_FUSED (nothing launched) where the token count
 * picks a tile without a gate + up form: the caller then runs the plain
 * GEMM and its own SiLU. */
/* A chunk's single-tensor GEMM whose epilogue adds a residual of the
 * output's shape: out = w . q (the f32 epilogue) + res. SLLM_SHIM_NOT_FUSED
 * (nothing launched) where the token count picks a tile without that form. */
SLLM_HIDDEN int         sllm_shim_gemm_res(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                                           const sllm_gfx950_act *act, size_t m, float *out, const float *res);
SLLM_HIDDEN int         sllm_shim_gemm_glu(const uint8_t *w_gate, const uint8_t *w_up, size_t n_rows, size_t n,
                                           const int8_t *q, const sllm_gfx950_act *act, size_t m, float *out);

/* noalloc.hip: the address on `device` (current) of the static array behind
 * sllm_gfx950_gemv_batch_noalloc; 0 or the HIP error */
SLLM_HIDDEN int         sllm_noalloc_resolve(int device, void **out);

#endif /* SLLM_SHIM_INTERNAL_H */
