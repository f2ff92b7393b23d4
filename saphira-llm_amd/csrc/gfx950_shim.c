/*
 * gfx950_shim.c -- the thin C11 shim between the host code and HIP.
 *
 * Loads the gfx950 code objects built from i2s_kernels.hip and
 * decode_kernels.hip (embedded in this library at build time) with
 * hipModuleLoadData, launches its entry points
 * with hipModuleLaunchKernel on one library-owned stream, and owns the device
 * buffers: registered weight tensors, per-call scratch and job tables.
 *
 * Argument structs passed by value (gemv_job) mirror the device structs in
 * i2s_kernels.hip field for field; their sizes are asserted below.
 */
#define _POSIX_C_SOURCE 200809L

#include "shim_internal.h"

#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ */
/* the embedded code object                                            */
/* ------------------------------------------------------------------ */

#ifndef SLLM_GFX950_HSACO
#error "SLLM_GFX950_HSACO must name the gfx950 code object to embed"
#endif

extern const unsigned char sllm_gfx950_code_object[];
extern const unsigned char sllm_gfx950_code_object_end[];
__asm__(".section .rodata.sllm_gfx950_code_object,\"a\",@progbits\n"
        ".balign 4096\n"
        ".hidden sllm_gfx950_code_object\n"
        ".globl sllm_gfx950_code_object\n"
        "sllm_gfx950_code_object:\n"
        ".incbin \"" SLLM_GFX950_HSACO "\"\n"
        ".hidden sllm_gfx950_code_object_end\n"
        ".globl sllm_gfx950_code_object_end\n"
        "sllm_gfx950_code_object_end:\n"
        ".byte 0\n"
        ".previous\n");

#ifndef SLLM_GFX950_DEC_HSACO
#error "SLLM_GFX950_DEC_HSACO must name the decode code object to embed"
#endif

extern const unsigned char sllm_gfx950_decode_object[];
__asm__(".section .rodata.sllm_gfx950_decode_object,\"a\",@progbits\n"
        ".balign 4096\n"
        ".hidden sllm_gfx950_decode_object\n"
        ".globl sllm_gfx950_decode_object\n"
        "sllm_gfx950_decode_object:\n"
        ".incbin \"" SLLM_GFX950_DEC_HSACO "\"\n"
        ".byte 0\n"
        ".previous\n");

/* ------------------------------------------------------------------ */
/* device-side argument layouts (k_gemv_job, k_wg_desc: shim_internal.h) */
/* ------------------------------------------------------------------ */

_Static_assert(sizeof(sllm_gfx950_act) == 8, "sllm_gfx950_act must match sllm_i2s_act");

enum { LPR_4 = 0, LPR_8 = 1, LPR_16 = 2, N_LPR = 3 };
static const int k_lpr_value[N_LPR] = { 4, 8, 16 };
static const char *const k_stream_names[N_LPR] = {
    "sllm_k_gemv_stream_l4", "sllm_k_gemv_stream_l8", "sllm_k_gemv_stream_l16"
};

#define QUANT_THREADS 256
#define QUANT_HOST_THREADS 1024   /* sllm_k_quant_host: QH_THREADS */

/* ------------------------------------------------------------------ */
/* library state                                                       */
/* ------------------------------------------------------------------ */

typedef struct reg_tensor {
    const uint8_t *host;
    size_t         bytes;    /* n_rows*n/4 + 32 */
    uint8_t       *dev;
    size_t         refs;     /* registrations of this exact range */
    int            acquired; /* the kernel row uploaded it on first use */
} reg_tensor;

/* One row for the list quantiser (mirror of quant_job in i2s_kernels.hip). */
typedef struct k_quant_job {
    const float     *x;
    int8_t          *q;
    sllm_gfx950_act *act;
    uint32_t         n;
    uint32_t         pad;
} k_quant_job;

_Static_assert(sizeof(k_quant_job) == 32, "k_quant_job must match quant_job in i2s_kernels.hip");

/*
 * A batch of GEMVs as launches: one list-quantiser launch for the distinct
 * activations of streaming jobs that carry f32 x, one slab launch, one
 * streaming launch. Device tables, in this order: quant list, jobs, slab
 * workgroup descriptors, streaming workgroup descriptors.
 */
struct sllm_gfx950_plan {
    void      *tables_dev;
    void      *scratch_dev;    /* q / act of streaming jobs that quantise without giving buffers */
    uint32_t   n_quant;
    uint32_t   n_jobs;
    uint32_t   slab_wg;        /* multiple of 8 (empty descriptors pad it) */
    uint32_t   st_wg, st_lds, st_threads;
    int        st_lpr_idx;
    uint64_t   slab_target;    /* bytes of packed weights per slab */
};

static struct {
    int            open;
    int            device;
    int            cu;
    size_t         hbm;
    char           name[520];
    hipModule_t    mod, dec_mod;
    hipFunction_t  k_quant, k_quant_list, k_quant_host, k_host_done;
    hipFunction_t  k_slab;
    hipFunction_t  k_stream[N_LPR];
    hipFunction_t  k_copy;
    hipFunction_t  k_gemm[15];
    hipFunction_t  k_gemm_t[5];
    hipFunction_t  k_gemm_s;             /* plans of a few tokens as one stream per workgroup */
    hipFunction_t  k_gemm_rope[2];       /* dk2x2, dk4x4 with the chunk's cache store */
    hipFunction_t  k_gemm_glu[2];        /* dk2x2, dk4x4 gate + up with silu(gate) * up */
    hipFunction_t  k_gemm_res[4];        /* dk2x2, dk4x4, dq1x1, dq2x1 with a residual added */
    int            force_gemm_tile;
    hipFunction_t  k_checksum;
    hipStream_t    stream;
    hipEvent_t     ev_start, ev_stop;
    hipEvent_t    *events;
    int            n_events;
    /* tuning overrides (0 / -1 = automatic) */
    int            force_path, force_variant, force_lpr, force_waves, force_rows, slab_kib;
    /* q / act for sllm_gfx950_linear when the caller gives none */
    void          *lin_scratch;
    /* registry for the host-pointer row */
    reg_tensor    *regs;
    size_t         n_regs, cap_regs;
    /* the host-pointer row's staging: pinned host memory the kernels read
     * and write directly (pin_q: the list-quantiser table, act and q as
     * last returned; pin_io: x in, int32 rows out), and the device copy of
     * the quantised vector the GEMVs read, valid for the host buffer last_q
     * while its bytes equal pin_q's */
    uint8_t       *pin_q, *pin_q_dev;
    size_t         pin_q_cap;
    uint8_t       *pin_io, *pin_io_dev;
    size_t         pin_io_cap;
    int8_t        *dq;
    size_t         dq_cap;
    const int8_t  *last_q;
    size_t         last_n;
    uint32_t       seq;          /* last value asked of the pinned done word */
    /* the device address of noalloc.hip's static array on this device */
    void          *noalloc_dev;
} g;

/* sllm_gfx950_gemv_batch_noalloc: host staging for its tables (static, so
 * that the call allocates nothing), guarded by its own lock */
static pthread_mutex_t g_noalloc_mtx = PTHREAD_MUTEX_INITIALIZER;
static struct {
    k_quant_job quant[SLLM_GFX950_NOALLOC_MAX_JOBS];
    k_gemv_job  jobs[SLLM_GFX950_NOALLOC_MAX_JOBS];
    uint8_t     is_slab[SLLM_GFX950_NOALLOC_MAX_JOBS];
    uint8_t     tables[SLLM_GFX950_NOALLOC_SCRATCH_BYTES];
} g_noalloc;

static pthread_mutex_t g_mtx = PTHREAD_MUTEX_INITIALIZER;
static char g_err[512];

static int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

/* A failed HIP call: out of device or pinned memory is the reference's
 * SLLM_ERR_NOMEM, anything else SLLM_GFX950_ERR_HIP. */
static int hip_fail(hipError_t e, const char *what) {
    const int status = e == hipErrorOutOfMemory ? SLLM_GFX950_ERR_NOMEM : SLLM_GFX950_ERR_HIP;
    return fail(status, "%s: %s (%d)", what, hipGetErrorString(e), (int) e);
}

#define HIP_TRY(call)                                                      \
    do {                                                                   \
        const hipError_t e_ = (call);                                      \
        if (e_ != hipSuccess) return hip_fail(e_, #call);                  \
    } while (0)

const char *sllm_gfx950_last_error(void) { return g_err; }

const char *sllm_gfx950_status_string(int status) {
    switch (status) {
    case SLLM_GFX950_OK:                 return "ok";
    case SLLM_GFX950_ERR_ARG:            return "invalid-argument";
    case SLLM_GFX950_ERR_NOMEM:          return "out-of-memory";
    case SLLM_GFX950_ERR_IO:             return "io-error";
    case SLLM_GFX950_ERR_UNSUPPORTED:    return "unsupported";
    case SLLM_GFX950_ERR_GGUF_MAGIC:     return "gguf-bad-magic";
    case SLLM_GFX950_ERR_GGUF_VERSION:   return "gguf-unsupported-version";
    case SLLM_GFX950_ERR_GGUF_TRUNCATED: return "gguf-truncated";
    case SLLM_GFX950_ERR_GGUF_TYPE:      return "gguf-bad-value-type";
    case SLLM_GFX950_ERR_GGUF_TENSOR:    return "gguf-bad-tensor";
    case SLLM_GFX950_ERR_GGUF_ALIGNMENT: return "gguf-bad-alignment";
    case SLLM_GFX950_ERR_GGUF_LAYOUT:    return "gguf-bad-layout";
    case SLLM_GFX950_ERR_GGUF_KEYDUP:    return "gguf-duplicate-key";
    case SLLM_GFX950_ERR_ARCH:           return "unsupported-architecture";
    case SLLM_GFX950_ERR_KV_MISSING:     return "missing-metadata";
    case SLLM_GFX950_ERR_TENSOR_SHAPE:   return "wrong-tensor-shape";
    case SLLM_GFX950_ERR_TOO_LARGE:      return "exceeds-limit";
    case SLLM_GFX950_ERR_NO_DEVICE:      return "no-gfx950-device";
    case SLLM_GFX950_ERR_HIP:            return "hip-error";
    case SLLM_GFX950_ERR_NOT_REGISTERED: return "tensor-not-registered";
    default:                             return "unknown-status";
    }
}

/* ------------------------------------------------------------------ */
/* lifecycle                                                           */
/* ------------------------------------------------------------------ */

static int load_functions(void) {
    HIP_TRY(hipModuleGetFunction(&g.k_quant, g.mod, "sllm_k_quant_act"));
    HIP_TRY(hipModuleGetFunction(&g.k_quant_list, g.mod, "sllm_k_quant_list"));
    HIP_TRY(hipModuleGetFunction(&g.k_quant_host, g.mod, "sllm_k_quant_host"));
    HIP_TRY(hipModuleGetFunction(&g.k_host_done, g.mod, "sllm_k_host_done"));
    HIP_TRY(hipModuleGetFunction(&g.k_copy, g.mod, "sllm_k_copy"));
    HIP_TRY(hipModuleGetFunction(&g.k_checksum, g.mod, "sllm_k_checksum"));
    HIP_TRY(hipModuleGetFunction(&g.k_slab, g.mod, "sllm_k_gemv_slab"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[0], g.mod, "sllm_k_gemm_mfma_s1x1"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[1], g.mod, "sllm_k_gemm_mfma_2x2"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[2], g.mod, "sllm_k_gemm_mfma_4x2"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[3], g.mod, "sllm_k_gemm_mfma_l128"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[4], g.mod, "sllm_k_gemm_mfma_l128s"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[5], g.mod, "sllm_k_gemm_dl1x1"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[6], g.mod, "sllm_k_gemm_dl2x1"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[7], g.mod, "sllm_k_gemm_dl2x2"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[8], g.mod, "sllm_k_gemm_dl4x4"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[9], g.mod, "sllm_k_gemm_dk4x4"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[10], g.mod, "sllm_k_gemm_dk4x2"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[11], g.mod, "sllm_k_gemm_dk2x4"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[12], g.mod, "sllm_k_gemm_dk2x2"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[13], g.mod, "sllm_k_gemm_dq1x1"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm[14], g.mod, "sllm_k_gemm_dq2x1"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_rope[0], g.mod, "sllm_k_gemm_dk2x2_rope"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_rope[1], g.mod, "sllm_k_gemm_dk4x4_rope"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_glu[0], g.mod, "sllm_k_gemm_dk2x2_glu"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_glu[1], g.mod, "sllm_k_gemm_dk4x4_glu"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_res[0], g.mod, "sllm_k_gemm_dk2x2_res"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_res[1], g.mod, "sllm_k_gemm_dk4x4_res"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_res[2], g.mod, "sllm_k_gemm_dq1x1_res"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_res[3], g.mod, "sllm_k_gemm_dq2x1_res"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_t[0], g.mod, "sllm_k_gemm_tdl1x1"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_t[1], g.mod, "sllm_k_gemm_tdl2x1"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_t[2], g.mod, "sllm_k_gemm_tdk2x2"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_t[3], g.mod, "sllm_k_gemm_tdk4x2"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_t[4], g.mod, "sllm_k_gemm_tdk4x4"));
    HIP_TRY(hipModuleGetFunction(&g.k_gemm_s, g.mod, "sllm_k_gemm_s1"));
    for (int i = 0; i < N_LPR; ++i) HIP_TRY(hipModuleGetFunction(&g.k_stream[i], g.mod, k_stream_names[i]));
    g.force_variant = -1;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_open(int device) {
    pthread_mutex_lock(&g_mtx);
    int st = SLLM_GFX950_OK;
    if (g.open) {
        if (device != g.device) {
            st = fail(SLLM_GFX950_ERR_ARG, "already open on device %d", g.device);
        }
        pthread_mutex_unlock(&g_mtx);
        return st;
    }
    /* what has been created, for the unwind on failure */
    int have_mod = 0, have_dec = 0, have_stream = 0, have_ev0 = 0, have_ev1 = 0;
    int count = 0;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceCount(&count);
    if (e == hipErrorNoDevice || (e == hipSuccess && count <= 0)) {
        st = fail(SLLM_GFX950_ERR_NO_DEVICE, "no HIP device");
        goto out;
    }
    if (e != hipSuccess) { st = hip_fail(e, "hipGetDeviceCount"); goto out; }
    if (device < 0 || device >= count) {
        st = fail(SLLM_GFX950_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, count);
        goto out;
    }
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) {
        st = hip_fail(e, "hipGetDeviceProperties");
        goto out;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        st = fail(SLLM_GFX950_ERR_NO_DEVICE, "device %d is %s, not gfx950", device, prop.gcnArchName);
        goto out;
    }
    if ((e = hipSetDevice(device)) != hipSuccess) { st = hip_fail(e, "hipSetDevice"); goto out; }
    if ((e = hipModuleLoadData(&g.mod, sllm_gfx950_code_object)) != hipSuccess) {
        st = hip_fail(e, "hipModuleLoadData");
        goto unwind;
    }
    have_mod = 1;
    if ((st = load_functions()) != SLLM_GFX950_OK) goto unwind;
    if ((e = hipModuleLoadData(&g.dec_mod, sllm_gfx950_decode_object)) != hipSuccess) {
        st = hip_fail(e, "hipModuleLoadData(decode)");
        goto unwind;
    }
    have_dec = 1;
    if ((e = hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking)) != hipSuccess) {
        st = hip_fail(e, "hipStreamCreateWithFlags");
        goto unwind;
    }
    have_stream = 1;
    if ((e = hipEventCreate(&g.ev_start)) != hipSuccess) { st = hip_fail(e, "hipEventCreate"); goto unwind; }
    have_ev0 = 1;
    if ((e = hipEventCreate(&g.ev_stop)) != hipSuccess) { st = hip_fail(e, "hipEventCreate"); goto unwind; }
    have_ev1 = 1;
    if ((e = hipMalloc(&g.lin_scratch, SLLM_GFX950_MAX_K + 256)) != hipSuccess) {
        g.lin_scratch = NULL;
        st = hip_fail(e, "hipMalloc(row scratch)");
        goto unwind;
    }
    /* the no-allocation batch's device array, resolved once for this device
     * with the device current */
    {
        const int rc = sllm_noalloc_resolve(device, &g.noalloc_dev);
        if (rc != 0) {
            st = hip_fail((hipError_t) rc, "hipGetSymbolAddress(no-allocation scratch)");
            goto unwind;
        }
    }
    g.device = device;
    g.cu = prop.multiProcessorCount;
    g.hbm = prop.totalGlobalMem;
    snprintf(g.name, sizeof g.name, "%s (%s)", prop.name, prop.gcnArchName);
    g.open = 1;
    goto out;
unwind:
    if (g.lin_scratch) hipFree(g.lin_scratch);
    if (have_ev1) hipEventDestroy(g.ev_stop);
    if (have_ev0) hipEventDestroy(g.ev_start);
    if (have_stream) hipStreamDestroy(g.stream);
    if (have_dec) hipModuleUnload(g.dec_mod);
    if (have_mod) hipModuleUnload(g.mod);
    memset(&g, 0, sizeof g);
out:
    pthread_mutex_unlock(&g_mtx);
    return st;
}

void sllm_gfx950_close(void) {
    pthread_mutex_lock(&g_mtx);
    if (g.open) {
        hipStreamSynchronize(g.stream);
        for (size_t i = 0; i < g.n_regs; ++i) hipFree(g.regs[i].dev);
        free(g.regs);
        if (g.pin_q) hipHostFree(g.pin_q);
        if (g.pin_io) hipHostFree(g.pin_io);
        if (g.dq) hipFree(g.dq);
        if (g.lin_scratch) hipFree(g.lin_scratch);
        for (int i = 0; i < g.n_events; ++i) hipEventDestroy(g.events[i]);
        free(g.events);
        hipEventDestroy(g.ev_start);
        hipEventDestroy(g.ev_stop);
        hipStreamDestroy(g.stream);
        hipModuleUnload(g.dec_mod);
        hipModuleUnload(g.mod);
        memset(&g, 0, sizeof g);
    }
    pthread_mutex_unlock(&g_mtx);
}

int sllm_gfx950_is_open(void) { return g.open; }

int sllm_gfx950_device_info(char *name, size_t name_len, int *cu, size_t *hbm) {
    if (!g.open) return fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open");
    if (name && name_len) snprintf(name, name_len, "%s", g.name);
    if (cu) *cu = g.cu;
    if (hbm) *hbm = g.hbm;
    return SLLM_GFX950_OK;
}

#define NEED_OPEN()                                                             \
    do {                                                                        \
        if (!g.open) return fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open"); \
    } while (0)

/* ------------------------------------------------------------------ */
/* memory, stream, timing                                              */
/* ------------------------------------------------------------------ */

int sllm_gfx950_malloc(void **dptr, size_t bytes) {
    NEED_OPEN();
    if (dptr == NULL) return fail(SLLM_GFX950_ERR_ARG, "malloc: NULL out pointer");
    *dptr = NULL;
    const hipError_t e = hipMalloc(dptr, bytes ? bytes : 1);
    if (e == hipErrorOutOfMemory) return fail(SLLM_GFX950_ERR_NOMEM, "hipMalloc(%zu)", bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc");
    return SLLM_GFX950_OK;
}

int sllm_gfx950_free(void *dptr) {
    NEED_OPEN();
    if (dptr) HIP_TRY(hipFree(dptr));
    return SLLM_GFX950_OK;
}

int sllm_gfx950_h2d(void *dst, const void *src, size_t bytes) {
    NEED_OPEN();
    if (bytes == 0) return SLLM_GFX950_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g.stream));
    HIP_TRY(hipStreamSynchronize(g.stream));
    return SLLM_GFX950_OK;
}

int sllm_gfx950_d2h(void *dst, const void *src, size_t bytes) {
    NEED_OPEN();
    if (bytes == 0) return SLLM_GFX950_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g.stream));
    HIP_TRY(hipStreamSynchronize(g.stream));
    return SLLM_GFX950_OK;
}

int sllm_gfx950_sync(void) {
    NEED_OPEN();
    HIP_TRY(hipStreamSynchronize(g.stream));
    return SLLM_GFX950_OK;
}

void *sllm_gfx950_stream(void) { return g.open ? (void *) g.stream : NULL; }

int sllm_gfx950_timer_start(void) {
    NEED_OPEN();
    HIP_TRY(hipEventRecord(g.ev_start, g.stream));
    return SLLM_GFX950_OK;
}

int sllm_gfx950_timer_stop(float *ms) {
    NEED_OPEN();
    HIP_TRY(hipEventRecord(g.ev_stop, g.stream));
    HIP_TRY(hipEventSynchronize(g.ev_stop));
    float t = 0.0f;
    HIP_TRY(hipEventElapsedTime(&t, g.ev_start, g.ev_stop));
    if (ms) *ms = t;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_events_reserve(int n) {
    NEED_OPEN();
    if (n < 0 || n > (1 << 20)) return fail(SLLM_GFX950_ERR_ARG, "events: bad count %d", n);
    if (n <= g.n_events) return SLLM_GFX950_OK;
    HIP_TRY(hipStreamSynchronize(g.stream));
    hipEvent_t *ev = realloc(g.events, (size_t) n * sizeof *ev);
    if (ev == NULL) return fail(SLLM_GFX950_ERR_NOMEM, "events");
    g.events = ev;
    /* all or nothing: a failure destroys what this call created */
    for (int i = g.n_events; i < n; ++i) {
        const hipError_t e = hipEventCreate(&g.events[i]);
        if (e != hipSuccess) {
            while (i-- > g.n_events) hipEventDestroy(g.events[i]);
            return hip_fail(e, "hipEventCreate(events)");
        }
    }
    g.n_events = n;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_event_record(int i) {
    NEED_OPEN();
    if (i < 0 || i >= g.n_events) return fail(SLLM_GFX950_ERR_ARG, "event %d not reserved", i);
    HIP_TRY(hipEventRecord(g.events[i], g.stream));
    return SLLM_GFX950_OK;
}

int sllm_gfx950_event_elapsed(int i, int j, float *ms) {
    NEED_OPEN();
    if (i < 0 || j < 0 || i >= g.n_events || j >= g.n_events || ms == NULL) {
        return fail(SLLM_GFX950_ERR_ARG, "event_elapsed: bad arguments");
    }
    HIP_TRY(hipEventSynchronize(g.events[j]));
    HIP_TRY(hipEventElapsedTime(ms, g.events[i], g.events[j]));
    return SLLM_GFX950_OK;
}

/* ------------------------------------------------------------------ */
/* launches                                                            */
/* ------------------------------------------------------------------ */

static int launch(hipFunction_t f, uint32_t grid, uint32_t block, uint32_t lds, void **args) {
    if (grid == 0) return SLLM_GFX950_OK;
    HIP_TRY(hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, lds, g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

/* what decode.c builds on (shim_internal.h) */
int sllm_shim_is_open(void) { return g.open; }
hipStream_t sllm_shim_stream(void) { return g.stream; }
int sllm_shim_cu(void) { return g.cu; }

int sllm_shim_fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

int sllm_shim_hip_fail(hipError_t e, const char *what) { return hip_fail(e, what); }

int sllm_shim_decode_function(const char *name, hipFunction_t *f) {
    if (!g.open) return fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open");
    HIP_TRY(hipModuleGetFunction(f, g.dec_mod, name));
    return SLLM_GFX950_OK;
}

int sllm_shim_launch(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t block, uint32_t lds, void **args) {
    if (gx == 0 || gy == 0) return SLLM_GFX950_OK;
    HIP_TRY(hipModuleLaunchKernel(f, gx, gy, 1, block, 1, 1, lds, g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

int sllm_shim_launch_3d(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block, uint32_t lds,
                        void **args) {
    if (gx == 0 || gy == 0 || gz == 0) return SLLM_GFX950_OK;
    HIP_TRY(hipModuleLaunchKernel(f, gx, gy, gz, block, 1, 1, lds, g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

static uint32_t stream_grid(uint64_t n16) {
    const uint64_t cap = (uint64_t) (g.cu > 0 ? g.cu : 256) * 8;
    const uint64_t want = (n16 + 255) / 256;
    return (uint32_t) (want < cap ? (want ? want : 1) : cap);
}

int sllm_gfx950_copy(void *dst, const void *src, size_t bytes) {
    NEED_OPEN();
    if (dst == NULL || src == NULL || bytes % 16 || ((uintptr_t) dst & 15u) || ((uintptr_t) src & 15u)) {
        return fail(SLLM_GFX950_ERR_ARG, "copy: pointers 16-byte aligned, bytes a multiple of 16");
    }
    uint64_t n16 = bytes / 16;
    void *args[] = { (void *) &src, &dst, &n16 };
    return launch(g.k_copy, n16 ? stream_grid(n16) : 0, 256, 0, args);
}

int sllm_gfx950_checksum(const void *src, size_t bytes, uint32_t *partials, uint32_t n_partials) {
    NEED_OPEN();
    if (src == NULL || partials == NULL || n_partials == 0 || bytes % 16 || ((uintptr_t) src & 15u)) {
        return fail(SLLM_GFX950_ERR_ARG, "checksum: bad arguments");
    }
    uint64_t n16 = bytes / 16;
    void *args[] = { (void *) &src, &n16, &partials };
    return launch(g.k_checksum, n_partials, 256, 0, args);
}

int sllm_gfx950_diag_expf(uint32_t first, uint32_t stride, uint32_t n, float *out) {
    NEED_OPEN();
    if (n == 0) return SLLM_GFX950_OK;
    if (out == NULL) return fail(SLLM_GFX950_ERR_ARG, "diag_expf: NULL output");
    hipFunction_t f;
    HIP_TRY(hipModuleGetFunction(&f, g.dec_mod, "sllm_k_diag_expf"));
    const uint32_t grid = n / 256 + 1 < 4096u ? n / 256 + 1 : 4096u;
    void *args[] = { &first, &stride, &n, &out };
    return launch(f, grid, 256, 0, args);
}

int sllm_gfx950_quant_act(const float *x, size_t n, size_t n_tok, int8_t *q,
                          sllm_gfx950_act *act) {
    NEED_OPEN();
    if (n_tok == 0) return SLLM_GFX950_OK;
    if (x == NULL || q == NULL || act == NULL) return fail(SLLM_GFX950_ERR_ARG, "quant_act: NULL pointer");
    if (n == 0 || n > UINT32_MAX || n_tok > INT32_MAX) return fail(SLLM_GFX950_ERR_ARG, "quant_act: bad size n=%zu m=%zu", n, n_tok);
    if ((n & 3u) == 0 && (((uintptr_t) x & 15u) != 0 || ((uintptr_t) q & 3u) != 0)) {
        return fail(SLLM_GFX950_ERR_ARG, "quant_act: x must be 16-byte and q 4-byte aligned");
    }
    uint32_t n32 = (uint32_t) n;
    void *args[] = { (void *) &x, &n32, &q, &act };
    return launch(g.k_quant, (uint32_t) n_tok, QUANT_THREADS, 0, args);
}

/*
 * Launch geometry.
 *
 * Slab kernel (K <= SLAB_MAX_K: every BitNet-2B projection; the default):
 * blocks of four waves, each owning a slab of consecutive rows of one job
 * (whole groups of 4 * 64/LPR rows), sized to about slab_kib KiB of packed
 * weights so that every workgroup streams the same bytes. The geometry
 * follows K: variant 0 runs 8 lanes x 5 chunks per row
 * (K <= 2560), variant 1 16 lanes x 7 chunks (K <= 7168). A job carrying
 * f32 x is quantised inside the kernel: no quantiser launch.
 *
 * Streaming kernel (larger K, or forced with path 1): LPR lanes per row, W
 * waves looping over groups of 64/LPR rows inside a slab of rows_per_wg rows,
 * reading a quantised row staged in LDS; jobs carrying f32 x are quantised
 * first, by one list-quantiser launch per batch.
 *
 * Batches describe every workgroup with a (job, rows) descriptor, padded
 * with empty ones to a multiple of 8 so that the kernel can hand each XCD a
 * contiguous eighth of the table.
 */
#define SLAB_THREADS     256
#define SLAB_MAX_K       7168
#define SLAB_MAX_ROWS    1024
#define SLAB_DEFAULT_KIB 136     /* 32 slabs per BitNet-2B FFN matrix: 2-4 % faster than 34 (128 KiB) */

typedef struct slab_geom { int lpr, cpl; } slab_geom;
static const slab_geom k_slab_geom[2] = { { 8, 5 }, { 16, 7 } };

static int slab_variant_for(size_t k) {
    const size_t chunks = k / 64;
    if (g.force_variant >= 0) {
        const slab_geom *v = &k_slab_geom[g.force_variant];
        if ((size_t) v->lpr * (size_t) v->cpl >= chunks) return g.force_variant;
    }
    for (int i = 0; i < 2; ++i) {
        if ((size_t) k_slab_geom[i].lpr * (size_t) k_slab_geom[i].cpl >= chunks) return i;
    }
    return -1;
}

int sllm_shim_slab_variant(uint32_t k) { return slab_variant_for(k); }
uint32_t sllm_shim_slab_group_rows(int variant) { return variant == 0 ? 4 * 64 / 8 : 4 * 64 / 16; }

/* does a job of this shape take the slab kernel (else the streaming one) */
static int slab_path(size_t n_rows, size_t k) {
    if (g.force_path == 1 || k > SLAB_MAX_K) return 0;
    /* the slab kernel addresses a tensor with 32-bit offsets, and aims the
     * loads it must not make at 0xFFFF0000, past every slab tensor */
    return (uint64_t) n_rows * (k / 4) + 32 <= 0xFFFF0000u;
}

/* Slabs of a job: about `target` bytes of weights each, at least one group
 * each, and few enough groups per slab for its dots to fit in LDS. */
static uint64_t slab_default_target(void) { return (uint64_t) (g.slab_kib ? g.slab_kib : SLAB_DEFAULT_KIB) * 1024u; }

static uint32_t slab_count(size_t n_rows, size_t k, int variant, uint64_t target) {
    const uint64_t group = 4u * (uint64_t) (64 / k_slab_geom[variant].lpr);
    const uint64_t n_groups = (n_rows + group - 1) / group;
    const uint64_t max_groups = SLAB_MAX_ROWS / group;
    uint64_t slabs = ((uint64_t) n_rows * (k / 4) + target / 2) / target;
    if (slabs < (n_groups + max_groups - 1) / max_groups) slabs = (n_groups + max_groups - 1) / max_groups;
    if (slabs > n_groups) slabs = n_groups;
    if (slabs == 0) slabs = 1;
    return (uint32_t) slabs;
}


typedef struct stream_shape {
    int      lpr_idx;
    int      waves;
    uint32_t rows_per_wg;
} stream_shape;

static int lpr_index(int lpr) {
    for (int i = 0; i < N_LPR; ++i) if (k_lpr_value[i] == lpr) return i;
    return -1;
}

static stream_shape stream_shape_for(void) {
    stream_shape s;
    s.lpr_idx = g.force_lpr ? lpr_index(g.force_lpr) : LPR_8;
    s.waves = g.force_waves ? g.force_waves : 2;
    const uint32_t rpw = (uint32_t) (64 / k_lpr_value[s.lpr_idx]);
    s.rows_per_wg = g.force_rows ? (uint32_t) g.force_rows : 2u * (uint32_t) s.waves * rpw;
    return s;
}

int sllm_gfx950_set_tuning(int path, int variant, int lanes_per_row, int waves, int rows_per_wg,
                           int slab_kib) {
    if (path < 0 || path > 2) return fail(SLLM_GFX950_ERR_ARG, "path must be 0 (auto), 1 (streaming) or 2 (slab)");
    if (variant < -1 || variant > 1) return fail(SLLM_GFX950_ERR_ARG, "slab variant must be -1 (auto), 0 or 1");
    if (lanes_per_row != 0 && lpr_index(lanes_per_row) < 0) {
        return fail(SLLM_GFX950_ERR_ARG, "lanes per row must be 4, 8 or 16");
    }
    if (waves < 0 || waves > 16) return fail(SLLM_GFX950_ERR_ARG, "waves must be 0..16");
    if (rows_per_wg < 0) return fail(SLLM_GFX950_ERR_ARG, "rows per workgroup must be >= 0");
    if (slab_kib < 0 || slab_kib > 65536) return fail(SLLM_GFX950_ERR_ARG, "slab KiB must be 0..65536");
    g.force_path = path;
    g.force_variant = variant;
    g.force_lpr = lanes_per_row;
    g.force_waves = waves;
    g.force_rows = rows_per_wg;
    g.slab_kib = slab_kib;
    return SLLM_GFX950_OK;
}

static int check_weights(const uint8_t *w, size_t n_rows, size_t n) {
    if (w == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv: NULL weights");
    if (n == 0 || n % SLLM_GFX950_QK != 0) return fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "gemv: K=%zu is not a positive multiple of 128", n);
    if (n > SLLM_GFX950_MAX_K) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemv: K=%zu above %d", n, SLLM_GFX950_MAX_K);
    if (n_rows > UINT32_MAX / 2) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemv: %zu rows", n_rows);
    if (((uintptr_t) w & 15u) != 0) return fail(SLLM_GFX950_ERR_ARG, "gemv: weights must be 16-byte aligned");
    return SLLM_GFX950_OK;
}

/* Validate one public job and translate it (variant filled in later). */
static int job_to_kernel(const sllm_gfx950_gemv_job *j, size_t i, k_gemv_job *kj) {
    int st = check_weights(j->w, j->n_rows, j->n);
    if (st != SLLM_GFX950_OK) return st;
    if (j->out == NULL && j->rows_out == NULL) return fail(SLLM_GFX950_ERR_ARG, "job %zu: no output", i);
    if (j->x != NULL) {
        if (((uintptr_t) j->x & 15u) != 0) return fail(SLLM_GFX950_ERR_ARG, "job %zu: x must be 16-byte aligned", i);
        if (j->q != NULL && ((uintptr_t) j->q & 15u) != 0) return fail(SLLM_GFX950_ERR_ARG, "job %zu: q must be 16-byte aligned", i);
        if ((j->q == NULL) != (j->act == NULL)) return fail(SLLM_GFX950_ERR_ARG, "job %zu: give both q and act, or neither", i);
    } else {
        if (j->q == NULL || ((uintptr_t) j->q & 15u) != 0) return fail(SLLM_GFX950_ERR_ARG, "job %zu: q must be given and 16-byte aligned", i);
        if (j->out != NULL && j->act == NULL) return fail(SLLM_GFX950_ERR_ARG, "job %zu: the epilogue needs act", i);
    }
    *kj = (k_gemv_job) { j->w, j->x, j->q, j->act, j->out, j->rows_out, (uint32_t) j->n_rows,
                         (uint32_t) j->n, 0, 0 };
    return SLLM_GFX950_OK;
}

static size_t align256(size_t v) { return (v + 255u) & ~(size_t) 255u; }

/* streaming jobs that quantise x into plan scratch (carry x, no q / act) */
static int takes_scratch(const sllm_gfx950_gemv_job *j) {
    return j->x != NULL && j->q == NULL && !slab_path(j->n_rows, j->n);
}

/* scratch bytes for one quantised row of width k: q, then act */
static size_t row_scratch(size_t k) { return align256(k) + 256; }

/* Bytes of plan scratch: one quantised row per distinct (x, K) among the
 * jobs that take scratch. */
static size_t plan_scratch_bytes(const sllm_gfx950_gemv_job *jobs, size_t n_jobs) {
    size_t bytes = 0;
    for (size_t i = 0; i < n_jobs; ++i) {
        if (!takes_scratch(&jobs[i])) continue;
        size_t e = 0;
        while (e < i && !(takes_scratch(&jobs[e]) && jobs[e].x == jobs[i].x && jobs[e].n == jobs[i].n)) ++e;
        if (e == i) bytes += row_scratch(jobs[i].n);
    }
    return bytes;
}

/* workgroups a job takes (streaming: and the rows each one owns) */
static uint32_t job_workgroups(const k_gemv_job *kj, int slab, uint32_t *rows, uint64_t target) {
    if (slab) {
        *rows = 0;
        return slab_count(kj->n_rows, kj->k, (int) kj->variant, target);
    }
    *rows = stream_shape_for().rows_per_wg;
    return (kj->n_rows + *rows - 1) / *rows;
}

static uint64_t pad8(uint64_t v) { return (v + 7u) & ~(uint64_t) 7u; }

/*
 * Lay a batch out. `kj` (n_jobs entries) receives the jobs in submission
 * order -- streaming jobs that carried x now read their quantised row -- and
 * `kq` (n_jobs entries) the quant list: one row per distinct (x, q) among
 * streaming jobs that carry x, into the job's q / act or into plan scratch
 * (p->scratch_dev, sized by plan_scratch_bytes) shared by every scratch job
 * with the same (x, K). Sets the plan's counts; the descriptors are written
 * by plan_descriptors.
 */
static int plan_layout(const sllm_gfx950_gemv_job *jobs, size_t n_jobs, sllm_gfx950_plan *p,
                       k_quant_job *kq, k_gemv_job *kj, uint8_t *is_slab) {
    const stream_shape ss = stream_shape_for();
    uint64_t slab_wg = 0, st_wg = 0;
    size_t st_lds = 0, scratch_at = 0;
    p->n_quant = 0;
    for (size_t i = 0; i < n_jobs; ++i) {
        k_gemv_job *j = &kj[i];
        int st = job_to_kernel(&jobs[i], i, j);
        if (st != SLLM_GFX950_OK) return st;
        is_slab[i] = (uint8_t) slab_path(j->n_rows, j->k);
        if (is_slab[i]) {
            j->variant = (uint32_t) slab_variant_for(j->k);
        } else if (j->x != NULL) {
            const int scratch = j->q == NULL;
            uint32_t e = 0;
            for (; e < p->n_quant; ++e) {
                if (kq[e].x != j->x || kq[e].n != j->k || (int) kq[e].pad != scratch) continue;
                if (scratch || kq[e].q == j->q) break;
            }
            if (e == p->n_quant) {
                if (scratch) {
                    uint8_t *row = (uint8_t *) p->scratch_dev + scratch_at;
                    scratch_at += row_scratch(j->k);
                    kq[e] = (k_quant_job) { j->x, (int8_t *) row,
                                            (sllm_gfx950_act *) (row + align256(j->k)), j->k, 1 };
                } else {
                    kq[e] = (k_quant_job) { j->x, j->q, j->act, j->k, 0 };
                }
                p->n_quant++;
            }
            j->q = kq[e].q;             /* the GEMV reads the quantised row */
            j->act = kq[e].act;
            j->x = NULL;
        }
    }
    /* Slabs of the default size fill the chip with a batch of 35 MB and up;
     * a smaller batch (one FFN set, 13 MB) gets slabs sized so that its
     * workgroups still cover every CU once. */
    uint64_t slab_bytes = 0;
    for (size_t i = 0; i < n_jobs; ++i) {
        if (is_slab[i]) slab_bytes += (uint64_t) kj[i].n_rows * (kj[i].k / 4);
    }
    p->slab_target = slab_default_target();
    if (g.slab_kib == 0 && slab_bytes > 0 && slab_bytes < p->slab_target * (uint64_t) g.cu) {
        p->slab_target = (slab_bytes + (uint64_t) g.cu - 1) / (uint64_t) g.cu;
    }
    for (size_t i = 0; i < n_jobs; ++i) {
        k_gemv_job *j = &kj[i];
        uint32_t rows;
        const uint64_t wg = job_workgroups(j, is_slab[i], &rows, p->slab_target);
        if (is_slab[i]) {
            slab_wg += wg;
        } else {
            st_wg += wg;
            if (j->k > st_lds) st_lds = j->k;
        }
    }
    slab_wg = pad8(slab_wg);
    st_wg = pad8(st_wg);
    if (slab_wg > INT32_MAX || st_wg > INT32_MAX) return fail(SLLM_GFX950_ERR_TOO_LARGE, "batch: too many workgroups");
    p->n_jobs = (uint32_t) n_jobs;
    p->slab_wg = (uint32_t) slab_wg;
    p->st_wg = (uint32_t) st_wg;
    p->st_lds = (uint32_t) st_lds;
    p->st_threads = (uint32_t) (64 * ss.waves);
    p->st_lpr_idx = ss.lpr_idx;
    return SLLM_GFX950_OK;
}

/* One descriptor per workgroup: slab jobs into sd, streaming jobs into td,
 * each in job order and padded with empty descriptors. */
static void plan_descriptors(const sllm_gfx950_plan *p, const k_gemv_job *kj, const uint8_t *is_slab,
                             k_wg_desc *sd, k_wg_desc *td) {
    uint32_t ns = 0, nt = 0;
    for (uint32_t i = 0; i < p->n_jobs; ++i) {
        uint32_t rows;
        const uint32_t wg = job_workgroups(&kj[i], is_slab[i], &rows, p->slab_target);
        for (uint32_t w = 0; w < wg; ++w) {
            if (is_slab[i]) {
                sd[ns++] = (k_wg_desc) { i, w, wg, w == 0 ? WG_PUBLISH : 0 };
            } else {
                const uint32_t b = w * rows, e = b + rows < kj[i].n_rows ? b + rows : kj[i].n_rows;
                td[nt++] = (k_wg_desc) { i, b, e, 0 };
            }
        }
    }
    while (ns < p->slab_wg) sd[ns++] = (k_wg_desc) { 0, 0, 0, 0 };
    while (nt < p->st_wg) td[nt++] = (k_wg_desc) { 0, 0, 0, 0 };
}

static int launch_quant(const float *x, uint32_t n, uint32_t n_tok, int8_t *q, sllm_gfx950_act *act) {
    void *args[] = { (void *) &x, &n, &q, &act };
    return launch(g.k_quant, n_tok, QUANT_THREADS, 0, args);
}

static int plan_launch(const sllm_gfx950_plan *p, int event) {
    int st = SLLM_GFX950_OK;
    const uint8_t *base = p->tables_dev;
    const k_quant_job *kq = (const k_quant_job *) base;
    const k_gemv_job *jobs = (const k_gemv_job *) (base + p->n_quant * sizeof(k_quant_job));
    const k_wg_desc *sd = (const k_wg_desc *) (jobs + p->n_jobs);
    const k_wg_desc *td = sd + p->slab_wg;
    k_gemv_job none;
    memset(&none, 0, sizeof none);
    uint32_t zero = 0;
    if (p->n_quant) {
        void *args[] = { (void *) &kq };
        st = launch(g.k_quant_list, p->n_quant, QUANT_THREADS, 0, args);
    }
    if (st == SLLM_GFX950_OK && event >= 0) st = sllm_gfx950_event_record(event);
    if (st == SLLM_GFX950_OK && p->slab_wg) {
        uint32_t n = p->slab_wg;
        void *args[] = { (void *) &jobs, (void *) &sd, &n, &none, &zero };
        st = launch(g.k_slab, p->slab_wg, SLAB_THREADS, 0, args);
    }
    if (st == SLLM_GFX950_OK && p->st_wg) {
        uint32_t n = p->st_wg;
        void *args[] = { (void *) &jobs, (void *) &td, &n, &none, &zero };
        st = launch(g.k_stream[p->st_lpr_idx], p->st_wg, p->st_threads, p->st_lds, args);
    }
    return st;
}

int sllm_gfx950_plan_create(const sllm_gfx950_gemv_job *jobs, size_t n_jobs,
                            sllm_gfx950_plan **plan) {
    NEED_OPEN();
    if (plan == NULL) return fail(SLLM_GFX950_ERR_ARG, "plan: NULL out pointer");
    *plan = NULL;
    if (jobs == NULL || n_jobs == 0 || n_jobs > UINT32_MAX / 2) return fail(SLLM_GFX950_ERR_ARG, "plan: bad job list");
    sllm_gfx950_plan *p = calloc(1, sizeof *p);
    k_quant_job *kq = malloc(n_jobs * sizeof *kq);
    k_gemv_job *kj = malloc(n_jobs * sizeof *kj);
    uint8_t *is_slab = malloc(n_jobs);
    uint8_t *host = NULL;
    int st = SLLM_GFX950_OK;
    if (p == NULL || kq == NULL || kj == NULL || is_slab == NULL) {
        st = fail(SLLM_GFX950_ERR_NOMEM, "plan: host tables");
    }
    if (st == SLLM_GFX950_OK) {
        const size_t scratch = plan_scratch_bytes(jobs, n_jobs);
        if (scratch) {
            hipError_t e = hipMalloc(&p->scratch_dev, scratch);
            if (e != hipSuccess) st = hip_fail(e, "plan: activation scratch");
        }
    }
    if (st == SLLM_GFX950_OK) st = plan_layout(jobs, n_jobs, p, kq, kj, is_slab);
    if (st == SLLM_GFX950_OK) {
        const size_t qbytes = p->n_quant * sizeof *kq, jbytes = n_jobs * sizeof *kj;
        const size_t dbytes = ((size_t) p->slab_wg + p->st_wg) * sizeof(k_wg_desc);
        const size_t bytes = qbytes + jbytes + dbytes;
        host = malloc(bytes);
        if (host == NULL) st = fail(SLLM_GFX950_ERR_NOMEM, "plan: table staging");
        if (st == SLLM_GFX950_OK) {
            memcpy(host, kq, qbytes);
            memcpy(host + qbytes, kj, jbytes);
            k_wg_desc *sd = (k_wg_desc *) (host + qbytes + jbytes);
            plan_descriptors(p, kj, is_slab, sd, sd + p->slab_wg);
            hipError_t e = hipMalloc(&p->tables_dev, bytes);
            if (e == hipSuccess) e = hipMemcpy(p->tables_dev, host, bytes, hipMemcpyHostToDevice);
            if (e != hipSuccess) st = hip_fail(e, "plan: job tables");
        }
    }
    free(host);
    free(kq);
    free(kj);
    free(is_slab);
    if (st != SLLM_GFX950_OK) {
        if (p) {
            if (p->tables_dev) hipFree(p->tables_dev);
            if (p->scratch_dev) hipFree(p->scratch_dev);
            free(p);
        }
        return st;
    }
    *plan = p;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_plan_run(const sllm_gfx950_plan *p) {
    NEED_OPEN();
    if (p == NULL) return fail(SLLM_GFX950_ERR_ARG, "plan_run: NULL plan");
    return plan_launch(p, -1);
}

int sllm_gfx950_plan_run_marked(const sllm_gfx950_plan *p, int event) {
    NEED_OPEN();
    if (p == NULL) return fail(SLLM_GFX950_ERR_ARG, "plan_run: NULL plan");
    if (event < 0 || event >= g.n_events) return fail(SLLM_GFX950_ERR_ARG, "plan_run_marked: event %d not reserved", event);
    return plan_launch(p, event);
}

/* Free a plan whose launches have all finished. */
static void plan_free(sllm_gfx950_plan *p) {
    if (g.open) {
        hipFree(p->tables_dev);
        if (p->scratch_dev) hipFree(p->scratch_dev);
    }
    free(p);
}

void sllm_gfx950_plan_destroy(sllm_gfx950_plan *p) {
    if (p == NULL) return;
    if (g.open) hipStreamSynchronize(g.stream);
    plan_free(p);
}

/* A batch is a plan used once; its tables are freed after the stream drains. */
int sllm_gfx950_gemv_batch(const sllm_gfx950_gemv_job *jobs, size_t n_jobs) {
    NEED_OPEN();
    if (n_jobs == 0) return SLLM_GFX950_OK;
    sllm_gfx950_plan *p = NULL;
    int st = sllm_gfx950_plan_create(jobs, n_jobs, &p);
    if (st != SLLM_GFX950_OK) return st;
    st = plan_launch(p, -1);
    if (st == SLLM_GFX950_OK) {
        /* the tables are freed below: wait for the launch, and report it */
        const hipError_t e = hipStreamSynchronize(g.stream);
        if (e != hipSuccess) st = hip_fail(e, "gemv_batch");
    }
    if (st == SLLM_GFX950_OK) plan_free(p);
    else sllm_gfx950_plan_destroy(p);
    return st;
}

/* A batch laid out in the static device array: quantised rows of streaming
 * jobs first, then the tables, all staged on the host in static buffers and
 * copied in on the library stream. */
int sllm_gfx950_gemv_batch_noalloc(const sllm_gfx950_gemv_job *jobs, size_t n_jobs) {
    NEED_OPEN();
    if (n_jobs == 0) return SLLM_GFX950_OK;
    if (jobs == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv_batch_noalloc: NULL job list");
    if (n_jobs > SLLM_GFX950_NOALLOC_MAX_JOBS) {
        return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemv_batch_noalloc: %zu jobs, at most %d", n_jobs,
                    SLLM_GFX950_NOALLOC_MAX_JOBS);
    }
    const size_t cap = SLLM_GFX950_NOALLOC_SCRATCH_BYTES;
    const size_t rows = align256(plan_scratch_bytes(jobs, n_jobs));
    if (rows > cap) {
        return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemv_batch_noalloc: %zu bytes of quantised rows, the array holds %zu",
                    rows, cap);
    }
    pthread_mutex_lock(&g_noalloc_mtx);
    sllm_gfx950_plan p;
    memset(&p, 0, sizeof p);
    p.scratch_dev = g.noalloc_dev;
    int st = plan_layout(jobs, n_jobs, &p, g_noalloc.quant, g_noalloc.jobs, g_noalloc.is_slab);
    if (st == SLLM_GFX950_OK) {
        const size_t qbytes = p.n_quant * sizeof(k_quant_job), jbytes = n_jobs * sizeof(k_gemv_job);
        const size_t dbytes = ((size_t) p.slab_wg + p.st_wg) * sizeof(k_wg_desc);
        const size_t bytes = qbytes + jbytes + dbytes;
        if (rows + bytes > cap) {
            st = fail(SLLM_GFX950_ERR_TOO_LARGE, "gemv_batch_noalloc: %zu bytes of rows and tables, the array holds %zu",
                      rows + bytes, cap);
        } else {
            uint8_t *host = g_noalloc.tables;
            memcpy(host, g_noalloc.quant, qbytes);
            memcpy(host + qbytes, g_noalloc.jobs, jbytes);
            k_wg_desc *sd = (k_wg_desc *) (host + qbytes + jbytes);
            plan_descriptors(&p, g_noalloc.jobs, g_noalloc.is_slab, sd, sd + p.slab_wg);
            p.tables_dev = (uint8_t *) g.noalloc_dev + rows;
            hipError_t e = hipMemcpyAsync(p.tables_dev, host, bytes, hipMemcpyHostToDevice, g.stream);
            if (e != hipSuccess) st = hip_fail(e, "gemv_batch_noalloc: tables");
            if (st == SLLM_GFX950_OK) st = plan_launch(&p, -1);
            /* the array and the host staging are free again once the stream drains */
            e = hipStreamSynchronize(g.stream);
            if (st == SLLM_GFX950_OK && e != hipSuccess) st = hip_fail(e, "gemv_batch_noalloc: synchronise");
        }
    }
    pthread_mutex_unlock(&g_noalloc_mtx);
    return st;
}

/* One job, passed to the kernel by value (no descriptor table). A
 * streaming job carrying x is quantised first (into its q / act, or the
 * library's row scratch); the slab kernel quantises in-kernel. */
static int single_launch(const sllm_gfx950_gemv_job *j) {
    k_gemv_job kj;
    int st = job_to_kernel(j, 0, &kj);
    if (st != SLLM_GFX950_OK) return st;
    if (kj.n_rows == 0) return SLLM_GFX950_OK;
    const k_gemv_job *no_jobs = NULL;
    const k_wg_desc *no_descs = NULL;
    uint32_t zero = 0;
    if (slab_path(kj.n_rows, kj.k)) {
        kj.variant = (uint32_t) slab_variant_for(kj.k);
        uint32_t rows, flags = 0;
        uint32_t wg = job_workgroups(&kj, 1, &rows, slab_default_target());
        if (g.slab_kib == 0) {
            /* The slab size targets batches, whose many jobs fill the chip;
             * a launch of its own spreads over one group of rows per
             * workgroup, up to one workgroup per CU. */
            const uint32_t group = 4u * (uint32_t) (64 / k_slab_geom[kj.variant].lpr);
            const uint32_t n_groups = (kj.n_rows + group - 1) / group;
            const uint32_t want = n_groups < (uint32_t) g.cu ? n_groups : (uint32_t) g.cu;
            if (wg < want) wg = want;
        }
        void *args[] = { (void *) &no_jobs, (void *) &no_descs, &zero, &kj, &flags };
        return launch(g.k_slab, wg, SLAB_THREADS, 0, args);
    }
    if (kj.x != NULL) {
        if (kj.q == NULL) {
            kj.q = (int8_t *) g.lin_scratch;
            kj.act = (sllm_gfx950_act *) ((uint8_t *) g.lin_scratch + SLLM_GFX950_MAX_K);
        }
        st = launch_quant(kj.x, kj.k, 1, kj.q, kj.act);
        if (st != SLLM_GFX950_OK) return st;
        kj.x = NULL;
    }
    const stream_shape ss = stream_shape_for();
    uint32_t rows;
    const uint32_t wg = job_workgroups(&kj, 0, &rows, slab_default_target());
    void *args[] = { (void *) &no_jobs, (void *) &no_descs, &zero, &kj, &rows };
    return launch(g.k_stream[ss.lpr_idx], wg, (uint32_t) (64 * ss.waves), kj.k, args);
}

int sllm_gfx950_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                     int32_t *rows_out) {
    NEED_OPEN();
    if (rows_out == NULL || q == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv: NULL q or rows_out");
    const sllm_gfx950_gemv_job j = { w, n_rows, n, NULL, (int8_t *) q, NULL, NULL, rows_out };
    return single_launch(&j);
}

int sllm_gfx950_gemv_epilogue(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                              const sllm_gfx950_act *act, float *out) {
    NEED_OPEN();
    if (out == NULL || act == NULL || q == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv_epilogue: NULL q, act or out");
    const sllm_gfx950_gemv_job j = { w, n_rows, n, NULL, (int8_t *) q, (sllm_gfx950_act *) act, out, NULL };
    return single_launch(&j);
}

/* ------------------------------------------------------------------ */
/* batched GEMM (i2s_kernels.hip: gemm_args)                           */
/* ------------------------------------------------------------------ */

typedef struct k_gemm_args {
    const int8_t          *q;
    const sllm_gfx950_act *act;
    const uint8_t         *w[3];
    float                 *out[3];
    int32_t               *out_i[3];
    uint32_t               n_rows[3];
    uint32_t               tiles[3];
    uint32_t               k, m, n_jobs, pad;
} k_gemm_args;

_Static_assert(sizeof(k_gemm_args) == 128, "k_gemm_args must match gemm_args in i2s_kernels.hip");

/* tile shapes per workgroup: tokens x rows (shape 0 splits K over its four
 * waves instead of spreading them along the rows; shapes 3 and 4 stage their
 * tile through LDS -- 3 with two buffers, one workgroup per CU; 4 with one,
 * two per CU; shapes 5..8 copy it straight into an LDS ring). Shapes 3 and
 * up need K % 256 == 0. */
#define N_GEMM_TILES 15
#define GEMM_DL_FIRST 5
static const uint32_t k_gemm_tokens[N_GEMM_TILES] = { 16, 32, 64, 128, 128, 16, 32, 32, 64, 64, 64, 32, 32, 16, 32 };
static const uint32_t k_gemm_rows[N_GEMM_TILES] = { 16, 128, 128, 128, 128, 64, 64, 128, 256, 256, 128, 256, 128, 64, 64 };
/* threads per workgroup: shapes 9..12 are two K groups of four waves */
static const uint32_t k_gemm_threads[N_GEMM_TILES] = { 256, 256, 256, 256, 256, 256, 256, 256, 256, 512, 512, 512, 512,
                                                       1024, 1024 };

/* workgroups of tile shape t for these jobs and tokens */
static uint64_t gemm_grid(int t, const sllm_gfx950_gemm_job *jobs, size_t n_jobs, size_t m) {
    uint64_t gx = 0;
    for (size_t j = 0; j < n_jobs; ++j) gx += (jobs[j].n_rows + k_gemm_rows[t] - 1) / k_gemm_rows[t];
    return gx * ((m + k_gemm_tokens[t] - 1) / k_gemm_tokens[t]);
}

int sllm_gfx950_set_gemm_tile(int tile) {
    if (tile < 0 || tile > N_GEMM_TILES) return fail(SLLM_GFX950_ERR_ARG, "set_gemm_tile: 0 (auto) .. %d", N_GEMM_TILES);
    g.force_gemm_tile = tile;
    return SLLM_GFX950_OK;
}

/* The launch of a GEMM over 1 to 3 jobs: arguments checked, tile shape
 * chosen, gemm_args filled. SLLM_GFX950_OK with *gx == 0: nothing to do. */
static int gemm_prepare(const sllm_gfx950_gemm_job *jobs, size_t n_jobs, size_t n, const int8_t *q,
                        const sllm_gfx950_act *act, size_t m, k_gemm_args *a, int *tile_out, uint64_t *gx_out,
                        uint64_t *gy_out) {
    *gx_out = 0;
    if (jobs == NULL || n_jobs < 1 || n_jobs > 3) return fail(SLLM_GFX950_ERR_ARG, "gemm: 1 to 3 jobs");
    if (m == 0) return SLLM_GFX950_OK;
    if (q == NULL || ((uintptr_t) q & 15u) != 0) return fail(SLLM_GFX950_ERR_ARG, "gemm: q must be given and 16-byte aligned");
    if (m > (size_t) UINT32_MAX / 2) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemm: m = %zu too large", m);
    for (size_t j = 0; j < n_jobs; ++j) {
        const int st = check_weights(jobs[j].w, jobs[j].n_rows, n);
        if (st != SLLM_GFX950_OK) return st;
        if (jobs[j].out == NULL && jobs[j].rows_out == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm: job %zu has no output", j);
        if (jobs[j].out != NULL && act == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm: the epilogue needs act");
        if ((uint64_t) m * jobs[j].n_rows > (uint64_t) 1 << 40) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemm: m x rows too large");
    }
    int tile = g.force_gemm_tile - 1;
    if (tile < 0 && n % 256 == 0) {
        /* measured on MI355X (K = 2560 and 6912, 4 to 512 tokens): the
         * direct-load tiles win everywhere. Up to 64 tokens the sixteen-wave
         * 16 x 64 / 32 x 64 tiles (four K groups; each tensor streamed once
         * per token tile); to 256 tokens the eight-wave 32 x 128, or 32 x 64
         * when that grid would cover under half the CUs; above 256 tokens the
         * eight-wave 64 x 256 when its grid covers three quarters of the
         * CUs, else 32 x 128. */
        const uint64_t cu = (uint64_t) (g.cu > 0 ? g.cu : 256);
        if (m <= 16) tile = 13;
        else if (m <= 64) tile = gemm_grid(14, jobs, n_jobs, m) * 4 >= cu * 3 ? 14 : 13;
        else if (m <= 256) tile = gemm_grid(12, jobs, n_jobs, m) * 2 >= cu ? 12 : 14;
        else tile = gemm_grid(9, jobs, n_jobs, m) * 4 >= cu * 3 ? 9 : 12;
    } else if (tile < 0) {
        /* K % 256 != 0: split-K tiles up to 64 tokens, else 64 x 128 */
        tile = m <= 64 ? 0 : 2;
    }
    if (tile >= 3 && n % 256 != 0) tile = 2;
    const uint32_t rows_per_wg = k_gemm_rows[tile], tok_per_wg = k_gemm_tokens[tile];
    memset(a, 0, sizeof *a);
    uint64_t gx = 0;
    for (size_t j = 0; j < 3; ++j) {
        const size_t jj = j < n_jobs ? j : n_jobs - 1;      /* unused slots repeat the last job, no tiles */
        a->w[j] = jobs[jj].w;
        a->out[j] = jobs[jj].out;
        a->out_i[j] = jobs[jj].rows_out;
        a->n_rows[j] = (uint32_t) jobs[jj].n_rows;
        a->tiles[j] = j < n_jobs ? (uint32_t) ((jobs[j].n_rows + rows_per_wg - 1) / rows_per_wg) : 0u;
        gx += a->tiles[j];
    }
    a->q = q; a->act = act; a->k = (uint32_t) n; a->m = (uint32_t) m; a->n_jobs = (uint32_t) n_jobs;
    const uint64_t gy = (m + tok_per_wg - 1) / tok_per_wg;
    if (gx > INT32_MAX || gy > 65535) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemm: grid too large");
    *tile_out = tile;
    *gx_out = gx;
    *gy_out = gy;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_gemm_multi(const sllm_gfx950_gemm_job *jobs, size_t n_jobs, size_t n, const int8_t *q,
                           const sllm_gfx950_act *act, size_t m) {
    NEED_OPEN();
    k_gemm_args a;
    int tile = 0;
    uint64_t gx, gy;
    const int st = gemm_prepare(jobs, n_jobs, n, q, act, m, &a, &tile, &gx, &gy);
    if (st != SLLM_GFX950_OK || gx == 0) return st;
    void *args[] = { &a };
    HIP_TRY(hipModuleLaunchKernel(g.k_gemm[tile], (uint32_t) gx, (uint32_t) gy, 1, k_gemm_threads[tile], 1, 1, 0,
                                  g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

int sllm_shim_gemm_qkv_rope(const sllm_gfx950_gemm_job jobs[3], size_t n, const int8_t *q,
                            const sllm_gfx950_act *act, size_t m, const k_gemm_rope *r) {
    NEED_OPEN();
    k_gemm_args a;
    int tile = 0;
    uint64_t gx, gy;
    const int st = gemm_prepare(jobs, 3, n, q, act, m, &a, &tile, &gx, &gy);
    if (st != SLLM_GFX950_OK || gx == 0) return st;
    const int which = tile == 12 ? 0 : (tile == 9 ? 1 : -1);
    if (which < 0 || r->hd == 0 || k_gemm_rows[tile] % r->hd != 0 || r->half == 0 || r->half % 4 != 0 ||
        2 * r->half > r->hd || r->hd % 8 != 0)
        return SLLM_SHIM_NOT_FUSED;
    for (int j = 0; j < 3; ++j)
        if (jobs[j].out == NULL || jobs[j].rows_out != NULL || jobs[j].n_rows % r->hd != 0) return SLLM_SHIM_NOT_FUSED;
    k_gemm_rope rr = *r;
    void *args[] = { &a, &rr };
    HIP_TRY(hipModuleLaunchKernel(g.k_gemm_rope[which], (uint32_t) gx, (uint32_t) gy, 1, k_gemm_threads[tile], 1, 1, 0,
                                  g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

int sllm_shim_gemm_glu(const uint8_t *w_gate, const uint8_t *w_up, size_t n_rows, size_t n, const int8_t *q,
                       const sllm_gfx950_act *act, size_t m, float *out) {
    NEED_OPEN();
    if (out == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm_glu: no output");
    const sllm_gfx950_gemm_job jobs[2] = { { w_gate, n_rows, out, NULL }, { w_up, n_rows, out, NULL } };
    k_gemm_args a;
    int tile = 0;
    uint64_t gx, gy;
    const int st = gemm_prepare(jobs, 2, n, q, act, m, &a, &tile, &gx, &gy);
    if (st != SLLM_GFX950_OK || gx == 0) return st;
    const int which = tile == 12 ? 0 : (tile == 9 ? 1 : -1);
    if (which < 0) return SLLM_SHIM_NOT_FUSED;
    /* one tile per BN / 2 rows of each tensor: the same grid as the pair */
    const uint32_t half_rows = k_gemm_rows[tile] / 2;
    a.tiles[0] = (uint32_t) ((n_rows + half_rows - 1) / half_rows);
    a.tiles[1] = a.tiles[2] = 0;
    a.n_jobs = 1;
    void *args[] = { &a };
    HIP_TRY(hipModuleLaunchKernel(g.k_gemm_glu[which], a.tiles[0], (uint32_t) gy, 1, k_gemm_threads[tile], 1, 1, 0,
                                  g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

int sllm_shim_gemm_res(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q, const sllm_gfx950_act *act,
                       size_t m, float *out, const float *res) {
    NEED_OPEN();
    if (out == NULL || res == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm_res: output and residual must be given");
    const sllm_gfx950_gemm_job job = { w, n_rows, out, NULL };
    k_gemm_args a;
    int tile = 0;
    uint64_t gx, gy;
    const int st = gemm_prepare(&job, 1, n, q, act, m, &a, &tile, &gx, &gy);
    if (st != SLLM_GFX950_OK || gx == 0) return st;
    const int which = tile == 12 ? 0 : (tile == 9 ? 1 : (tile == 13 ? 2 : (tile == 14 ? 3 : -1)));
    if (which < 0) return SLLM_SHIM_NOT_FUSED;
    void *args[] = { &a, (void *) &res };
    HIP_TRY(hipModuleLaunchKernel(g.k_gemm_res[which], (uint32_t) gx, (uint32_t) gy, 1, k_gemm_threads[tile], 1, 1, 0,
                                  g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

/* ------------------------------------------------------------------ */
/* GEMM plans (i2s_kernels.hip: gemm_table, gemm_tjob)                 */
/* ------------------------------------------------------------------ */

typedef struct k_gemm_tjob {
    const uint8_t         *w;
    const int8_t          *q;
    const sllm_gfx950_act *act;
    float                 *out;
    int32_t               *out_i;
    uint32_t               n_rows, k, tile0, pad;
} k_gemm_tjob;

typedef struct k_gemm_table {
    const k_gemm_tjob *jobs;
    const uint32_t    *tile_job;
    uint32_t           m, pad;
} k_gemm_table;

_Static_assert(sizeof(k_gemm_tjob) == 56, "k_gemm_tjob must match gemm_tjob in i2s_kernels.hip");
_Static_assert(sizeof(k_gemm_table) == 24, "k_gemm_table must match gemm_table in i2s_kernels.hip");

/* the plan kernels: the tile shapes 6, 7, 13, 11 and 10 over a table */
static const int k_gemm_t_shape[5] = { 5, 6, 12, 10, 9 };

/* a streamed plan (i2s_kernels.hip: gemm_srec, gemm_stream) */
typedef struct k_gemm_srec {
    const uint8_t         *w;
    const int8_t          *q;
    float                 *out;
    int32_t               *out_i;
    const sllm_gfx950_act *act;
    const float           *ws;
    uint32_t               k, rows, n_rows, vec;
} k_gemm_srec;

typedef struct k_gemm_stream {
    const k_gemm_srec *recs;
    const uint32_t    *range;
    uint32_t           m, gy, n_ranges, pad;
} k_gemm_stream;

_Static_assert(sizeof(k_gemm_srec) == 64, "k_gemm_srec must match gemm_srec in i2s_kernels.hip");
_Static_assert(sizeof(k_gemm_stream) == 32, "k_gemm_stream must match gemm_stream in i2s_kernels.hip");

#define GS_ROWS 128u          /* rows per streamed tile */
#define GS_STEPS 2u           /* 256-k super-steps per iteration */
#define GS_TOKENS 4           /* plans of at most this many tokens stream (measured on the 96 FFN */
                              /* tensors: 4 tokens 90.7 against 93.1 us, 16 tokens 105.7 against 102.6) */
#define GS_RMAX 64u           /* tiles per run, as the kernel's LDS holds them */

struct sllm_gfx950_gemm_plan {
    uint8_t      *tables_dev;     /* jobs, then the row tile -> job map; or the stream's tables */
    k_gemm_table  table;
    k_gemm_stream stream;
    uint32_t      gx, gy;
    int           kind;           /* index into k_gemm_t, or 5: the stream */
};

/* The stream's tables: every tile of rows_per rows of the jobs in order,
 * cut into runs of about equal iteration counts (ss 256-k super-steps
 * each), at most GS_RMAX tiles per run and at least one run per CU where
 * there are tiles enough. Host memory: recs, then range[n_runs + 1]. */
static int gemm_stream_tables(const sllm_gfx950_gemm_plan_job *jobs, size_t n_jobs, uint32_t rows_per, uint32_t ss,
                              uint8_t **host_out, size_t *bytes_out, uint32_t *n_tiles_out, uint32_t *n_runs_out) {
    uint64_t n_tiles = 0, total = 0;
    for (size_t j = 0; j < n_jobs; ++j) {
        const uint64_t t = (jobs[j].n_rows + rows_per - 1) / rows_per;
        n_tiles += t;
        total += t * ((jobs[j].n / 256 + ss - 1) / ss);
    }
    if (n_tiles == 0 || n_tiles > UINT32_MAX / 2) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemm_plan: tiles");
    uint32_t n_runs = (uint32_t) ((n_tiles + 47) / 48);
    if (n_runs < (uint32_t) g.cu) n_runs = (uint32_t) g.cu;
    if (n_runs > n_tiles) n_runs = (uint32_t) n_tiles;
    uint32_t *it = malloc(n_tiles * sizeof *it);
    if (it == NULL) return fail(SLLM_GFX950_ERR_NOMEM, "gemm_plan: host tables");
    uint8_t *host = NULL;
    for (;;) {
        const size_t bytes = n_tiles * sizeof(k_gemm_srec) + ((size_t) n_runs + 1) * sizeof(uint32_t);
        free(host);
        host = malloc(bytes);
        if (host == NULL) {
            free(it);
            return fail(SLLM_GFX950_ERR_NOMEM, "gemm_plan: host tables");
        }
        k_gemm_srec *rec = (k_gemm_srec *) host;
        uint32_t *range = (uint32_t *) (host + n_tiles * sizeof(k_gemm_srec));
        uint32_t t = 0;
        for (size_t j = 0; j < n_jobs; ++j) {
            const sllm_gfx950_gemm_plan_job *J = &jobs[j];
            const size_t kb = J->n / 4;
            const int vec = J->n_rows % 4 == 0 && ((uintptr_t) J->out & 15u) == 0 && ((uintptr_t) J->rows_out & 15u) == 0;
            for (size_t n0 = 0; n0 < J->n_rows; n0 += rows_per, ++t) {
                const size_t rows = J->n_rows - n0 < rows_per ? J->n_rows - n0 : rows_per;
                rec[t] = (k_gemm_srec) { J->w + n0 * kb, J->q, J->out ? J->out + n0 : NULL,
                                         J->rows_out ? J->rows_out + n0 : NULL, J->act,
                                         (const float *) (J->w + J->n_rows * kb), (uint32_t) J->n, (uint32_t) rows,
                                         (uint32_t) J->n_rows, (uint32_t) vec };
                it[t] = (uint32_t) ((J->n / 256 + ss - 1) / ss);
            }
        }
        /* run r ends at the tile boundary nearest to (r + 1) total / n_runs */
        uint64_t done = 0;
        t = 0;
        for (uint32_t r = 0; r < n_runs; ++r) {
            range[r] = t;
            const uint64_t target = total * (r + 1) / n_runs;
            uint32_t cnt = 0;
            uint64_t acc = 0;
            while (t < n_tiles && cnt < GS_RMAX &&
                   (cnt == 0 || r + 1 == n_runs || 2 * (done + acc) + it[t] <= 2 * target)) {
                acc += it[t];
                ++t;
                ++cnt;
            }
            done += acc;
        }
        range[n_runs] = t;
        if (t == n_tiles) {
            *host_out = host;
            *bytes_out = bytes;
            *n_tiles_out = (uint32_t) n_tiles;
            *n_runs_out = n_runs;
            free(it);
            return SLLM_GFX950_OK;
        }
        n_runs += 8;                            /* a run hit GS_RMAX: cut finer */
    }
}

static int gemm_plan_stream(const sllm_gfx950_gemm_plan_job *jobs, size_t n_jobs, size_t m,
                            sllm_gfx950_gemm_plan **plan) {
    uint8_t *host = NULL;
    size_t bytes = 0;
    uint32_t n_tiles = 0, n_runs = 0;
    int st = gemm_stream_tables(jobs, n_jobs, GS_ROWS, GS_STEPS, &host, &bytes, &n_tiles, &n_runs);
    if (st != SLLM_GFX950_OK) return st;
    sllm_gfx950_gemm_plan *p = calloc(1, sizeof *p);
    if (p == NULL) {
        free(host);
        return fail(SLLM_GFX950_ERR_NOMEM, "gemm_plan: host tables");
    }
    hipError_t e = hipMalloc((void **) &p->tables_dev, bytes);
    if (e != hipSuccess) {
        p->tables_dev = NULL;
    } else {
        e = hipMemcpy(p->tables_dev, host, bytes, hipMemcpyHostToDevice);
    }
    free(host);
    if (e != hipSuccess) {
        if (p->tables_dev) hipFree(p->tables_dev);
        free(p);
        return hip_fail(e, "gemm_plan: tables");
    }
    const uint32_t gy = (uint32_t) ((m + 15) / 16);    /* 16 tokens per token tile */
    const uint32_t *range = (const uint32_t *) (p->tables_dev + (size_t) n_tiles * sizeof(k_gemm_srec));
    p->stream = (k_gemm_stream) { (const k_gemm_srec *) p->tables_dev, range, (uint32_t) m, gy, n_runs, 0 };
    p->gx = 8u * gy * ((n_runs + 7u) / 8u);
    p->gy = 1;
    p->kind = 5;
    *plan = p;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_gemm_plan_create(const sllm_gfx950_gemm_plan_job *jobs, size_t n_jobs, size_t m,
                                 sllm_gfx950_gemm_plan **plan) {
    NEED_OPEN();
    if (plan == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm_plan: NULL out pointer");
    *plan = NULL;
    if (jobs == NULL || n_jobs == 0 || n_jobs > UINT32_MAX / 2) return fail(SLLM_GFX950_ERR_ARG, "gemm_plan: bad job list");
    if (m == 0 || m > (size_t) 65535 * 16) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemm_plan: m = %zu", m);
    for (size_t j = 0; j < n_jobs; ++j) {
        const sllm_gfx950_gemm_plan_job *J = &jobs[j];
        const int st = check_weights(J->w, J->n_rows, J->n);
        if (st != SLLM_GFX950_OK) return st;
        if (J->n % 256 != 0) return fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "gemm_plan: job %zu K=%zu is not a multiple of 256", j, J->n);
        if (J->q == NULL || ((uintptr_t) J->q & 15u) != 0) return fail(SLLM_GFX950_ERR_ARG, "gemm_plan: job %zu q must be given and 16-byte aligned", j);
        if (J->out == NULL && J->rows_out == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm_plan: job %zu has no output", j);
        if (J->out != NULL && J->act == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm_plan: job %zu: the epilogue needs act", j);
        if ((uint64_t) m * J->n_rows > (uint64_t) 1 << 40) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemm_plan: m x rows too large");
    }
    /* the tile: forced, or by token count (measured on the FFN tensors of
     * 32 weight sets: the stream up to GS_TOKENS, 32 x 128 up to 32 tokens,
     * 64 x 256 above) */
    int kind = -1;
    for (int i = 0; i < 5; ++i) if (g.force_gemm_tile - 1 == k_gemm_t_shape[i]) kind = i;
    if (kind < 0 && g.force_gemm_tile == 0 && m <= GS_TOKENS) {
        /* the stream, where every job's outputs are within its buffers' 32-bit offsets */
        int ok = 1;
        for (size_t j = 0; j < n_jobs; ++j) if ((uint64_t) m * jobs[j].n_rows * 4 > 0x7FFFFFFFu) ok = 0;
        if (ok) return gemm_plan_stream(jobs, n_jobs, m, plan);
    }
    if (kind < 0) kind = m <= 32 ? 2 : 4;
    const int shape = k_gemm_t_shape[kind];
    const uint32_t rows_per = k_gemm_rows[shape], tok_per = k_gemm_tokens[shape];
    uint64_t gx = 0;
    for (size_t j = 0; j < n_jobs; ++j) gx += (jobs[j].n_rows + rows_per - 1) / rows_per;
    const uint64_t gy = (m + tok_per - 1) / tok_per;
    if (gx == 0) return fail(SLLM_GFX950_ERR_ARG, "gemm_plan: no rows");
    if (gx > INT32_MAX || gy > 65535) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemm_plan: grid too large");
    const size_t jbytes = n_jobs * sizeof(k_gemm_tjob), bytes = jbytes + (size_t) gx * sizeof(uint32_t);
    uint8_t *host = malloc(bytes);
    sllm_gfx950_gemm_plan *p = calloc(1, sizeof *p);
    if (host == NULL || p == NULL) {
        free(host);
        free(p);
        return fail(SLLM_GFX950_ERR_NOMEM, "gemm_plan: host tables");
    }
    k_gemm_tjob *kj = (k_gemm_tjob *) host;
    uint32_t *tile_job = (uint32_t *) (host + jbytes);
    uint32_t tile = 0;
    for (size_t j = 0; j < n_jobs; ++j) {
        const uint32_t tiles = (uint32_t) ((jobs[j].n_rows + rows_per - 1) / rows_per);
        kj[j] = (k_gemm_tjob) { jobs[j].w, jobs[j].q, jobs[j].act, jobs[j].out, jobs[j].rows_out,
                                (uint32_t) jobs[j].n_rows, (uint32_t) jobs[j].n, tile, 0 };
        for (uint32_t t = 0; t < tiles; ++t) tile_job[tile + t] = (uint32_t) j;
        tile += tiles;
    }
    hipError_t e = hipMalloc((void **) &p->tables_dev, bytes);
    if (e != hipSuccess) {
        p->tables_dev = NULL;
    } else {
        e = hipMemcpy(p->tables_dev, host, bytes, hipMemcpyHostToDevice);
    }
    free(host);
    if (e != hipSuccess) {
        if (p->tables_dev) hipFree(p->tables_dev);
        free(p);
        return hip_fail(e, "gemm_plan: tables");
    }
    p->table = (k_gemm_table) { (const k_gemm_tjob *) p->tables_dev,
                                (const uint32_t *) (p->tables_dev + jbytes), (uint32_t) m, 0 };
    p->gx = (uint32_t) gx;
    p->gy = (uint32_t) gy;
    p->kind = kind;
    *plan = p;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_gemm_plan_run(const sllm_gfx950_gemm_plan *p) {
    NEED_OPEN();
    if (p == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemm_plan_run: NULL plan");
    if (p->kind >= 5) {
        k_gemm_stream sa = p->stream;
        void *sargs[] = { &sa };
        HIP_TRY(hipModuleLaunchKernel(g.k_gemm_s, p->gx, 1, 1, 512, 1, 1, 0, g.stream, sargs, NULL));
        return SLLM_GFX950_OK;
    }
    k_gemm_table t = p->table;
    void *args[] = { &t };
    HIP_TRY(hipModuleLaunchKernel(g.k_gemm_t[p->kind], p->gx, p->gy, 1, k_gemm_threads[k_gemm_t_shape[p->kind]],
                                  1, 1, 0, g.stream, args, NULL));
    return SLLM_GFX950_OK;
}

void sllm_gfx950_gemm_plan_destroy(sllm_gfx950_gemm_plan *p) {
    if (p == NULL) return;
    if (g.open) {
        hipStreamSynchronize(g.stream);
        hipFree(p->tables_dev);
    }
    free(p);
}

int sllm_gfx950_gemm(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                     const sllm_gfx950_act *act, size_t m, float *out, int32_t *rows_out) {
    NEED_OPEN();
    if (m == 0) return SLLM_GFX950_OK;
    const sllm_gfx950_gemm_job job = { w, n_rows, out, rows_out };
    return sllm_gfx950_gemm_multi(&job, 1, n, q, act, m);
}

int sllm_gfx950_linear_batch(const uint8_t *w, size_t n_rows, size_t n, const float *x, size_t m,
                             int8_t *q, sllm_gfx950_act *act, float *out, int32_t *rows_out) {
    NEED_OPEN();
    if (m == 0) return SLLM_GFX950_OK;
    if (x == NULL || q == NULL || act == NULL) return fail(SLLM_GFX950_ERR_ARG, "linear_batch: NULL x, q or act");
    int st = check_weights(w, n_rows, n);
    if (st == SLLM_GFX950_OK) st = sllm_gfx950_quant_act(x, n, m, q, act);
    if (st == SLLM_GFX950_OK) st = sllm_gfx950_gemm(w, n_rows, n, q, act, m, out, rows_out);
    return st;
}

int sllm_gfx950_linear(const uint8_t *w, size_t n_rows, size_t n, const float *x,
                       int8_t *q, sllm_gfx950_act *act, float *out) {
    NEED_OPEN();
    if (x == NULL || out == NULL) return fail(SLLM_GFX950_ERR_ARG, "linear: NULL x or out");
    const sllm_gfx950_gemv_job j = { w, n_rows, n, x, q, act, out, NULL };
    return single_launch(&j);
}

/* ------------------------------------------------------------------ */
/* the host-pointer kernel row                                         */
/* ------------------------------------------------------------------ */

/* registry kept sorted by host address; lookups accept interior pointers */
static ptrdiff_t reg_find(const void *host) {
    const uint8_t *h = host;
    size_t lo = 0, hi = g.n_regs;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (g.regs[mid].host + g.regs[mid].bytes <= h) lo = mid + 1;
        else hi = mid;
    }
    if (lo < g.n_regs && g.regs[lo].host <= h && h < g.regs[lo].host + g.regs[lo].bytes) return (ptrdiff_t) lo;
    return -1;
}

/* Upload [h, h + bytes) into a new registry entry at sorted position pos
 * (g_mtx held). */
static int reg_insert(const uint8_t *h, size_t bytes, size_t pos, size_t refs, int acquired) {
    if (g.n_regs == g.cap_regs) {
        const size_t cap = g.cap_regs ? 2 * g.cap_regs : 256;
        reg_tensor *r = realloc(g.regs, cap * sizeof *r);
        if (r == NULL) return fail(SLLM_GFX950_ERR_NOMEM, "register: registry");
        g.regs = r;
        g.cap_regs = cap;
    }
    uint8_t *dev = NULL;
    hipError_t e = hipMalloc((void **) &dev, bytes);
    if (e == hipSuccess) e = hipMemcpy(dev, h, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (dev) hipFree(dev);
        return hip_fail(e, "register: upload");
    }
    memmove(&g.regs[pos + 1], &g.regs[pos], (g.n_regs - pos) * sizeof *g.regs);
    g.regs[pos] = (reg_tensor) { h, bytes, dev, refs, acquired };
    g.n_regs++;
    return SLLM_GFX950_OK;
}

/* the sorted position of h, and whether [h, h + bytes) overlaps an entry */
static size_t reg_pos(const uint8_t *h, size_t bytes, int *overlap) {
    size_t pos = 0;
    while (pos < g.n_regs && g.regs[pos].host < h) ++pos;
    *overlap = (pos < g.n_regs && g.regs[pos].host < h + bytes) ||
               (pos > 0 && g.regs[pos - 1].host + g.regs[pos - 1].bytes > h);
    return pos;
}

int sllm_gfx950_tensor_register(const void *packed, size_t n_rows, size_t n) {
    NEED_OPEN();
    if (packed == NULL) return fail(SLLM_GFX950_ERR_ARG, "register: NULL tensor");
    if (n % SLLM_GFX950_QK != 0 || n == 0) return fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "register: K=%zu is not a positive multiple of 128", n);
    const size_t bytes = n_rows * (n / 4) + 32;
    pthread_mutex_lock(&g_mtx);
    int st = SLLM_GFX950_OK, overlap;
    const uint8_t *h = packed;
    const size_t pos = reg_pos(h, bytes, &overlap);
    if (pos < g.n_regs && g.regs[pos].host == h && g.regs[pos].bytes == bytes) {
        /* a second model over the same image: share the device copy */
        g.regs[pos].refs++;
    } else if (overlap) {
        st = fail(SLLM_GFX950_ERR_ARG, "register: tensor overlaps a registered one");
    } else {
        st = reg_insert(h, bytes, pos, 1, 0);
    }
    pthread_mutex_unlock(&g_mtx);
    return st;
}

int sllm_gfx950_tensor_acquire(const void *packed, size_t n_rows, size_t n) {
    NEED_OPEN();
    if (packed == NULL) return fail(SLLM_GFX950_ERR_ARG, "acquire: NULL tensor");
    if (n % SLLM_GFX950_QK != 0 || n == 0) return fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "acquire: K=%zu is not a positive multiple of 128", n);
    const size_t bytes = n_rows * (n / 4) + 32;
    const uint8_t *h = packed;
    pthread_mutex_lock(&g_mtx);
    int st = SLLM_GFX950_OK;
    const ptrdiff_t i = reg_find(h);
    if (i >= 0 && h + bytes <= g.regs[i].host + g.regs[i].bytes) {
        /* already on the device: registered, or acquired by an earlier GEMV */
    } else {
        int overlap;
        const size_t pos = reg_pos(h, bytes, &overlap);
        st = overlap ? fail(SLLM_GFX950_ERR_ARG, "acquire: tensor overlaps a registered one")
                     : reg_insert(h, bytes, pos, 0, 1);
    }
    pthread_mutex_unlock(&g_mtx);
    return st;
}

int sllm_gfx950_tensor_release_acquired(void) {
    NEED_OPEN();
    pthread_mutex_lock(&g_mtx);
    /* kernels reading a copy may still be in flight: wait, then free */
    const hipError_t e = hipStreamSynchronize(g.stream);
    size_t keep = 0;
    for (size_t i = 0; i < g.n_regs; ++i) {
        reg_tensor r = g.regs[i];
        if (r.acquired && r.refs == 0) {
            hipFree(r.dev);
            continue;
        }
        r.acquired = 0;               /* registered as well: it stays, as registered */
        g.regs[keep++] = r;
    }
    g.n_regs = keep;
    pthread_mutex_unlock(&g_mtx);
    return e != hipSuccess ? hip_fail(e, "release_acquired") : SLLM_GFX950_OK;
}

int sllm_gfx950_tensor_unregister(const void *packed) {
    NEED_OPEN();
    pthread_mutex_lock(&g_mtx);
    const ptrdiff_t i = reg_find(packed);
    int st = SLLM_GFX950_OK;
    if (i < 0 || g.regs[i].host != (const uint8_t *) packed) {
        st = fail(SLLM_GFX950_ERR_NOT_REGISTERED, "unregister: %p is not a registered tensor", packed);
    } else if (--g.regs[i].refs == 0 && !g.regs[i].acquired) {
        /* the copy goes either way; a failed wait is still reported
         * (an acquired copy stays until release_acquired) */
        const hipError_t e = hipStreamSynchronize(g.stream);
        hipFree(g.regs[i].dev);
        memmove(&g.regs[i], &g.regs[i + 1], (g.n_regs - (size_t) i - 1) * sizeof *g.regs);
        g.n_regs--;
        if (e != hipSuccess) st = hip_fail(e, "unregister");
    }
    pthread_mutex_unlock(&g_mtx);
    return st;
}

const void *sllm_gfx950_tensor_device(const void *host) {
    if (!g.open || host == NULL) return NULL;
    pthread_mutex_lock(&g_mtx);
    const ptrdiff_t i = reg_find(host);
    const void *d = i < 0 ? NULL : g.regs[i].dev + ((const uint8_t *) host - g.regs[i].host);
    pthread_mutex_unlock(&g_mtx);
    return d;
}

static size_t align16(size_t v) { return (v + 15u) & ~(size_t) 15u; }

/* pin_q layout: the done word (a line of its own), act, then q */
#define PIN_Q_DONE 0u
#define PIN_Q_ACT  64u
#define PIN_Q_Q    128u

static int pinned_reserve(uint8_t **host, uint8_t **dev, size_t *cap, size_t bytes) {
    if (bytes <= *cap) return SLLM_GFX950_OK;
    HIP_TRY(hipStreamSynchronize(g.stream));
    if (*host) HIP_TRY(hipHostFree(*host));
    *host = *dev = NULL;
    *cap = 0;
    bytes = (bytes + 4095u) & ~(size_t) 4095u;
    /* coherent (fine-grained) whatever HIP_HOST_COHERENT says: the host
     * spins on a completion word the device stores into this memory */
    HIP_TRY(hipHostMalloc((void **) host, bytes, hipHostMallocCoherent));
    HIP_TRY(hipHostGetDevicePointer((void **) dev, *host, 0));
    *cap = bytes;
    return SLLM_GFX950_OK;
}

/* Room for a quantised vector of n and for max(4n, io) bytes of x / rows. */
static int hostrow_reserve(size_t n, size_t io) {
    if (PIN_Q_Q + n > g.pin_q_cap) {
        g.last_q = NULL;                    /* the kept copy goes with the old buffer */
        int st = pinned_reserve(&g.pin_q, &g.pin_q_dev, &g.pin_q_cap, PIN_Q_Q + n);
        if (st != SLLM_GFX950_OK) return st;
        /* the next wait is for seq + 1: the fresh word must not read as it */
        __atomic_store_n((uint32_t *) (g.pin_q + PIN_Q_DONE), g.seq, __ATOMIC_RELEASE);
    }
    if (io > g.pin_io_cap) {
        int st = pinned_reserve(&g.pin_io, &g.pin_io_dev, &g.pin_io_cap, io);
        if (st != SLLM_GFX950_OK) return st;
    }
    if (align16(n) + 16 > g.dq_cap) {             /* q, then act at align16(n) */
        g.last_q = NULL;
        HIP_TRY(hipStreamSynchronize(g.stream));
        if (g.dq) HIP_TRY(hipFree(g.dq));
        g.dq = NULL;
        g.dq_cap = 0;
        HIP_TRY(hipMalloc((void **) &g.dq, align16(n) + 16));
        g.dq_cap = align16(n) + 16;
    }
    return SLLM_GFX950_OK;
}

/* The reference's hot-path functions cannot return a status; failing
 * silently (zeros) would read as a wrong answer, and falling back to a CPU
 * kernel would hide that the GPU row is broken. So: say why, and stop. */
static void die(const char *fn, int st) {
    fprintf(stderr, "libsllm_gfx950: %s failed: %s: %s\n", fn, sllm_gfx950_status_string(st), g_err);
    abort();
}

static uint64_t now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t) ts.tv_sec * 1000000000u + (uint64_t) ts.tv_nsec;
}

/* Wait until the device has stored `seq` to the pinned done word: a spin on
 * host memory sees it about 5 us sooner than a stream synchronisation. After
 * 20 ms the wait becomes hipStreamSynchronize, which also reports a failed
 * launch. */
static int host_wait(uint32_t seq, const char *what) {
    const volatile uint32_t *done = (const volatile uint32_t *) (g.pin_q + PIN_Q_DONE);
    const uint64_t t0 = now_ns();
    for (unsigned spins = 0; __atomic_load_n(done, __ATOMIC_ACQUIRE) != seq; ++spins) {
        if ((spins & 255u) == 255u && now_ns() - t0 > 20000000u) {
            hipError_t e = hipStreamSynchronize(g.stream);
            if (e != hipSuccess) return hip_fail(e, what);
            if (__atomic_load_n(done, __ATOMIC_ACQUIRE) != seq) {
                return fail(SLLM_GFX950_ERR_HIP, "%s: the stream drained without the completion word", what);
            }
            break;
        }
        __builtin_ia32_pause();
    }
    return SLLM_GFX950_OK;
}

/*
 * The host-pointer row. A call of the reference's hot path hands over host
 * buffers and expects the result in host buffers on return, so each call is
 * one launch and one wait -- on a pinned word the device sets last, which
 * the host sees sooner than a stream synchronisation. The data moves through
 * pinned host memory that the kernels read and write themselves (no
 * copy-engine transfers):
 *   quant_act: x is copied into pinned memory; one workgroup
 *              (sllm_k_quant_host) reads it and writes q / act to the device
 *              (for the GEMVs that follow) and to pinned memory (for the
 *              caller);
 *   gemv:      the device copy of q is reused when q is the buffer the last
 *              quant_act filled and still holds those bytes (the reference
 *              quantises once and runs two or three GEMVs on the result);
 *              otherwise q goes up first. The GEMV writes its int32 rows
 *              straight into pinned memory; sllm_k_host_done follows it.
 */
void sllm_gfx950_i2s_quant_act(const float *x, size_t n, int8_t *q_out, sllm_gfx950_act *out) {
    if (!g.open) die("sllm_gfx950_i2s_quant_act", fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open"));
    if (x == NULL || q_out == NULL || out == NULL || n == 0) return;
    if (n > UINT32_MAX / 4) die("sllm_gfx950_i2s_quant_act", fail(SLLM_GFX950_ERR_ARG, "quant_act: n=%zu", n));
    pthread_mutex_lock(&g_mtx);
    int st = hostrow_reserve(n, n * sizeof(float));
    if (st == SLLM_GFX950_OK) {
        memcpy(g.pin_io, x, n * sizeof(float));
        const float *xd = (const float *) g.pin_io_dev;
        uint32_t n32 = (uint32_t) n;
        int8_t *qd = g.dq, *qh = (int8_t *) (g.pin_q_dev + PIN_Q_Q);
        sllm_gfx950_act *ad = (sllm_gfx950_act *) (g.dq + align16(n));
        sllm_gfx950_act *ah = (sllm_gfx950_act *) (g.pin_q_dev + PIN_Q_ACT);
        uint32_t *done = (uint32_t *) (g.pin_q_dev + PIN_Q_DONE);
        uint32_t seq = ++g.seq;
        void *args[] = { (void *) &xd, &n32, &qd, &ad, &qh, &ah, &done, &seq };
        g.last_q = NULL;
        st = launch(g.k_quant_host, 1, QUANT_HOST_THREADS, 0, args);
        if (st == SLLM_GFX950_OK) st = host_wait(seq, "quant_act");
    }
    if (st == SLLM_GFX950_OK) {
        memcpy(q_out, g.pin_q + PIN_Q_Q, n);
        memcpy(out, g.pin_q + PIN_Q_ACT, sizeof *out);
        g.last_q = q_out;
        g.last_n = n;
    }
    pthread_mutex_unlock(&g_mtx);
    if (st != SLLM_GFX950_OK) die("sllm_gfx950_i2s_quant_act", st);
}

void sllm_gfx950_i2s_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                          int32_t *rows_out) {
    if (!g.open) die("sllm_gfx950_i2s_gemv", fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open"));
    if (w == NULL || q == NULL || rows_out == NULL) return;          /* src/i2s_gemm.c:262-264 */
    if (n_rows == 0) return;
    if (n < SLLM_GFX950_QK) {                                        /* dot is 0 below one block */
        memset(rows_out, 0, n_rows * sizeof *rows_out);
        return;
    }
    pthread_mutex_lock(&g_mtx);
    int st = SLLM_GFX950_OK;
    const ptrdiff_t i = reg_find(w);
    const size_t need = n_rows * (n / 4);
    if (i < 0 || w + need > g.regs[i].host + g.regs[i].bytes) {
        st = fail(SLLM_GFX950_ERR_NOT_REGISTERED, "weights %p (+%zu bytes) are not inside a registered tensor", (const void *) w, need);
    }
    if (st == SLLM_GFX950_OK) st = hostrow_reserve(n, n_rows * sizeof(int32_t));
    if (st == SLLM_GFX950_OK && !(q == g.last_q && n == g.last_n && memcmp(q, g.pin_q + PIN_Q_Q, n) == 0)) {
        memcpy(g.pin_q + PIN_Q_Q, q, n);
        hipError_t e = hipMemcpyAsync(g.dq, g.pin_q + PIN_Q_Q, n, hipMemcpyHostToDevice, g.stream);
        if (e != hipSuccess) {
            g.last_q = NULL;
            st = hip_fail(e, "gemv upload");
        } else {
            g.last_q = q;
            g.last_n = n;
        }
    }
    if (st == SLLM_GFX950_OK) {
        const uint8_t *wd = g.regs[i].dev + (w - g.regs[i].host);
        st = sllm_gfx950_gemv(wd, n_rows, n, g.dq, (int32_t *) g.pin_io_dev);
    }
    if (st == SLLM_GFX950_OK) {
        uint32_t *done = (uint32_t *) (g.pin_q_dev + PIN_Q_DONE);
        uint32_t seq = ++g.seq;
        void *args[] = { &done, &seq };
        st = launch(g.k_host_done, 1, 64, 0, args);
        if (st == SLLM_GFX950_OK) st = host_wait(seq, "gemv");
        if (st == SLLM_GFX950_OK) memcpy(rows_out, g.pin_io, n_rows * sizeof(int32_t));
    }
    pthread_mutex_unlock(&g_mtx);
    if (st != SLLM_GFX950_OK) die("sllm_gfx950_i2s_gemv", st);
}

int32_t sllm_gfx950_i2s_dot(const uint8_t *w, const int8_t *q, size_t n) {
    if (w == NULL || q == NULL || n < SLLM_GFX950_QK) return 0;      /* src/i2s_gemm.c:247-249 */
    int32_t d = 0;
    sllm_gfx950_i2s_gemv(w, 1, n, q, &d);
    return d;
}
