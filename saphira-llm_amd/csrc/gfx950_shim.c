/*
 * gfx950_shim.c -- the thin C11 shim between the host code and HIP.
 *
 * Loads the gfx950 code object built from i2s_kernels.hip (embedded in this
 * library at build time) with hipModuleLoadData, launches its entry points
 * with hipModuleLaunchKernel on one library-owned stream, and owns the device
 * buffers: registered weight tensors, per-call scratch and job tables.
 *
 * Argument structs passed by value (gemv_job) mirror the device structs in
 * i2s_kernels.hip field for field; their sizes are asserted below.
 */
#define _POSIX_C_SOURCE 200809L

#include <saphira_amd/sllm_gfx950.h>

#include <hip/hip_runtime_api.h>

#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

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

/* ------------------------------------------------------------------ */
/* device-side argument layouts (mirrors of i2s_kernels.hip)           */
/* ------------------------------------------------------------------ */

typedef struct k_gemv_job {
    const uint8_t         *w;
    const int8_t          *q;
    const sllm_gfx950_act *act;
    float                 *out_f;
    int32_t               *out_i;
    uint32_t               n_rows;
    uint32_t               k;
    uint32_t               wg_begin;
    uint32_t               rows_per_wg;
} k_gemv_job;

_Static_assert(sizeof(k_gemv_job) == 56, "k_gemv_job must match gemv_job in i2s_kernels.hip");
_Static_assert(sizeof(sllm_gfx950_act) == 8, "sllm_gfx950_act must match sllm_i2s_act");

enum { LPR_4 = 0, LPR_8 = 1, LPR_16 = 2, N_LPR = 3 };
static const int k_lpr_value[N_LPR] = { 4, 8, 16 };
static const char *const k_gemv_names[N_LPR] = {
    "sllm_k_gemv_l4", "sllm_k_gemv_l8", "sllm_k_gemv_l16"
};
static const char *const k_group_names[N_LPR] = {
    "sllm_k_gemv_group_l4", "sllm_k_gemv_group_l8", "sllm_k_gemv_group_l16"
};

#define QUANT_THREADS 256

/* ------------------------------------------------------------------ */
/* library state                                                       */
/* ------------------------------------------------------------------ */

typedef struct reg_tensor {
    const uint8_t *host;
    size_t         bytes;    /* n_rows*n/4 + 32 */
    uint8_t       *dev;
} reg_tensor;

struct sllm_gfx950_plan {
    void    *jobs_dev;
    uint32_t n_jobs;
    uint32_t n_wg;
    uint32_t lds;
    int      lpr_idx;
    int      threads;
};

static struct {
    int            open;
    int            device;
    int            cu;
    size_t         hbm;
    char           name[520];
    hipModule_t    mod;
    hipFunction_t  k_quant;
    hipFunction_t  k_gemv[N_LPR];
    hipFunction_t  k_group[N_LPR];
    hipFunction_t  k_copy;
    hipFunction_t  k_checksum;
    hipStream_t    stream;
    hipEvent_t     ev_start, ev_stop;
    hipEvent_t    *events;
    int            n_events;
    /* tuning override (0 = automatic) */
    int            force_lpr, force_waves, force_rows;
    /* registry for the host-pointer row */
    reg_tensor    *regs;
    size_t         n_regs, cap_regs;
    /* scratch for the host-pointer row and for per-call job tables */
    void          *scratch;
    size_t         scratch_bytes;
    void          *jobs_dev;
    size_t         jobs_cap;
} g;

static pthread_mutex_t g_mtx = PTHREAD_MUTEX_INITIALIZER;
static char g_err[512];

static int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

static int hip_fail(hipError_t e, const char *what) {
    return fail(SLLM_GFX950_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int) e);
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
    case SLLM_GFX950_ERR_UNSUPPORTED:    return "unsupported";
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
    HIP_TRY(hipModuleGetFunction(&g.k_copy, g.mod, "sllm_k_copy"));
    HIP_TRY(hipModuleGetFunction(&g.k_checksum, g.mod, "sllm_k_checksum"));
    for (int i = 0; i < N_LPR; ++i) {
        HIP_TRY(hipModuleGetFunction(&g.k_gemv[i], g.mod, k_gemv_names[i]));
        HIP_TRY(hipModuleGetFunction(&g.k_group[i], g.mod, k_group_names[i]));
    }
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
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) {
        st = fail(SLLM_GFX950_ERR_NO_DEVICE, "no HIP device (%s)", hipGetErrorString(e));
        goto out;
    }
    if (device < 0 || device >= count) {
        st = fail(SLLM_GFX950_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, count);
        goto out;
    }
    hipDeviceProp_t prop;
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
        goto out;
    }
    if ((st = load_functions()) != SLLM_GFX950_OK) {
        hipModuleUnload(g.mod);
        goto out;
    }
    if ((e = hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking)) != hipSuccess) {
        hipModuleUnload(g.mod);
        st = hip_fail(e, "hipStreamCreateWithFlags");
        goto out;
    }
    if ((e = hipEventCreate(&g.ev_start)) != hipSuccess ||
        (e = hipEventCreate(&g.ev_stop)) != hipSuccess) {
        hipStreamDestroy(g.stream);
        hipModuleUnload(g.mod);
        st = hip_fail(e, "hipEventCreate");
        goto out;
    }
    g.device = device;
    g.cu = prop.multiProcessorCount;
    g.hbm = prop.totalGlobalMem;
    snprintf(g.name, sizeof g.name, "%s (%s)", prop.name, prop.gcnArchName);
    g.open = 1;
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
        if (g.scratch) hipFree(g.scratch);
        if (g.jobs_dev) hipFree(g.jobs_dev);
        for (int i = 0; i < g.n_events; ++i) hipEventDestroy(g.events[i]);
        free(g.events);
        hipEventDestroy(g.ev_start);
        hipEventDestroy(g.ev_stop);
        hipStreamDestroy(g.stream);
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
    while (g.n_events < n) {
        HIP_TRY(hipEventCreate(&g.events[g.n_events]));
        g.n_events++;
    }
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

/* Shape of one GEMV launch. */
typedef struct gemv_shape {
    int      lpr_idx;
    int      waves;
    uint32_t rows_per_wg;
} gemv_shape;

static int lpr_index(int lpr) {
    for (int i = 0; i < N_LPR; ++i) if (k_lpr_value[i] == lpr) return i;
    return -1;
}

/*
 * Automatic launch shape. A row is split over `lpr` lanes (each takes every
 * lpr-th 16-byte chunk); a wave therefore covers 64/lpr rows per pass. Prefer
 * the split that keeps every lane busy (chunks per row divisible by lpr), then
 * enough waves to cover the chip.
 */
static gemv_shape choose_shape(size_t n_rows, size_t n) {
    gemv_shape s;
    const size_t chunks = n / 64;
    int best = LPR_4;
    if (g.force_lpr) {
        best = lpr_index(g.force_lpr);
    } else {
        /* smallest lpr whose rows-per-wave still gives >= 2 waves per CU */
        const size_t cu = g.cu > 0 ? (size_t) g.cu : 256;
        best = LPR_16;
        for (int i = 0; i < N_LPR; ++i) {
            const size_t rpw = 64 / (size_t) k_lpr_value[i];
            const size_t waves = (n_rows + rpw - 1) / rpw;
            if (waves >= 2 * cu && chunks % (size_t) k_lpr_value[i] == 0) { best = i; break; }
        }
    }
    s.lpr_idx = best;
    s.waves = g.force_waves ? g.force_waves : 4;
    const uint32_t rpw = (uint32_t) (64 / k_lpr_value[best]);
    s.rows_per_wg = g.force_rows ? (uint32_t) g.force_rows : (uint32_t) s.waves * rpw;
    return s;
}

int sllm_gfx950_set_gemv_shape(int lanes_per_row, int waves, int rows_per_wg) {
    if (lanes_per_row != 0 && lpr_index(lanes_per_row) < 0) {
        return fail(SLLM_GFX950_ERR_ARG, "lanes per row must be 4, 8 or 16");
    }
    if (waves < 0 || waves > 16) return fail(SLLM_GFX950_ERR_ARG, "waves must be 0..16");
    if (rows_per_wg < 0) return fail(SLLM_GFX950_ERR_ARG, "rows per workgroup must be >= 0");
    if (rows_per_wg > 0) {
        const int l = lanes_per_row ? lanes_per_row : 4;
        if (rows_per_wg % (64 / l) != 0) {
            return fail(SLLM_GFX950_ERR_ARG, "rows per workgroup must be a multiple of %d", 64 / l);
        }
    }
    g.force_lpr = lanes_per_row;
    g.force_waves = waves;
    g.force_rows = rows_per_wg;
    return SLLM_GFX950_OK;
}

static int check_gemv_args(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q) {
    if (w == NULL || q == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv: NULL pointer");
    if (n % SLLM_GFX950_QK != 0) return fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "gemv: K=%zu is not a multiple of 128", n);
    if (n > SLLM_GFX950_MAX_K) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemv: K=%zu above %d", n, SLLM_GFX950_MAX_K);
    if (n_rows > UINT32_MAX / 2) return fail(SLLM_GFX950_ERR_TOO_LARGE, "gemv: %zu rows", n_rows);
    if (((uintptr_t) w & 15u) != 0 || ((uintptr_t) q & 15u) != 0) {
        return fail(SLLM_GFX950_ERR_ARG, "gemv: weights and activations must be 16-byte aligned");
    }
    return SLLM_GFX950_OK;
}

static int gemv_launch(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                       const sllm_gfx950_act *act, float *out, int32_t *rows_out) {
    NEED_OPEN();
    int st = check_gemv_args(w, n_rows, n, q);
    if (st != SLLM_GFX950_OK) return st;
    if (out == NULL && rows_out == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv: no output");
    if (out != NULL && act == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv: epilogue needs act");
    if (n_rows == 0 || n == 0) return SLLM_GFX950_OK;
    const gemv_shape s = choose_shape(n_rows, n);
    k_gemv_job job = { w, q, act, out, rows_out, (uint32_t) n_rows, (uint32_t) n, 0, s.rows_per_wg };
    const uint32_t grid = (uint32_t) ((n_rows + s.rows_per_wg - 1) / s.rows_per_wg);
    void *args[] = { &job };
    return launch(g.k_gemv[s.lpr_idx], grid, (uint32_t) (64 * s.waves), (uint32_t) n, args);
}

int sllm_gfx950_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                     int32_t *rows_out) {
    if (rows_out == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv: NULL rows_out");
    return gemv_launch(w, n_rows, n, q, NULL, NULL, rows_out);
}

int sllm_gfx950_gemv_epilogue(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                              const sllm_gfx950_act *act, float *out) {
    if (out == NULL || act == NULL) return fail(SLLM_GFX950_ERR_ARG, "gemv_epilogue: NULL out/act");
    return gemv_launch(w, n_rows, n, q, act, out, NULL);
}

int sllm_gfx950_linear(const uint8_t *w, size_t n_rows, size_t n, const float *x,
                       int8_t *q, sllm_gfx950_act *act, float *out) {
    NEED_OPEN();
    int st = check_gemv_args(w, n_rows, n, q);
    if (st != SLLM_GFX950_OK) return st;
    if ((st = sllm_gfx950_quant_act(x, n, 1, q, act)) != SLLM_GFX950_OK) return st;
    return sllm_gfx950_gemv_epilogue(w, n_rows, n, q, act, out);
}

/* Build the device job table for a batch; all jobs share one launch shape. */
static int build_jobs(const sllm_gfx950_gemv_job *jobs, size_t n_jobs, k_gemv_job *kj,
                      gemv_shape *shape_out, uint32_t *n_wg_out, uint32_t *lds_out) {
    size_t max_rows = 0, max_k = 0, total_rows = 0;
    for (size_t i = 0; i < n_jobs; ++i) {
        const sllm_gfx950_gemv_job *j = &jobs[i];
        int st = check_gemv_args(j->w, j->n_rows, j->n, j->q);
        if (st != SLLM_GFX950_OK) return st;
        if (j->out == NULL && j->rows_out == NULL) return fail(SLLM_GFX950_ERR_ARG, "batch job %zu: no output", i);
        if (j->out != NULL && j->act == NULL) return fail(SLLM_GFX950_ERR_ARG, "batch job %zu: epilogue needs act", i);
        if (j->n_rows > max_rows) max_rows = j->n_rows;
        if (j->n > max_k) max_k = j->n;
        total_rows += j->n_rows;
    }
    /* one shape for the whole launch, judged on the total row count and the
     * largest K (any shape is correct for any K; the choice only moves lane
     * utilisation) */
    const gemv_shape s = choose_shape(total_rows, max_k);
    uint64_t wg = 0;
    for (size_t i = 0; i < n_jobs; ++i) {
        const sllm_gfx950_gemv_job *j = &jobs[i];
        kj[i] = (k_gemv_job) { j->w, j->q, j->act, j->out, j->rows_out, (uint32_t) j->n_rows,
                               (uint32_t) j->n, (uint32_t) wg, s.rows_per_wg };
        wg += (j->n_rows + s.rows_per_wg - 1) / s.rows_per_wg;
    }
    if (wg > UINT32_MAX) return fail(SLLM_GFX950_ERR_TOO_LARGE, "batch: too many workgroups");
    *shape_out = s;
    *n_wg_out = (uint32_t) wg;
    *lds_out = (uint32_t) max_k;
    (void) max_rows;
    return SLLM_GFX950_OK;
}

static int launch_group(const void *jobs_dev, uint32_t n_jobs, uint32_t n_wg, uint32_t lds,
                        const gemv_shape *s) {
    void *args[] = { (void *) &jobs_dev, &n_jobs };
    return launch(g.k_group[s->lpr_idx], n_wg, (uint32_t) (64 * s->waves), lds, args);
}

int sllm_gfx950_gemv_batch(const sllm_gfx950_gemv_job *jobs, size_t n_jobs) {
    NEED_OPEN();
    if (n_jobs == 0) return SLLM_GFX950_OK;
    if (jobs == NULL || n_jobs > UINT32_MAX) return fail(SLLM_GFX950_ERR_ARG, "batch: bad job list");
    k_gemv_job *kj = malloc(n_jobs * sizeof *kj);
    if (kj == NULL) return fail(SLLM_GFX950_ERR_NOMEM, "batch: host job table");
    gemv_shape s;
    uint32_t n_wg = 0, lds = 0;
    int st = build_jobs(jobs, n_jobs, kj, &s, &n_wg, &lds);
    const size_t bytes = n_jobs * sizeof *kj;
    if (st == SLLM_GFX950_OK && bytes > g.jobs_cap) {
        /* the previous table may still be read by an enqueued launch */
        hipError_t e = hipStreamSynchronize(g.stream);
        if (e == hipSuccess && g.jobs_dev) e = hipFree(g.jobs_dev);
        g.jobs_dev = NULL;
        g.jobs_cap = 0;
        if (e == hipSuccess) e = hipMalloc(&g.jobs_dev, bytes);
        if (e != hipSuccess) st = hip_fail(e, "batch: job table");
        else g.jobs_cap = bytes;
    }
    if (st == SLLM_GFX950_OK) {
        /* synchronous upload: the host table is freed below, and a launch
         * already enqueued may be reading the device table */
        hipError_t e = hipStreamSynchronize(g.stream);
        if (e == hipSuccess) e = hipMemcpy(g.jobs_dev, kj, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) st = hip_fail(e, "batch: job upload");
    }
    free(kj);
    if (st != SLLM_GFX950_OK) return st;
    return launch_group(g.jobs_dev, (uint32_t) n_jobs, n_wg, lds, &s);
}

int sllm_gfx950_plan_create(const sllm_gfx950_gemv_job *jobs, size_t n_jobs,
                            sllm_gfx950_plan **plan) {
    NEED_OPEN();
    if (plan == NULL) return fail(SLLM_GFX950_ERR_ARG, "plan: NULL out pointer");
    *plan = NULL;
    if (jobs == NULL || n_jobs == 0 || n_jobs > UINT32_MAX) return fail(SLLM_GFX950_ERR_ARG, "plan: bad job list");
    k_gemv_job *kj = malloc(n_jobs * sizeof *kj);
    sllm_gfx950_plan *p = calloc(1, sizeof *p);
    if (kj == NULL || p == NULL) {
        free(kj);
        free(p);
        return fail(SLLM_GFX950_ERR_NOMEM, "plan: host tables");
    }
    gemv_shape s;
    int st = build_jobs(jobs, n_jobs, kj, &s, &p->n_wg, &p->lds);
    if (st == SLLM_GFX950_OK) {
        hipError_t e = hipMalloc(&p->jobs_dev, n_jobs * sizeof *kj);
        if (e == hipSuccess) e = hipMemcpy(p->jobs_dev, kj, n_jobs * sizeof *kj, hipMemcpyHostToDevice);
        if (e != hipSuccess) st = hip_fail(e, "plan: job table");
    }
    free(kj);
    if (st != SLLM_GFX950_OK) {
        if (p->jobs_dev) hipFree(p->jobs_dev);
        free(p);
        return st;
    }
    p->n_jobs = (uint32_t) n_jobs;
    p->lpr_idx = s.lpr_idx;
    p->threads = 64 * s.waves;
    *plan = p;
    return SLLM_GFX950_OK;
}

int sllm_gfx950_plan_run(const sllm_gfx950_plan *p) {
    NEED_OPEN();
    if (p == NULL) return fail(SLLM_GFX950_ERR_ARG, "plan_run: NULL plan");
    const gemv_shape s = { p->lpr_idx, p->threads / 64, 0 };
    return launch_group(p->jobs_dev, p->n_jobs, p->n_wg, p->lds, &s);
}

void sllm_gfx950_plan_destroy(sllm_gfx950_plan *p) {
    if (p == NULL) return;
    if (g.open) {
        hipStreamSynchronize(g.stream);
        hipFree(p->jobs_dev);
    }
    free(p);
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

int sllm_gfx950_tensor_register(const void *packed, size_t n_rows, size_t n) {
    NEED_OPEN();
    if (packed == NULL) return fail(SLLM_GFX950_ERR_ARG, "register: NULL tensor");
    if (n % SLLM_GFX950_QK != 0 || n == 0) return fail(SLLM_GFX950_ERR_TENSOR_SHAPE, "register: K=%zu is not a positive multiple of 128", n);
    const size_t bytes = n_rows * (n / 4) + 32;
    pthread_mutex_lock(&g_mtx);
    int st = SLLM_GFX950_OK;
    const uint8_t *h = packed;
    size_t pos = 0;
    while (pos < g.n_regs && g.regs[pos].host < h) ++pos;
    if ((pos < g.n_regs && g.regs[pos].host < h + bytes) ||
        (pos > 0 && g.regs[pos - 1].host + g.regs[pos - 1].bytes > h)) {
        st = fail(SLLM_GFX950_ERR_ARG, "register: tensor overlaps a registered one");
        goto out;
    }
    if (g.n_regs == g.cap_regs) {
        const size_t cap = g.cap_regs ? 2 * g.cap_regs : 256;
        reg_tensor *r = realloc(g.regs, cap * sizeof *r);
        if (r == NULL) { st = fail(SLLM_GFX950_ERR_NOMEM, "register: registry"); goto out; }
        g.regs = r;
        g.cap_regs = cap;
    }
    uint8_t *dev = NULL;
    hipError_t e = hipMalloc((void **) &dev, bytes);
    if (e == hipSuccess) e = hipMemcpy(dev, h, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (dev) hipFree(dev);
        st = hip_fail(e, "register: upload");
        goto out;
    }
    memmove(&g.regs[pos + 1], &g.regs[pos], (g.n_regs - pos) * sizeof *g.regs);
    g.regs[pos] = (reg_tensor) { h, bytes, dev };
    g.n_regs++;
out:
    pthread_mutex_unlock(&g_mtx);
    return st;
}

int sllm_gfx950_tensor_unregister(const void *packed) {
    NEED_OPEN();
    pthread_mutex_lock(&g_mtx);
    const ptrdiff_t i = reg_find(packed);
    int st = SLLM_GFX950_OK;
    if (i < 0 || g.regs[i].host != (const uint8_t *) packed) {
        st = fail(SLLM_GFX950_ERR_NOT_REGISTERED, "unregister: %p is not a registered tensor", packed);
    } else {
        hipStreamSynchronize(g.stream);
        hipFree(g.regs[i].dev);
        memmove(&g.regs[i], &g.regs[i + 1], (g.n_regs - (size_t) i - 1) * sizeof *g.regs);
        g.n_regs--;
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

static int scratch_reserve(size_t bytes) {
    if (bytes <= g.scratch_bytes) return SLLM_GFX950_OK;
    HIP_TRY(hipStreamSynchronize(g.stream));
    if (g.scratch) HIP_TRY(hipFree(g.scratch));
    g.scratch = NULL;
    g.scratch_bytes = 0;
    HIP_TRY(hipMalloc(&g.scratch, bytes));
    g.scratch_bytes = bytes;
    return SLLM_GFX950_OK;
}

static size_t align16(size_t v) { return (v + 15u) & ~(size_t) 15u; }

/* The reference's hot-path functions cannot return a status; failing
 * silently (zeros) would read as a wrong answer, and falling back to a CPU
 * kernel would hide that the GPU row is broken. So: say why, and stop. */
static void die(const char *fn, int st) {
    fprintf(stderr, "libsllm_gfx950: %s failed: %s: %s\n", fn, sllm_gfx950_status_string(st), g_err);
    abort();
}

void sllm_gfx950_i2s_quant_act(const float *x, size_t n, int8_t *q_out, sllm_gfx950_act *out) {
    if (!g.open) die("sllm_gfx950_i2s_quant_act", fail(SLLM_GFX950_ERR_NO_DEVICE, "library not open"));
    if (x == NULL || q_out == NULL || out == NULL || n == 0) return;
    pthread_mutex_lock(&g_mtx);
    const size_t off_q = align16(n * sizeof(float));
    const size_t off_a = off_q + align16(n);
    int st = scratch_reserve(off_a + 16);
    uint8_t *s = g.scratch;
    if (st == SLLM_GFX950_OK) {
        hipError_t e = hipMemcpyAsync(s, x, n * sizeof(float), hipMemcpyHostToDevice, g.stream);
        if (e != hipSuccess) st = hip_fail(e, "quant_act upload");
    }
    if (st == SLLM_GFX950_OK) st = sllm_gfx950_quant_act((const float *) s, n, 1, (int8_t *) (s + off_q), (sllm_gfx950_act *) (s + off_a));
    if (st == SLLM_GFX950_OK) {
        hipError_t e = hipMemcpyAsync(q_out, s + off_q, n, hipMemcpyDeviceToHost, g.stream);
        if (e == hipSuccess) e = hipMemcpyAsync(out, s + off_a, sizeof *out, hipMemcpyDeviceToHost, g.stream);
        if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
        if (e != hipSuccess) st = hip_fail(e, "quant_act download");
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
    const size_t off_o = align16(n);
    if (st == SLLM_GFX950_OK) st = scratch_reserve(off_o + n_rows * sizeof(int32_t));
    uint8_t *s = g.scratch;
    if (st == SLLM_GFX950_OK) {
        hipError_t e = hipMemcpyAsync(s, q, n, hipMemcpyHostToDevice, g.stream);
        if (e != hipSuccess) st = hip_fail(e, "gemv upload");
    }
    if (st == SLLM_GFX950_OK) {
        const uint8_t *wd = g.regs[i].dev + (w - g.regs[i].host);
        st = sllm_gfx950_gemv(wd, n_rows, n, (const int8_t *) s, (int32_t *) (s + off_o));
    }
    if (st == SLLM_GFX950_OK) {
        hipError_t e = hipMemcpyAsync(rows_out, s + off_o, n_rows * sizeof(int32_t), hipMemcpyDeviceToHost, g.stream);
        if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
        if (e != hipSuccess) st = hip_fail(e, "gemv download");
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
