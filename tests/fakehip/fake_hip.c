/*
 * fake_hip.c -- a host-memory stand-in for the HIP runtime, for CPU tests of
 * the library's failure paths. TEST INFRASTRUCTURE ONLY.
 *
 * The library's C sources (gfx950_shim.c, decode.c, gguf_load.c,
 * dispatch.c) are linked against this file instead of libamdhip64 into
 * tests/fakehip/libsllm_gfx950_fakehip.so. It reports one gfx950 device;
 * device and pinned memory are host memory; copies and fills are memcpy /
 * memset; kernel launches do nothing, except the two the host-pointer row
 * waits on (sllm_k_host_done, sllm_k_quant_host), whose completion word it
 * sets. Numbers are not the point: with any HIP call made to fail on demand,
 * the tests show which status reaches the caller and that nothing is left
 * allocated.
 *
 *   fakehip_fail(fn, err, skip)  the (skip+1)-th call of `fn` from now ("*":
 *                                of any call below) returns `err`, once, and
 *                                does nothing else
 *   fakehip_fired()              whether the armed failure has happened
 *   fakehip_live()               resources held: memory, modules, streams,
 *                                events, graphs
 *   fakehip_calls()              HIP calls made so far
 */
#include <hip/hip_runtime_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define FAKE_EXPORT __attribute__((visibility("default")))

static char     g_fail_fn[64];
static int      g_fail_err;
static long     g_fail_skip = -1;     /* < 0: disarmed */
static int      g_fired;
static long     g_live;
static unsigned long g_calls;

FAKE_EXPORT void fakehip_fail(const char *fn, int err, unsigned skip) {
    snprintf(g_fail_fn, sizeof g_fail_fn, "%s", fn);
    g_fail_err = err;
    g_fail_skip = (long) skip;
    g_fired = 0;
}
FAKE_EXPORT void fakehip_clear(void) { g_fail_skip = -1; g_fired = 0; }
FAKE_EXPORT int  fakehip_fired(void) { return g_fired; }
FAKE_EXPORT long fakehip_live(void) { return g_live; }
FAKE_EXPORT unsigned long fakehip_calls(void) { return g_calls; }

static int inject(const char *fn) {
    ++g_calls;
    if (g_fail_skip < 0) return 0;
    if (strcmp(g_fail_fn, "*") != 0 && strcmp(g_fail_fn, fn) != 0) return 0;
    if (g_fail_skip-- > 0) return 0;
    g_fired = 1;
    return 1;
}
#define INJECT() do { if (inject(__func__)) return (hipError_t) g_fail_err; } while (0)

/* device and pinned memory: host memory behind a small header */
typedef struct fake_block { size_t bytes; uint64_t magic; } fake_block;
#define FAKE_MAGIC 0x66616b6568697021ull

static void *fake_alloc(size_t bytes) {
    fake_block *b = calloc(1, sizeof *b + 64 + bytes);
    if (b == NULL) return NULL;
    b->bytes = bytes;
    b->magic = FAKE_MAGIC;
    ++g_live;
    return (uint8_t *) (b + 1) + 64;            /* 16-byte-plus alignment, as the device's */
}

static hipError_t fake_release(void *p) {
    if (p == NULL) return hipSuccess;
    fake_block *b = (fake_block *) ((uint8_t *) p - 64) - 1;
    if (b->magic != FAKE_MAGIC) { fprintf(stderr, "fake_hip: free of %p, not an allocation\n", p); abort(); }
    b->magic = 0;
    free(b);
    --g_live;
    return hipSuccess;
}

hipError_t hipMalloc(void **p, size_t bytes) {
    *p = NULL;
    INJECT();
    *p = fake_alloc(bytes);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void *p) { ++g_calls; return fake_release(p); }
hipError_t hipHostMalloc(void **p, size_t bytes, unsigned int flags) {
    (void) flags;
    *p = NULL;
    INJECT();
    *p = fake_alloc(bytes);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void *p) { ++g_calls; return fake_release(p); }
hipError_t hipHostGetDevicePointer(void **d, void *h, unsigned int flags) {
    (void) flags;
    INJECT();
    *d = h;
    return hipSuccess;
}

hipError_t hipGetDeviceCount(int *n) { *n = 0; INJECT(); *n = 1; return hipSuccess; }
hipError_t hipGetDeviceProperties(hipDeviceProp_t *p, int d) {
    INJECT();
    if (d != 0) return hipErrorInvalidDevice;
    memset(p, 0, sizeof *p);
    snprintf(p->name, sizeof p->name, "fake");
    snprintf(p->gcnArchName, sizeof p->gcnArchName, "gfx950:sramecc+:xnack-");
    p->multiProcessorCount = 256;
    p->totalGlobalMem = (size_t) 288 << 30;
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { INJECT(); return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
const char *hipGetErrorString(hipError_t e) {
    static char buf[64];
    snprintf(buf, sizeof buf, "fake HIP error %d", (int) e);
    return buf;
}

/* modules: a function handle carries its name, for the launches emulated */
typedef struct fake_fn { char name[96]; } fake_fn;
typedef struct fake_mod { fake_fn fns[64]; int n; } fake_mod;

hipError_t hipModuleLoadData(hipModule_t *m, const void *image) {
    (void) image;
    *m = NULL;
    INJECT();
    fake_mod *fm = calloc(1, sizeof *fm);
    if (fm == NULL) return hipErrorOutOfMemory;
    ++g_live;
    *m = (hipModule_t) fm;
    return hipSuccess;
}
hipError_t hipModuleUnload(hipModule_t m) {
    ++g_calls;
    if (m == NULL) return hipErrorInvalidResourceHandle;
    free(m);
    --g_live;
    return hipSuccess;
}
hipError_t hipModuleGetFunction(hipFunction_t *f, hipModule_t m, const char *name) {
    *f = NULL;
    INJECT();
    fake_mod *fm = (fake_mod *) m;
    for (int i = 0; i < fm->n; ++i) {
        if (strcmp(fm->fns[i].name, name) == 0) { *f = (hipFunction_t) &fm->fns[i]; return hipSuccess; }
    }
    if (fm->n == 64) return hipErrorOutOfMemory;
    snprintf(fm->fns[fm->n].name, sizeof fm->fns[fm->n].name, "%s", name);
    *f = (hipFunction_t) &fm->fns[fm->n++];
    return hipSuccess;
}
hipError_t hipModuleLaunchKernel(hipFunction_t f, unsigned int gx, unsigned int gy, unsigned int gz,
                                 unsigned int bx, unsigned int by, unsigned int bz, unsigned int lds,
                                 hipStream_t s, void **args, void **extra) {
    (void) gx; (void) gy; (void) gz; (void) bx; (void) by; (void) bz; (void) lds; (void) s; (void) extra;
    INJECT();
    const char *name = ((const fake_fn *) f)->name;
    if (strcmp(name, "sllm_k_host_done") == 0) {
        **(uint32_t **) args[0] = *(uint32_t *) args[1];
    } else if (strcmp(name, "sllm_k_quant_host") == 0) {
        **(uint32_t **) args[6] = *(uint32_t *) args[7];
    }
    return hipSuccess;
}

/* streams, events, graphs */
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned int flags) {
    (void) flags;
    *s = NULL;
    INJECT();
    *s = (hipStream_t) malloc(1);
    ++g_live;
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) { ++g_calls; free(s); --g_live; return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t s) { (void) s; INJECT(); return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t *e) { *e = NULL; INJECT(); *e = (hipEvent_t) malloc(1); ++g_live; return hipSuccess; }
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned flags) { (void) flags; return hipEventCreate(e); }
hipError_t hipEventDestroy(hipEvent_t e) { ++g_calls; free(e); --g_live; return hipSuccess; }
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) { (void) e; (void) s; INJECT(); return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t e) { (void) e; INJECT(); return hipSuccess; }
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b) {
    (void) a; (void) b;
    INJECT();
    *ms = 0.0f;
    return hipSuccess;
}
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode mode) { (void) s; (void) mode; INJECT(); return hipSuccess; }
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t *g) {
    (void) s;
    *g = NULL;
    INJECT();
    *g = (hipGraph_t) malloc(1);
    ++g_live;
    return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t *x, hipGraph_t g, hipGraphNode_t *node, char *log, size_t n) {
    (void) g; (void) node; (void) log; (void) n;
    *x = NULL;
    INJECT();
    *x = (hipGraphExec_t) malloc(1);
    ++g_live;
    return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t x, hipStream_t s) { (void) x; (void) s; INJECT(); return hipSuccess; }
hipError_t hipGraphExecDestroy(hipGraphExec_t x) { ++g_calls; free(x); --g_live; return hipSuccess; }
hipError_t hipGraphDestroy(hipGraph_t g) { ++g_calls; free(g); --g_live; return hipSuccess; }

/* copies and fills */
hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind k) {
    (void) k;
    INJECT();
    if (n) memmove(d, s, n);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind k, hipStream_t st) {
    (void) k; (void) st;
    INJECT();
    if (n) memmove(d, s, n);
    return hipSuccess;
}
hipError_t hipMemcpy2DAsync(void *d, size_t dp, const void *s, size_t sp, size_t w, size_t h,
                            hipMemcpyKind k, hipStream_t st) {
    (void) k; (void) st;
    INJECT();
    for (size_t r = 0; r < h; ++r) memmove((uint8_t *) d + r * dp, (const uint8_t *) s + r * sp, w);
    return hipSuccess;
}
hipError_t hipMemset(void *d, int v, size_t n) { INJECT(); memset(d, v, n); return hipSuccess; }
hipError_t hipMemsetAsync(void *d, int v, size_t n, hipStream_t st) { (void) st; INJECT(); memset(d, v, n); return hipSuccess; }
hipError_t hipMemset2DAsync(void *d, size_t pitch, int v, size_t w, size_t h, hipStream_t st) {
    (void) st;
    INJECT();
    for (size_t r = 0; r < h; ++r) memset((uint8_t *) d + r * pitch, v, w);
    return hipSuccess;
}

/* noalloc.hip's static device array (a HIP translation unit in the real
 * build): host memory here, resolved the same way once per device */
static unsigned char g_noalloc_array[1u << 20];
__attribute__((visibility("hidden"))) int sllm_noalloc_resolve(int device, void **out) {
    *out = NULL;
    if (inject("hipGetSymbolAddress")) return g_fail_err;
    if (device != 0) return (int) hipErrorInvalidDevice;
    *out = g_noalloc_array;
    return 0;
}
