// noalloc.hip -- the device array behind sllm_gfx950_gemv_batch_noalloc.
//
// A batch of GEMVs needs device memory beyond its inputs and outputs: the
// job table, one descriptor per workgroup and, for streaming jobs that
// quantise an activation without giving q / act buffers, the quantised rows.
// sllm_gfx950_gemv_batch allocates them per call; the no-allocation variant
// places them in this file-scope array instead, one copy per device, which
// the device holds until the process ends.
//
// Host code never uses the array's name as a device address: its address on
// a device comes from hipGetSymbolAddress, resolved once per device with that
// device current (at sllm_gfx950_open), and only that address is handed to
// copies and kernels.
#include <hip/hip_runtime.h>

#include <stddef.h>

#include <saphira_amd/sllm_gfx950.h>

#define SLLM_NOALLOC_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[SLLM_GFX950_NOALLOC_SCRATCH_BYTES];

static void *g_scratch_dev[SLLM_NOALLOC_MAX_DEVICES];

// The array's address on `device`, which must be the current device; looked
// up on the first call for that device and kept. 0, or the HIP error.
extern "C" __attribute__((visibility("hidden"))) int sllm_noalloc_resolve(int device, void **out) {
    *out = nullptr;
    if (device < 0 || device >= SLLM_NOALLOC_MAX_DEVICES) return (int) hipErrorInvalidDevice;
    if (g_scratch_dev[device] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int) e;
        if (p == nullptr) return (int) hipErrorInvalidSymbol;
        g_scratch_dev[device] = p;
    }
    *out = g_scratch_dev[device];
    return 0;
}
