// sgpu_scratch.hip -- the fixed device scratch of the allocation-free split-K entry point
// (sgpu_sgemm_splitk_noalloc): the partial tiles and tile counters of sgemm_splitk in a
// file-scope device array, compiled into libswitchgpu.so, so the entry point never allocates.
//
// Host code never uses the array's name as an address (in host code it names a host-side
// stand-in): at set-up, once per device with that device current, hipGetSymbolAddress
// resolves the device's own copy, and that pointer is what the kernels get and what is
// cleared.  Every call on a device shares that device's copy.
#include <hip/hip_runtime.h>

#include "sgpu_internal.h"
#include "switch_gpu.h"

// Partial tiles first (SGPU_SCRATCH_FLOATS floats), then SGPU_SCRATCH_TILES counters.
static __device__ __align__(256) unsigned char scratch[(size_t)SGPU_SCRATCH_FLOATS * 4 + (size_t)SGPU_SCRATCH_TILES * 4];

static void* g_scratch[SGPU_MAX_DEVICES];

extern "C" int sgpu_internal_scratch_setup(int dev) {
    if (dev < 0 || dev >= SGPU_MAX_DEVICES) return SGPU_ERR_INVALID_ARG;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return SGPU_ERR_NO_KERNEL;
    // the counters start at zero; every launch leaves them at zero again
    e = hipMemset(static_cast<unsigned char*>(p) + (size_t)SGPU_SCRATCH_FLOATS * 4, 0,
                  (size_t)SGPU_SCRATCH_TILES * 4);
    if (e != hipSuccess) return (int)e;
    e = hipDeviceSynchronize();
    if (e != hipSuccess) return (int)e;
    g_scratch[dev] = p;
    return SGPU_OK;
}

extern "C" int sgpu_internal_scratch(int dev, float** ws, unsigned** cnt) {
    if (dev < 0 || dev >= SGPU_MAX_DEVICES || !g_scratch[dev]) return SGPU_ERR_NOT_INITIALIZED;
    *ws = static_cast<float*>(g_scratch[dev]);
    *cnt = reinterpret_cast<unsigned*>(static_cast<unsigned char*>(g_scratch[dev]) + (size_t)SGPU_SCRATCH_FLOATS * 4);
    return SGPU_OK;
}
