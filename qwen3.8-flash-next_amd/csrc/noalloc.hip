/*
 * noalloc.hip -- the scratch of qmoe_layer_forward_noalloc: one block of
 * device memory at file scope, so that every GPU the library runs on holds
 * its own copy from the moment the code object is loaded there until the
 * process ends, and nothing is allocated at call time.
 *
 * In host code `scratch` names a host-side stand-in, not device memory:
 * the block's device address on the current GPU comes from
 * hipGetSymbolAddress, looked up once per device on the first call there
 * and kept; only that address is ever handed to kernels.
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "qmoe_internal.h"

static __device__ __align__(256) unsigned char scratch[QK_NOALLOC_SCRATCH_BYTES];

#define QK_NOALLOC_MAX_DEVICES 64

static void *g_scratch[QK_NOALLOC_MAX_DEVICES]; /* the block's address per device */
static std::mutex g_lock;

extern "C" int qk_noalloc_scratch(void **ptr) {
    *ptr = nullptr;
    int dev = 0;
    hipError_t rc = hipGetDevice(&dev);
    if (rc != hipSuccess) return (int)rc;
    if (dev < 0 || dev >= QK_NOALLOC_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> hold(g_lock);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != hipSuccess) return (int)rc;
        if (!p) return (int)hipErrorInvalidSymbol;
        g_scratch[dev] = p;
    }
    *ptr = g_scratch[dev];
    return 0;
}
