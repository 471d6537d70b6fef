/*
 * scratch.hip - the workspace of the allocation-free forward
 * (prism_forward_noalloc): one file-scope device array, `scratch`.
 *
 * Every GPU the library runs on holds its own copy of the array, at its own
 * address, from the first call below on that device until the process ends.
 * In host code the name `scratch` stands for the host-side shadow of the
 * array, not a device address, so it is never passed to a kernel or a copy:
 * scratch_device_address() takes the device address once per device, with
 * that device current, through hipGetSymbolAddress, and keeps it; the engine
 * uses only that pointer (kernel arguments, fill launches).
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "ctx.h"

static __device__ __align__(256) unsigned char scratch[PRISM_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_addr[PRISM_SCRATCH_MAX_DEVICES] = {};
}  // namespace

hipError_t scratch_device_address(int device, void** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= PRISM_SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
    if (!g_scratch_addr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_addr[device] = p;
    }
    *out = g_scratch_addr[device];
    return hipSuccess;
}
