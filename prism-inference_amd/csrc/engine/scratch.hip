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
 *
 * Calls on one GPU share its array, so they are put in order: the same first
 * call creates the device's completion event, each call's stream waits for
 * the previous call's event and records it again after its own launches, and
 * a host mutex per device keeps those two steps of concurrent callers from
 * interleaving.
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "ctx.h"

static __device__ __align__(256) unsigned char scratch[PRISM_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_addr[PRISM_SCRATCH_MAX_DEVICES] = {};
/* per device: the last call's completion and the lock that orders calls */
hipEvent_t g_scratch_done[PRISM_SCRATCH_MAX_DEVICES] = {};
std::mutex g_scratch_call_mu[PRISM_SCRATCH_MAX_DEVICES];
}  // namespace

hipError_t scratch_device_address(int device, void** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= PRISM_SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
    if (!g_scratch_addr[device]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        hipEvent_t ev = nullptr;
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return e;
        g_scratch_done[device] = ev;
        g_scratch_addr[device] = p;
    }
    *out = g_scratch_addr[device];
    return hipSuccess;
}

hipEvent_t scratch_done_event(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return device >= 0 && device < PRISM_SCRATCH_MAX_DEVICES ? g_scratch_done[device] : nullptr;
}

std::mutex& scratch_call_mutex(int device) { return g_scratch_call_mu[device]; }
