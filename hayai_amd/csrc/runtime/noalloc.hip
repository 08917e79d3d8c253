// The fixed scratch array of the no-allocation FFN entry point (hh_ffn_dev_noalloc).
//
// Some callers cannot allocate device memory at call time (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).  For them the FFN's intermediate
// lives in this file-scope device array instead of the engine's growable workspaces.  Every
// GPU the library runs on holds its own copy of the array for the life of the process; its
// device address is looked up once per device (noalloc_scratch, called by engine creation
// with the device current) and only that address is handed to kernels.  The array's name in
// host code is a host-side stand-in, never a device address.
//
// All calls on one GPU share the array: calls that overlap on one GPU (two engines' streams,
// or one engine from two threads) race on it.  Nothing in it must start at zero: each call
// writes the intermediate in full before reading it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "engine.h"

static __device__ __align__(256) unsigned char scratch[HH_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void* g_scratch[kMaxDevices] = {};
}  // namespace

namespace hh {

hh_status noalloc_scratch(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices)
        return fail(HH_ERR_INVALID, "noalloc scratch: device %d beyond the %d this build tracks", device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_mutex);
    if (!g_scratch[device]) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(noalloc scratch)");
        if (!p) return fail(HH_ERR_RUNTIME, "hipGetSymbolAddress(noalloc scratch) returned a null address");
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return HH_OK;
}

}  // namespace hh
