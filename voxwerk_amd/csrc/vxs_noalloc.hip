// vxs_noalloc.hip — the fixed device scratch of vxs_sample_noalloc.
//
// vxs_sample stages its host inputs in buffers the context allocates and grows. For callers that
// may not allocate (tight serving loops, harnesses that forbid hipMalloc), vxs_sample_noalloc
// stages them in this array instead: a file-scope device array of kNoAllocScratchBytes, one copy
// per GPU, held until the process ends. Host code never passes the array's name to a kernel or a
// copy (in host code it only stands for the symbol): set-up looks up its device address once per
// device, with that device current, and every use goes through that address. A per-device lock,
// held by vxs_sample_noalloc for the whole (synchronous) call, keeps calls on one GPU from
// overlapping in its scratch, whichever threads or contexts make them.
#include <hip/hip_runtime.h>

#include <mutex>

#include "vxs_internal.h"

namespace vxs {
namespace {

__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};
std::mutex g_use[kMaxDevices];  // held while a call stages, samples and fetches on that device

}  // namespace

hipError_t noalloc_scratch(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    return hipSuccess;
}

std::mutex& noalloc_lock(int device) { return g_use[device]; }

}  // namespace vxs
