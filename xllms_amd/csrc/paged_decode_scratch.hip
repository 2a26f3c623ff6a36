// Fixed device scratch of the allocation-free decode entry point
// (nxt_paged_attention_noalloc): the split-K partials and the unit prefix
// live in a file-scope __device__ array instead of a hipMalloc'd workspace.
//
// Each device the library runs on holds its own copy of the array until the
// process ends.  Host code never uses the array's name as a device address:
// the first call on a device (that device current) looks its address up with
// hipGetSymbolAddress, and every later use goes through that pointer.
// Every no-alloc call on one device shares the array, so the entry point
// orders such calls on the GPU (noalloc_gate.h): two whose kernels overlapped
// would race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "paged_decode_scratch.h"

namespace {

static __device__ __align__(256) char scratch[xhip::kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices];

}  // namespace

namespace xhip {

hipError_t noalloc_scratch(int device, void **ptr, size_t *bytes) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        // `device` is the caller's current device: the lookup resolves this
        // device's copy of the array
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_ptr[device] = p;
    }
    *ptr = g_ptr[device];
    *bytes = kNoAllocScratchBytes;
    return hipSuccess;
}

}  // namespace xhip
