// The caller-free scratch of the no-allocation entry point
// (xl_shared_forward_noalloc): one static device array, which every GPU the
// library runs on holds from the module's load until the process ends, used
// in place of a workspace the caller would otherwise allocate.
//
// Host code never passes `scratch` itself to a kernel (in host code the name
// is a host-side stand-in, not a device address): once per device, with that
// device current, hipGetSymbolAddress gives the device's own address of its
// copy, which is kept per device and handed to the kernels as a plain pointer.
// Every call on a GPU shares that GPU's array and sees the last call's
// contents; calls that overlap on one GPU (through any context or stream) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "xl_internal.hpp"

static __device__ __align__(256) uint8_t scratch[xl::kNoAllocScratchBytes];

namespace xl::dev {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};
}  // namespace

hipError_t noalloc_scratch(int device, void** out) {
    if (device < 0 || device >= kMaxDevices || !out) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != device) return hipErrorInvalidDevice;   // the caller makes the device current first
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    return hipSuccess;
}

}  // namespace xl::dev
