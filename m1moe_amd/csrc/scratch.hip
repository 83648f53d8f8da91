// Fixed-size device scratch for m1moe_moe_prefill_noalloc, the prefill entry
// point that allocates nothing.
//
// `scratch` is a file-scope device array: every GPU that loads this code
// object holds its own copy, at its own address, until the process ends.  On
// the host the name is only a shadow symbol, never a device address:
// static_scratch_attach looks each device's address up once, with that
// device current, and host code passes the pointer it returns to kernels.
// Every call on one GPU shares that GPU's copy and finds the previous call's
// contents in it; calls that overlap on one GPU (two streams, two contexts)
// race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.hpp"

namespace m1moe {
namespace {

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t* g_addr[kMaxDevices] = {};

}  // namespace

int static_scratch_attach(int device, uint8_t** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_addr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return (int)e;
        if (cur != device) return (int)hipErrorInvalidDevice;   // the caller makes it current
        void* p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return (int)e;
        if (!p || (reinterpret_cast<uintptr_t>(p) & 255)) return (int)hipErrorInvalidSymbol;
        g_addr[device] = static_cast<uint8_t*>(p);
    }
    *out = g_addr[device];
    return (int)hipSuccess;
}

}  // namespace m1moe
