// Scratch of the allocation-free verify entry point (kyro_spec_verify_noalloc): a fixed-size
// array in this library's code object, one copy per device, held until the process ends.
//
// The array's name is a host-side stand-in in host code, not a device address: passing it to a
// kernel would fault. Its address on a device comes from hipGetSymbolAddress with that device
// current, once per device (at kyro_ctx_create), and only that address is handed to kernels.
#include <mutex>

#include "kernels.hpp"

namespace kyro {

namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices];  // the array's device address on each device (null: not set up)

}  // namespace

hipError_t noalloc_scratch(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

}  // namespace kyro
