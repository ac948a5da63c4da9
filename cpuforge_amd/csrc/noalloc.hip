// Fixed device scratch for the entry points that allocate nothing
// (cfattn_bwd_noalloc): a file-scope device array, resolved once per device
// to its address on that device.
//
// Host code never passes the array's name to a kernel or a copy: on the
// host that name is only a stand-in symbol, and a kernel given it would
// fault.  noalloc_init_device() looks the array up with hipGetSymbolAddress
// while the device is current and keeps the device address; every user
// takes that address from noalloc_scratch().
//
// Every call on one device shares that device's array, and it keeps the
// last call's contents.  Calls that overlap on one device race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "cfattn_kernels.hpp"

namespace cfattn {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};
}  // namespace

hipError_t noalloc_init_device(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return hipSuccess;
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_ptr[device] = p;
    return hipSuccess;
}

void* noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    return g_ptr[device];
}

}  // namespace cfattn
