// noalloc.hip — the fixed device scratch of the allocation-free projection entry point
// (ovfq_project_noalloc_dev).
//
// `scratch` is a file-scope device array: every GPU the library runs on holds its own copy, at its own address,
// until the process ends. In host code the name `scratch` is only a host-side stand-in for the symbol, so host
// code never passes it to a kernel: noalloc_scratch_init resolves the device address of the current device's
// copy once (hipGetSymbolAddress) and every later use goes through that address.
#include <hip/hip_runtime.h>

#include <mutex>

#include "ovfq_launch.h"

namespace ovfq {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {nullptr};

}  // namespace

hipError_t noalloc_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return hipSuccess;
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current first
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[device] = p;
    return hipSuccess;
}

void* noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    return g_ptr[device];
}

}  // namespace ovfq
