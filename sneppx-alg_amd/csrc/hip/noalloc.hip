// noalloc.hip - the scratch buffer of the allocation-free entry point
// (SNEPPX_qlinear_w4a16_noalloc): a file-scope device array of
// SNEPPX_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until
// the process ends, so a call needs no device allocation at all.
//
// In host code the array's name is a host-side stand-in, not a device
// address.  Its address on a device comes from hipGetSymbolAddress, looked up
// once per device (with that device current, at the entry point's first call
// there) and kept in g_scratch[dev]; only that pointer is ever handed to
// kernels.  Each device has its own copy at its own address.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "launch.h"
#include "sneppx_qlinear.h"
#include "../snx_internal.h"

static __device__ __align__(256) uint8_t scratch[SNEPPX_NOALLOC_SCRATCH_BYTES];

namespace {
std::atomic<void*> g_scratch[snx::kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

extern "C" void* snx_noalloc_scratch(size_t bytes, const char* who) {
    if (bytes > (size_t)SNEPPX_NOALLOC_SCRATCH_BYTES) {
        snx_set_error("%s: this call needs %zu bytes of scratch, more than the %zu of the "
                      "library's static buffer", who, bytes, (size_t)SNEPPX_NOALLOC_SCRATCH_BYTES);
        return nullptr;
    }
    const int dev = snx::current_device();
    if (dev < 0) {
        snx_set_error("%s: no current device (or device index beyond %d)", who, snx::kMaxDevices - 1);
        return nullptr;
    }
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            snx_set_error("%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                          hipGetErrorString(e));
            return nullptr;
        }
        g_scratch[dev].store(p, std::memory_order_release);
    }
    return p;
}
