// launch.h - per-device launch facts shared by the kernel launchers: the
// current device's CU count, and a kernel's one-time opt-in to more than
// 64 KB of dynamic LDS.  Both are kept per device (devices 0..63), since a
// process may drive several GPUs and each holds its own function attributes.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

namespace snx {

constexpr int kMaxDevices = 64;

// the current device, or -1 when it cannot be read or is beyond kMaxDevices
inline int current_device() {
    int d = 0;
    return hipGetDevice(&d) == hipSuccess && d >= 0 && d < kMaxDevices ? d : -1;
}

// CU count of the current device (256, the MI355X's, if it cannot be read)
inline int cu_count() {
    static std::atomic<int> ncu[kMaxDevices];   // 0: not asked yet
    const int d = current_device();
    if (d < 0) return 256;
    int n = ncu[d].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || n <= 0)
        n = 256;
    ncu[d].store(n, std::memory_order_relaxed);
    return n;
}

// Opts kernel `fn` into `bytes` of dynamic LDS on the current device, once
// per device; `done` is the caller's mask for that kernel (bit d: device d).
inline hipError_t lds_optin(const void* fn, int bytes, std::atomic<uint64_t>& done) {
    const int d = current_device();
    if (d < 0) return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    const uint64_t bit = 1ull << d;
    if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) done.fetch_or(bit, std::memory_order_acq_rel);
    return e;
}

}  // namespace snx
