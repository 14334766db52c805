// Host-side helper: a kernel that takes more than 64 KiB of dynamic LDS needs its
// hipFuncAttributeMaxDynamicSharedMemorySize raised before the first launch.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

namespace apex_hip {

// Raise `kernel`'s dynamic LDS limit to `bytes` once per device (the current one);
// `done` holds one bit per device (devices 0..63; others set it on every call).
// Safe to call from several threads.
template <typename F>
hipError_t allow_dynamic_lds(F *kernel, size_t bytes, std::atomic<uint64_t> &done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    const uint64_t bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit))
        return hipSuccess;
    e = hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)bytes);
    if (e == hipSuccess && bit)
        done.fetch_or(bit, std::memory_order_release);
    return e;
}

} // namespace apex_hip
