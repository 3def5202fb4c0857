// Per-device launch set-up shared by the kernel launchers, safe under
// concurrent first calls from several threads: dynamic LDS above the 64 KiB
// default (one hipFuncSetAttribute per device and kernel) and the CU count.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <mutex>
#include <map>
#include <utility>

namespace kk {

// gfx950: 160 KiB of LDS per workgroup.
constexpr size_t kLdsOptInBytes = 160 * 1024;

// Raises `kernel`'s dynamic-LDS limit on the current device to at least
// `bytes` when a launch needs more than the 64 KiB default. The limit only
// grows (a later launch with a larger K raises it again), and the kernel's
// static LDS plus `bytes` must fit the 160 KiB the hardware has, which
// hipFuncSetAttribute checks. hipSuccess or the HIP error.
inline hipError_t opt_in_lds(const void *kernel, size_t bytes) {
    if (bytes <= 64 * 1024) return hipSuccess;
    if (bytes > kLdsOptInBytes) return hipErrorInvalidValue;
    int device = 0;
    hipError_t rc = hipGetDevice(&device);
    if (rc != hipSuccess) return rc;
    static std::mutex mutex;
    static std::map<std::pair<int, const void *>, size_t> granted;
    std::lock_guard<std::mutex> lock(mutex);
    size_t &have = granted[{device, kernel}];
    if (have >= bytes) return hipSuccess;
    rc = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (rc == hipSuccess) have = bytes;
    return rc;
}

// Compute units of `device`, read once per device (256 when the query fails).
inline int cu_count(int device) {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cached[kMaxDevices];
    if (device < 0 || device >= kMaxDevices) return 256;
    int v = cached[device].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || v <= 0) v = 256;
    cached[device].store(v, std::memory_order_relaxed);
    return v;
}

} // namespace kk
