// kernel_attr.h -- host helper: a kernel's dynamic-LDS limit, set once per
// (kernel, device, size) and safe to call from several host threads (the
// asynchronous worker and callers launch concurrently).
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <set>
#include <tuple>

namespace tessa {

inline int ensure_lds_limit(const void *kernel, int bytes) {
    static std::mutex mu;
    static std::set<std::tuple<const void *, int, int>> done;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_tuple(kernel, dev, bytes);
    if (done.count(key)) return 0;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) return -1;
    done.insert(key);
    return 0;
}

}  // namespace tessa
