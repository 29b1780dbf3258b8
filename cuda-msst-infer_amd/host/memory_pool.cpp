// memory_pool.cpp — see memory_pool.h.
#include "memory_pool.h"

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

namespace cudasep {

DeviceMemoryPool& DeviceMemoryPool::instance() {
    static DeviceMemoryPool pool;
    return pool;
}

DeviceMemoryPool::~DeviceMemoryPool() {
    // The runtime may already be torn down at static destruction; the
    // driver reclaims device memory with the process, so errors are ignored.
    for (auto& kv : free_) (void)hipFree(kv.second);
}

size_t DeviceMemoryPool::round_size(size_t bytes) {
    if (bytes == 0) bytes = 1;
    constexpr size_t kSmall = 256, kLarge = 2u << 20, kSplit = 1u << 20;
    if (bytes < kSplit) return (bytes + kSmall - 1) / kSmall * kSmall;
    return (bytes + kLarge - 1) / kLarge * kLarge;
}

void* DeviceMemoryPool::allocate(size_t bytes) {
    const size_t need = round_size(bytes);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        throw std::runtime_error("DeviceMemoryPool: hipGetDevice failed");
    {
        std::lock_guard<std::mutex> lock(mu_);
        auto it = free_.lower_bound({dev, need});
        if (it != free_.end() && it->first.first == dev && it->first.second <= 2 * need) {
            void* p = it->second;
            const size_t sz = it->first.second;
            free_.erase(it);
            cached_ -= sz;
            in_use_ += sz;
            live_[p] = Block{sz, dev};
            return p;
        }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, need);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        release_cached();
        e = hipMalloc(&p, need);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            throw std::runtime_error("DeviceMemoryPool: hipMalloc of " + std::to_string(need) +
                                     " bytes failed: " + hipGetErrorString(e));
        }
    }
    std::lock_guard<std::mutex> lock(mu_);
    in_use_ += need;
    live_[p] = Block{need, dev};
    return p;
}

void DeviceMemoryPool::deallocate(void* ptr) {
    if (!ptr) return;
    std::lock_guard<std::mutex> lock(mu_);
    auto it = live_.find(ptr);
    if (it == live_.end()) return;  // not ours
    const Block b = it->second;
    live_.erase(it);
    in_use_ -= b.size;
    cached_ += b.size;
    free_.emplace(std::make_pair(b.device, b.size), ptr);
}

void DeviceMemoryPool::release_cached() {
    std::lock_guard<std::mutex> lock(mu_);
    for (auto& kv : free_) (void)hipFree(kv.second);
    free_.clear();
    cached_ = 0;
}

size_t DeviceMemoryPool::cached_bytes() const {
    std::lock_guard<std::mutex> lock(mu_);
    return cached_;
}

size_t DeviceMemoryPool::in_use_bytes() const {
    std::lock_guard<std::mutex> lock(mu_);
    return in_use_;
}

}  // namespace cudasep
