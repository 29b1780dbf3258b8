// memory_pool.h — caching device allocator behind cudasep::Tensor.
//
// Plays the role of the reference's CudaMemoryPool (src/memory_pool.h:29-96):
// freed blocks are kept per device and handed out again, so the per-op
// temporaries of an inference loop stop calling hipMalloc/hipFree after the
// first iteration.  Own policy: requests are rounded up to 256 B below
// 1 MiB and to 2 MiB above; a cached block is reused for a request when its
// size is within [request, 2 x request] (best fit).  Thread safe (one
// mutex).  On hipMalloc failure the cache is released and the allocation
// retried once; a second failure throws std::runtime_error.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>

namespace cudasep {

class DeviceMemoryPool {
public:
    static DeviceMemoryPool& instance();

    void* allocate(size_t bytes);
    void deallocate(void* ptr);
    // hipFree every cached (unused) block of every device.
    void release_cached();

    size_t cached_bytes() const;
    size_t in_use_bytes() const;

private:
    DeviceMemoryPool() = default;
    ~DeviceMemoryPool();
    DeviceMemoryPool(const DeviceMemoryPool&) = delete;
    DeviceMemoryPool& operator=(const DeviceMemoryPool&) = delete;

    static size_t round_size(size_t bytes);

    struct Block {
        size_t size;
        int device;
    };
    mutable std::mutex mu_;
    // (device, size) -> cached pointers
    std::multimap<std::pair<int, size_t>, void*> free_;
    std::unordered_map<void*, Block> live_;
    size_t cached_ = 0, in_use_ = 0;
};

}  // namespace cudasep
