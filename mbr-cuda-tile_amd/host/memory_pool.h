// Caching device allocator behind Tensor::empty (the role of CudaMemoryPool,
// src/memory_pool.h:21-190).
//
// Freed blocks are kept per device in size-keyed free lists and handed out again for a
// request of at most their size and at least half of it, so steady-state inference makes
// no hipMalloc/hipFree calls.  Sizes are rounded to 512 B up to 1 MiB and to 2 MiB above
// (the HBM page fragment of MI355X), which keeps the waste of large activation buffers
// below 2 MiB each on a 288 GB device.  When hipMalloc fails, the cache of that device is
// released and the allocation retried once before the error is thrown.  Blocks are reused
// in stream order: all tensor work runs on HipContext::stream(), so a block freed by the
// host can be handed out at once.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace cudasep {

class HipMemoryPool {
public:
    struct Stats {
        size_t allocations = 0;    // hipMalloc calls
        size_t deallocations = 0;  // blocks returned to the cache
        size_t cache_hits = 0;
        size_t total_allocated = 0;
        size_t total_freed = 0;    // bytes given back with hipFree
        size_t active_bytes = 0;
        size_t peak_bytes = 0;
        size_t cached_bytes = 0;
    };

    static HipMemoryPool& instance();

    void* allocate(size_t bytes);   // nullptr for 0 bytes; throws std::runtime_error
    void deallocate(void* ptr);     // returns a block to its device's cache
    void trim_cached_memory();      // hipFree every cached block
    void release_all();             // hipFree cached and active blocks
    Stats get_stats() const;
    void print_stats() const;
    static size_t round_up(size_t bytes);

    HipMemoryPool(const HipMemoryPool&) = delete;
    HipMemoryPool& operator=(const HipMemoryPool&) = delete;

private:
    HipMemoryPool() = default;
    ~HipMemoryPool();
    struct Block {
        size_t size;
        int device;
    };
    void release_cached_locked(int device);  // device < 0: every device

    mutable std::mutex mutex_;
    std::map<int, std::multimap<size_t, void*>> free_;  // device -> size -> block
    std::unordered_map<void*, Block> active_;
    Stats stats_;
};

}  // namespace cudasep
