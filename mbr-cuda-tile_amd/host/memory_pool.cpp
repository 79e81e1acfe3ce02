#include "memory_pool.h"

#include <hip/hip_runtime.h>

#include <iostream>
#include <stdexcept>
#include <string>

namespace cudasep {

namespace {
constexpr size_t kSmall = 512;
constexpr size_t kSmallLimit = size_t(1) << 20;
constexpr size_t kLarge = size_t(2) << 20;

int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) d = 0;
    return d;
}
}  // namespace

HipMemoryPool& HipMemoryPool::instance() {
    // Never destroyed: tensors held in static storage may be released after main returns,
    // when the HIP runtime may already be gone, so the pool does not free at exit.
    static HipMemoryPool* pool = new HipMemoryPool();
    return *pool;
}

HipMemoryPool::~HipMemoryPool() = default;

size_t HipMemoryPool::round_up(size_t bytes) {
    if (bytes <= kSmallLimit) return (bytes + kSmall - 1) / kSmall * kSmall;
    return (bytes + kLarge - 1) / kLarge * kLarge;
}

void* HipMemoryPool::allocate(size_t requested) {
    if (requested == 0) return nullptr;
    const size_t size = round_up(requested);
    const int dev = current_device();
    std::lock_guard<std::mutex> lock(mutex_);
    auto& lists = free_[dev];
    auto it = lists.lower_bound(size);
    if (it != lists.end() && it->first <= 2 * size) {
        void* p = it->second;
        const size_t got = it->first;
        lists.erase(it);
        active_[p] = Block{got, dev};
        stats_.cache_hits++;
        stats_.active_bytes += got;
        stats_.cached_bytes -= got;
        if (stats_.active_bytes > stats_.peak_bytes) stats_.peak_bytes = stats_.active_bytes;
        return p;
    }
    void* p = nullptr;
    hipError_t err = hipMalloc(&p, size);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        release_cached_locked(dev);
        err = hipMalloc(&p, size);
        if (err != hipSuccess) {
            (void)hipGetLastError();
            throw std::runtime_error("HipMemoryPool: hipMalloc failed for " + std::to_string(size) +
                                     " bytes: " + hipGetErrorString(err));
        }
    }
    active_[p] = Block{size, dev};
    stats_.allocations++;
    stats_.total_allocated += size;
    stats_.active_bytes += size;
    if (stats_.active_bytes > stats_.peak_bytes) stats_.peak_bytes = stats_.active_bytes;
    return p;
}

void HipMemoryPool::deallocate(void* ptr) {
    if (ptr == nullptr) return;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = active_.find(ptr);
    if (it == active_.end()) {
        (void)hipFree(ptr);  // not from this pool
        return;
    }
    const Block b = it->second;
    active_.erase(it);
    free_[b.device].emplace(b.size, ptr);
    stats_.active_bytes -= b.size;
    stats_.cached_bytes += b.size;
    stats_.deallocations++;
}

void HipMemoryPool::release_cached_locked(int device) {
    int prev = -1;
    (void)hipGetDevice(&prev);
    for (auto& [dev, lists] : free_) {
        if (device >= 0 && dev != device) continue;
        if (lists.empty()) continue;
        (void)hipSetDevice(dev);
        // blocks may still be read by queued work of this device
        (void)hipDeviceSynchronize();
        for (auto& [size, p] : lists) {
            (void)hipFree(p);
            stats_.total_freed += size;
            stats_.cached_bytes -= size;
        }
        lists.clear();
    }
    if (prev >= 0) (void)hipSetDevice(prev);
}

void HipMemoryPool::trim_cached_memory() {
    std::lock_guard<std::mutex> lock(mutex_);
    release_cached_locked(-1);
}

void HipMemoryPool::release_all() {
    std::lock_guard<std::mutex> lock(mutex_);
    release_cached_locked(-1);
    for (auto& [p, b] : active_) {
        (void)hipSetDevice(b.device);
        (void)hipFree(p);
        stats_.total_freed += b.size;
    }
    active_.clear();
    stats_.active_bytes = 0;
}

HipMemoryPool::Stats HipMemoryPool::get_stats() const {
    std::lock_guard<std::mutex> lock(mutex_);
    return stats_;
}

void HipMemoryPool::print_stats() const {
    const Stats s = get_stats();
    std::cout << "[MemPool] allocs=" << s.allocations << " deallocs=" << s.deallocations
              << " cache_hits=" << s.cache_hits << " active=" << (s.active_bytes >> 20) << "MB"
              << " cached=" << (s.cached_bytes >> 20) << "MB"
              << " peak=" << (s.peak_bytes >> 20) << "MB" << std::endl;
}

}  // namespace cudasep
