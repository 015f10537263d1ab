// Caching device allocator (host-side logic only, no HIP types).
//
// Counterpart of the reference's cuda_pool_alloc / cuda_pool_free
// (src/tensor/tensor.cc:22-68): freed blocks are kept and handed out again
// instead of going back to the driver, because hipMalloc/hipFree
// synchronise the device.  Differences, for a device with 288 GB of HBM:
//   - requests are rounded to size classes (512 B granules up to 1 MiB,
//     2 MiB granules above) and served best-fit from the cache when the
//     cached block wastes at most a quarter of the rounded size, so
//     near-identical scratch sizes share blocks;
//   - when the backing allocator reports out-of-memory, every cached block
//     is released and the request retried once (the reference never frees);
//   - statistics are kept for tests and tuning.
// Thread-safe (one mutex).  Blocks are never split or merged.  Reuse is
// stream-ordered for a single stream, as in the reference.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>

namespace vvh {

// Backing allocator interface: alloc returns 0 on success, 1 when out of
// memory, 2 on any other failure.
struct RawAllocator {
    virtual ~RawAllocator() = default;
    virtual int alloc(void** p, std::size_t bytes) = 0;
    virtual int free(void* p) = 0;
};

struct PoolStats {
    std::uint64_t bytes_in_use = 0;
    std::uint64_t bytes_cached = 0;
    std::uint64_t peak_reserved = 0;
    std::uint64_t alloc_calls = 0;
    std::uint64_t cache_hits = 0;
    std::uint64_t driver_allocs = 0;
    std::uint64_t oom_releases = 0;
};

class CachingPool {
public:
    static constexpr std::size_t kSmallGranule = 512;
    static constexpr std::size_t kSmallLimit = std::size_t(1) << 20;
    static constexpr std::size_t kLargeGranule = std::size_t(2) << 20;

    explicit CachingPool(RawAllocator* raw) : raw_(raw) {}

    static std::size_t round_size(std::size_t bytes)
    {
        const std::size_t g = bytes <= kSmallLimit ? kSmallGranule : kLargeGranule;
        if (bytes > SIZE_MAX - g) return 0;  // overflow -> caller rejects
        return (bytes + g - 1) / g * g;
    }

    // 0 = ok, 1 = out of memory, 2 = backing failure, 3 = bad size.
    int alloc(void** p, std::size_t bytes)
    {
        *p = nullptr;
        if (bytes == 0) return 0;
        const std::size_t rs = round_size(bytes);
        if (rs == 0) return 3;
        std::lock_guard<std::mutex> lock(mu_);
        stats_.alloc_calls++;
        auto it = free_.lower_bound(rs);
        if (it != free_.end() && it->first - rs <= rs / 4) {
            *p = it->second;
            live_.emplace(*p, it->first);
            stats_.bytes_cached -= it->first;
            stats_.bytes_in_use += it->first;
            free_.erase(it);
            stats_.cache_hits++;
            return 0;
        }
        int rc = raw_->alloc(p, rs);
        if (rc == 1 && !free_.empty()) {
            release_locked();
            stats_.oom_releases++;
            rc = raw_->alloc(p, rs);
        }
        if (rc != 0) {
            *p = nullptr;
            return rc == 1 ? 1 : 2;
        }
        stats_.driver_allocs++;
        live_.emplace(*p, rs);
        stats_.bytes_in_use += rs;
        const std::uint64_t reserved = stats_.bytes_in_use + stats_.bytes_cached;
        if (reserved > stats_.peak_reserved) stats_.peak_reserved = reserved;
        return 0;
    }

    // Returns 0 if p was cached, 1 if p was not from the pool (the caller
    // frees it for real), -1 if the backing free failed.
    int free(void* p)
    {
        if (!p) return 0;
        std::lock_guard<std::mutex> lock(mu_);
        auto it = live_.find(p);
        if (it == live_.end()) return 1;
        free_.emplace(it->second, p);
        stats_.bytes_in_use -= it->second;
        stats_.bytes_cached += it->second;
        live_.erase(it);
        return 0;
    }

    bool owns(void* p)
    {
        std::lock_guard<std::mutex> lock(mu_);
        return live_.count(p) != 0;
    }

    // Releases every cached block to the backing allocator; returns the
    // number of backing frees that failed.
    int release_cached()
    {
        std::lock_guard<std::mutex> lock(mu_);
        return release_locked();
    }

    PoolStats stats()
    {
        std::lock_guard<std::mutex> lock(mu_);
        return stats_;
    }

private:
    int release_locked()
    {
        int failures = 0;
        for (auto& kv : free_) {
            if (raw_->free(kv.second) != 0) failures++;
            stats_.bytes_cached -= kv.first;
        }
        free_.clear();
        return failures;
    }

    RawAllocator* raw_;
    std::mutex mu_;
    std::multimap<std::size_t, void*> free_;       // rounded size -> block
    std::unordered_map<void*, std::size_t> live_;  // block -> rounded size
    PoolStats stats_;
};

}  // namespace vvh
