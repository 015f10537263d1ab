// CPU test of the caching allocator logic (vvllm_amd/csrc/pool.h) with a
// fake backing allocator that can run out of memory on demand.  Counterpart
// of the allocator behaviour in src/tensor/tensor.cc:22-68 (which the
// reference does not test).
#include <cstdio>
#include <cstdlib>
#include <set>

#include "pool.h"

using vvh::CachingPool;

namespace
{

int g_failures = 0;
#define EXPECT(cond)                                                         \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::fprintf(stderr, "%s:%d: EXPECT failed: %s\n", __FILE__, __LINE__, #cond); \
            g_failures++;                                                    \
        }                                                                    \
    } while (0)

struct FakeRaw final : vvh::RawAllocator {
    std::size_t capacity;
    std::size_t used = 0;
    int allocs = 0, frees = 0;
    bool broken = false;
    std::set<void*> live;
    explicit FakeRaw(std::size_t cap) : capacity(cap) {}
    int alloc(void** p, std::size_t bytes) override
    {
        if (broken) return 2;
        if (used + bytes > capacity) return 1;
        *p = std::malloc(bytes);
        used += bytes;
        allocs++;
        live.insert(*p);
        sizes[*p] = bytes;
        return 0;
    }
    int free(void* p) override
    {
        if (!live.count(p)) return 2;
        live.erase(p);
        used -= sizes[p];
        frees++;
        std::free(p);
        return 0;
    }
    std::unordered_map<void*, std::size_t> sizes;
};

void test_rounding()
{
    EXPECT(CachingPool::round_size(1) == 512);
    EXPECT(CachingPool::round_size(512) == 512);
    EXPECT(CachingPool::round_size(513) == 1024);
    EXPECT(CachingPool::round_size(1 << 20) == (1 << 20));
    EXPECT(CachingPool::round_size((1 << 20) + 1) == (std::size_t(2) << 20));
    EXPECT(CachingPool::round_size(std::size_t(288) << 30) == (std::size_t(288) << 30));
    EXPECT(CachingPool::round_size(SIZE_MAX - 3) == 0);  // overflow is reported as 0
}

void test_reuse_and_stats()
{
    FakeRaw raw(1 << 30);
    CachingPool pool(&raw);
    void* a = nullptr;
    EXPECT(pool.alloc(&a, 0) == 0 && a == nullptr);  // zero bytes -> null, like device_allocate
    EXPECT(pool.alloc(&a, 1000) == 0 && a != nullptr);
    EXPECT(raw.allocs == 1);
    EXPECT(pool.free(a) == 0);
    void* b = nullptr;
    EXPECT(pool.alloc(&b, 900) == 0);  // same 1024-byte class -> cached block
    EXPECT(b == a && raw.allocs == 1);
    auto s = pool.stats();
    EXPECT(s.cache_hits == 1 && s.bytes_in_use == 1024 && s.bytes_cached == 0);
    EXPECT(pool.free(b) == 0);
    // best fit, but never a block wasting more than a quarter of the request
    void* c = nullptr;
    EXPECT(pool.alloc(&c, 400) == 0);  // 512 class: the cached 1024 block is too wasteful
    EXPECT(c != a && raw.allocs == 2);
    void* d = nullptr;
    EXPECT(pool.alloc(&d, 1024) == 0 && d == a);
    // not from the pool -> reported, caller frees for real
    int local = 0;
    EXPECT(pool.free(&local) == 1);
    EXPECT(pool.free(nullptr) == 0);
    EXPECT(pool.owns(c) && pool.owns(d));
    pool.free(c);
    pool.free(d);
    s = pool.stats();
    EXPECT(s.bytes_in_use == 0 && s.bytes_cached == 1536 && s.peak_reserved == 1536);
    EXPECT(pool.release_cached() == 0);
    EXPECT(raw.live.empty() && pool.stats().bytes_cached == 0);
}

void test_oom_release_and_retry()
{
    FakeRaw raw(8 << 20);  // 8 MiB device
    CachingPool pool(&raw);
    void* p[4];
    for (auto& x : p) EXPECT(pool.alloc(&x, std::size_t(2) << 20) == 0);
    EXPECT(raw.used == (std::size_t(8) << 20));
    void* q = nullptr;
    EXPECT(pool.alloc(&q, 100) == 1 && q == nullptr);  // nothing cached to release -> OOM
    pool.free(p[0]);
    pool.free(p[1]);
    // 4 MiB request: no 4 MiB block cached; cache flushed, retry succeeds
    EXPECT(pool.alloc(&q, std::size_t(4) << 20) == 0 && q != nullptr);
    auto s = pool.stats();
    EXPECT(s.oom_releases == 1 && s.bytes_cached == 0);
    EXPECT(s.bytes_in_use == (std::size_t(8) << 20));
    pool.free(q);
    pool.free(p[2]);
    pool.free(p[3]);
    raw.broken = true;
    void* r = nullptr;
    EXPECT(pool.alloc(&r, std::size_t(32) << 20) == 2);  // backing failure other than OOM
    raw.broken = false;
    EXPECT(pool.alloc(&r, SIZE_MAX - 1) == 3);
    EXPECT(pool.release_cached() == 0 && raw.live.empty());
}

}  // namespace

int main()
{
    test_rounding();
    test_reuse_and_stats();
    test_oom_release_and_retry();
    if (g_failures) {
        std::fprintf(stderr, "test_pool: %d failure(s)\n", g_failures);
        return 1;
    }
    std::printf("test_pool: all passed\n");
    return 0;
}
