// CPU test of omhip::CachingPool with a fake device allocator: reuse,
// rounding, flush-and-retry on allocation failure (the reference pool's OOM
// path, src/cuda/cuda_kernels.cu:220-245), unknown-pointer free, trim/clear
// accounting, concurrent use and cross-stream reuse (stream tags and fences).
// Exit status 0 = all checks passed.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <set>
#include <thread>
#include <vector>

#include "../../omnimatchdeeplearningtool_amd/csrc/caching_pool.hpp"

static int g_fail = 0;
#define CHECK(c)                                                               \
    do {                                                                       \
        if (!(c)) { std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c); ++g_fail; } \
    } while (0)

struct FakeDevice {
    size_t capacity;
    size_t used = 0;
    std::atomic<int> allocs{0}, frees{0}, failures{0};
    std::set<void*> live;
    std::mutex m;
    void* alloc(size_t n) {
        std::lock_guard<std::mutex> l(m);
        if (used + n > capacity) { ++failures; return nullptr; }
        void* p = std::malloc(n);
        used += n;
        live.insert(p);
        ++allocs;
        return p;
    }
    void release(void* p, size_t n) {
        std::lock_guard<std::mutex> l(m);
        if (live.erase(p)) { used -= n; ++frees; std::free(p); }
    }
};

int main() {
    // --- reuse and rounding ---
    {
        FakeDevice dev{1 << 20};
        std::vector<std::pair<void*, size_t>> sizes;  // pointer -> rounded size, for the fake free
        omhip::CachingPool pool([&](size_t n) { void* p = dev.alloc(n); if (p) sizes.push_back({p, n}); return p; },
                                [&](void* p) { for (auto& s : sizes) if (s.first == p) dev.release(p, s.second); });
        CHECK(omhip::CachingPool::roundUp(1) == 512);
        CHECK(omhip::CachingPool::roundUp(512) == 512);
        CHECK(omhip::CachingPool::roundUp(513) == 1024);
        void* a = pool.allocate(1000);
        CHECK(a != nullptr);
        CHECK(pool.usedBytes() == 1024 && pool.heldBytes() == 1024);
        pool.release(a);
        CHECK(pool.usedBytes() == 0 && pool.heldBytes() == 1024 && pool.cachedBlocks() == 1);
        void* b = pool.allocate(700);            // fits the cached 1024 block (<= 2x)
        CHECK(b == a);
        CHECK(dev.allocs == 1);
        pool.release(b);
        void* big = pool.allocate(2000);         // 2048: nothing cached that large -> fresh block
        CHECK(big != a && dev.allocs == 2);
        pool.release(big);                       // cache: {1024, 2048}
        void* c = pool.allocate(600);            // 1024: the smallest cached block that fits
        CHECK(c == a && dev.allocs == 2);
        void* d = pool.allocate(300);            // 512: the cached 2048 block is more than 2x -> fresh block
        CHECK(d != big && dev.allocs == 3);
        pool.release(c);
        pool.release(d);
        pool.trim();
        CHECK(pool.heldBytes() == 0 && pool.cachedBlocks() == 0 && dev.used == 0);
    }
    // --- allocation failure: cached blocks are flushed and the allocation retried ---
    {
        FakeDevice dev{4096};
        std::vector<std::pair<void*, size_t>> sizes;
        omhip::CachingPool pool([&](size_t n) { void* p = dev.alloc(n); if (p) sizes.push_back({p, n}); return p; },
                                [&](void* p) { for (auto& s : sizes) if (s.first == p) dev.release(p, s.second); });
        void* x = pool.allocate(2048);
        void* y = pool.allocate(1024);
        CHECK(x && y);
        pool.release(x);                          // 2048 cached, 1024 live, device full except 1024
        void* z = pool.allocate(3000);            // 3072: fails, flush frees the cached 2048, retry succeeds
        CHECK(z != nullptr);
        CHECK(dev.failures == 1);
        CHECK(pool.cachedBlocks() == 0);
        void* w = pool.allocate(4096);            // nothing to flush: stays a failure
        CHECK(w == nullptr);
        pool.release(y);
        pool.release(z);
        pool.clear();
        CHECK(dev.used == 0 && pool.heldBytes() == 0);
    }
    // --- unknown pointer goes to the raw free ---
    {
        int rawFrees = 0;
        omhip::CachingPool pool([](size_t n) { return std::malloc(n); }, [&](void* p) { ++rawFrees; std::free(p); });
        void* foreign = std::malloc(64);
        CHECK(pool.release(foreign) == false);
        CHECK(rawFrees == 1);
        CHECK(pool.release(nullptr) == true);
    }
    // --- concurrent allocate / release ---
    {
        FakeDevice dev{64 << 20};
        std::mutex sm;
        std::vector<std::pair<void*, size_t>> sizes;
        omhip::CachingPool pool(
            [&](size_t n) { void* p = dev.alloc(n); if (p) { std::lock_guard<std::mutex> l(sm); sizes.push_back({p, n}); } return p; },
            [&](void* p) { std::lock_guard<std::mutex> l(sm); for (auto& s : sizes) if (s.first == p) dev.release(p, s.second); });
        std::vector<std::thread> th;
        std::atomic<int> nullCount{0};
        for (int t = 0; t < 8; ++t)
            th.emplace_back([&, t] {
                for (int i = 0; i < 2000; ++i) {
                    void* p = pool.allocate(512 * (1 + (i + t) % 7));
                    if (!p) { ++nullCount; continue; }
                    pool.release(p);
                }
            });
        for (auto& x : th) x.join();
        CHECK(nullCount == 0);
        CHECK(pool.usedBytes() == 0);
        pool.clear();
        CHECK(dev.used == 0);
    }
    // --- streams: a block freed on stream 1 goes back to stream 1 at once, to stream 2 only
    // once its fence has completed (or the stream was retired); flushes drain first ---
    {
        FakeDevice dev{1 << 20};
        std::vector<std::pair<void*, size_t>> sizes;
        int drains = 0;
        omhip::CachingPool pool([&](size_t n) { void* p = dev.alloc(n); if (p) sizes.push_back({p, n}); return p; },
                                [&](void* p) { for (auto& s : sizes) if (s.first == p) dev.release(p, s.second); },
                                [](void* f) { return *static_cast<bool*>(f); }, [&] { ++drains; });
        auto makeFence = [] { return omhip::CachingPool::Fence(new bool(false), [](void* p) { delete static_cast<bool*>(p); }); };
        auto done = [](const omhip::CachingPool::Fence& f) { *static_cast<bool*>(f.get()) = true; };
        void* a = pool.allocate(1000, 1);
        auto f1 = makeFence();
        pool.release(a, 1, f1);
        void* b = pool.allocate(1000, 2);         // the fence is pending: stream 2 gets a fresh block
        CHECK(b != a && dev.allocs == 2);
        void* c = pool.allocate(1000, 1);         // stream 1 itself: stream order protects the block
        CHECK(c == a);
        pool.release(c, 1, f1);
        done(f1);
        void* d = pool.allocate(1000, 2);         // fence completed: free for every stream
        CHECK(d == a);
        pool.release(d, 1, nullptr);              // no fence: only stream 1 (or a retire) may take it
        void* e = pool.allocate(1000, 2);
        CHECK(e != a && e != b);
        pool.retire(1);                           // stream 1 synchronised: its blocks are idle
        void* g = pool.allocate(1000, 2);
        CHECK(g == a);
        pool.release(g, 1, nullptr);
        auto f2 = makeFence();
        pool.fenceTag(1, f2);                     // stream 1 stops being current
        void* h = pool.allocate(1000, 3);
        CHECK(h != a);
        done(f2);
        void* i = pool.allocate(1000, 3);
        CHECK(i == a);
        pool.release(b, 2, makeFence());          // pending fence on a cached block ...
        CHECK(drains == 0);
        pool.trim();                              // ... so the flush drains the device first
        CHECK(drains == 1 && pool.cachedBlocks() == 0);
        pool.release(e, 2);
        pool.release(h, 3);
        pool.release(i, 3);
        pool.clear();
        CHECK(dev.used == 0);
    }
    std::printf(g_fail ? "FAILED %d\n" : "ALL PASSED\n", g_fail);
    return g_fail ? 1 : 0;
}
