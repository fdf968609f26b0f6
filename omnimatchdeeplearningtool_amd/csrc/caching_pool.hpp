// caching_pool.hpp — size-bucketed caching allocator behind omHipMalloc/omHipFree.
//
// Behaviour follows the reference pool (src/cuda/cuda_kernels.cu:167-281):
// freed blocks stay cached; an allocation takes the smallest cached block that
// is large enough; when the raw allocator fails, every cached block is released
// and the allocation is retried once; freeing an unknown pointer hands it to the
// raw free. Differences by design: sizes are rounded up to a 512-byte granule
// (so near-equal requests share blocks), a cached block is only reused for a
// request of at least half its size (no large block pinned by a tiny tensor),
// and the pool keeps byte counters for omHipPoolStats.
//
// The raw allocator is injected, so the same class is unit-tested on the CPU
// with a fake device (allocation failure, flush-and-retry, unknown pointers).
#pragma once

#include <cstddef>
#include <functional>
#include <map>
#include <mutex>
#include <unordered_map>

namespace omhip {

class CachingPool {
public:
    using RawAlloc = std::function<void*(size_t)>;   // returns nullptr on failure
    using RawFree = std::function<void(void*)>;

    static constexpr size_t kGranule = 512;

    CachingPool(RawAlloc fnAlloc, RawFree fnFree)
        : m_fnAlloc(std::move(fnAlloc)), m_fnFree(std::move(fnFree)) {}

    ~CachingPool() = default;  // the owner calls clear() while the device is alive

    static size_t roundUp(size_t nBytes) {
        if (nBytes == 0) nBytes = 1;
        return (nBytes + kGranule - 1) / kGranule * kGranule;
    }

    void* allocate(size_t nBytes) {
        const size_t nRounded = roundUp(nBytes);
        std::lock_guard<std::mutex> lock(m_mutex);
        auto it = m_free.lower_bound(nRounded);
        if (it != m_free.end() && it->first <= 2 * nRounded) {
            void* p = it->second;
            m_free.erase(it);
            m_nUsed += m_live[p];
            return p;
        }
        void* p = m_fnAlloc(nRounded);
        if (!p) {
            releaseCachedLocked();
            p = m_fnAlloc(nRounded);
            if (!p) return nullptr;
        }
        m_live[p] = nRounded;
        m_nHeld += nRounded;
        m_nUsed += nRounded;
        return p;
    }

    // Returns false if the pointer was unknown (it is then passed to the raw free).
    bool release(void* p) {
        if (!p) return true;
        std::lock_guard<std::mutex> lock(m_mutex);
        auto it = m_live.find(p);
        if (it == m_live.end()) {
            m_fnFree(p);
            return false;
        }
        m_free.emplace(it->second, p);
        m_nUsed -= it->second;
        return true;
    }

    // Drops every cached (free) block; live blocks stay valid.
    void trim() {
        std::lock_guard<std::mutex> lock(m_mutex);
        releaseCachedLocked();
    }

    // Frees everything, live blocks included (device teardown).
    void clear() {
        std::lock_guard<std::mutex> lock(m_mutex);
        for (auto& kv : m_live) m_fnFree(kv.first);
        m_live.clear();
        m_free.clear();
        m_nHeld = m_nUsed = 0;
    }

    size_t heldBytes() const { std::lock_guard<std::mutex> lock(m_mutex); return m_nHeld; }
    size_t usedBytes() const { std::lock_guard<std::mutex> lock(m_mutex); return m_nUsed; }
    size_t cachedBlocks() const { std::lock_guard<std::mutex> lock(m_mutex); return m_free.size(); }

private:
    void releaseCachedLocked() {
        for (auto& kv : m_free) {
            m_fnFree(kv.second);
            m_nHeld -= kv.first;
            m_live.erase(kv.second);
        }
        m_free.clear();
    }

    RawAlloc m_fnAlloc;
    RawFree m_fnFree;
    mutable std::mutex m_mutex;
    std::unordered_map<void*, size_t> m_live;   // every block the pool owns -> rounded size
    std::multimap<size_t, void*> m_free;        // cached blocks by size
    size_t m_nHeld = 0;
    size_t m_nUsed = 0;
};

}  // namespace omhip
