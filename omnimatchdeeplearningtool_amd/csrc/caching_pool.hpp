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
// Streams. A block is released with the tag of the stream that was current at
// the free, and optionally a fence: a marker that completes once everything
// enqueued on that stream before the free has run. A request tagged with the
// same stream takes the block at once (stream order protects it); a request
// from another stream takes it only when its tag is 0 (no pending use) or its
// fence has completed. Before the cached blocks are flushed to the raw free, the
// injected drain waits until every fence has completed.
//
// The raw allocator, fence test and drain are injected, so the same class is
// unit-tested on the CPU with a fake device (allocation failure, flush-and-retry,
// unknown pointers, cross-stream reuse).
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <unordered_map>

namespace omhip {

class CachingPool {
public:
    using RawAlloc = std::function<void*(size_t)>;   // returns nullptr on failure
    using RawFree = std::function<void(void*)>;
    using Fence = std::shared_ptr<void>;             // completion marker (nullptr: none)
    using FenceReady = std::function<bool(void*)>;   // has the marker completed?
    using Drain = std::function<void()>;             // waits for every marker

    static constexpr size_t kGranule = 512;

    CachingPool(RawAlloc fnAlloc, RawFree fnFree, FenceReady fnReady = nullptr, Drain fnDrain = nullptr)
        : m_fnAlloc(std::move(fnAlloc)), m_fnFree(std::move(fnFree)), m_fnReady(std::move(fnReady)),
          m_fnDrain(std::move(fnDrain)) {}

    ~CachingPool() = default;  // the owner calls clear() while the device is alive

    static size_t roundUp(size_t nBytes) {
        if (nBytes == 0) nBytes = 1;
        return (nBytes + kGranule - 1) / kGranule * kGranule;
    }

    // A block of at least nBytes for work tagged `tag` (the current stream).
    void* allocate(size_t nBytes, uintptr_t tag = 0) {
        const size_t nRounded = roundUp(nBytes);
        std::lock_guard<std::mutex> lock(m_mutex);
        for (auto it = m_free.lower_bound(nRounded); it != m_free.end() && it->first <= 2 * nRounded; ++it) {
            if (!usableLocked(it->second, tag)) continue;
            void* p = it->second.p;
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
    bool release(void* p, uintptr_t tag = 0, Fence fence = nullptr) {
        if (!p) return true;
        std::lock_guard<std::mutex> lock(m_mutex);
        auto it = m_live.find(p);
        if (it == m_live.end()) {
            m_fnFree(p);
            return false;
        }
        m_free.emplace(it->second, Entry{p, tag, std::move(fence)});
        m_nUsed -= it->second;
        return true;
    }

    // Attaches `fence` to every cached block tagged `tag` that has none (the
    // stream stops being the current one: later work elsewhere must wait for it).
    void fenceTag(uintptr_t tag, const Fence& fence) {
        std::lock_guard<std::mutex> lock(m_mutex);
        for (auto& kv : m_free)
            if (kv.second.tag == tag && !kv.second.fence) kv.second.fence = fence;
    }

    // Every use on stream `tag` has finished: its cached blocks become free for all.
    void retire(uintptr_t tag) {
        std::lock_guard<std::mutex> lock(m_mutex);
        for (auto& kv : m_free)
            if (kv.second.tag == tag) {
                kv.second.tag = 0;
                kv.second.fence.reset();
            }
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
    struct Entry {
        void* p;
        uintptr_t tag;
        Fence fence;
    };

    bool usableLocked(Entry& e, uintptr_t tag) {
        if (e.tag == 0 || e.tag == tag) return true;
        if (e.fence && m_fnReady && m_fnReady(e.fence.get())) {
            e.tag = 0;
            e.fence.reset();
            return true;
        }
        return false;
    }

    void releaseCachedLocked() {
        if (m_free.empty()) return;
        if (m_fnDrain) m_fnDrain();   // no cached block may still be in use
        for (auto& kv : m_free) {
            m_fnFree(kv.second.p);
            m_nHeld -= kv.first;
            m_live.erase(kv.second.p);
        }
        m_free.clear();
    }

    RawAlloc m_fnAlloc;
    RawFree m_fnFree;
    FenceReady m_fnReady;
    Drain m_fnDrain;
    mutable std::mutex m_mutex;
    std::unordered_map<void*, size_t> m_live;   // every block the pool owns -> rounded size
    std::multimap<size_t, Entry> m_free;        // cached blocks by size
    size_t m_nHeld = 0;
    size_t m_nUsed = 0;
};

}  // namespace omhip
