// runtime.cpp — device bring-up, library stream, caching pool, copies.
//
// Mirrors the reference runtime (src/cuda/cuda_kernels.cu:63-158 streams,
// :167-281 pool, :287-438 device management) with one library-owned
// non-blocking stream: host copies are enqueued on that stream and then waited
// for, so ordering with the kernels is explicit instead of relying on the
// legacy default stream.
#include "omhip_internal.hpp"
#include "caching_pool.hpp"
#include "../../include/omhip.h"

#include <atomic>
#include <map>
#include <cstdarg>
#include <cstring>
#include <memory>
#include <mutex>
#include <vector>

namespace omhip {
namespace {

std::mutex g_initMutex;
std::atomic<bool> g_inited{false};
int g_device = 0;
hipStream_t g_ownStream = nullptr;
std::atomic<hipStream_t> g_userStream{nullptr};
// Transfer stream and the two ordering events (created on first use).
hipStream_t g_xferStream = nullptr;
hipEvent_t g_evXfer = nullptr, g_evCompute = nullptr;
std::mutex g_xferMutex;
int g_cuCount = 0;
int g_maxShared = 65536;
std::unique_ptr<CachingPool> g_pool;
std::mutex g_wsMutex;
std::vector<void (*)()> g_cleanupHooks;

// Library workspace: one block per (stream, slot), so partials written on one
// stream are never overwritten by work enqueued on another, and the two users
// of one call (split-K partials, slot 0; a call's own temporary such as
// flipped weights or an im2col buffer, slot 1) never share memory. A block that is
// outgrown is retired, not freed: it goes back to the pool only once the event
// recorded after its last use has completed and no executable graph exists
// (a graph captured earlier may hold its address in its nodes).
struct WsBlock {
    void* p = nullptr;
    size_t bytes = 0;
};
struct RetiredWs {
    void* p;
    hipEvent_t done;
};
std::map<std::pair<hipStream_t, int>, WsBlock> g_ws;   // (stream, slot)
std::vector<RetiredWs> g_wsRetired;
int g_liveGraphs = 0;   // executable graphs not yet destroyed (guarded by g_wsMutex)
std::map<hipStream_t, int> g_graphsOn;   // live graphs per capture stream (guarded by g_wsMutex)
// Set once a second stream has been current: from then on every omHipFree
// records a fence on the freeing stream, so another stream reuses the block only
// after that stream's earlier work has finished.
std::atomic<bool> g_multiStream{false};

// Graph handle: the executable graph and the stream it was captured on (its
// nodes use that stream's workspace, so replays are ordered on that stream).
struct GraphHandle {
    hipGraphExec_t exec;
    hipStream_t stream;
};
thread_local hipStream_t t_captureStream = nullptr;

thread_local char t_err[512] = {0};

int initLocked(int nDev) {
    hipError_t e = hipSetDevice(nDev);
    if (e != hipSuccess) return fail("hipSetDevice(%d): %s", nDev, hipGetErrorString(e));
    (void)hipGetLastError();  // clear a stale error left by an earlier failure
    e = hipStreamCreateWithFlags(&g_ownStream, hipStreamNonBlocking);
    if (e != hipSuccess) return fail("hipStreamCreate: %s", hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, nDev);
    if (e != hipSuccess) return fail("hipGetDeviceProperties: %s", hipGetErrorString(e));
    g_cuCount = prop.multiProcessorCount;
    g_maxShared = static_cast<int>(prop.sharedMemPerBlock);
    g_device = nDev;
    g_pool = std::make_unique<CachingPool>(
        [](size_t n) -> void* {
            void* p = nullptr;
            return hipMalloc(&p, n) == hipSuccess ? p : ((void)hipGetLastError(), nullptr);
        },
        [](void* p) { (void)hipFree(p); },
        [](void* ev) {
            const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(ev));
            if (e != hipSuccess) (void)hipGetLastError();   // hipErrorNotReady
            return e == hipSuccess;
        },
        [] { (void)hipDeviceSynchronize(); });
    return 0;
}

uintptr_t tagOf(hipStream_t s) { return reinterpret_cast<uintptr_t>(s); }

// A fence on stream s: an event recorded now (nullptr while s records a graph,
// or when the event cannot be made; the block then keeps its stream tag only).
CachingPool::Fence fenceOn(hipStream_t s) {
    if (capturing(s)) return nullptr;
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (hipEventRecord(ev, s) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipEventDestroy(ev);
        return nullptr;
    }
    return CachingPool::Fence(static_cast<void*>(ev), [](void* e) { (void)hipEventDestroy(static_cast<hipEvent_t>(e)); });
}

int ensureInit(int nDev, bool bExplicit) {
    if (g_inited.load(std::memory_order_acquire)) {
        if (bExplicit && nDev != g_device) {
            hipError_t e = hipSetDevice(nDev);
            if (e != hipSuccess) return fail("hipSetDevice(%d): %s", nDev, hipGetErrorString(e));
        }
        return 0;
    }
    std::lock_guard<std::mutex> lock(g_initMutex);
    if (g_inited.load(std::memory_order_relaxed)) return 0;
    int rc = initLocked(nDev);
    if (rc == 0) g_inited.store(true, std::memory_order_release);
    return rc;
}

}  // namespace

hipStream_t transferStream() {
    if (ensureInit(0, false)) return nullptr;
    std::lock_guard<std::mutex> lock(g_xferMutex);
    if (!g_xferStream) {
        // default priority, like the compute stream
        if (hipStreamCreateWithFlags(&g_xferStream, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&g_evXfer, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&g_evCompute, hipEventDisableTiming) != hipSuccess) {
            (void)fail("transfer stream: %s", hipGetErrorString(hipGetLastError()));
            return nullptr;
        }
    }
    return g_xferStream;
}

hipStream_t stream() {
    hipStream_t s = g_userStream.load(std::memory_order_acquire);
    if (s) return s;
    if (!g_inited.load(std::memory_order_acquire)) ensureInit(0, false);
    return g_ownStream;
}

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(t_err, sizeof(t_err), fmt, ap);
    va_end(ap);
    return -1;
}

void clearError() { t_err[0] = 0; }

int cuCount() {
    if (!g_inited.load(std::memory_order_acquire)) ensureInit(0, false);
    return g_cuCount > 0 ? g_cuCount : 256;
}

int maxSharedPerBlock() { return g_maxShared; }

void onCleanup(void (*fn)()) {
    std::lock_guard<std::mutex> lock(g_wsMutex);
    g_cleanupHooks.push_back(fn);
}

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;   // unknown: treat as recording, the caller then refuses to allocate
    }
    return st != hipStreamCaptureStatusNone;
}

int publish(hipStream_t s, const char* what) {
    if (capturing(s))
        return fail("%s: not built yet while the stream records a graph; run the sequence once before capture", what);
    OMHIP_CHECK(hipStreamSynchronize(s));
    return 0;
}

namespace {
// Returns retired blocks whose last use has finished to the pool (g_wsMutex held).
void reapRetiredLocked() {
    if (g_liveGraphs > 0) return;
    for (size_t i = 0; i < g_wsRetired.size();) {
        if (hipEventQuery(g_wsRetired[i].done) == hipSuccess) {
            (void)hipEventDestroy(g_wsRetired[i].done);
            g_pool->release(g_wsRetired[i].p);
            g_wsRetired[i] = g_wsRetired.back();
            g_wsRetired.pop_back();
        } else {
            (void)hipGetLastError();   // hipErrorNotReady
            ++i;
        }
    }
}
}  // namespace

void* workspace(size_t bytes, int slot) {
    if (!g_inited.load(std::memory_order_acquire) && ensureInit(0, false)) return nullptr;
    const hipStream_t s = stream();
    std::lock_guard<std::mutex> lock(g_wsMutex);
    WsBlock& w = g_ws[{s, slot}];
    if (bytes <= w.bytes) return w.p;
    if (capturing(s)) {
        (void)fail("workspace of %zu bytes needed while the stream records a graph (it holds %zu); "
                   "run the sequence once before capture", bytes, w.bytes);
        return nullptr;
    }
    reapRetiredLocked();
    if (w.p) {
        hipEvent_t ev = nullptr;
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess || hipEventRecord(ev, s) != hipSuccess) {
            (void)fail("workspace: event: %s", hipGetErrorString(hipGetLastError()));
            if (ev) (void)hipEventDestroy(ev);
            return nullptr;
        }
        g_wsRetired.push_back({w.p, ev});
        w = WsBlock{};
    }
    const size_t want = (bytes + (1u << 20) - 1) / (1u << 20) * (1u << 20);   // 1 MiB steps
    void* p = g_pool->allocate(want, tagOf(s));
    if (!p) {
        (void)fail("workspace: out of device memory (%zu bytes)", want);
        return nullptr;
    }
    if (slot == kWsCounters && byteFill(p, 0, want)) {   // counters start at zero, kernels leave them so
        g_pool->release(p, tagOf(s));
        return nullptr;
    }
    w.p = p;
    w.bytes = want;
    return p;
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipInit(int nDeviceId) {
    clearError();
    return ensureInit(nDeviceId, true);
}

int omHipGetDeviceCount(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int omHipGetDeviceName(int nDeviceId, char* pNameBuf, int nBufSize) {
    clearError();
    if (!pNameBuf || nBufSize <= 0) return fail("omHipGetDeviceName: bad buffer");
    hipDeviceProp_t prop;
    OMHIP_CHECK(hipGetDeviceProperties(&prop, nDeviceId));
    std::snprintf(pNameBuf, static_cast<size_t>(nBufSize), "%s (%s)", prop.name, prop.gcnArchName);
    return 0;
}

int omHipGetMemInfo(int nDeviceId, size_t* pFreeMem, size_t* pTotalMem) {
    clearError();
    if (ensureInit(nDeviceId, true)) return -1;
    size_t f = 0, t = 0;
    OMHIP_CHECK(hipMemGetInfo(&f, &t));
    if (pFreeMem) *pFreeMem = f;
    if (pTotalMem) *pTotalMem = t;
    return 0;
}

int omHipGetComputeCapability(int nDeviceId, int* pMajor, int* pMinor) {
    clearError();
    hipDeviceProp_t prop;
    OMHIP_CHECK(hipGetDeviceProperties(&prop, nDeviceId));
    if (pMajor) *pMajor = prop.major;
    if (pMinor) *pMinor = prop.minor;
    return 0;
}

int omHipSynchronize(void) {
    clearError();
    OMHIP_CHECK(hipStreamSynchronize(stream()));
    return 0;
}

int omHipSyncComputeStream(void) { return omHipSynchronize(); }

int omHipCleanup(void) {
    clearError();
    std::lock_guard<std::mutex> lock(g_initMutex);
    if (!g_inited.load(std::memory_order_acquire)) return 0;
    (void)hipDeviceSynchronize();   // every stream that used a workspace or a table
    std::vector<void (*)()> hooks;
    {
        std::lock_guard<std::mutex> wsLock(g_wsMutex);
        g_ws.clear();
        for (auto& r : g_wsRetired) (void)hipEventDestroy(r.done);
        g_wsRetired.clear();   // their memory goes with the pool below
        hooks = g_cleanupHooks;
    }
    for (auto fn : hooks) fn();
    if (g_pool) g_pool->clear();
    g_pool.reset();
    {
        std::lock_guard<std::mutex> xl(g_xferMutex);
        if (g_xferStream) {
            (void)hipStreamSynchronize(g_xferStream);
            (void)hipStreamDestroy(g_xferStream);
        }
        if (g_evXfer) (void)hipEventDestroy(g_evXfer);
        if (g_evCompute) (void)hipEventDestroy(g_evCompute);
        g_xferStream = nullptr;
        g_evXfer = g_evCompute = nullptr;
    }
    (void)hipStreamDestroy(g_ownStream);
    g_ownStream = nullptr;
    g_userStream.store(nullptr, std::memory_order_release);
    g_inited.store(false, std::memory_order_release);
    return 0;
}

int omHipForceReset(void) {
    clearError();
    if (!g_inited.load(std::memory_order_acquire)) {
        (void)hipGetLastError();
        return 0;
    }
    (void)hipDeviceSynchronize();   // every kernel has finished (its status is not ours to report)
    (void)hipGetLastError();        // clear the sticky error left by a failed call
    const int rc = omHipCleanup();  // pool, workspaces, tables and streams; the next call re-initialises
    (void)hipGetLastError();
    return rc;
}

int omHipReleaseStream(void* pStream) {
    clearError();
    if (!pStream || !g_inited.load(std::memory_order_acquire)) return 0;
    const hipStream_t s = static_cast<hipStream_t>(pStream);
    if (capturing(s)) return fail("omHipReleaseStream: the stream records a graph");
    {
        std::lock_guard<std::mutex> lock(g_wsMutex);
        auto g = g_graphsOn.find(s);
        if (g != g_graphsOn.end() && g->second > 0)
            return fail("omHipReleaseStream: %d graph(s) captured on this stream still exist; destroy them first",
                        g->second);
    }
    OMHIP_CHECK(hipStreamSynchronize(s));
    g_pool->retire(tagOf(s));   // every block freed on the stream is idle now
    std::lock_guard<std::mutex> lock(g_wsMutex);
    for (auto it = g_ws.begin(); it != g_ws.end();) {
        if (it->first.first != s) {
            ++it;
            continue;
        }
        if (it->second.p) {
            if (g_liveGraphs > 0) {
                // a graph captured on this stream may still replay: keep the block until it is gone
                hipEvent_t ev = nullptr;
                OMHIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
                OMHIP_CHECK(hipEventRecord(ev, s));
                g_wsRetired.push_back({it->second.p, ev});
            } else {
                g_pool->release(it->second.p);
            }
        }
        it = g_ws.erase(it);
    }
    if (g_userStream.load(std::memory_order_acquire) == s) g_userStream.store(nullptr, std::memory_order_release);
    return 0;
}

int omHipGetStream(void** ppStream) {
    clearError();
    if (!ppStream) return fail("omHipGetStream: null output");
    *ppStream = static_cast<void*>(stream());
    return 0;
}

int omHipSetStream(void* pStream) {
    clearError();
    if (ensureInit(0, false)) return -1;
    const hipStream_t prev = stream();
    const hipStream_t next = pStream ? static_cast<hipStream_t>(pStream) : g_ownStream;
    if (next != prev) {
        // blocks freed on the previous stream become reusable elsewhere once its
        // work so far has finished; later frees carry a fence of their own
        g_multiStream.store(true, std::memory_order_release);
        CachingPool::Fence f = fenceOn(prev);
        if (f) g_pool->fenceTag(tagOf(prev), f);
    }
    g_userStream.store(static_cast<hipStream_t>(pStream), std::memory_order_release);
    return 0;
}

const char* omHipGetLastError(void) { return t_err; }

int omHipMalloc(void** ppDevPtr, size_t nBytes) {
    clearError();
    if (!ppDevPtr) return fail("omHipMalloc: null output");
    *ppDevPtr = nullptr;
    if (ensureInit(0, false)) return -1;
    void* p = g_pool->allocate(nBytes, tagOf(stream()));
    if (!p) return fail("omHipMalloc(%zu): out of device memory after flushing the pool", nBytes);
    *ppDevPtr = p;
    return 0;
}

int omHipFree(void* pDevPtr) {
    clearError();
    if (!pDevPtr) return 0;
    if (!g_inited.load(std::memory_order_acquire) || !g_pool) {
        OMHIP_CHECK(hipFree(pDevPtr));
        return 0;
    }
    // The free is ordered on the current stream: later work on that stream may
    // reuse the block at once (stream order protects it); work on another stream
    // only once the fence recorded here has completed.
    const hipStream_t s = stream();
    g_pool->release(pDevPtr, tagOf(s), g_multiStream.load(std::memory_order_acquire) ? fenceOn(s) : nullptr);
    return 0;
}

int omHipPoolStats(size_t* pHeldBytes, size_t* pUsedBytes) {
    clearError();
    if (pHeldBytes) *pHeldBytes = g_pool ? g_pool->heldBytes() : 0;
    if (pUsedBytes) *pUsedBytes = g_pool ? g_pool->usedBytes() : 0;
    return 0;
}

int omHipPoolTrim(void) {
    clearError();
    if (!g_pool) return 0;
    g_pool->trim();   // drains the device first
    return 0;
}

int omHipCopyH2D(void* pDst, const void* pSrc, size_t nBytes) {
    clearError();
    if (nBytes == 0) return 0;
    if (!pDst || !pSrc) return fail("omHipCopyH2D: null pointer");
    hipStream_t s = stream();
    OMHIP_CHECK(hipMemcpyAsync(pDst, pSrc, nBytes, hipMemcpyHostToDevice, s));
    OMHIP_CHECK(hipStreamSynchronize(s));
    return 0;
}

int omHipCopyD2H(void* pDst, const void* pSrc, size_t nBytes) {
    clearError();
    if (nBytes == 0) return 0;
    if (!pDst || !pSrc) return fail("omHipCopyD2H: null pointer");
    hipStream_t s = stream();
    OMHIP_CHECK(hipMemcpyAsync(pDst, pSrc, nBytes, hipMemcpyDeviceToHost, s));
    OMHIP_CHECK(hipStreamSynchronize(s));
    return 0;
}

int omHipCopyD2D(void* pDst, const void* pSrc, size_t nBytes) {
    clearError();
    if (nBytes == 0) return 0;
    if (!pDst || !pSrc) return fail("omHipCopyD2D: null pointer");
    OMHIP_CHECK(hipMemcpyAsync(pDst, pSrc, nBytes, hipMemcpyDeviceToDevice, stream()));
    return 0;
}

int omHipMemset(void* pDev, int nValue, size_t nBytes) {
    clearError();
    if (nBytes == 0) return 0;
    if (!pDev) return fail("omHipMemset: null pointer");
    // a kernel, not hipMemsetAsync, so the call may sit inside a captured graph
    return byteFill(pDev, (unsigned char)nValue, nBytes);
}

// ---- transfer stream, pinned host memory (cuda_kernels.cu:388-417, :4887-4900) ----

int omHipMallocHost(void** ppPtr, size_t nBytes) {
    clearError();
    if (!ppPtr) return fail("omHipMallocHost: null output");
    *ppPtr = nullptr;
    if (ensureInit(0, false)) return -1;
    OMHIP_CHECK(hipHostMalloc(ppPtr, nBytes, hipHostMallocDefault));
    return 0;
}

int omHipFreeHost(void* pPtr) {
    clearError();
    if (!pPtr) return 0;
    OMHIP_CHECK(hipHostFree(pPtr));
    return 0;
}

int omHipAsyncCopyH2D(void* pDst, const void* pSrc, size_t nBytes) {
    clearError();
    if (nBytes == 0) return 0;
    if (!pDst || !pSrc) return fail("omHipAsyncCopyH2D: null pointer");
    hipStream_t x = transferStream();
    if (!x) return -1;
    OMHIP_CHECK(hipMemcpyAsync(pDst, pSrc, nBytes, hipMemcpyHostToDevice, x));
    return 0;
}

int omHipAsyncCopyD2H(void* pDst, const void* pSrc, size_t nBytes) {
    clearError();
    if (nBytes == 0) return 0;
    if (!pDst || !pSrc) return fail("omHipAsyncCopyD2H: null pointer");
    hipStream_t x = transferStream();
    if (!x) return -1;
    OMHIP_CHECK(hipMemcpyAsync(pDst, pSrc, nBytes, hipMemcpyDeviceToHost, x));
    return 0;
}

int omHipSyncTransferStream(void) {
    clearError();
    hipStream_t x = transferStream();
    if (!x) return -1;
    OMHIP_CHECK(hipStreamSynchronize(x));
    return 0;
}

int omHipComputeWaitTransfer(void) {
    clearError();
    hipStream_t x = transferStream();
    if (!x) return -1;
    OMHIP_CHECK(hipEventRecord(g_evXfer, x));
    OMHIP_CHECK(hipStreamWaitEvent(stream(), g_evXfer, 0));
    return 0;
}

int omHipTransferWaitCompute(void) {
    clearError();
    hipStream_t x = transferStream();
    if (!x) return -1;
    OMHIP_CHECK(hipEventRecord(g_evCompute, stream()));
    OMHIP_CHECK(hipStreamWaitEvent(x, g_evCompute, 0));
    return 0;
}

// ---- graphs on the compute stream (cuda_kernels.cu OPT-3.5: omCudaGraph*) ----

int omHipGraphBeginCapture(void) {
    clearError();
    if (ensureInit(0, false)) return -1;
    const hipStream_t s = stream();
    // relaxed: the pool may still call hipMalloc while a graph is recorded
    OMHIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
    t_captureStream = s;
    return 0;
}

int omHipGraphEndCapture(void** ppGraphExec) {
    clearError();
    if (!ppGraphExec) return fail("omHipGraphEndCapture: null output");
    *ppGraphExec = nullptr;
    const hipStream_t s = t_captureStream ? t_captureStream : stream();
    t_captureStream = nullptr;
    hipGraph_t g = nullptr;
    OMHIP_CHECK(hipStreamEndCapture(s, &g));
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail("hipGraphInstantiate: %s", hipGetErrorString(e));
    {
        std::lock_guard<std::mutex> lock(g_wsMutex);
        ++g_liveGraphs;
        ++g_graphsOn[s];
    }
    *ppGraphExec = static_cast<void*>(new GraphHandle{exec, s});
    return 0;
}

int omHipGraphLaunch(void* pGraphExec) {
    clearError();
    if (!pGraphExec) return fail("omHipGraphLaunch: null graph");
    const GraphHandle* h = static_cast<const GraphHandle*>(pGraphExec);
    OMHIP_CHECK(hipGraphLaunch(h->exec, h->stream));
    return 0;
}

int omHipGraphDestroy(void* pGraphExec) {
    clearError();
    if (!pGraphExec) return 0;
    GraphHandle* h = static_cast<GraphHandle*>(pGraphExec);
    // replays still running may use retired workspaces: let them finish first.
    // The whole device is waited for, so a handle that outlives its capture
    // stream never touches that stream.
    const hipError_t es = hipDeviceSynchronize();
    const hipError_t ed = hipGraphExecDestroy(h->exec);
    {
        std::lock_guard<std::mutex> lock(g_wsMutex);
        --g_liveGraphs;
        auto g = g_graphsOn.find(h->stream);
        if (g != g_graphsOn.end() && --g->second <= 0) g_graphsOn.erase(g);
    }
    delete h;
    OMHIP_CHECK(es);
    OMHIP_CHECK(ed);
    return 0;
}

}  // extern "C"
