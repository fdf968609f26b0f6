// omhip_internal.hpp — shared plumbing of libomhip: stream access, error
// reporting and launch checks. Host-side only declarations; kernels live in the
// .hip files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <mutex>

namespace omhip {

// Stream every entry point enqueues on (library stream unless omHipSetStream
// installed a caller stream). Initialises device 0 lazily if omHipInit was not
// called, so a forgotten init degrades to the reference's default device.
hipStream_t stream();

// Library transfer stream for the asynchronous host copies (created on
// first use); nullptr with the error recorded on failure.
hipStream_t transferStream();

// Sets nBytes bytes at p to value with a kernel on the library stream (safe
// inside a captured graph). 0 or -1.
int byteFill(void* p, unsigned char value, size_t nBytes);

// Records a message for omHipGetLastError (thread-local) and returns -1.
int fail(const char* fmt, ...);

// Clears the thread-local error message (called at the top of every entry).
void clearError();

// Device workspace of at least `bytes` for the current stream (one block per
// stream and slot, grown on demand; an outgrown block stays allocated until its
// last use has finished and no executable graph exists). Reuse is ordered by
// the stream. Slot 0 holds split-K partial sums, slot 1 a call's temporary
// operand (flipped weights, an im2col buffer) that slot-0 users read, slot 2
// per-tile arrival counters: zero-filled when (re)allocated, and every kernel
// that counts on them returns them to zero; slot 3 the intermediates of a
// composed layer (the attention block's projections), which the ops it calls
// do not touch. nullptr with the error recorded on OOM, or when the block must
// grow while the stream records a graph.
enum WsSlot { kWsPartials = 0, kWsOperand = 1, kWsCounters = 2, kWsStaging = 3 };
void* workspace(size_t bytes, int slot = kWsPartials);

// Whether stream s is recording a graph.
bool capturing(hipStream_t s);

// Makes a lookup table that a kernel just built on stream s visible to every
// stream: waits for s. Fails (-1, naming `what`) while s records a graph.
int publish(hipStream_t s, const char* what);

// Sets a kernel's dynamic-LDS limit once per call site (each template
// instantiation of the enclosing function has its own), thread-safely;
// evaluates to the status of that single hipFuncSetAttribute call.
#define OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kernel, bytes)                                          \
    ([&]() -> hipError_t {                                                                      \
        static std::once_flag omhip_once_;                                                      \
        static hipError_t omhip_status_ = hipSuccess;                                           \
        std::call_once(omhip_once_, [&] {                                                       \
            omhip_status_ = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),          \
                                                hipFuncAttributeMaxDynamicSharedMemorySize,     \
                                                static_cast<int>(bytes));                       \
        });                                                                                     \
        return omhip_status_;                                                                   \
    }())

// Registers a function that omHipCleanup runs before the pool is released
// (for caches of pool-owned device buffers).
void onCleanup(void (*fn)());

// Device properties cached at init.
int cuCount();           // compute units of the current device
int maxSharedPerBlock(); // bytes

}  // namespace omhip

// Evaluates a HIP call; on error records "<call>: <hip error string>" and
// returns -1 from the calling entry point.
#define OMHIP_CHECK(expr)                                                          \
    do {                                                                           \
        hipError_t omhip_err_ = (expr);                                            \
        if (omhip_err_ != hipSuccess)                                              \
            return ::omhip::fail("%s failed: %s (%s:%d)", #expr,                   \
                                 hipGetErrorString(omhip_err_), __FILE__, __LINE__); \
    } while (0)

// Checks the launch that was just enqueued.
#define OMHIP_CHECK_LAUNCH() OMHIP_CHECK(hipGetLastError())
