// omhip_internal.hpp — shared plumbing of libomhip: stream access, error
// reporting and launch checks. Host-side only declarations; kernels live in the
// .hip files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>

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

// Library-owned device workspace of at least `bytes` (grown on demand, kept
// until omHipCleanup). Reuse is ordered by the single stream; nullptr on OOM.
void* workspace(size_t bytes);

// Registers a function that omHipCleanup runs before the pool is released
// (for caches of pool-owned device buffers).
void onCleanup(void (*fn)());

// Device properties cached at init.
int cuCount();          // compute units of the current device
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
