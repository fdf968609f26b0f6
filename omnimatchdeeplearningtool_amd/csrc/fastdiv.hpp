// Unsigned division by a divisor fixed at launch time.
//
// For 1 <= d < 2^31, with s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1
// (which fits in 32 bits because 2^s - d < d), q = (umulhi(x, m) + x) >> s
// equals floor(x / d) for every 0 <= x < 2^32 when the sum is taken in 33 bits
// (Granlund & Montgomery, "Division by Invariant Integers using
// Multiplication", PLDI 1994, section 4). Callers keep x < 2^31, so the sum
// fits in 32 bits: umulhi(x, m) < x. Three VALU operations instead of the
// compiler's ~25 for a signed division by a runtime value.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace omhip {

struct FastDiv {
    uint32_t d, m, s;

    static FastDiv make(uint32_t d) {
        uint32_t s = 0;
        while ((1ull << s) < d) ++s;
        const uint64_t m = ((((1ull << s) - d) << 32) / d) + 1;
        return {d, (uint32_t)m, s};
    }

    __host__ __device__ __forceinline__ uint32_t div(uint32_t x) const {
#if defined(__HIP_DEVICE_COMPILE__)
        return (__umulhi(x, m) + x) >> s;
#else
        return (uint32_t)((((uint64_t)x * m) >> 32) + x) >> s;
#endif
    }
};

}  // namespace omhip
