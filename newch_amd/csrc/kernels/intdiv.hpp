// Division of 32-bit indices by a loop-invariant divisor with a multiply-high and a shift
// (Granlund & Montgomery, "Division by invariant integers using multiplication", PLDI 1994,
// round-up variant): q = (umulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1.
// The add is done in 64 bits, so it is exact for every n < 2^32 (checked exhaustively over edge
// divisors and randomly by the host-logic tests through nc_hip_check_intdiv, which also checks the
// 32-bit form div31 for dividends below 2^31).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nchip {

struct IntDiv {
    uint32_t d;
    uint32_t m;
    uint32_t s;

    __host__ __device__ IntDiv() : d(1), m(0), s(0) {}
    __host__ explicit IntDiv(uint32_t div) {
        d = div;
        s = 0;
        while (s < 32 && (uint64_t(1) << s) < div) s++;
        m = (uint32_t)(((uint64_t(1) << 32) * ((uint64_t(1) << s) - div)) / div + 1);
    }
    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t t = __umulhi(n, m);
#else
        const uint32_t t = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
        return (uint32_t)(((uint64_t)t + n) >> s);
    }
    // the same for n < 2^31: t <= n, so t + n cannot wrap 32 bits
    __host__ __device__ __forceinline__ uint32_t div31(uint32_t n) const { return div31(n, m, s); }
    __host__ __device__ __forceinline__ static uint32_t div31(uint32_t n, uint32_t m, uint32_t s) {
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t t = __umulhi(n, m);
#else
        const uint32_t t = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
        return (t + n) >> s;
    }
};

}  // namespace nchip
