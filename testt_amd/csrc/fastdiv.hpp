// Division of non-negative 31-bit integers by a divisor fixed at launch time, with one 32-bit
// multiply-high, one add and one shift instead of a full integer division.
//
// Method (Granlund & Montgomery, "Division by invariant integers using multiplication", 1994):
// with s = ceil(log2 d) and m = floor(2^32 * (2^s - d) / d) + 1, for 0 <= n < 2^31,
//   floor(n / d) = (mulhi(n, m) + n) >> s.
// mulhi(n, m) < n < 2^31, so the sum cannot overflow 32 bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace soupk {

struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t s;

  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t divisor) : d(divisor), m(0), s(0) {
    while ((uint64_t{1} << s) < divisor) ++s;
    m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << s) - divisor)) / divisor +
                              1);
  }

  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t hi = __umulhi(n, m);
#else
    const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> 32);
#endif
    return (hi + n) >> s;
  }
};

}  // namespace soupk
