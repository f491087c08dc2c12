// Magic-number unsigned 32-bit division (Granlund & Montgomery, "Division by
// Invariant Integers using Multiplication", PLDI 1994): for d >= 1,
// n / d == (umulhi(n, m) + n) >> s with s = ceil(log2 d) and
// m = floor(2^32 * (2^s - d) / d) + 1, exact for all n < 2^32.
// Header-only and free of HIP includes so host tests can exercise it.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define LMP_HD __host__ __device__ __forceinline__
#else
#define LMP_HD inline
#endif

namespace lmp_hip {

struct FastDiv {
  uint32_t d = 1, m = 0, s = 0;
  FastDiv() = default;
  explicit FastDiv(uint32_t divisor) : d(divisor) {
    s = 0;
    while ((uint64_t(1) << s) < divisor) ++s;
    m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - divisor)) / divisor + 1);
  }
  LMP_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t hi = __umulhi(n, m);
#else
    const uint32_t hi = uint32_t((uint64_t(n) * m) >> 32);
#endif
    return uint32_t((uint64_t(hi) + n) >> s);
  }
};

}  // namespace lmp_hip
