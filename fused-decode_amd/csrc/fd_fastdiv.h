// Division of 32-bit unsigned integers by a divisor fixed at launch time, with
// one multiply-high, one add and one shift (Granlund & Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, section 4). The row
// decomposition of every elementwise kernel uses it in place of integer
// division, which gfx950 has no instruction for.
//
// For d >= 1 let l = ceil(log2 d) and m = floor(2^32 * (2^l - d) / d) + 1 (< 2^32).
// Then for every n < 2^32:  n / d == (mulhi(n, m) + n) >> l, with the sum
// taken in 64 bits. Plain C++ so the host can verify it exhaustively.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FD_HD __host__ __device__ __forceinline__
#else
#define FD_HD inline
#endif

namespace fd {

struct FastDiv {
  uint32_t d;  // divisor
  uint32_t m;  // magic multiplier
  uint32_t s;  // shift, ceil(log2 d)

  FastDiv() : d(1), m(1), s(0) {}
  explicit FastDiv(uint32_t divisor) {
    d = divisor ? divisor : 1;
    uint32_t l = 0;
    while (l < 32 && (uint64_t(1) << l) < d) ++l;
    s = l;
    m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  }

  FD_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t hi = __umulhi(n, m);
#else
    const uint32_t hi = uint32_t((uint64_t(n) * m) >> 32);
#endif
    return uint32_t((uint64_t(hi) + n) >> s);
  }
  // quotient and remainder
  FD_HD uint32_t divmod(uint32_t n, uint32_t& r) const {
    const uint32_t q = div(n);
    r = n - q * d;
    return q;
  }
};

}  // namespace fd
