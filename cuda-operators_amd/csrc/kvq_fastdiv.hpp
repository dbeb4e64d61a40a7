// kvq_fastdiv.hpp -- division of 32-bit unsigned values by a divisor fixed for
// a whole launch, as a multiply-high and two shifts (Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, Fig. 4.1):
//   l = ceil(log2 d),  m = floor(2^32 (2^l - d) / d) + 1,
//   t = mulhi(m, n),   q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0),
// exact for every n < 2^32 and 1 <= d < 2^32.  The host builds the constants;
// kernels divide.  Plain C++ as well, so the CPU tests compile it with g++.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define KVQ_HD __host__ __device__
#else
#define KVQ_HD
#endif

namespace kvq {

struct FastDiv {
    uint32_t d, m;
    int sh1, sh2;
};

inline FastDiv make_fastdiv(uint32_t d) {
    int l = 0;
    while ((uint64_t(1) << l) < d) l++;
    const uint64_t m = (uint64_t(1) << 32) * ((uint64_t(1) << l) - d) / d + 1;
    return FastDiv{d, static_cast<uint32_t>(m), l < 1 ? l : 1, l > 1 ? l - 1 : 0};
}

KVQ_HD inline uint32_t fastdiv(uint32_t n, const FastDiv& f) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t t = __umulhi(f.m, n);
#else
    const uint32_t t = static_cast<uint32_t>((static_cast<uint64_t>(f.m) * n) >> 32);
#endif
    return (t + ((n - t) >> f.sh1)) >> f.sh2;
}

}  // namespace kvq
