// Exhaustive / randomized check of the kernels' exact division by invariant
// integers (make_fastdiv / fast_div in i8conv_device.hpp), built with g++ by
// tests/test_host.py.  Prints "ok <checked>" or the first failure; exit 0 on
// success.
#include <stdint.h>
#include <stdio.h>

#include <random>

#include "i8conv_device.hpp"

using i8conv::FastDiv;
using i8conv::fast_div;
using i8conv::make_fastdiv;

static uint64_t checked = 0;

static bool one(uint32_t n, uint32_t d, const FastDiv &f) {
  ++checked;
  if (fast_div(n, f) != n / d) {
    printf("FAIL n=%u d=%u got=%u want=%u\n", n, d, fast_div(n, f), n / d);
    return false;
  }
  return true;
}

int main() {
  const uint32_t kMaxN = 0x7fffffffu;  // dividends are < 2^31
  // every divisor up to 4096 against every dividend up to 2^16 and the
  // dividends next to each multiple of d near the top of the range
  for (uint32_t d = 1; d <= 4096; ++d) {
    const FastDiv f = make_fastdiv(d);
    for (uint32_t n = 0; n < (1u << 16); ++n)
      if (!one(n, d, f)) return 1;
    const uint32_t top = kMaxN / d * d;
    for (uint32_t q = 0; q < 64 && q * d <= top; ++q) {
      const uint32_t m = top - q * d;
      if (!one(m, d, f) || (m > 0 && !one(m - 1, d, f)) || (m < kMaxN && !one(m + 1, d, f)))
        return 1;
    }
    if (!one(kMaxN, d, f)) return 1;
  }
  // random divisors over the whole range, powers of two and their neighbours
  std::mt19937_64 rng(12345);
  for (int i = 0; i < 200000; ++i) {
    uint32_t d = uint32_t(rng() % 0x80000000u) + 1u;
    if (i % 4 == 1) d = 1u << (rng() % 32);
    if (i % 4 == 2) d = (1u << (rng() % 31 + 1)) - 1u;
    if (i % 4 == 3) d = (1u << (rng() % 31)) + 1u;
    if (d > 0x80000000u) d = 0x80000000u;
    const FastDiv f = make_fastdiv(d);
    for (int j = 0; j < 16; ++j) {
      const uint32_t n = uint32_t(rng() % (uint64_t(kMaxN) + 1));
      const uint32_t q = n / d;
      if (!one(n, d, f) || !one(q * d, d, f) || (q > 0 && !one(q * d - 1, d, f)))
        return 1;
    }
  }
  printf("ok %llu\n", (unsigned long long)checked);
  return 0;
}
