// Host build of the kernels' requantization (requant1 in i8conv_device.hpp),
// driven by tests/test_requant.py: reads "acc mult shift zp" lines on stdin
// and prints one result per line, which the test compares with the CPU
// checker's restatement and with exact rational arithmetic.
#include <stdint.h>
#include <stdio.h>

#include "i8conv_device.hpp"

int main() {
  long long acc, mult, shift, zp;
  while (scanf("%lld %lld %lld %lld", &acc, &mult, &shift, &zp) == 4)
    printf("%d\n", i8conv::requant1(int32_t(acc), int32_t(mult), int32_t(shift), int32_t(zp)));
  return 0;
}
