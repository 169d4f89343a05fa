// Host build of the kernels' requantization (requant1, requant1_short and
// requant1_odd in i8conv_device.hpp), driven by tests/test_requant.py: reads
// "acc mult shift zp" lines on stdin and prints, per line, requant1's
// result, the short form's and the odd-multiplier form's (each form
// requant1's again where it does not apply) and 1 or 0 for whether the odd
// form applies, which the test compares with exact rational arithmetic.
#include <stdint.h>
#include <stdio.h>

#include "i8conv_device.hpp"

int main() {
  long long acc, mult, shift, zp;
  while (scanf("%lld %lld %lld %lld", &acc, &mult, &shift, &zp) == 4) {
    const int32_t a = int32_t(acc), m = int32_t(mult), s = int32_t(shift), z = int32_t(zp);
    const int32_t full = i8conv::requant1(a, m, s, z);
    const int32_t brief =
        i8conv::requant_short_ok(s) && i8conv::requant_short_zp_ok(z)
            ? i8conv::requant1_short(a, i8conv::requant_short_am(m), m, i8conv::requant_short_hh(s),
                                     i8conv::requant_short_sh(s), z)
            : full;
    const i8conv::RequantOdd o = i8conv::requant_odd_params(m, s, z);
    const int32_t odd = o.ok ? i8conv::requant1_odd(a, o.mo, o.k, o.sh) : full;
    printf("%d %d %d %d\n", full, brief, odd, o.ok ? 1 : 0);
  }
  return 0;
}
