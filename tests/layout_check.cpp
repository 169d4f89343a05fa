// Check of the LDS layouts the kernels read MFMA fragments from
// (i8conv_device.hpp, i8conv_internal.hpp), built with g++ by
// tests/test_host.py.  For every layout: the swizzle permutes the 16-byte
// chunks of a row, its inverse undoes it, and every fragment read (lane l:
// row or pixel l % 16 from a multiple of 16, chunk l / 16 of either
// k-half) satisfies gfx950's ds_read_b128 bank rule as measured with the
// LDS probe: 32 consecutive lanes on 32 distinct 16-byte units modulo 512
// bytes and 4 consecutive lanes on 4 distinct units modulo 128 bytes.  The
// same rule must reject the layouts the probe measured 2-way (an XOR of the
// row's low bits, 80- and 144-byte pitches).  Prints "ok <checked>" or the
// first failure; exit 0 on success.
#include <stdio.h>

#include <functional>
#include <set>

#include "i8conv_internal.hpp"

using namespace i8conv;

static int checked = 0;

// unit(l): the 16-byte unit lane l reads
static bool rule_ok(const std::function<long(int)> &unit) {
  for (int h = 0; h < 64; h += 32) {
    std::set<long> s;
    for (int l = h; l < h + 32; ++l) s.insert(((unit(l) % 32) + 32) % 32);
    if (s.size() != 32) return false;
  }
  for (int q = 0; q < 64; q += 4) {
    std::set<long> s;
    for (int l = q; l < q + 4; ++l) s.insert(((unit(l) % 8) + 8) % 8);
    if (s.size() != 4) return false;
  }
  return true;
}

static bool expect(bool cond, const char *what, int a, int b) {
  ++checked;
  if (!cond) printf("FAIL %s (%d, %d)\n", what, a, b);
  return cond;
}

int main() {
  bool ok = true;
  // swz128: 128-byte rows, 8 chunks
  for (int r = 0; r < 512 && ok; ++r) {
    std::set<int> phys;
    for (int c = 0; c < 8; ++c) {
      const int off = swz128(r, c);
      ok &= expect(off / 128 == r, "swz128 stays in its row", r, c);
      phys.insert((off % 128) / 16);
      ok &= expect(swz128_chunk(r, (off % 128) / 16) == c, "swz128_chunk inverts swz128", r, c);
    }
    ok &= expect(phys.size() == 8, "swz128 permutes the chunks", r, 0);
  }
  for (int r0 = 0; r0 < 512 && ok; r0 += 16)
    for (int kh = 0; kh < 2; ++kh)
      ok &= expect(rule_ok([&](int l) { return swz128(r0 + l % 16, 4 * kh + l / 16) / 16; }),
                   "swz128 fragment read conflict-free", r0, kh);
  // swz128x: a permutation of each row's chunks with its inverse (2-way by
  // the rule: checked below)
  for (int r = 0; r < 512 && ok; ++r) {
    std::set<int> phys;
    for (int c = 0; c < 8; ++c) {
      const int off = swz128x(r, c);
      ok &= expect(off / 128 == r, "swz128x stays in its row", r, c);
      phys.insert((off % 128) / 16);
      ok &= expect(swz128x_chunk(r, (off % 128) / 16) == c, "swz128x_chunk inverts swz128x", r, c);
    }
    ok &= expect(phys.size() == 8, "swz128x permutes the chunks", r, 0);
  }
  // swz64: 64-byte pixels, 4 chunks
  for (int p = 0; p < 512 && ok; ++p) {
    std::set<int> phys;
    for (int c = 0; c < 4; ++c) {
      const int off = swz64(p, c);
      ok &= expect(off / 64 == p, "swz64 stays in its pixel", p, c);
      phys.insert((off % 64) / 16);
      ok &= expect(swz64_chunk(p, (off % 64) / 16) == c, "swz64_chunk inverts swz64", p, c);
    }
    ok &= expect(phys.size() == 4, "swz64 permutes the chunks", p, 0);
  }
  for (int p0 = 0; p0 < 512 && ok; p0 += 16)
    ok &= expect(rule_ok([&](int l) { return swz64(p0 + l % 16, l / 16) / 16; }),
                 "swz64 fragment read conflict-free", p0, 0);
  // row kernel pitch: a fragment of 16 consecutive padded columns from any
  // start, any 64-channel group and either k-half
  for (int c = 64; c <= 1024 && ok; c += 64) {
    const int units = int(halo_row_layout(64, c, kRowPadUnits).units);
    for (int x0 = 0; x0 < 48 && ok; ++x0)
      for (int ch = 0; ch < c / 16; ch += 4)
        ok &= expect(rule_ok([&](int l) { return long(units) * (x0 + l % 16) + ch + l / 16; }),
                     "row-kernel pitch conflict-free", c, x0);
  }
  // deep-channel split-K planes: every full 16-pixel fragment of every
  // shape (images n, output h x w; the padded image is the output plus 2
  // for a 3x3 stride-1 filter whatever the padding), at every tap and
  // k-half, with the row and image strides of deep_row_units /
  // deep_image_units
  for (int oh = 1; oh <= 20 && ok; ++oh)
    for (int ow = 1; ow <= 20 && ok; ++ow)
      for (int n = 1; n <= 8 && ok; ++n) {
          const long M = long(n) * oh * ow;
          if (M > 512) break;
          const long hp = oh + 2, wp = ow + 2;  // 3x3, stride 1: out = padded - 2
          const long S = deep_row_units(wp, ow), I = deep_image_units(hp, S, oh, ow);
          for (long f = 0; (f + 1) * 16 <= M && ok; ++f)
            for (int t = 0; t < 9 && ok; ++t)
              for (int kh = 0; kh < 2; ++kh)
                ok &= expect(rule_ok([&](int l) {
                               const long m = 16 * f + l % 16;
                               const long b = m / (oh * ow), rem = m % (oh * ow);
                               return b * I + (rem / ow) * S + (rem % ow) * kDeepUnits +
                                      (t / 3) * S + (t % 3) * kDeepUnits + 4 * kh + l / 16;
                             }),
                             "deep-channel plane fragment conflict-free", int(M), int(f));
      }
  // without the row alignment (S = 10 wp) the 7x7 fragments conflict
  ok &= expect(!rule_ok([](int l) {
                 const long m = l % 16, S = 90;
                 return (m / 7) * S + (m % 7) * kDeepUnits + l / 16;
               }),
               "unaligned deep-channel rows rejected", 0, 0);
  // the rule rejects what the probe measured as 2-way
  ok &= expect(!rule_ok([](int l) { return long(swz128x(l % 16, l / 16) / 16); }),
               "swz128x (xor-of-row-bits) layout rejected", 0, 0);
  ok &= expect(!rule_ok([](int l) { return long(5 * (l % 16) + l / 16); }), "80-byte pitch rejected",
               0, 0);
  ok &= expect(!rule_ok([](int l) { return long(9 * (l % 16) + l / 16); }), "144-byte pitch rejected",
               0, 0);
  if (!ok) return 1;
  printf("ok %d\n", checked);
  return 0;
}
