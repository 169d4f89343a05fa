// Seeded synthetic data.  SplitMix64 (Steele, Lea, Flood, "Fast splittable
// pseudorandom number generators", OOPSLA 2014): the state advances by the
// golden-ratio increment and each output is the state passed through the
// variant-13 finalizer of MurmurHash3.  Value = lo + (next() mod span).
// The reference draws from std::mt19937 + std::uniform_int_distribution
// (conv_lab.cu:149-157), whose value stream is implementation-defined; this
// generator is fully specified so every host produces the same bytes.
#include <stdint.h>

#include "i8conv.h"

namespace {

inline uint64_t splitmix64_next(uint64_t *state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

extern "C" void i8conv_fill_int8(int8_t *dst, size_t count, int lo, int hi,
                                 uint64_t *state) {
  const uint64_t span = uint64_t(int64_t(hi) - int64_t(lo) + 1);
  for (size_t i = 0; i < count; ++i)
    dst[i] = int8_t(int64_t(lo) + int64_t(splitmix64_next(state) % span));
}

extern "C" void i8conv_fill_int32(int32_t *dst, size_t count, int32_t lo,
                                  int32_t hi, uint64_t *state) {
  const uint64_t span = uint64_t(int64_t(hi) - int64_t(lo) + 1);
  for (size_t i = 0; i < count; ++i)
    dst[i] = int32_t(int64_t(lo) + int64_t(splitmix64_next(state) % span));
}
