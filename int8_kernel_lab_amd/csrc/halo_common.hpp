// Building blocks shared by the kernels that keep whole padded input rows
// in LDS and stream the filter through an LDS ring (kernel_halo.hip,
// kernel_row.hip): kernel-argument pinning, the per-wave filter ring and
// the row-aligned input-row copy.
#pragma once

#include "i8conv_internal.hpp"

namespace i8conv {

__device__ __forceinline__ v4i add_wrap4(v4i a, v4i b) {
  // int32 addition with two's-complement wrap, like the MFMA accumulator.
  return __builtin_bit_cast(v4i, __builtin_bit_cast(v4u, a) + __builtin_bit_cast(v4u, b));
}

// Loads every 32-bit word of a kernel-argument struct into SGPRs here, in
// one batch, instead of where each field is first used.
template <class T>
__device__ __forceinline__ void pin_sgprs(const T &v) {
  static_assert(sizeof(T) % 4 == 0, "argument block of whole words");
  uint32_t w[sizeof(T) / 4];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (int i = 0; i < int(sizeof(T) / 4); ++i) asm volatile("" ::"s"(w[i]));
}

// s_waitcnt vmcnt(min(n, 63)) for a wave-uniform run-time n (the counter
// field is six bits; waiting for fewer outstanding copies is always safe).
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n > 63 ? 63 : n) {
#define I8_VM(N) \
  case N: asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); break;
    I8_VM(0) I8_VM(1) I8_VM(2) I8_VM(3) I8_VM(4) I8_VM(5) I8_VM(6) I8_VM(7)
    I8_VM(8) I8_VM(9) I8_VM(10) I8_VM(11) I8_VM(12) I8_VM(13) I8_VM(14) I8_VM(15)
    I8_VM(16) I8_VM(17) I8_VM(18) I8_VM(19) I8_VM(20) I8_VM(21) I8_VM(22) I8_VM(23)
    I8_VM(24) I8_VM(25) I8_VM(26) I8_VM(27) I8_VM(28) I8_VM(29) I8_VM(30) I8_VM(31)
    I8_VM(32) I8_VM(33) I8_VM(34) I8_VM(35) I8_VM(36) I8_VM(37) I8_VM(38) I8_VM(39)
    I8_VM(40) I8_VM(41) I8_VM(42) I8_VM(43) I8_VM(44) I8_VM(45) I8_VM(46) I8_VM(47)
    I8_VM(48) I8_VM(49) I8_VM(50) I8_VM(51) I8_VM(52) I8_VM(53) I8_VM(54) I8_VM(55)
    I8_VM(56) I8_VM(57) I8_VM(58) I8_VM(59) I8_VM(60) I8_VM(61) I8_VM(62)
#undef I8_VM
    default: asm volatile("s_waitcnt vmcnt(63)" ::: "memory"); break;
  }
}

// The filter staging ring: chunk c = bytes [128c, 128c + 128) of the
// workgroup's 64*FN filter rows, in ring slot c % slots.  Each wave copies
// and reads only its own 16*FN rows of every slot, so a chunk needs no
// barrier: the wave's own copy counter says when its rows have landed, and
// only the wave itself reuses them.
template <int FN, int kSteps>
struct FilterRing {
  static constexpr int kRows = 64 * FN;
  static constexpr int kChunks = (kSteps + 1) / 2;
  static constexpr int kChunkBytes = kRows * 128;
  static constexpr int kCopies = kRows * 8 / 64 / 4;  // per wave per chunk
  v4u wd;
  uint32_t lds;  // LDS address of slot 0
  const int8_t *ptr;
  int slots, wave, lane;
  mutable int cur;  // ring slot of the next chunk take() waits for
  // Per copy j of this lane: the filter byte offset of its 16 bytes in
  // chunk 0, and the bound on 128*c below which chunk c's bytes exist (0
  // for channels past N, so every chunk reads zeros there).
  uint32_t base[kCopies];
  int klim[kCopies];

  __device__ __forceinline__ void init(int tile_n, int gemm_n, int gemm_k) {
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      const int slot = (kCopies * wave + j) * 64 + lane;  // rows 16*FN*wave + [0, 16*FN)
      const int r = slot >> 3;
      const int chunk16 = swz128_chunk(r, slot & 7);
      const int oc = tile_n + r;
      base[j] = uint32_t(oc) * uint32_t(gemm_k) + uint32_t(chunk16 * 16);
      klim[j] = oc < gemm_n ? gemm_k - chunk16 * 16 : 0;
    }
  }
  // Copies chunk c into ring slot `slot` (== c % slots).
  __device__ __forceinline__ void issue(int c, int slot) const {
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      const uint32_t off = c * 128 < klim[j] ? base[j] + uint32_t(c * 128) : kOutOfRange;
      lds_copy16(wd, lds + slot * kChunkBytes + (kCopies * wave + j) * 1024, off);
    }
  }
  // Chunk c has landed once no more than `after` later chunks are
  // outstanding: copies return in issue order, and everything issued before
  // the ring (bias, input rows) is older than every chunk.
  __device__ __forceinline__ void wait(int c) const {
    const int after = min(slots - 1, kChunks - 1 - c);
    switch (after) {
      case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
      case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(1 * kCopies) : "memory"); break;
      case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kCopies) : "memory"); break;
      case 3: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * kCopies) : "memory"); break;
      case 4: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * kCopies) : "memory"); break;
      case 5: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * kCopies) : "memory"); break;
      case 6: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 * kCopies) : "memory"); break;
      default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(7 * kCopies) : "memory"); break;
    }
  }
  // Waits for chunk c, moves its two k-steps into this wave's fragments and
  // refills its slot with chunk c + slots.  Chunks are taken in order, so
  // `cur` (the slot of the next chunk to take) advances by one per take.
  // Taking chunk 0 also publishes the input rows: every wave has then waited
  // for its own row copies (older than its chunk-0 copies), and one barrier
  // makes all of them visible to all waves.
  __device__ __forceinline__ void take(int c, v4i (&wf)[kSteps][FN]) const {
    wait(c);
    if (c == 0) __syncthreads();
    const int slot = cur;
    cur = slot + 1 == slots ? 0 : slot + 1;
    const int8_t *src = ptr + slot * kChunkBytes;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = 2 * c + h;
      if (t >= kSteps) break;
#pragma unroll
      for (int i = 0; i < FN; ++i)
        wf[t][i] = *reinterpret_cast<const v4i *>(
            src + swz128(wave * 16 * FN + i * 16 + (lane & 15), 4 * h + (lane >> 4)));
    }
    if (c + slots < kChunks) {
      // this wave's reads of its rows must be done before they are refilled
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(c + slots, slot);
    }
  }
};

// Copies padded input rows [vr0, vr0 + nrows) into LDS at lds0, rows
// row_bytes apart (HaloRowLayout).  A virtual row vr = batch * hp + padded
// row; rows outside the image (padding, or past the last image) read as
// zeros.  Copy q covers units [64j, 64j + 64) of row rr (q = rr *
// row_copies + j), the four waves taking every fourth copy; copies never
// straddle rows, so the row arithmetic is wave-uniform.  Unit `slot` of a
// row is unit u of padded column pix (slot = pix*units + u); units c/16 and
// up are the pad.  Its byte offset in x is
//   ((b*h + iy)*w + pix - pad_w)*c + 16u = row_off + pix*c + 16u.
template <class Div>
__device__ __forceinline__ void copy_input_rows(v4u xd, uint32_t lds0, int vr0, int nrows,
                                                int wave, int lane, int row_copies,
                                                const Div &div_row_copies, int row_bytes,
                                                const Div &div_hp, int hp, int units,
                                                const Div &div_units, int n, int h, int wd,
                                                int c, int pad_h, int pad_w) {
  const int copies = nrows * row_copies;
  for (int q = wave; q < copies; q += 4) {
    const int rr = int(fast_div(uint32_t(q), div_row_copies));
    const int j = q - rr * row_copies;
    const int vr = vr0 + rr;
    const int b = int(fast_div(uint32_t(vr), div_hp));
    const int iy = vr - b * hp - pad_h;
    const bool row_ok = b < n && unsigned(iy) < unsigned(h);
    // modulo 2^32: exact wherever it is used (the sum below is in [0, 2^31))
    const uint32_t row_off = uint32_t((b * h + iy) * wd - pad_w) * uint32_t(c);
    const int slot = j * 64 + lane;
    const int pix = int(fast_div(uint32_t(slot), div_units));
    const int u = slot - pix * units;
    const bool ok = row_ok && u < (c >> 4) && unsigned(pix - pad_w) < unsigned(wd);
    const uint32_t off = ok ? row_off + uint32_t(pix * c + 16 * u) : kOutOfRange;
    lds_copy16(xd, lds0 + rr * row_bytes + j * 1024, off);
  }
}

// Stages this wave's bias (16*FN channels from oc0) into LDS at `dst` (256
// bytes per wave) with one dword copy: the first copy of the wave, so every
// later wait on the copy stream also covers it.  (A register load of the
// bias would need a compiler-inserted wait, which cannot see the copies and
// so would wait for everything, stores included.)
template <int FN>
__device__ __forceinline__ void stage_bias(const int32_t *bias, int gemm_n, int oc0,
                                           const int8_t *dst, int lane) {
  const int oc = oc0 + lane;
  const uint32_t off = lane < 16 * FN && oc < gemm_n ? uint32_t(oc) * 4u : kOutOfRange;
  lds_copy4(make_desc(bias, uint32_t(gemm_n) * 4u), lds_addr(dst), off);
}

}  // namespace i8conv
