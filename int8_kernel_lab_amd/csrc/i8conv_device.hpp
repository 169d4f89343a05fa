// Device-side building blocks shared by every gfx950 kernel of the lab:
// exact fast division, buffer resources with hardware zero-fill, the INT8
// MFMA wrapper and the LDS swizzles.  Also compiled by the host (and by g++
// in the CPU tests) for the parts marked I8_HD.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define I8_HD __host__ __device__
#else
#define I8_HD
#endif

namespace i8conv {

// ---------------------------------------------------------------------------
// Exact unsigned division by a runtime divisor d (1 <= d <= 2^31) for
// dividends n < 2^31, by multiplication with M = ceil(2^(31+L) / d),
// L = max(1, ceil(log2 d)).  The round-up method (Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994):
// n*M / 2^(31+L) = n/d + e*n/2^(31+L) with 0 <= e < 1 and
// e*n/2^(31+L) < 2^-L <= 1/d, so the floor is exactly n/d.
// 2^31 <= M <= 2^32; M == 2^32 (only d == 1) is stored as add = 1, mul = 0.
struct FastDiv {
  uint32_t mul;
  uint32_t add;
  uint32_t shift;  // L - 1
  uint32_t divisor;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{};
  f.divisor = d;
  uint32_t l = 1;
  while (l < 32 && (uint64_t(1) << l) < d) ++l;  // l = max(1, ceil(log2 d))
  const uint64_t num = uint64_t(1) << (31 + l);
  const uint64_t m = (num + d - 1) / d;
  if (m == (uint64_t(1) << 32)) {
    f.mul = 0;
    f.add = 1;
  } else {
    f.mul = uint32_t(m);
    f.add = 0;
  }
  f.shift = l - 1;
  return f;
}

// The same divider without the divisor: three words, for kernels that keep
// every argument in SGPRs.
struct FastDiv3 {
  uint32_t mul;
  uint32_t add;
  uint32_t shift;
};

inline FastDiv3 make_fastdiv3(uint32_t d) {
  const FastDiv f = make_fastdiv(d);
  return FastDiv3{f.mul, f.add, f.shift};
}

template <class D>
I8_HD inline uint32_t fast_div(uint32_t n, const D &f) {
  const uint32_t hi = uint32_t((uint64_t(n) * f.mul) >> 32);
  return (hi + (f.add ? n : 0u)) >> f.shift;
}

// Kernel argument block.  All element offsets fit in int32 (the ABI rejects
// tensors above 2^31-1 bytes).
struct ConvArgs {
  const int8_t *x;
  const int8_t *w;
  const int32_t *bias;
  int32_t *y;        // final output (NHWK int32)
  int32_t *partial;  // split-K partial sums [splits][M][N], else nullptr
  int n, h, wd, c, k, r, s;
  int pad_h, pad_w, stride_h, stride_w, dil_h, dil_w;
  int out_h, out_w;
  int gemm_m, gemm_n, gemm_k;
  uint32_t x_bytes, w_bytes;
  FastDiv div_c, div_s, div_ow, div_ohw;
  // split-K: stages [split * stages_per_split, ...) of 128 k-bytes each
  int stages_per_split;
  int splits;
  // pipelined GEMM: pixel rows a tile stores (its tile height, or fewer:
  // the tile's last rows then read as zeros and are not stored)
  int m_step;
  // pipelined GEMM only: requantized int8 output from its epilogue when
  // q_y != nullptr (y unused), with per-channel multipliers and shifts
  // (16-byte aligned, N % 4 == 0) and the zero point
  const int32_t *q_mult;
  const int32_t *q_shift;
  int32_t q_zp;
  int8_t *q_y;
};

// The lab's int32 -> int8 requantization of one value:
//   clamp(zp + round(acc * mult / 2^shift), -128, 127)
// with shift clamped to [0, 62], the product exact in int64 (|acc|, |mult|
// <= 2^31, so |p| <= 2^62) and ties rounded away from zero:
//   round(p / 2^s) = floor((p + 2^(s-1) - [p < 0]) / 2^s)   (s >= 1)
// (for p < 0, -floor((|p| + h) / 2^s) = floor((p + h - 1) / 2^s) with
// h = 2^(s-1)), one add and one arithmetic shift.  Host and device: a CPU
// test checks it against the checker's own restatement.
I8_HD inline int32_t requant1(int32_t acc, int32_t mult, int32_t shift, int32_t zp) {
  const int s = shift < 0 ? 0 : (shift > 62 ? 62 : shift);
  const int64_t p = int64_t(acc) * int64_t(mult);
  const int64_t h = s > 0 ? (int64_t(1) << (s - 1)) - (p < 0 ? 1 : 0) : 0;
  const int64_t q = ((p + h) >> s) + zp;
  return int32_t(q < -128 ? -128 : (q > 127 ? 127 : q));
}

// Short form of requant1 for shift >= 33 and |zp| <= 2^30 (the usual Q31
// scales), from per-channel constants am = |mult|, hh = 2^(s-33), sh = s - 32
// (s = min(shift, 62)).  In sign-magnitude form round-half-away needs no tie
// correction: with a = |acc|,
//   round(|p| / 2^s) = floor((a*am + 2^(s-1)) / 2^s)
//                    = (hi32(a*am) + hh) >> sh
// because 2^(s-1) = hh * 2^32 adds nothing to the low word (no carry).  The
// quotient is below 2^30 (a*am <= 2^62), so zp plus the signed quotient stays
// inside int32; the sign is that of acc xor mult (a zero acc or mult gives a
// zero quotient).  One 32-bit high multiply instead of a 64-bit product,
// 64-bit add and shift.  Equal to requant1 wherever requant_short_ok holds.
I8_HD inline bool requant_short_ok(int32_t shift) { return shift >= 33; }
I8_HD inline bool requant_short_zp_ok(int32_t zp) { return zp >= -(1 << 30) && zp <= (1 << 30); }
I8_HD inline uint32_t requant_short_am(int32_t mult) {
  return mult < 0 ? 0u - uint32_t(mult) : uint32_t(mult);
}
// (1 for shifts the short form does not take, so that hh stays defined)
I8_HD inline uint32_t requant_short_sh(int32_t shift) {
  return shift < 33 ? 1u : uint32_t((shift > 62 ? 62 : shift) - 32);
}
I8_HD inline uint32_t requant_short_hh(int32_t shift) { return 1u << (requant_short_sh(shift) - 1); }
I8_HD inline int32_t requant1_short(int32_t acc, uint32_t am, int32_t mult, uint32_t hh,
                                    uint32_t sh, int32_t zp) {
  const uint32_t a = acc < 0 ? 0u - uint32_t(acc) : uint32_t(acc);
  const uint32_t r = (uint32_t((uint64_t(a) * am) >> 32) + hh) >> sh;
  const uint32_t sg = uint32_t((acc ^ mult) >> 31);
  const int32_t v = int32_t((r ^ sg) - sg) + zp;
  return v < -128 ? -128 : (v > 127 ? 127 : v);
}

// Odd-multiplier form of requant1: one signed high multiply, one add, one
// arithmetic shift and the clamp per value.  Write mult = mo * 2^t with mo
// odd (t = trailing zeros) and s' = min(shift, 62) - t:
// acc * mult / 2^s = acc * mo / 2^s'.  (mult = 0 takes mo = 0 and sh = 1:
// (0 + k) >> 1 = zp.)  For
// s' = 32 + sh with 1 <= sh <= 30, p = acc * mo and hi = floor(p / 2^32):
//   p >= 0:            round(p / 2^s') = floor((hi + hh) / 2^sh)
//                      (2^(s'-1) = hh * 2^32 with hh = 2^(sh-1) adds nothing
//                      to the low word);
//   p < 0, p not a multiple of 2^32:
//                      hi = -floor(|p| / 2^32) - 1, and
//                      -floor((-hi - 1 + hh) / 2^sh) = floor((hi + hh) / 2^sh)
//                      (since -floor(x / d) = floor((-x + d - 1) / d) and
//                      2^sh - hh = hh).
// The one case left out, p < 0 a multiple of 2^32, needs acc * mo = 0 mod 2^32,
// so acc = 0 (mo is odd, hence invertible mod 2^32), and then p = 0: it
// never occurs.  So round(acc * mult / 2^s) = (hi + hh) >> sh exactly, and
// with k = hh + zp * 2^sh (adding a multiple of 2^sh commutes with the
// shift) zp + round(...) = (hi + k) >> sh.  |hi| <= 2^30 (|p| < 2^62), so
// hi + k stays in int32 whenever |k| <= 2^30: together with 1 <= sh <= 30
// that is the form's domain (RequantOdd::ok).  Equal to requant1 there.
struct RequantOdd {
  int32_t mo, k, sh;
  bool ok;
};
I8_HD inline RequantOdd requant_odd_params(int32_t mult, int32_t shift, int32_t zp) {
  const int s = shift < 0 ? 0 : (shift > 62 ? 62 : shift);
  // trailing zeros (a uniform mult gives one s_ff1 on the device)
  const int t = mult == 0 ? 0 : __builtin_ctz(uint32_t(mult));
  RequantOdd r;
  r.mo = mult == 0 ? 0 : int32_t(int64_t(mult) >> t);
  const int sh = mult == 0 ? 1 : s - t - 32;
  r.ok = sh >= 1 && sh <= 30;
  const int64_t k = r.ok ? (int64_t(1) << (sh - 1)) + int64_t(zp) * (int64_t(1) << sh) : 0;
  r.ok = r.ok && k >= -(int64_t(1) << 30) && k <= (int64_t(1) << 30);
  r.k = r.ok ? int32_t(k) : 0;
  r.sh = r.ok ? sh : 1;
  return r;
}
I8_HD inline int32_t requant1_odd(int32_t acc, int32_t mo, int32_t k, int32_t sh) {
#if defined(__HIP_DEVICE_COMPILE__)
  // one v_mul_hi_i32: written as a 64-bit product, the compiler made it a
  // full 64 x 64 multiply (three quarter-rate operations) where it could
  // not see that mo is a sign-extended 32-bit value
  const int32_t hi = __mulhi(acc, mo);
#else
  const int32_t hi = int32_t((int64_t(acc) * int64_t(mo)) >> 32);
#endif
  const int32_t v = (hi + k) >> sh;
  return v < -128 ? -128 : (v > 127 ? 127 : v);
}

#if defined(__HIPCC__)

typedef int v4i __attribute__((ext_vector_type(4)));

// An offset at or beyond num_records makes a raw buffer load return zeros:
// that is how padding taps, m >= M and n >= N rows are zero-filled.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base,
                                                             uint32_t bytes) {
  // dword3 0x00020000: raw (stride 0) buffer, 32-bit format, gfx9 family.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base),
                                           (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ v4i load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Raw buffer descriptor as four dwords (same fields as make_rsrc), for the
// inline-asm copy below.
__device__ __forceinline__ v4u make_desc(const void *base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return v4u{uint32_t(b), uint32_t(b >> 32) & 0xffffu, bytes, 0x00020000u};
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return uint32_t(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const void *)p));
}

// One wave-wide 16-byte-per-lane copy from a buffer into LDS: lane i's 16
// bytes at buffer offset `voffset` land at LDS address lds_base + 16*i
// (zeros when voffset is out of range).  Issued as inline asm so that the
// compiler does not model it: it would otherwise wait for every copy in
// flight before any later LDS read.  The caller owns the vmcnt accounting
// (these copies complete in issue order with the wave's other vector
// memory loads).  The LDS address goes in as an M0 operand: the compiler
// writes M0 itself before the asm (and so knows it is in use).
// The asm starts with s_nop 4, five wait states: a vector memory
// instruction that reads an SGPR written by a VALU instruction (a
// v_readlane restoring a spilled SGPR of the descriptor, a readfirstlane)
// needs five wait states after that write, and M0 one after an SALU write.
// The compiler's hazard check cannot see the copy inside the asm, so it
// does not pad before it; in SGPR-heavy kernels it has placed such a
// v_readlane two instructions before the copy.
__device__ __forceinline__ void lds_copy16(v4u desc, uint32_t lds_base, uint32_t voffset) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voffset), "s"(desc), "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
      : "memory");
}

// As lds_copy16 with 4 bytes per lane: lane i's dword at buffer offset
// `voffset` lands at lds_base + 4*i (zero when out of range).
__device__ __forceinline__ void lds_copy4(v4u desc, uint32_t lds_base, uint32_t voffset) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dword %0, %1, 0 offen lds"
      :
      : "v"(voffset), "s"(desc), "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
      : "memory");
}

// Four consecutive int32 from `base` (bias), element e at index i0 + e,
// zero where i0 + e >= count; no branches.
__device__ __forceinline__ v4i load_bias4(const int32_t *base, int count, int i0) {
  const auto r = make_rsrc(base, uint32_t(count) * 4u);
  v4i v;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    v[e] = __builtin_amdgcn_raw_buffer_load_b32(r, uint32_t(i0 + e) * 4u, 0, 0);
  return v;
}

// Final-output stores.  The 16-byte stores go through a buffer resource
// over the workgroup's output rows (out_window) with one of two cache
// policies (the aux operand of the gfx950 buffer-store builtins), chosen per
// kernel by measurement:
//  * kStoreThrough, sc1 (bit 4): device-scope write-through.  For kernels
//    whose stores are spread over their whole run (the row-streaming
//    kernels) and for split-K partial sums: without it the lines stay dirty
//    in the L2 and the release at the end of the kernel writes them back
//    after the last wave has finished, which the next launch on the stream
//    waits for (28x28x128 layer: 7.8 -> 7.1 us per launch; split-K on the
//    deep-K layer 15.1 -> 14.6 us).  The pipelined GEMM uses it too, with
//    each wave storing a pixel row's channel fragments back to back so that
//    whole lines arrive together: the layers then write exactly their output
//    bytes (stride-2 3x3 layer: 14.1 us; 15.5 us and 1.29x the output bytes
//    with evict-first stores issued one channel fragment at a time).
//  * kStoreStream, nt (bit 1): evict-first lines written back by the L2.
//    Partly written lines leave the L2 as partial writes, so it pays only
//    where every store covers whole lines.
// (sc1 and nt together made the K = 36 row-kernel layer 25 % slower.)
// Write-through sends each store's bytes on at once, so the pieces must be
// whole 32-byte memory sectors: a wave's 16-channel slice of a pixel (64
// bytes) starts on a sector only when the pixel pitch N * 4 is a multiple of
// 32.  Other channel counts store ordinarily, and the L2 merges the slices
// into whole lines (K = 36 layer: 1.33x the output bytes written through,
// 1.00x ordinary, 4.08 -> 4.13 us).
// The 4-byte stores of a channel tail (N % 4 != 0) stay ordinary: each
// covers a sliver of a line, and only ordinary stores are merged into whole
// lines in the L2 (non-temporal ones went to HBM as partial writes and made
// such layers several times slower).
constexpr int kStoreThrough = 16;
constexpr int kStoreStream = 2;
// Final outputs above this size store evict-first instead of write-through.
constexpr int64_t kStreamOutputBytes = int64_t(128) << 20;

template <int kPolicy>
__device__ __forceinline__ void store_out4(__amdgpu_buffer_rsrc_t out, uint32_t byte_off, v4i v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, out, byte_off, 0, kPolicy);
}

// Write-through for sector-aligned pixel pitches (N % 8 == 0), else ordinary.
// Kernels pick the policy once per launch or per epilogue, not per store: a
// per-store branch cost 2-4 % on the GEMM layers.
__device__ __forceinline__ bool sector_pitch(int gemm_n) { return (gemm_n & 7) == 0; }

// A workgroup's output window: a buffer resource over pixels (GEMM rows)
// [m0, m0 + rows) of an [M][N] int32 tensor, clamped to M, so that
// store_out4 offsets are byte offsets from pixel m0 and fit 32 bits even
// where the whole output does not.  ok is false when the window itself is
// 2 GiB or more (absurdly wide N): the caller then takes its element path.
struct OutWindow {
  __amdgpu_buffer_rsrc_t r;
  bool ok;
};

__device__ __forceinline__ OutWindow out_window(int32_t *y, int64_t gemm_m, int n, int64_t m0,
                                                int64_t rows) {
  const int64_t rr = min(rows, gemm_m - m0);
  const int64_t bytes = rr > 0 ? rr * int64_t(n) * 4 : 0;
  OutWindow w;
  w.ok = bytes < (int64_t(1) << 31);
  w.r = make_rsrc(y + m0 * int64_t(n), w.ok ? uint32_t(bytes) : 0u);
  return w;
}
__device__ __forceinline__ void store_out1(int32_t *dst, int32_t v) { *dst = v; }

// Four consecutive channels requantized and packed into one dword (byte e =
// channel e, the NHWK int8 order).
__device__ __forceinline__ uint32_t requant4(v4i acc, v4i mult, v4i shift, int32_t zp) {
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    packed |= (uint32_t(requant1(acc[e], mult[e], shift[e], zp)) & 0xffu) << (8 * e);
  return packed;
}

// requant4 through requant1_odd (mo, k, sh from requant_odd_params); the
// low bytes are gathered with two byte permutes: v_perm_b32 selector bytes
// 0-3 pick from its second operand, 4-7 from its first, 0x0c gives zero.
__device__ __forceinline__ uint32_t requant4_odd(v4i acc, v4i mo, v4i k, v4i sh) {
  int32_t y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = requant1_odd(acc[e], mo[e], k[e], sh[e]);
  const uint32_t lo = __builtin_amdgcn_perm(uint32_t(y[1]), uint32_t(y[0]), 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(uint32_t(y[3]), uint32_t(y[2]), 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// D = A x B + C over int8 -> int32.  A is 16 rows (lane % 16) by 64 k,
// B is 64 k by 16 columns (lane % 16); lane l supplies 16 k-bytes of its
// row/column for k-block l / 16.  Any mapping of the 64 k positions onto
// (k-block, byte) is valid as long as A and B use the same one.
// Result: lane l holds C[4 * (l / 16) + v][l % 16] in element v.
__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

#endif  // __HIPCC__

// LDS bank rule for ds_read_b128 on gfx950, measured with the LDS probe
// (kernel_probe.hip): a wave's read runs at full rate when every 32
// consecutive lanes address distinct 16-byte units modulo 512 bytes and
// every 4 consecutive lanes distinct units modulo 128 bytes; a pattern that
// breaks either takes about 1.4x as long (2-way), and 8 or 16 lanes on one
// unit position 5.5x and 11x.  An MFMA fragment read has lane l on row
// (or pixel) l % 16 and 16-byte chunk l / 16 (+ 4 for the second k-half),
// so lanes 0..31 cover 16 rows x 2 chunks and lanes 4k..4k+3 four
// consecutive rows of one chunk.

// LDS layout of a [rows][128-byte] operand tile: 16-byte chunk j of row r
// lives at r*128 + 16*(j ^ f(r)) with f(r) = 2*((r + (r >> 2)) & 3) +
// ((r >> 2) & 1).  Rows r, r + 4, r + 8, r + 12 share a 512-byte unit
// position modulo 4 rows, and f gives them four distinct values of f >> 1,
// so chunks j and j ^ 1 of the four land on eight distinct units; f of four
// consecutive rows takes four distinct values.  (The earlier form
// j ^ (r & 7) ^ ((r >> 3) & 1) broke the 32-lane condition: 123 against
// 173 bytes per clock per compute unit in the probe.)
I8_HD inline int swz128_f(int row) { return 2 * ((row + (row >> 2)) & 3) + ((row >> 2) & 1); }
I8_HD inline int swz128(int row, int chunk) { return row * 128 + ((chunk ^ swz128_f(row)) << 4); }
// Inverse: the logical chunk stored in physical 16-byte slot `phys` of
// `row` (a DMA writes slots in order, so each lane fetches the chunk its
// slot holds).
I8_HD inline int swz128_chunk(int row, int phys) { return phys ^ swz128_f(row); }

// The XOR-of-row-bits layout of 128-byte rows: chunk j of row r at
// r*128 + 16*(j ^ (r & 7) ^ ((r >> 3) & 1)).  Each 16 lanes of a fragment
// read cover all sixteen 4-bank groups, but it breaks the 32-lane
// condition: fragment reads are 2-way conflicts.  The pipelined GEMM keeps
// it all the same: there the conflict-free swz128 measured 1-2 % slower
// (A/B, configs 3 and 5b and 256x256 layers; the GEMM's time is not in its
// LDS reads), so swz128x is its layout.  Its own inverse.
I8_HD inline int swz128x(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7) ^ ((row >> 3) & 1)) << 4);
}
I8_HD inline int swz128x_chunk(int row, int phys) { return phys ^ (row & 7) ^ ((row >> 3) & 1); }

// LDS layout of a [pixels][64-byte] halo/strip patch: chunk j of pixel p at
// p*64 + 16*(j ^ g(p)), g(p) = 2*(((p >> 1) ^ (p >> 3)) & 1).  Pixels p and
// p + 8 share a unit position modulo 512 bytes and get g values 0 and 2, so
// chunks j, j ^ 1 of both cover four distinct units; consecutive pixels p,
// p + 2 of one parity get different g.  Conflict-free for sixteen
// consecutive pixels by the rule above (the earlier j ^ ((p >> 2) & 3) was
// not: 122 against 173 bytes per clock).
I8_HD inline int swz64_g(int pixel) { return 2 * (((pixel >> 1) ^ (pixel >> 3)) & 1); }
I8_HD inline int swz64(int pixel, int chunk) { return pixel * 64 + ((chunk ^ swz64_g(pixel)) << 4); }
// Inverse, as for swz128_chunk.
I8_HD inline int swz64_chunk(int pixel, int phys) { return phys ^ swz64_g(pixel); }

}  // namespace i8conv
