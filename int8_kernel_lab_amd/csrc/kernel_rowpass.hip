// Row-streaming 3x3 kernel for 128-channel layers on gfx950 INT8 MFMA,
// with copy-only waves that stream the operands to the MFMA waves row by
// row (the headline kernel of the 28x28x128 layer).
//
// Why.  A row-streaming workgroup (kernel_row.hip) copies its padded input
// rows and its filter slice (16 output channels x 9 x 128 bytes per MFMA
// wave) into LDS before most of its MFMAs can run.  At kernel start the L2s
// are cold and all 256 compute units copy at once; one compute unit's
// copies land at about 65 GB/s whatever the access pattern or wave count,
// so the ~108 KB of a 28x28x128 workgroup take ~1.7 us, and a wave that
// issues copies stalls while the memory pipeline is full.
//
// How.  Eight waves: four MFMA waves (16 output channels each) and four
// copy waves.  The copy waves issue the copies in the order the MFMA waves
// consume them, in chunks: padded input row r (both 64-channel groups),
// preceded for r <= 2 by the taps of filter row r (input row r feeds output
// rows r - fy, so filter row r is first needed at input row r), the bias
// first of all.  Each copy wave follows each chunk with a flag copy (below)
// and never waits; the MFMA waves walk the input rows, wait for each row's
// chunk just before reading it, and store output row o once it is complete
// (one row after input row o + 2).  The MFMAs start after the first chunk
// (~9 KB) instead of all the copies, and the stores are spread over the
// walk.
//
// Flags.  A copy wave's loads return in the order it issued them (the
// property that makes vmcnt a count of the oldest loads outstanding), and
// an LDS-DMA load writes LDS when it returns.  So after issuing its copies
// of chunk c a copy wave issues one more: a 4-byte LDS-DMA copy, from lane
// 0 only (the copy writes only the active lanes), of a device word holding
// 1 into its flag word of chunk c.  Once that flag reads 1, all of the
// wave's copies of chunk c are in LDS.  The copy waves thus issue all their
// copies without a single wait: a wave that waits for chunk c before
// signalling it (vmcnt, then an LDS add) cannot issue meanwhile, and the
// compute unit's loads in flight drop (28x28x128: 6.44 -> 6.14 us per
// launch, same box).  With 4 fragments per row the registers do not hold both
// groups: the walk then runs twice, group 0 (accumulating every output row
// of the block) and group 1 (completing and storing them).
//
// Layouts.  Input: one LDS plane per (group, padded row): wp pixels x 96
// bytes (the group's 64 channels, then 32 bytes of padding).  A fragment
// read (16 pixels x 4 chunks) is then conflict-free by gfx950's
// ds_read_b128 bank rule (i8conv_device.hpp): a pitch of 6 units puts
// lanes 0..31 on 32 distinct units modulo 512 bytes and four consecutive
// pixels on distinct units modulo 128; the earlier 80-byte pitch (5 units)
// made every fragment read a 2-way conflict.  Filter: per MFMA wave, 18
// 1 KB halves (group-major, then tap): 16 output channels x 64 bytes in the
// swz64 layout, copied with the swizzle applied at the source.
//
// Reuse and MFMAs are as in kernel_row.hip: the fragment of input row ir at
// column offset fx feeds output rows ir - fy for fy = 0, 1, 2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "halo_common.hpp"

namespace i8conv {

// Set by a wave of rowpass_kernel whose bounded chunk wait gave up (below);
// read and cleared by rowpass_wait_expired on the host.
__device__ __attribute__((aligned(4))) unsigned int g_wait_expired;

namespace {

constexpr int kGroups = 2;      // 64-channel groups: c == 128
constexpr int kUnits = 6;       // 16-byte units per pixel in a plane (4 data + 2 pad)
constexpr int kTaps = 9;
constexpr int kHalves = kTaps * kGroups;  // 1 KB filter halves per wave
// Channel groups per row walk: 2 (one pass over the rows, both groups per
// row) where the registers allow it, 1 (two passes, group 0 then group 1)
// for 4 fragments per row, whose single-pass form would spill.
constexpr int walk_groups(int nfr) { return nfr == 4 ? 1 : 2; }
// How a walk stores its output rows: element stores (a misaligned output or
// N % 4 != 0); 16-byte stores, with a branch per row on the block's row
// count; 16-byte stores of a block that has all the walk's rows (no branch).
constexpr int kStoreElem = 0, kStoreVec = 1, kStoreFull = 2;

// The arguments of the walk (the copy waves' come preloaded: PreGeo and
// the kernel's leading pointers, below).
struct PassArgs {
  int32_t *y;
  uint32_t y_bytes;  // output bytes (< 2^31: checked at launch)
  // requantized int8 output (kQ instances): per-channel multiplier and
  // shift, zero point, output (y_bytes then counts int8 bytes)
  const int32_t *qmult, *qshift;
  int8_t *qy;
  int32_t qzp;
  int out_h, out_w, gemm_n;
  int plane_copies;  // 1 KB copies per plane: ceil(wp * kUnits / 64)
  int rows_in;       // input rows per block: R + 2
  int spin_limit;    // polls of a bounded chunk wait (wait_spin_limit())
};

// Cross-wave signals in LDS: flag words set by LDS-DMA flag copies behind
// each chunk (see the top of this file), polled by the MFMA waves.
// The wait is bounded: after spin_limit polls (each a read and a sleep of
// about 64 cycles; by default 2^20, some tens of ms in all, far beyond any
// real copy time) it gives up, so that every wave always reaches the end of
// the kernel.  The host lowers the limit only to test the give-up path
// (i8conv_set_wait_spin_limit: 0 gives up at the first wait).  A
// wave that gives up goes on with LDS contents that may not have landed,
// so it records the give-up in g_wait_expired (a vector store to global
// memory); the host reads and clears that word with i8conv_wait_expired()
// after synchronizing, and must treat the output of the launches since the
// last check as wrong when it is set.
// The source word of every flag copy.
__device__ __attribute__((aligned(16))) int g_flag_one[4] = {1, 1, 1, 1};

// A compiler-visible read of the four flag words (one per copy wave) of a
// chunk at LDS address addr, issued ahead of its use: the compiler waits
// for it where the value is tested, a row later.
__device__ __forceinline__ v4i flag_peek(uint32_t addr) {
  return *reinterpret_cast<volatile __attribute__((address_space(3))) v4i *>(size_t(addr));
}

// All four copy waves' copies of the chunk have landed (wave-uniform).
__device__ __forceinline__ bool flags_set(v4i f) {
  return __builtin_amdgcn_readfirstlane(f[0] & f[1] & f[2] & f[3]) != 0;
}

// The workgroup barrier after wave 0 zeroes the chunk flags.  It waits for
// LDS operations only (wave 0's flag writes): __syncthreads' release fence
// could also wait for the copy waves' loads in flight, which are free to
// land at any time (nothing reads them before their flags).
__device__ __forceinline__ void flag_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ void flag_wait(uint32_t addr, int spin_limit) {
  for (int spin = 0; spin < spin_limit; ++spin) {
    v4i v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    if (flags_set(v)) return;
    __builtin_amdgcn_s_sleep(1);
  }
  // the chunk never arrived: every lane stores the same word (one global
  // vector store, agent scope), the host finds it set after the launch.  A
  // relaxed atomic store is a plain global store; a volatile one through a
  // generic pointer was a flat store plus a wait for all memory operations,
  // which the compiler then also assumed after every wait.
  __hip_atomic_store(&g_wait_expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// State of one wave's row walk over output rows [OLO, OHI) of the block
// (input rows OLO .. OHI + 1), NG channel groups at a time: NG == 1 walks
// the rows twice (group 0, then group 1; the two-pass form), NG == 2 once
// with both groups per row (the single-pass form).
template <int R, int NFR, int NG, bool kQ, int OLO, int OHI>
struct PassState {
  v4i wf[NG][kTaps];       // this wave's 16 channels, the walk's groups, all taps (t = fy*3 + fx)
  v4i acc[R][NFR];         // output rows of the block
  v4i frag[NG][3][NFR];    // fragments of the next input row (column offsets 0, 1, 2)
  int colofs[3][NFR];      // LDS offset of this lane's column + fx / k-block in a plane
  const int8_t *planes;    // group-0 planes, then group-1 planes
  const int8_t *halves;    // this wave's filter halves: (group, tap) 1 KB each
  const int8_t *bias_lds;  // this wave's 16 bias values
  int plane_bytes;
  uint32_t flags;          // LDS address of the chunk flags: 16 bytes per chunk
  v4i peeked;              // flags of the next row's chunk, read one row ahead
  v4i lastpeek;            // flags of the walk's last chunk (read at step OLO + kDecide - 1)
  // Output, vector path: a buffer resource over y, this lane's byte offset
  // of output row 0 per fragment (out of range where the column or the
  // channels fall outside the layer: the store is dropped, no branch), and
  // the byte stride between output rows (a scalar offset per row).
  __amdgpu_buffer_rsrc_t yr;
  uint32_t voff[NFR];
  uint32_t row_stride;
  // kQ: this lane's four channels' multiplier and shift, and their odd
  // multiplier, k and sh for requant4_odd, which the wave takes when every
  // one of its channels is in that form's domain (qodd; else requant4)
  v4i qm, qs;
  v4i qmo, qk, qsh;
  bool qodd;

  // steps of a walk that test each row's chunk flags before the walk tests
  // its last chunk's
  static constexpr int kDecide = 4;

  // The requantizing two-group full-store walk's MFMA order within a step:
  // the row that the step completes (fy = 2) first, interleaved with the
  // fy = 1 row, then fy = 0 with the rest of fy = 1 (entries: fy, block
  // g * 3 + fx; each entry is NFR MFMAs), so that at least four accumulator
  // chains alternate; the completed row is requantized and stored in the
  // same step, six MFMAs after its last, one step earlier than the order
  // below allows, and the walk's last row in its last step.  28x28x128 with
  // int8 output: 6.52-6.57 -> 6.19-6.21 us per launch (same box); with int32
  // output the same order measured 4.84 -> 4.87 us, so that walk keeps the
  // (g, fx, fy) order and stores each row in the step after.
  static constexpr int kOrderFy[18] = {2, 2, 1, 2, 2, 1, 2, 2, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1};
  static constexpr int kOrderB[18] = {0, 1, 0, 2, 3, 1, 4, 5, 2, 0, 1, 3, 2, 3, 4, 4, 5, 5};
  // index of the MFMA after which row ir - 2's stores go: six after its last
  static constexpr int early_sa(int ir) {
    int n = 0, done = 0;
    for (int e = 0; e < 18; ++e) {
      const int o = ir - kOrderFy[e];
      if (o >= OLO && o < OHI) {
        n += NFR;
        if (kOrderFy[e] == 2) done = n;
      }
    }
    return done + 5 < n - 1 ? done + 5 : n - 1;
  }
  static constexpr int mfmas_in_step(int ir) {
    int n = 0;
    for (int fy = 0; fy < 3; ++fy) n += (ir - fy >= OLO && ir - fy < OHI) ? 1 : 0;
    return n * NG * 3 * NFR;
  }
  static constexpr int reads_in_step(int ir) {
    return ir + 1 < OHI + 2 ? NG * 3 * NFR + (ir + 1 - OLO <= 2 ? NG * 3 : 0) : 0;
  }
  // MFMAs and LDS reads (the next row's fragments and taps) of step ir.
  // Scheduling groups: MFMA m is preceded by the LDS reads that spread NR
  // reads evenly over NM MFMAs (ceil((m+1) NR / NM) - ceil(m NR / NM)).
  // With NS > 0, the NS buffer stores of the step go right after MFMA SA.
  template <int NR, int NM, int SA, int NS, int M>
  __device__ static __forceinline__ void interleave_one() {
    constexpr int r = ((M + 1) * NR + NM - 1) / NM - (M * NR + NM - 1) / NM;
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (NS > 0 && M == SA) __builtin_amdgcn_sched_group_barrier(0x040, NS, 0);
  }
  template <int NR, int NM, int SA, int NS, size_t... M>
  __device__ static __forceinline__ void interleave(std::index_sequence<M...>) {
    (interleave_one<NR, NM, SA, NS, int(M)>(), ...);
  }

  template <int G>
  __device__ __forceinline__ void load_row(const PassArgs &p, int r) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int8_t *plane = planes + ((G + g) * p.rows_in + r) * plane_bytes;
#pragma unroll
      for (int fx = 0; fx < 3; ++fx)
#pragma unroll
        for (int j = 0; j < NFR; ++j)
          frag[g][fx][j] = *reinterpret_cast<const v4i *>(plane + colofs[fx][j]);
    }
  }

  // Chunk of (first group G, padded input row r): chunks are numbered in the
  // order the copy waves issue them (group-major when NG == 1).
  template <int G>
  __device__ __forceinline__ uint32_t counter(const PassArgs &p, int r) const {
    return flags + 16u * uint32_t((G / NG) * p.rows_in + r);
  }

  template <int G, int FY>
  __device__ __forceinline__ void take_taps(int lane) {
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int fx = 0; fx < 3; ++fx)
        wf[g][FY * 3 + fx] = *reinterpret_cast<const v4i *>(
            halves + ((G + g) * kTaps + FY * 3 + fx) * 1024 + swz64(lane & 15, lane >> 4));
  }

  // Input row IR of the walk from group G: once the next row's chunk has
  // landed, its fragments (and, in the walk's first rows, the next filter
  // row's taps: input row OLO + t first needs filter row t) are read,
  // interleaved with the MFMAs of this row into output rows IR - fy
  // (compile-time valid ones); in the last walk, output row IR - 3 is then
  // stored.  The flags of the chunk after next are read here and tested
  // one row later, so a chunk that has landed costs no wait.
  template <int G, int IR, int kMode, bool kTest>
  __device__ __forceinline__ void step(const PassArgs &p, int rows_out, int m_row0, int oc0,
                                       int lane) {
    // Output row IR - 3 was completed by the previous row's MFMAs.
    // kStoreFull: its two stores (with kQ, requantized in the odd form) go
    // between this row's MFMAs, after the sixth, by which time the MFMAs
    // that completed it have drained.
    // Otherwise (a branch per row: element stores, or a block with fewer
    // rows than the walk) it is stored first thing.
    constexpr bool kEarly = kMode == kStoreFull && NG == 2 && kQ;
    constexpr bool kEarlyHere = kEarly && G + NG == kGroups && IR - 2 >= OLO && IR - 2 < OHI;
    constexpr bool kStoreHere = !kEarly && G + NG == kGroups && IR >= OLO + 3;
    constexpr bool kInStep = kStoreHere && kMode == kStoreFull;
    if constexpr (kStoreHere && !kInStep)
      store_row<IR - 3>(p, kMode != kStoreElem, rows_out, m_row0, oc0, lane);
    v4i cur[NG][3][NFR];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int fx = 0; fx < 3; ++fx)
#pragma unroll
        for (int j = 0; j < NFR; ++j) cur[g][fx][j] = frag[g][fx][j];
    if (IR + 1 < OHI + 2) {
      if constexpr (kTest) {
        const v4i seen = peeked;
        if (IR + 2 < OHI + 2) peeked = flag_peek(counter<G>(p, IR + 2));
        // the last chunk's flags, tested before the steps that may skip
        // their flag tests (walk)
        if (IR + 1 == OLO + kDecide) lastpeek = flag_peek(counter<G>(p, OHI + 1));
        if (!flags_set(seen)) flag_wait(counter<G>(p, IR + 1), p.spin_limit);
        // keeps the compiler from moving the plain LDS reads of load_row
        // (and take_taps) above the flag test on the path that skips
        // flag_wait (whose asm already orders them); the hardware issues a
        // wave's LDS operations in order, so no wait instruction is needed
        asm volatile("" ::: "memory");
      }
      constexpr int fy_next = IR + 1 - OLO;
      if (fy_next <= 2) take_taps<G, (fy_next <= 2 ? fy_next : 0)>(lane);
      load_row<G>(p, IR + 1);
    }
    if constexpr (kEarly) {
#pragma unroll
      for (int e = 0; e < 18; ++e) {
        const int fy = kOrderFy[e], bb = kOrderB[e], g = bb / 3, fx = bb % 3;
        const int o = IR - fy;
        if (o >= OLO && o < OHI) {
#pragma unroll
          for (int j = 0; j < NFR; ++j)
            acc[o][j] = mfma16(wf[g][fy * 3 + fx], cur[g][fx][j], acc[o][j]);
        }
      }
    } else {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int fx = 0; fx < 3; ++fx) {
#pragma unroll
        for (int fy = 0; fy < 3; ++fy) {
          const int o = IR - fy;  // a constant once the loops are unrolled
          if (o >= OLO && o < OHI) {
#pragma unroll
            for (int j = 0; j < NFR; ++j)
              acc[o][j] = mfma16(wf[g][fy * 3 + fx], cur[g][fx][j], acc[o][j]);
          }
        }
      }
    }
    }
    if constexpr (kEarlyHere && kQ) {
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        __builtin_amdgcn_raw_buffer_store_b32(requant4_odd(acc[IR - 2][j], qmo, qk, qsh), yr,
                                              voff[j], (IR - 2) * row_stride, 0);
    } else if constexpr (kEarlyHere) {
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(acc[IR - 2][j], yr, voff[j],
                                               (IR - 2) * row_stride, kStoreThrough);
    }
    if constexpr (kInStep && kQ) {
      // kStoreFull with kQ: the wave takes the odd-multiplier form (qodd),
      // whose ~5 VALU operations per value the compiler spreads between
      // the MFMAs like the reads
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        __builtin_amdgcn_raw_buffer_store_b32(requant4_odd(acc[IR - 3][j], qmo, qk, qsh), yr,
                                              voff[j], (IR - 3) * row_stride, 0);
    } else if constexpr (kInStep) {
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(acc[IR - 3][j], yr, voff[j],
                                               (IR - 3) * row_stride, kStoreThrough);
    }
    // the next row's reads go between this row's MFMAs (issued all ahead of
    // them, they held the MFMAs back: 6.7 -> 6.5 us per launch on 28x28x128)
    constexpr int kNM = mfmas_in_step(IR);
    interleave<reads_in_step(IR), kNM, (kEarlyHere ? early_sa(IR) : (kNM < 6 ? kNM - 1 : 5)),
               ((kInStep || kEarlyHere) ? NFR : 0)>(
        std::make_index_sequence<kNM>{});
  }

  // Output row O: the accumulators already hold bias + dot products.  N % 4
  // == 0 (and an aligned output): one buffer store per fragment at a scalar
  // row offset, no address arithmetic: 16 bytes of int32 (write-through,
  // kStoreThrough), or with kQ the four requantized int8 values as one
  // dword (an ordinary store: a wave writes 16 bytes of a pixel's line, and
  // the L2 merges the four waves' pieces before writing it; 28x28x128 int8
  // output with the odd form: 7.35 us per launch, against 7.5 written
  // through and 8.2 evict-first, same box); otherwise element stores.
  template <int O>
  __device__ __forceinline__ void store_row(const PassArgs &p, bool vec, int rows_out, int m_row0,
                                            int oc0, int lane) {
    if (O >= rows_out) return;
    if constexpr (kQ) {
      if (vec) {
        // qodd is uniform over the wave: a scalar branch
        if (qodd) {
#pragma unroll
          for (int j = 0; j < NFR; ++j)
            __builtin_amdgcn_raw_buffer_store_b32(requant4_odd(acc[O][j], qmo, qk, qsh), yr,
                                                  voff[j], O * row_stride, 0);
        } else {
#pragma unroll
          for (int j = 0; j < NFR; ++j)
            __builtin_amdgcn_raw_buffer_store_b32(requant4(acc[O][j], qm, qs, p.qzp), yr, voff[j],
                                                  O * row_stride, kStoreStream);
        }
        return;
      }
      const int m_row = m_row0 + O * p.out_w;
#pragma unroll
      for (int j = 0; j < NFR; ++j) {
        const int col = 16 * j + (lane & 15);
        if (col >= p.out_w) continue;
        int8_t *dst = p.qy + size_t(m_row + col) * size_t(p.gemm_n) + oc0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (oc0 + e < p.gemm_n) dst[e] = int8_t(requant1(acc[O][j][e], qm[e], qs[e], p.qzp));
      }
      return;
    }
    if (vec) {
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(acc[O][j], yr, voff[j], O * row_stride,
                                               kStoreThrough);
      return;
    }
    const int m_row = m_row0 + O * p.out_w;
#pragma unroll
    for (int j = 0; j < NFR; ++j) {
      const int col = 16 * j + (lane & 15);
      if (col >= p.out_w) continue;
      int32_t *dst = p.y + size_t(m_row + col) * size_t(p.gemm_n) + oc0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (oc0 + e < p.gemm_n) store_out1(dst + e, acc[O][j][e]);
    }
  }

  // Steps OLO + From + I of the walk from group G, with or without the
  // next row's flag test.
  template <int G, int kMode, bool kTest, int From, size_t... I>
  __device__ __forceinline__ void steps(const PassArgs &p, int rows_out, int m_row0, int oc0,
                                        int lane, std::index_sequence<I...>) {
    (step<G, OLO + From + int(I), kMode, kTest>(p, rows_out, m_row0, oc0, lane), ...);
  }

  // The walk from group G over padded input rows OLO .. OHI + 1.  The first
  // kDecide steps test each next row's chunk flags; by then the copy waves
  // have usually landed every chunk (they issue all copies without
  // waiting), so the walk tests the flags of its last chunk once: if they
  // are set, every chunk of the walk has landed (each copy wave's loads
  // land in the order it issued them, its flag copy of a chunk after the
  // chunk's copies), and the remaining steps run without flag tests, whose
  // read-test-branch sequence left the MFMA pipe idle for some cycles per
  // row (28x28x128: ~20 ns per row step).
  template <int G, int kMode>
  __device__ __forceinline__ void walk(const PassArgs &p, int rows_out, int m_row0, int oc0,
                                       int lane) {
    constexpr int kSteps = OHI - OLO + 2;
    flag_wait(counter<G>(p, OLO), p.spin_limit);
    peeked = flag_peek(counter<G>(p, OLO + 1));
    take_taps<G, 0>(lane);
    load_row<G>(p, OLO);
    if (G == 0) {
      // the accumulators start at the bias (the oracle adds the bias first)
      const v4i bv = *reinterpret_cast<const v4i *>(bias_lds + 16 * (lane >> 4));
#pragma unroll
      for (int r = OLO; r < OHI; ++r)
#pragma unroll
        for (int j = 0; j < NFR; ++j) acc[r][j] = bv;
    }
    if constexpr (kDecide + 1 < kSteps) {
      steps<G, kMode, true, 0>(p, rows_out, m_row0, oc0, lane,
                               std::make_index_sequence<kDecide>{});
      if (flags_set(lastpeek))
        steps<G, kMode, false, kDecide>(p, rows_out, m_row0, oc0, lane,
                                        std::make_index_sequence<kSteps - kDecide>{});
      else
        steps<G, kMode, true, kDecide>(p, rows_out, m_row0, oc0, lane,
                                       std::make_index_sequence<kSteps - kDecide>{});
    } else {
      steps<G, kMode, true, 0>(p, rows_out, m_row0, oc0, lane,
                               std::make_index_sequence<kSteps>{});
    }
  }
};

// Eight waves: waves 0-3 only copy, waves 4-7 run the MFMAs (16 output
// channels each; wave w and MFMA wave w + 4 share a SIMD).  The copy waves
// come first so that they are launched first and start issuing a little
// earlier.  The copies are issued in chunks, in the order the MFMA waves
// consume them: padded input row r (of the walk's groups), preceded for
// r <= 2 by the filter taps of filter row r (the first row an input row
// needs them at: input row r feeds output rows r - fy), and the bias first
// of all.  Copy wave w copies MFMA wave w's filter halves and plane copies
// j = w + 4i of every row, then its flag copy of the chunk, and never
// waits; the MFMA waves wait for each row's chunk just before reading it:
// the MFMAs start after the first chunk instead of half or all of the
// copies.
//
// The copy waves' schedule, unrolled at compile time (R + 2 padded input
// rows per walk, NG groups per chunk, PW plane copies per row and group
// from this wave): chunk k's copies, then its flag, in order.  Straight-
// line code: a copy wave's scalar work per chunk is a few instructions, so
// its issue keeps up with the copies.  The wave waits for all of its loads
// once, at the end (before it ends, or walks rows itself).
//
// The first kPre chunks' copies go out before the workgroup barrier, their
// flag copies after it.  The barrier only orders the flags: wave 0 zeroes
// them before it, and no flag copy may land, nor an MFMA wave read a flag,
// before they are zero (LDS keeps the previous workgroup's words).  The copy
// waves, launched first, reach the barrier ~0.4 us before the last MFMA
// wave does, and their first copies are in flight meanwhile (28x28x128:
// 6.03 -> 5.84 us per launch, same box; the first two chunks: 5.85).
template <int R, int PW, int NG>
struct CopySchedule {
  static constexpr int kRows = R + 2;
  static constexpr int kChunks = (kGroups / NG) * kRows;
  static constexpr int kPre = 1;
  template <class Issue, size_t... K>
  __device__ static __forceinline__ void copies(Issue &issue, std::index_sequence<K...>) {
    (issue((int(K) / kRows) * NG, int(K) % kRows, PW, NG), ...);
  }
  template <class Signal, size_t... K>
  __device__ static __forceinline__ void flags(Signal &signal, std::index_sequence<K...>) {
    (signal(int(K)), ...);
  }
  template <class Issue, class Signal, size_t... K>
  __device__ static __forceinline__ void steps(Issue &issue, Signal &signal,
                                               std::index_sequence<K...>) {
    constexpr int k0 = kPre;
    ((issue((k0 + int(K)) / kRows * NG, (k0 + int(K)) % kRows, PW, NG), signal(k0 + int(K))),
     ...);
  }
  template <class Issue, class Signal>
  __device__ static __forceinline__ void run(Issue &issue, Signal &signal) {
    copies(issue, std::make_index_sequence<kPre>{});
    flag_barrier();
    flags(signal, std::make_index_sequence<kPre>{});
    steps(issue, signal, std::make_index_sequence<kChunks - kPre>{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
};

// One wave's walk over output rows [OLO, OHI) of its block: output set-up,
// then the walk(s) over the input rows, then the last row's store.
template <int R, int NFR, int NG, bool kQ, int OLO, int OHI>
__device__ __forceinline__ void run_walk(const PassArgs &p, const int8_t *smem, int wave, int lane,
                                         int b, int oy0, int rows_out, int tile_n, v4i qm,
                                         v4i qs) {
  PassState<R, NFR, NG, kQ, OLO, OHI> st;
  st.bias_lds = smem + wave * 256;
  st.planes = smem + kHaloBiasLds;
  st.plane_bytes = p.plane_copies * 1024;
  const int8_t *ring = st.planes + kGroups * p.rows_in * st.plane_bytes;
  st.halves = ring + wave * kHalves * 1024;
  st.flags = lds_addr(ring) + uint32_t(4 * kHalves * 1024);
#pragma unroll
  for (int fx = 0; fx < 3; ++fx)
#pragma unroll
    for (int j = 0; j < NFR; ++j) {
      // Not clamped to the padded row: every offset is then this lane's
      // column-0 offset plus a constant, which the compiler folds into the
      // reads' immediate offsets (one address add per row and group instead
      // of one per read; 28x28x128: 5.91 -> 5.66 us per launch).  Lanes past
      // the row read the next plane or the filter halves after the last one
      // (at most 66 columns x 96 bytes past a plane start, inside the
      // workgroup's LDS); they belong to output columns past out_w, which
      // are never stored.
      const int col = 16 * j + (lane & 15) + fx;
      st.colofs[fx][j] = col * (16 * kUnits) + 16 * (lane >> 4);
    }
  const int m_row0 = (b * p.out_h + oy0) * p.out_w;
  const int oc0 = tile_n + wave * 16 + 4 * (lane >> 4);
  // output element size: 4 (int32) or 1 (requantized int8)
  constexpr uint32_t esize = kQ ? 1u : 4u;
  const void *ybase = kQ ? static_cast<const void *>(p.qy) : static_cast<const void *>(p.y);
  const bool vec = (p.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(ybase) & (4 * esize - 1)) == 0;
  st.yr = make_rsrc(ybase, p.y_bytes);
  st.row_stride = uint32_t(p.out_w) * uint32_t(p.gemm_n) * esize;
#pragma unroll
  for (int j = 0; j < NFR; ++j) {
    const int col = 16 * j + (lane & 15);
    st.voff[j] = col < p.out_w && oc0 < p.gemm_n
                     ? (uint32_t(m_row0 + col) * uint32_t(p.gemm_n) + uint32_t(oc0)) * esize
                     : kOutOfRange;
  }
  if constexpr (kQ) {
    st.qm = qm;
    st.qs = qs;
    bool ok = true;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const RequantOdd o = requant_odd_params(st.qm[e], st.qs[e], p.qzp);
      // channels past N are never stored: they do not hold the wave back
      ok = ok && (oc0 + e >= p.gemm_n || o.ok);
      st.qmo[e] = o.mo;
      st.qk[e] = o.k;
      st.qsh[e] = o.sh;
    }
    st.qodd = __builtin_amdgcn_ballot_w64(!ok) == 0;
  }

  // The walk specialised for the (uniform) store path: each copy holds only
  // its own stores, and the 16-byte path's row steps no longer jump over
  // the element-store code (28x28x128: 5.52 -> 5.41 us per launch).
  auto walks = [&](auto mode) {
    constexpr int M = decltype(mode)::value;
    st.template walk<0, M>(p, rows_out, m_row0, oc0, lane);
    if constexpr (NG == 1) st.template walk<1, M>(p, rows_out, m_row0, oc0, lane);
    if constexpr (!(M == kStoreFull && NG == 2 && kQ))
      st.template store_row<OHI - 1>(p, M != kStoreElem, rows_out, m_row0, oc0, lane);
  };
  if (vec && rows_out >= OHI && (!kQ || st.qodd))
    walks(std::integral_constant<int, kStoreFull>{});
  else if (vec)
    walks(std::integral_constant<int, kStoreVec>{});
  else
    walks(std::integral_constant<int, kStoreElem>{});
}

// The MFMA waves walk every output row of the block.  (The requantizing
// instances once let the copy waves walk the block's last rows once their
// copies had landed, so that a second wave per SIMD shared the epilogue's
// VALU work: 8.97 -> 8.39 us per launch on 28x28x128 with int8 output; with
// the kernel arguments preloaded it measured 7.64-8.04 against 6.92-7.09 us
// without, same box, and was removed.)

// The kernel's leading arguments arrive preloaded in SGPRs (this file is
// built with -amdgpu-kernarg-preload-count=7: seven arguments, ten words):
// the base pointers of input, filter and bias and four words of the
// layer's geometry (n; h | wd << 16;
// pad_h | pad_w << 8 | blocks << 16, the row blocks per image; the output
// channels), which is everything the copy waves need to issue their
// copies.  The rest of the arguments (PassArgs) are loaded from the
// kernel-argument segment as usual, a cold scalar round trip (~0.3 us after
// a launch enqueued on a stream) that the MFMA waves take while the first
// chunk lands.  The grid is (channel tiles, row blocks, images).
template <int R, int NFR, int NG, bool kQ>
__global__ __launch_bounds__(2 * kThreads, 1) void rowpass_kernel(
    const int8_t *x_pre, const int8_t *w_pre, const int32_t *bias_pre, uint32_t n_pre,
    uint32_t hw_pre, uint32_t pads_pre, uint32_t gemm_n_pre, PassArgs p_arg) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const PassArgs &p = p_arg;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool copier = wave_id < 4;
  // the MFMA wave this wave is, 0..3 (or copies the filter halves and bias for)
  const int wave = wave_id & 3;

  // geometry from the preloaded words (c == 128, 3x3, stride 1, dilation 1);
  // bit 31 of n_pre: the grid groups images by XCD (below)
  const bool by_xcd = (n_pre >> 31) != 0;
  const int n = int(n_pre & 0xffffu);
  const int h = int(hw_pre & 0xffffu), wd = int(hw_pre >> 16);
  const int pad_h = int(pads_pre & 0xffu), pad_w = int((pads_pre >> 8) & 0xffu);
  const int blocks = int(pads_pre >> 16);
  const int gemm_n = int(gemm_n_pre);
  const int hp = h + 2 * pad_h;
  const int out_h = hp - 2;
  const int plane_copies = ((wd + 2 * pad_w) * kUnits + 63) / 64;
  constexpr int kRowsIn = R + 2;
  constexpr int kGemmK = 9 * 64 * kGroups;

  // grid: (channel tiles, row blocks, images), or with by_xcd (n % 8 == 0)
  // (8 x channel tiles, row blocks, images / 8) with blockIdx.x = x + 8 tn
  // and image 8 blockIdx.z + x.  Workgroup i of a launch runs on XCD i mod 8,
  // and i mod 8 = blockIdx.x mod 8 = x: every workgroup of an image (both
  // channel tiles, every row block) runs on one XCD, whose L2 then fetches
  // the image's rows from HBM once for all of them.
  const int tn = by_xcd ? int(blockIdx.x >> 3) : int(blockIdx.x);
  const int q = int(blockIdx.y);
  const int b = by_xcd ? int(8 * blockIdx.z + (blockIdx.x & 7)) : int(blockIdx.z);
  // out_h < 2^16 and q < blocks <= out_h: the products fit in 32 bits
  const int oy0 = int(uint32_t(q * out_h) / uint32_t(blocks));
  const int rows_out = int(uint32_t((q + 1) * out_h) / uint32_t(blocks)) - oy0;  // <= R
  const int tile_n = tn * 64;

  // LDS: [bias, 256 B per wave][planes: group 0 rows, group 1 rows]
  //      [filter halves: 18 KB per wave][chunk flags: 16 B per chunk]
  const int8_t *bias_lds = smem + wave * 256;
  const int8_t *planes = smem + kHaloBiasLds;
  const int plane_bytes = plane_copies * 1024;
  const int8_t *ring = planes + kGroups * kRowsIn * plane_bytes;
  const int8_t *halves = ring + wave * kHalves * 1024;
  const uint32_t flags = lds_addr(ring) + uint32_t(4 * kHalves * 1024);
  constexpr int nchunks = (kGroups / NG) * kRowsIn;

  // kQ: the multipliers and shifts of this lane's four output channels,
  // loaded by the MFMA waves first thing (the walk needs them before its
  // first row).  Channels past N read as zero (their values are never
  // stored).  Staged through LDS with the bias instead (16 active lanes per
  // copy wave) they measured 7.43-7.55 against 7.16-7.18 us per launch
  // (28x28x128, int8 output, same box).
  v4i qm{0, 0, 0, 0}, qs{0, 0, 0, 0};
  if constexpr (kQ) {
    if (!copier) {
      const int oc0 = tile_n + wave * 16 + 4 * (lane >> 4);
      const auto mr = make_rsrc(p.qmult, uint32_t(gemm_n) * 4u);
      const auto sr = make_rsrc(p.qshift, uint32_t(gemm_n) * 4u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qm[e] = __builtin_amdgcn_raw_buffer_load_b32(mr, uint32_t(oc0 + e) * 4u, 0, 0);
        qs[e] = __builtin_amdgcn_raw_buffer_load_b32(sr, uint32_t(oc0 + e) * 4u, 0, 0);
      }
    }
  }

  if (wave_id == 0 && lane < nchunks) {
    // every flag starts at zero before any copy can land
    asm volatile("ds_write_b128 %0, %1" ::"v"(flags + 16u * uint32_t(lane)), "v"(v4i{0, 0, 0, 0})
                 : "memory");
  }

  if (copier) {
    const v4u xd = make_desc(x_pre, uint32_t(n) * uint32_t(h) * uint32_t(wd) * uint32_t(64 * kGroups));
    const v4u wd_desc = make_desc(w_pre, uint32_t(gemm_n) * uint32_t(kGemmK));
    const uint32_t planes_lds = lds_addr(planes);
    // filter halves for MFMA wave `wave`: lane -> filter row 16*wave +
    // lane/4 and 16-byte chunk lane%4, holding the chunk swz64 puts there
    const int frow = lane >> 2;
    const int fchunk = swz64_chunk(frow, lane & 3);
    const int oc_copy = tile_n + wave * 16 + frow;
    const uint32_t fbase = oc_copy < gemm_n
                               ? uint32_t(oc_copy) * uint32_t(kGemmK) + uint32_t(16 * fchunk)
                               : kOutOfRange;
    const uint32_t halves_lds = lds_addr(halves);
    // Chunk (groups g0 .. g0 + ng - 1, row r): the bias (first chunk), the
    // filter taps of filter row r (r <= 2) and plane copies j = wave + 4i
    // of padded input row r.  Copy j covers units [64j, 64j + 64) of the
    // plane; unit u of pixel pix is slot pix*kUnits + u (u >= 4: padding,
    // left out of range -> zeros).
    auto issue_chunk = [&](int g0, int r, int pw, int ng) {
      if (g0 == 0 && r == 0) stage_bias<1>(bias_pre, gemm_n, tile_n + wave * 16, bias_lds, lane);
      for (int g = g0; g < g0 + ng; ++g) {
        if (r <= 2) {
#pragma unroll
          for (int fx = 0; fx < 3; ++fx) {
            const int t = 3 * r + fx;
            lds_copy16(wd_desc, halves_lds + uint32_t((g * kTaps + t) * 1024),
                       fbase + uint32_t(t * 128 + g * 64));
          }
        }
      }
      // padded row oy0 + r of image b; the rows past the image (a block
      // shorter than R at the bottom) fall into the next image's top rows
      // (oy0 + r < 2 hp), which are read but feed no stored output
      const int pr = oy0 + r;
      const int bb = b + (pr >= hp ? 1 : 0);
      const int iy = pr - (pr >= hp ? hp : 0) - pad_h;
      const bool row_ok = bb < n && unsigned(iy) < unsigned(h);
      // modulo 2^32: exact wherever it is used (the sums below are in [0, 2^31))
      const uint32_t row_off = uint32_t((bb * h + iy) * wd - pad_w) * uint32_t(64 * kGroups);
      for (int g = g0; g < g0 + ng; ++g) {
        for (int i = 0; i < pw; ++i) {
          const int j = wave + 4 * i;
          const int slot = j * 64 + lane;
          const int pix = slot / kUnits;
          const int u = slot - pix * kUnits;
          const bool ok = row_ok && u < 4 && unsigned(pix - pad_w) < unsigned(wd);
          const uint32_t off =
              ok ? row_off + uint32_t(64 * g + pix * 64 * kGroups + 16 * u) : kOutOfRange;
          lds_copy16(xd, planes_lds + uint32_t((g * kRowsIn + r) * plane_bytes + j * 1024), off);
        }
      }
    };
    // the flag copy of chunk c: lane 0 copies the word holding 1 into this
    // wave's flag word of the chunk (the other lanes are inactive)
    const v4u one = make_desc(g_flag_one, 16u);
    auto signal = [&](int c) {
      if (lane == 0) lds_copy4(one, flags + 16u * uint32_t(c) + 4u * uint32_t(wave), 0u);
    };
    // plane copies per row and group this wave issues: j = wave, wave + 4;
    // each schedule passes the workgroup barrier once (flag_barrier)
    const int pw = plane_copies > wave ? (plane_copies - wave + 3) / 4 : 0;
    if (pw == 0) CopySchedule<R, 0, NG>::run(issue_chunk, signal);
    else if (pw == 1) CopySchedule<R, 1, NG>::run(issue_chunk, signal);
    else CopySchedule<R, 2, NG>::run(issue_chunk, signal);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // the copy wave's work is done
    return;
  }
  // the remaining arguments, in one batch, while the first chunk lands
  pin_sgprs(p);
  // The MFMA waves issue ahead of the copy waves that share their SIMDs
  // (wave priority, not stream priority): 28x28x128, 5.47-5.48 -> 5.38-5.43
  // us per launch at K = 20, same box.
  __builtin_amdgcn_s_setprio(3);
  flag_barrier();
  run_walk<R, NFR, NG, kQ, 0, R>(p, smem, wave, lane, b, oy0, rows_out, tile_n, qm, qs);
}


// The preloaded leading arguments of rowpass_kernel.
struct PreArgs {
  const int8_t *x;
  const int8_t *w;
  const int32_t *bias;
  uint32_t n, hw, pads, gemm_n;
};

template <int R, int NFR, bool kQ>
int launch_q(const PreArgs &a, const PassArgs &h, dim3 grid, size_t lds, hipStream_t s) {
  auto kern = rowpass_kernel<R, NFR, walk_groups(NFR), kQ>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(lds));
    if (e != hipSuccess) {
      set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
  }
  I8_LAUNCH(kern, grid, dim3(2 * kThreads), lds, s, a.x, a.w, a.bias, a.n, a.hw, a.pads,
                     a.gemm_n, h);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("row kernel with copy waves, launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

template <int R, int NFR>
int launch_t(const PreArgs &a, const PassArgs &h, dim3 grid, size_t lds, hipStream_t s,
             bool requant) {
  return requant ? launch_q<R, NFR, true>(a, h, grid, lds, s)
                 : launch_q<R, NFR, false>(a, h, grid, lds, s);
}

}  // namespace

// Instances: R = 1..8 output rows per block with NFR = 1 or 2 fragments per
// output row (out_w <= 16, 32), R = 1..4 with NFR = 4 (out_w <= 64): an MFMA
// wave has 256 VGPRs when the workgroup runs eight waves, and R x NFR
// accumulators beyond 32 fragments would spill.
int rowpass_nfr(int out_w) {
  const int f = (out_w + 15) / 16;
  return f <= 2 ? f : (f <= 4 ? 4 : 0);
}

int rowpass_max_rows(int nfr) { return nfr == 4 ? 4 : 8; }

size_t rowpass_lds_bytes(int wp, int rows) {
  const size_t plane_copies = (size_t(wp) * kUnits + 63) / 64;
  return size_t(kHaloBiasLds) + size_t(kGroups) * size_t(rows + 2) * plane_copies * 1024 +
         size_t(4) * kHalves * 1024 + 512;  // + chunk flags (16 B x 2 x up to 10 rows)
}

int launch_rowpass(const ConvArgs &a, const PatchPlan &p, void *stream, const RequantArgs *q) {
  const int R = p.rows - 2;
  const int nfr = rowpass_nfr(a.out_w);
  const int wp = a.wd + 2 * a.pad_w;
  const size_t lds = rowpass_lds_bytes(wp, R);
  if (a.r != 3 || a.s != 3 || a.stride_h != 1 || a.stride_w != 1 || a.dil_h != 1 ||
      a.dil_w != 1 || a.c != 64 * kGroups || R < 1 || nfr == 0 || R > rowpass_max_rows(nfr) ||
      p.bn != 64 ||
      lds > size_t(kLdsBudget) || p.ranges < 1 || wp != a.out_w + 2 ||
      (wp * kUnits + 63) / 64 > 8 ||
      int64_t(a.out_h) > int64_t(p.ranges) * R ||
      int64_t(a.gemm_m) * a.gemm_n * 4 > int64_t(INT32_MAX)) {
    set_error("row plan (copy waves) out of range");
    return I8CONV_BAD_ARGUMENT;
  }
  if (a.h >= 65536 || a.wd >= 65536 || a.pad_h >= 256 || a.pad_w >= 256 || p.ranges >= 65536 ||
      a.n >= 65536 || a.pad_h < 0 || a.pad_w < 0) {
    set_error("row plan (copy waves): geometry beyond the packed kernel arguments");
    return I8CONV_BAD_ARGUMENT;
  }
  PreArgs pre;
  pre.x = a.x;
  pre.w = a.w;
  pre.bias = a.bias;
  // n % 8 == 0: the grid groups each image's workgroups on one XCD
  const bool by_xcd = a.n % 8 == 0;
  pre.n = uint32_t(a.n) | (by_xcd ? 0x80000000u : 0u);
  pre.hw = uint32_t(a.h) | uint32_t(a.wd) << 16;
  pre.pads = uint32_t(a.pad_h) | uint32_t(a.pad_w) << 8 | uint32_t(p.ranges) << 16;
  pre.gemm_n = uint32_t(a.gemm_n);
  PassArgs h{};
  h.y = a.y;
  h.y_bytes = uint32_t(int64_t(a.gemm_m) * a.gemm_n * (q ? 1 : 4));
  if (q) {
    h.qmult = q->mult;
    h.qshift = q->shift;
    h.qy = q->y;
    h.qzp = q->zero_point;
  }
  h.out_h = a.out_h;
  h.out_w = a.out_w;
  h.gemm_n = a.gemm_n;
  h.plane_copies = (wp * kUnits + 63) / 64;
  h.rows_in = R + 2;
  h.spin_limit = wait_spin_limit();
  const dim3 grid = by_xcd ? dim3(8 * unsigned(p.tiles_n), unsigned(p.ranges), unsigned(a.n / 8))
                           : dim3(unsigned(p.tiles_n), unsigned(p.ranges), unsigned(a.n));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define I8_PASS_CASE(RR)                                                         \
  if (R == RR) {                                                                 \
    if (nfr == 1) return launch_t<RR, 1>(pre, h, grid, lds, s, q != nullptr);    \
    if (nfr == 2) return launch_t<RR, 2>(pre, h, grid, lds, s, q != nullptr);    \
    if constexpr (RR <= 4) return launch_t<RR, 4>(pre, h, grid, lds, s, q != nullptr); \
  }
  I8_PASS_CASE(1) I8_PASS_CASE(2) I8_PASS_CASE(3) I8_PASS_CASE(4)
  I8_PASS_CASE(5) I8_PASS_CASE(6) I8_PASS_CASE(7) I8_PASS_CASE(8)
#undef I8_PASS_CASE
  set_error("no row-kernel (copy waves) instance for this plan");
  return I8CONV_BAD_ARGUMENT;
}

int rowpass_wait_expired(int *expired) {
  void *word = nullptr;
  hipError_t e = hipGetSymbolAddress(&word, HIP_SYMBOL(g_wait_expired));
  if (e != hipSuccess) {
    set_error(std::string("hipGetSymbolAddress(g_wait_expired): ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  e = hipDeviceSynchronize();
  unsigned int value = 0;
  if (e == hipSuccess) e = hipMemcpy(&value, word, sizeof(value), hipMemcpyDeviceToHost);
  if (e == hipSuccess && value != 0) e = hipMemset(word, 0, sizeof(value));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    set_error(std::string("reading g_wait_expired: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  *expired = value != 0 ? 1 : 0;
  return I8CONV_OK;
}

}  // namespace i8conv
