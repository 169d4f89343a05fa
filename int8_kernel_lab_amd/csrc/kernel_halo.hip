// Halo kernel on gfx950 INT8 MFMA: flattened pixel ranges, LDS-resident
// input rows, filter held in registers, output stored pass by pass.
//
// Work split.  The M = n*out_h*out_w output pixels, in NHW order, are cut
// into 16-pixel MFMA fragments and every workgroup takes an equal,
// contiguous range of fragments (and one 64*FN-channel slice of K).  Ranges
// ignore row and image boundaries, so all compute units get the same work
// and no fragment is partly empty except the very last one.
//
// Input.  Coordinates are taken in the zero-padded image: padded row
// py = oy*stride_h + fy*dil_h, padded column px = ox*stride_w + fx*dil_w,
// and "virtual row" vr = batch * (h + 2*pad_h) + py numbers the padded rows
// of all images consecutively.  A range needs the virtual rows from its
// first pixel's tap-0 row to its last pixel's last-tap row; those rows (all
// w + 2*pad_w columns, every 64-channel group) are copied into LDS once by
// the buffer unit (1 KB per wave instruction).  Copies never straddle rows,
// so everything about the row (image, input row, padding) is wave-uniform
// scalar arithmetic and a lane only finds its pixel in the row.  Padding
// rows/columns and rows between images come back as zeros because their
// buffer offsets are out of range.  LDS layout: a row is [pixel][c + 16
// bytes] (all channels of a pixel, then 16 bytes of padding), rows
// row_bytes apart (HaloRowLayout).  The pixel pitch is an odd number of
// 16-byte units (c % 32 == 0), so the 16 pixels of an MFMA fragment hit 16
// different 16-byte bank groups of the 64 x 4-byte LDS banks, and a fragment
// address is linear in the tap offset: the k loop spends one add per
// fragment per step on addressing.
//
// Issue cost.  A wave64 VALU instruction takes at least 4 cycles and the
// 32-bit multiplies 16, so per-copy address arithmetic is kept to a few
// instructions: row math is scalar, filter copy offsets are computed once
// per lane and advanced by a scalar per chunk, and every kernel argument is
// loaded into SGPRs in one batch before the first copy (otherwise the
// argument loads trail the copies, one cold scalar round trip each).
//
// Filter.  Each of the 4 waves owns 16*FN output channels and keeps its
// whole filter slice (16*FN x r*s*c bytes, kSteps 64-byte k-steps) in VGPRs
// for the life of the workgroup.  A fragment read straight from KRSC touches
// 16 rows x 64 bytes (16 half-used cache lines) and streams at a third of
// the rate of whole-line reads, so the slice is fetched with whole-line
// copies (8 rows x 128 bytes per instruction) into an LDS ring of up to 8
// slots (swz128 layout) and picked out of LDS in fragment order.  Each wave
// copies its own rows, so the ring needs no barriers.  The first pass
// consumes each 128-byte chunk as soon as it lands, so the filter fetch
// overlaps that pass's MFMAs.
//
// Compute.  Fragments run up to four at a time through all k-steps (B
// fragments read from LDS one step ahead), then get the bias and are stored;
// the next pass computes while those stores drain.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "halo_common.hpp"

namespace i8conv {
namespace {


constexpr int kPassFrags = 4;

struct HaloArgs {
  int hp;            // padded rows per image: h + 2*pad_h
  int pitch;         // LDS bytes per input pixel: c + 16
  int units;         // 16-byte units per pixel in LDS: c / 16 + 1
  int row_copies;    // 1 KB copies per padded input row
  int row_bytes;     // LDS bytes between consecutive rows
  int input_bytes;   // LDS bytes of the input rows (rows * row_bytes)
  int ranges;        // pixel ranges per channel slice
  int ring;          // filter staging slots in LDS (1..kHaloRing)
  int total_frags;   // ceil(M / 16)
  int tiles_n;
  FastDiv div_ohw, div_ow, div_hp, div_units, div_row_copies;
};

// Virtual padded row of output pixel m's tap-0 row; also returns its column.
__device__ __forceinline__ int pixel_vrow(const ConvArgs &a, const HaloArgs &p, int m, int &ox) {
  const int b = int(fast_div(uint32_t(m), p.div_ohw));
  const int rem = m - b * a.out_h * a.out_w;
  const int oy = int(fast_div(uint32_t(rem), p.div_ow));
  ox = rem - oy * a.out_w;
  return b * p.hp + oy * a.stride_h;
}

// LDS byte offset of k-step t (64 k-bytes): its tap's pixel offset plus its
// 64-channel group inside the pixel.  Wave-uniform.
__device__ __forceinline__ int step_offset(const ConvArgs &a, const HaloArgs &p, int t) {
  const int k0 = t * 64;
  const int tap = int(fast_div(uint32_t(k0), a.div_c));
  const int c0 = k0 - tap * a.c;
  const int fy = int(fast_div(uint32_t(tap), a.div_s));
  const int fx = tap - fy * a.s;
  return fy * a.dil_h * p.row_bytes + fx * a.dil_w * p.pitch + c0;
}

// NF fragments starting at f0 through all k-steps, then bias + stores.  The
// staging pass (kStage) also pulls the filter out of the ring, chunk by chunk,
// just before the steps that need it.
template <int FN, int kSteps, int NF, bool kStage>
__device__ __forceinline__ void halo_pass(const ConvArgs &a, const HaloArgs &p,
                                          const int8_t *smem, const FilterRing<FN, kSteps> &ring,
                                          v4i (&wf)[kSteps][FN], const int8_t *bias_lds,
                                          const int (&soff)[kSteps], int f0, int vr0, int m_first,
                                          int tile_n, int wave, int lane) {
  int vaddr[NF];
  int mpx[NF];
#pragma unroll
  for (int j = 0; j < NF; ++j) {
    int m = (f0 + j) * 16 + (lane & 15);
    mpx[j] = m < a.gemm_m ? m : -1;
    if (mpx[j] < 0) m = m_first;  // past the last pixel: computed, never stored
    int ox;
    const int vr = pixel_vrow(a, p, m, ox);
    vaddr[j] = (vr - vr0) * p.row_bytes + ox * a.stride_w * p.pitch + 16 * (lane >> 4);
  }
  v4i acc[NF][FN];
#pragma unroll
  for (int j = 0; j < NF; ++j)
#pragma unroll
    for (int i = 0; i < FN; ++i) acc[j][i] = v4i{0, 0, 0, 0};

  // The staging pass takes chunk 0 before its first B reads: that wait and
  // barrier are also what make every wave's input-row copies visible.
  if (kStage) ring.take(0, wf);
  v4i bcur[NF], bnxt[NF];
#pragma unroll
  for (int j = 0; j < NF; ++j) bcur[j] = *reinterpret_cast<const v4i *>(smem + vaddr[j] + soff[0]);
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    if (kStage && t > 0 && (t & 1) == 0) ring.take(t >> 1, wf);
    if (t + 1 < kSteps) {  // next step's B fragments, one step ahead of use
#pragma unroll
      for (int j = 0; j < NF; ++j)
        bnxt[j] = *reinterpret_cast<const v4i *>(smem + vaddr[j] + soff[t + 1]);
    }
    // keep those reads ahead of this step's MFMAs (the scheduler would
    // otherwise sink each read next to its use and expose the LDS latency)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
      for (int i = 0; i < FN; ++i) acc[j][i] = mfma16(wf[t][i], bcur[j], acc[j][i]);
    if (t + 1 < kSteps) {
#pragma unroll
      for (int j = 0; j < NF; ++j) bcur[j] = bnxt[j];
    }
  }

  // this wave's bias, staged in LDS by the first copy (see the prologue)
  v4i bv[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i)
    bv[i] = *reinterpret_cast<const v4i *>(bias_lds + (i * 16 + 4 * (lane >> 4)) * 4);
  // output window: the pass's NF fragments of 16 pixels from pixel 16*f0
  const OutWindow ow = out_window(a.y, a.gemm_m, a.gemm_n, int64_t(f0) * 16, NF * 16);
  const bool vec = (a.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && ow.ok;
#pragma unroll
  for (int j = 0; j < NF; ++j) {
    if (mpx[j] < 0) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int oc0 = tile_n + wave * 16 * FN + i * 16 + 4 * (lane >> 4);
      const v4i v = add_wrap4(acc[j][i], bv[i]);
      if (vec) {
        if (oc0 < a.gemm_n)
          store_out4<kStoreStream>(ow.r, (uint32_t(mpx[j] - f0 * 16) * uint32_t(a.gemm_n) + uint32_t(oc0)) * 4u, v);
      } else {
        int32_t *dst = a.y + size_t(mpx[j]) * size_t(a.gemm_n) + oc0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (oc0 + e < a.gemm_n) store_out1(dst + e, v[e]);
      }
    }
  }
}

template <int FN, int kSteps>
__global__ __launch_bounds__(kThreads, 1) void halo_kernel(ConvArgs a_arg, HaloArgs p_arg) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const ConvArgs a = a_arg;
  const HaloArgs p = p_arg;
  pin_sgprs(a);
  pin_sgprs(p);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int tn = int(blockIdx.x) % p.tiles_n;
  const int range = int(blockIdx.x) / p.tiles_n;
  const int f_begin = int((int64_t(range) * p.total_frags) / p.ranges);
  const int f_end = int((int64_t(range + 1) * p.total_frags) / p.ranges);
  const int tile_n = tn * 64 * FN;

  // ---- 0. bias of this wave's 16*FN channels -> LDS [wave * 256, +256) ----
  // The first copy of every wave, so each later wait on the copy stream also
  // covers it (its register form would need a compiler-inserted wait, which
  // cannot see these copies and so waits for everything, stores included).
  const int8_t *bias_lds = smem + wave * 256;
  stage_bias<FN>(a.bias, a.gemm_n, tile_n + wave * 16 * FN, bias_lds, lane);

  const v4u xd = make_desc(a.x, a.x_bytes);
  const int8_t *rows = smem + kHaloBiasLds;
  const uint32_t lds0 = lds_addr(rows);
  int ox_unused;
  const int m_first = f_begin * 16;
  const int m_last = min(f_end * 16, a.gemm_m) - 1;
  const int vr0 = __builtin_amdgcn_readfirstlane(pixel_vrow(a, p, m_first, ox_unused));
  const int vr1 = __builtin_amdgcn_readfirstlane(pixel_vrow(a, p, m_last, ox_unused)) +
                  (a.r - 1) * a.dil_h;

  // ---- 1. input rows -> LDS ------------------------------------------------
  copy_input_rows(xd, lds0, vr0, vr1 - vr0 + 1, wave, lane, p.row_copies, p.div_row_copies,
                  p.row_bytes, p.div_hp, p.hp, p.units, p.div_units, a.n, a.h, a.wd, a.c,
                  a.pad_h, a.pad_w);

  // ---- 2. start the filter ring --------------------------------------------
  FilterRing<FN, kSteps> ring;
  ring.wd = make_desc(a.w, a.w_bytes);
  ring.ptr = rows + p.input_bytes;
  ring.lds = lds_addr(ring.ptr);
  ring.slots = p.ring;
  ring.cur = 0;
  ring.wave = wave;
  ring.lane = lane;
  ring.init(tile_n, a.gemm_n, a.gemm_k);
  for (int c = 0; c < ring.slots && c < ring.kChunks; ++c) ring.issue(c, c);

  // ---- 3. passes of up to four fragments -------------------------------------
  int soff[kSteps];
#pragma unroll
  for (int t = 0; t < kSteps; ++t) soff[t] = step_offset(a, p, t);
  v4i wf[kSteps][FN];
  int f0 = f_begin;
  {
    const int nf = min(kPassFrags, f_end - f0);
    switch (nf) {
      case 4: halo_pass<FN, kSteps, 4, true>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
      case 3: halo_pass<FN, kSteps, 3, true>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
      case 2: halo_pass<FN, kSteps, 2, true>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
      default: halo_pass<FN, kSteps, 1, true>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
    }
    f0 += nf;
  }
  for (; f0 < f_end; f0 += kPassFrags) {
    switch (min(kPassFrags, f_end - f0)) {
      case 4: halo_pass<FN, kSteps, 4, false>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
      case 3: halo_pass<FN, kSteps, 3, false>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
      case 2: halo_pass<FN, kSteps, 2, false>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
      default: halo_pass<FN, kSteps, 1, false>(a, p, rows, ring, wf, bias_lds, soff, f0, vr0, m_first, tile_n, wave, lane); break;
    }
  }
}

template <int FN, int kSteps>
int launch_t(const ConvArgs &a, const HaloArgs &h, size_t blocks, size_t lds, hipStream_t s) {
  auto kern = halo_kernel<FN, kSteps>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(lds));
    if (e != hipSuccess) {
      set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
  }
  I8_LAUNCH(kern, dim3(unsigned(blocks)), dim3(kThreads), lds, s, a, h);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("halo kernel launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

bool halo_instance_exists(int fn, int steps) {
  return (fn == 1 && (steps == 9 || steps == 18 || steps == 36)) ||
         (fn == 2 && (steps == 9 || steps == 18));
}

int launch_halo_resident(const ConvArgs &a, const PatchPlan &p, void *stream) {
  const HaloRowLayout row = halo_row_layout(a.wd + 2 * a.pad_w, a.c, kHaloPadUnits);
  const int fn = p.bn / 64;
  const size_t lds = size_t(kHaloBiasLds) + size_t(p.rows) * size_t(row.row_bytes) +
                     size_t(p.ring) * halo_ring_slot_bytes(fn);
  HaloArgs h{};
  h.hp = a.h + 2 * a.pad_h;
  h.pitch = a.c + 16;
  h.units = int(row.units);
  h.row_copies = int(row.row_copies);
  h.row_bytes = int(std::min<int64_t>(row.row_bytes, kLdsBudget));
  h.input_bytes = int(std::min<size_t>(size_t(p.rows) * size_t(h.row_bytes), kLdsBudget));
  h.ranges = p.ranges;
  h.ring = p.ring;
  h.total_frags = (a.gemm_m + 15) / 16;
  h.tiles_n = p.tiles_n;
  h.div_ohw = make_fastdiv(uint32_t(a.out_h * a.out_w));
  h.div_ow = make_fastdiv(uint32_t(a.out_w));
  h.div_hp = make_fastdiv(uint32_t(h.hp));
  h.div_units = make_fastdiv(uint32_t(h.units));
  h.div_row_copies = make_fastdiv(uint32_t(h.row_copies));
  const size_t blocks = size_t(p.ranges) * p.tiles_n;
  const int steps = a.gemm_k / 64;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.c % 64 != 0 || !halo_instance_exists(fn, steps) || lds > size_t(kLdsBudget) ||
      p.rows < 1 || p.ranges < 1 || p.ring < 1 || p.ring > kHaloRing) {
    set_error("halo plan out of range");
    return I8CONV_BAD_ARGUMENT;
  }
  if (fn == 1 && steps == 9) return launch_t<1, 9>(a, h, blocks, lds, s);
  if (fn == 1 && steps == 18) return launch_t<1, 18>(a, h, blocks, lds, s);
  if (fn == 1 && steps == 36) return launch_t<1, 36>(a, h, blocks, lds, s);
  if (fn == 2 && steps == 9) return launch_t<2, 9>(a, h, blocks, lds, s);
  if (fn == 2 && steps == 18) return launch_t<2, 18>(a, h, blocks, lds, s);
  set_error("no halo instance for this plan");
  return I8CONV_BAD_ARGUMENT;
}

}  // namespace i8conv
