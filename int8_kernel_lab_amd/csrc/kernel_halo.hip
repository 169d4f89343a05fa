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
// the buffer unit (buffer_load_dwordx4 ... lds, 1 KB per wave instruction).
// Padding rows/columns and rows between images come back as zeros because
// their buffer offsets are out of range.  LDS layout: [group][row][col][64 B]
// with chunk j of pixel slot p at 16*(j ^ ((p >> 2) & 3)) (swz64).
//
// Filter.  Each of the 4 waves owns 16*FN output channels and loads its
// whole filter slice (16*FN x r*s*c bytes, kSteps 64-byte k-steps) into
// VGPRs in k order; the k loop consumes step t as soon as its registers
// land (the loads complete in issue order), so the fetch overlaps the first
// pass's MFMAs.
//
// Compute.  Fragments run four at a time through all k-steps (B fragments
// read from LDS one step ahead), then get the bias and are stored; the next
// pass computes while those stores drain.
#include <hip/hip_runtime.h>

#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i add_wrap(v4i a, v4i b) {
  return __builtin_bit_cast(v4i, __builtin_bit_cast(v4u, a) +
                                     __builtin_bit_cast(v4u, b));
}

constexpr int kPassFrags = 4;

struct HaloArgs {
  int wp;            // padded row width: w + 2*pad_w
  int hp;            // padded rows per image: h + 2*pad_h
  int groups;        // c / 64
  int group_bytes;   // LDS bytes per channel group (whole 4 KB copy rounds)
  int copies;        // buffer->LDS instructions per wave per group
  int ranges;        // pixel ranges per channel slice
  int total_frags;   // ceil(M / 16)
  int tiles_n;
  FastDiv div_ohw, div_ow, div_wp, div_hp;
};

// k-step t (64 k-bytes) -> LDS pixel-slot offset of its tap and the byte
// offset of its channel group.
__device__ __forceinline__ void step_geometry(const ConvArgs &a, const HaloArgs &p,
                                              int t, int &delta, int &gbase) {
  const int k0 = t * 64;
  const int tap = int(fast_div(uint32_t(k0), a.div_c));
  const int g = (k0 - tap * a.c) >> 6;
  const int fy = int(fast_div(uint32_t(tap), a.div_s));
  const int fx = tap - fy * a.s;
  delta = fy * a.dil_h * p.wp + fx * a.dil_w;
  gbase = g * p.group_bytes;
}

// Virtual padded row of output pixel m's tap-0 row; also returns its column.
__device__ __forceinline__ int pixel_vrow(const ConvArgs &a, const HaloArgs &p, int m, int &ox) {
  const int b = int(fast_div(uint32_t(m), p.div_ohw));
  const int rem = m - b * a.out_h * a.out_w;
  const int oy = int(fast_div(uint32_t(rem), p.div_ow));
  ox = rem - oy * a.out_w;
  return b * p.hp + oy * a.stride_h;
}

// NF fragments starting at f0 through all k-steps, then bias + stores.
template <int FN, int kSteps, int NF>
__device__ __forceinline__ void halo_pass(const ConvArgs &a, const HaloArgs &p,
                                          const int8_t *smem, const v4i (&wf)[kSteps][FN],
                                          const v4i (&bv)[FN], int f0, int vr0, int m_first,
                                          int tile_n, int wave, int lane) {
  const int chunk = lane >> 4;
  int lbase[NF];
  int mpx[NF];
#pragma unroll
  for (int j = 0; j < NF; ++j) {
    int m = (f0 + j) * 16 + (lane & 15);
    mpx[j] = m < a.gemm_m ? m : -1;
    if (mpx[j] < 0) m = m_first;  // past the last pixel: computed, never stored
    int ox;
    const int vr = pixel_vrow(a, p, m, ox);
    lbase[j] = (vr - vr0) * p.wp + ox * a.stride_w;
  }
  v4i acc[NF][FN];
#pragma unroll
  for (int j = 0; j < NF; ++j)
#pragma unroll
    for (int i = 0; i < FN; ++i) acc[j][i] = v4i{0, 0, 0, 0};

  v4i bcur[NF], bnxt[NF];
  int delta, gbase;
  step_geometry(a, p, 0, delta, gbase);
#pragma unroll
  for (int j = 0; j < NF; ++j)
    bcur[j] = *reinterpret_cast<const v4i *>(smem + gbase + swz64(lbase[j] + delta, chunk));
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    if (t + 1 < kSteps) {  // next step's B fragments, one step ahead of use
      step_geometry(a, p, t + 1, delta, gbase);
#pragma unroll
      for (int j = 0; j < NF; ++j)
        bnxt[j] = *reinterpret_cast<const v4i *>(smem + gbase + swz64(lbase[j] + delta, chunk));
    }
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
      for (int i = 0; i < FN; ++i) acc[j][i] = mfma16(wf[t][i], bcur[j], acc[j][i]);
    if (t + 1 < kSteps) {
#pragma unroll
      for (int j = 0; j < NF; ++j) bcur[j] = bnxt[j];
    }
  }

  const bool vec = (a.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
#pragma unroll
  for (int j = 0; j < NF; ++j) {
    if (mpx[j] < 0) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int oc0 = tile_n + wave * 16 * FN + i * 16 + 4 * (lane >> 4);
      const v4i v = add_wrap(acc[j][i], bv[i]);
      int32_t *dst = a.y + size_t(mpx[j]) * size_t(a.gemm_n) + oc0;
      if (vec) {
        if (oc0 < a.gemm_n) *reinterpret_cast<v4i *>(dst) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (oc0 + e < a.gemm_n) dst[e] = v[e];
      }
    }
  }
}

template <int FN, int kSteps>
__global__ __launch_bounds__(kThreads, 1) void halo_kernel(ConvArgs a, HaloArgs p) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int tn = int(blockIdx.x) % p.tiles_n;
  const int range = int(blockIdx.x) / p.tiles_n;
  const int f_begin = int((int64_t(range) * p.total_frags) / p.ranges);
  const int f_end = int((int64_t(range + 1) * p.total_frags) / p.ranges);
  const int tile_n = tn * 64 * FN;

  const auto xr = make_rsrc(a.x, a.x_bytes);
  const auto wr = make_rsrc(a.w, a.w_bytes);

  int ox_unused;
  const int m_first = f_begin * 16;
  const int m_last = min(f_end * 16, a.gemm_m) - 1;
  const int vr0 = pixel_vrow(a, p, m_first, ox_unused);
  const int vr1 = pixel_vrow(a, p, m_last, ox_unused) + (a.r - 1) * a.dil_h;
  const int slots = (vr1 - vr0 + 1) * p.wp;  // LDS pixel slots per group

  // ---- 1. input rows -> LDS (every channel group) -------------------------
  for (int g = 0; g < p.groups; ++g) {
    for (int j = 0; j < p.copies; ++j) {
      const int inst = wave + 4 * j;
      const int slot = inst * 64 + lane;
      const int pix = slot >> 2;
      uint32_t off = kOutOfRange;
      if (pix < slots) {
        const int rr = int(fast_div(uint32_t(pix), p.div_wp));
        const int px = pix - rr * p.wp - a.pad_w;
        const int vr = vr0 + rr;
        const int b = int(fast_div(uint32_t(vr), p.div_hp));  // vr / hp
        const int iy = vr - b * p.hp - a.pad_h;
        if (b < a.n && unsigned(iy) < unsigned(a.h) && unsigned(px) < unsigned(a.wd))
          off = uint32_t(((b * a.h + iy) * a.wd + px) * a.c + g * 64 +
                         swz64_chunk(pix, slot & 3) * 16);
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (__attribute__((address_space(3))) void *)(smem + g * p.group_bytes + inst * 1024),
          16, off, 0, 0, 0);
    }
  }

  asm volatile("" ::: "memory");  // keep every copy ahead of the filter loads

  // ---- 2. this wave's filter slice -> VGPRs, in k order ---------------------
  v4i wf[kSteps][FN];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int oc = tile_n + wave * 16 * FN + i * 16 + (lane & 15);
    const int row = oc < a.gemm_n ? oc * a.gemm_k + 16 * (lane >> 4) : -1;
#pragma unroll
    for (int t = 0; t < kSteps; ++t)
      wf[t][i] = load16(wr, row >= 0 ? uint32_t(row + t * 64) : kOutOfRange);
  }
  // The input rows are complete once every load issued before the filter
  // and bias loads has returned (loads return in order).
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kSteps * FN) : "memory");
  __syncthreads();
  v4i bv[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int oc0 = tile_n + wave * 16 * FN + i * 16 + 4 * (lane >> 4);
    bv[i] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (oc0 + e < a.gemm_n) bv[i][e] = a.bias[oc0 + e];
  }



  // ---- 3. passes of up to four fragments ------------------------------------
  for (int f0 = f_begin; f0 < f_end; f0 += kPassFrags) {
    switch (min(kPassFrags, f_end - f0)) {
      case 4: halo_pass<FN, kSteps, 4>(a, p, smem, wf, bv, f0, vr0, m_first, tile_n, wave, lane); break;
      case 3: halo_pass<FN, kSteps, 3>(a, p, smem, wf, bv, f0, vr0, m_first, tile_n, wave, lane); break;
      case 2: halo_pass<FN, kSteps, 2>(a, p, smem, wf, bv, f0, vr0, m_first, tile_n, wave, lane); break;
      default: halo_pass<FN, kSteps, 1>(a, p, smem, wf, bv, f0, vr0, m_first, tile_n, wave, lane); break;
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
  hipLaunchKernelGGL(kern, dim3(unsigned(blocks)), dim3(kThreads), lds, s, a, h);
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
  HaloArgs h{};
  h.wp = a.wd + 2 * a.pad_w;
  h.hp = a.h + 2 * a.pad_h;
  h.groups = a.c / 64;
  h.copies = p.copies;
  h.group_bytes = p.copies * 4 * 1024;
  h.ranges = p.ranges;
  h.total_frags = (a.gemm_m + 15) / 16;
  h.tiles_n = p.tiles_n;
  h.div_ohw = make_fastdiv(uint32_t(a.out_h * a.out_w));
  h.div_ow = make_fastdiv(uint32_t(a.out_w));
  h.div_wp = make_fastdiv(uint32_t(h.wp));
  h.div_hp = make_fastdiv(uint32_t(h.hp));
  const size_t lds = size_t(h.groups) * h.group_bytes;
  const size_t blocks = size_t(p.ranges) * p.tiles_n;
  const int fn = p.bn / 64;
  const int steps = a.gemm_k / 64;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.c % 64 != 0 || !halo_instance_exists(fn, steps) || lds > size_t(kLdsBudget)) {
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
