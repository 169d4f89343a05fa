// Pipelined generic implicit GEMM on gfx950 INT8 MFMA, for layers whose
// input channels are a multiple of 128 (every 128-byte k-stage then lies in
// one filter tap), and its split-K form.
//
// Same GEMM view and semantics as kernel_gemm.hip (generic_implicit_gemm.cuh
// :90-153 of the reference: M = n*out_h*out_w pixels, N = k output
// channels, K = r*s*c with k = (fy*s + fx)*c + ci); what changes is how the
// operands reach the MFMAs:
//   * each 128-byte k-stage of the BN filter rows and the BM im2col rows is
//     copied straight from global memory into LDS by the buffer unit
//     (buffer_load ... lds, 1 KB per wave instruction), no VGPR round trip;
//   * a ring of three stage buffers: stage s + 2 is in flight while stage s
//     feeds the MFMAs, one barrier per stage; the copies of stage s + 2 are
//     issued between the MFMA groups of stage s, or by copy waves (below);
//   * the LDS rows use the swz128x layout (see i8conv_device.hpp).  A copy writes lane
//     i's 16 bytes to LDS slot i of its 1 KB block, so the swizzle is applied
//     on the source side: the lane of slot (row, physical chunk) fetches the
//     logical chunk that belongs there;
//   * because a stage lies inside one tap, the tap decomposition is uniform
//     per stage: each lane keeps its rows' pixel origin and adds one tap
//     offset per stage, with two compares for padding;
//   * eight MFMA waves, two per SIMD, on the 256 x 128, 256 x 64 and
//     128 x 128 tiles (wave tiles 64 x 64 or 64 x 32), so one wave's MFMAs
//     run while the other waits on its fragment reads; four on the small
//     128 x 64 tile;
//   * on the 256 x 128 and 128 x 128 tiles with four or more k-stages per
//     workgroup, four more waves that only issue the copies: an MFMA wave
//     that also issues copies stalls whenever the buffer unit's queue is
//     full, and its MFMAs wait behind the stalled issue;
//   * accumulators stay in VGPRs (built with -amdgpu-mfma-vgpr-form);
//   * XCD-aware tile order (see below);
//   * fragments wholly past the last pixel row run no MFMAs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

constexpr int kRing = 3;  // stage buffers in LDS

typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i add_wrap(v4i a, v4i b) {
  // int32 addition with two's-complement wrap, like the MFMA accumulator.
  return __builtin_bit_cast(v4i, __builtin_bit_cast(v4u_t, a) + __builtin_bit_cast(v4u_t, b));
}

// Calls run(std::integral_constant<int, F>) with F = min(live, FMAX).
template <int F, int FMAX, class Run>
__device__ __forceinline__ void with_live_frags(int live, Run &run) {
  if constexpr (F < FMAX) {
    if (live <= F) {
      run(std::integral_constant<int, F>{});
      return;
    }
    with_live_frags<F + 1, FMAX>(live, run);
  } else {
    run(std::integral_constant<int, FMAX>{});
  }
}

// NCW == 0: every wave both copies and runs MFMAs.  NCW > 0: WM*WN MFMA
// waves plus NCW copy waves (waves WM*WN and up) that only issue the stage
// copies, so an MFMA wave never stalls on a copy issue.  The two roles run
// separate loops with the same one barrier per stage, so neither role's
// registers are live in the other's loop.
template <int BM, int BN, int WM, int WN, bool kSplit, int NCW>
__global__ __launch_bounds__(64 * (WM * WN + NCW)) void gemm_dma_kernel(ConvArgs a) {
  constexpr int NMW = WM * WN;             // MFMA waves
  constexpr int NW = NCW > 0 ? NCW : NMW;  // copy waves
  constexpr int TMW = BM / WM;  // pixels per wave
  constexpr int TNW = BN / WN;  // output channels per wave
  constexpr int FM = TMW / 16;
  constexpr int FN = TNW / 16;
  constexpr int kRows = BM + BN;             // LDS rows per stage: filter, then pixels
  constexpr int kTile = kRows * kStageBytes;  // bytes per stage buffer
  constexpr int kCopies = kRows / 8;          // 1 KB copies per stage
  constexpr int CPW = kCopies / NW;           // per wave
  constexpr int CPA = BN / 8 / NW;            // of which filter rows
  static_assert(kCopies % NW == 0 && (BN / 8) % NW == 0 && FM >= 1 && FN >= 1, "tile shape");
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool copier = NCW > 0 && wave_id >= NMW;  // a copy-only wave
  const int wave = copier ? wave_id - NMW : wave_id;  // index within its role
  const int wm = wave % WM;
  const int wn = wave / WM;

  // Workgroup i runs on XCD i % 8 (round-robin dispatch), and each XCD has
  // its own L2.  Tiles are handed out so that every XCD gets a contiguous
  // run of them (both channel tiles of a pixel tile, then the next pixel
  // tile): neighbouring pixel tiles share input rows, which then stay in
  // that XCD's L2 instead of being fetched into two.  A bijection on
  // [0, gridDim.x): the first 8 * (gridDim.x / 8) workgroups are permuted,
  // the rest keep their index.
  const int per_xcd = int(gridDim.x) / 8;
  int tile = int(blockIdx.x);
  if (tile < 8 * per_xcd) tile = (tile % 8) * per_xcd + tile / 8;
  const int tiles_n = (a.gemm_n + BN - 1) / BN;
  const int tile_m = (tile / tiles_n) * a.m_step;
  // pixel rows this tile stores; rows from m_end on read as zeros
  const int m_end = min(a.gemm_m, tile_m + a.m_step);
  const int tile_n = (tile % tiles_n) * BN;
  const int stages = a.gemm_k / kStageBytes;
  int s_begin = 0, s_end = stages;
  if (kSplit) {
    s_begin = int(blockIdx.y) * a.stages_per_split;
    s_end = min(stages, s_begin + a.stages_per_split);
  }

  const v4u xd = make_desc(a.x, a.x_bytes);
  const v4u wd = make_desc(a.w, a.w_bytes);
  const uint32_t lds0 = lds_addr(smem);

  // Copy j of this wave is block q = wave + NW*j of the stage: rows 8q..8q+7,
  // lane -> row 8q + lane/8, physical chunk lane%8.  Copies j < CPA are
  // filter rows (q < BN/8), the rest pixel rows.
  uint32_t abase[CPA];  // filter byte offset of this lane's chunk at stage 0
#pragma unroll
  for (int j = 0; j < CPA; ++j) {
    const int r = 8 * (wave + NW * j) + (lane >> 3);
    const int lc = swz128x_chunk(r, lane & 7);
    const int oc = tile_n + r;
    abase[j] = oc < a.gemm_n ? uint32_t(oc) * uint32_t(a.gemm_k) + uint32_t(lc * 16)
                             : kOutOfRange;
  }
  constexpr int CPB = CPW - CPA;
  int pix[CPB], iy0[CPB], ix0[CPB];
#pragma unroll
  for (int j = 0; j < CPB; ++j) {
    const int r = 8 * (wave + NW * (CPA + j)) + (lane >> 3);  // >= BN
    const int lc = swz128x_chunk(r, lane & 7);
    const int m = tile_m + r - BN;
    if (m < m_end) {
      const int b = int(fast_div(uint32_t(m), a.div_ohw));
      const int rem = m - b * a.out_h * a.out_w;
      const int oy = int(fast_div(uint32_t(rem), a.div_ow));
      const int ox = rem - oy * a.out_w;
      iy0[j] = oy * a.stride_h - a.pad_h;
      ix0[j] = ox * a.stride_w - a.pad_w;
      pix[j] = ((b * a.h + iy0[j]) * a.wd + ix0[j]) * a.c + lc * 16;
    } else {
      iy0[j] = -(1 << 29);  // every tap out of the image -> zeros
      ix0[j] = 0;
      pix[j] = 0;
    }
  }

  // Copies of one stage (stage buffers are numbered from the first stage of
  // this workgroup).  Copy j < CPA: filter rows; j >= CPA: pixel rows, at the
  // stage's tap offset, zero-filled where the tap falls in the padding.
  struct StageTap {
    uint32_t dst;
    int dy, dx, tap_off;
  };
  auto stage_tap = [&](int stage) {
    StageTap t;
    t.dst = lds0 + uint32_t(((stage - s_begin) % kRing) * kTile);
    // the stage's tap and channel offset (uniform)
    const int k0 = stage * kStageBytes;
    const int tap = int(fast_div(uint32_t(k0), a.div_c));
    const int ci0 = k0 - tap * a.c;
    const int fy = int(fast_div(uint32_t(tap), a.div_s));
    const int fx = tap - fy * a.s;
    t.dy = fy * a.dil_h;
    t.dx = fx * a.dil_w;
    t.tap_off = (t.dy * a.wd + t.dx) * a.c + ci0;
    return t;
  };
  auto copy = [&](const StageTap &t, int stage, int j) {
    if (j < CPA) {
      lds_copy16(wd, t.dst + uint32_t(wave + NW * j) * 1024u, abase[j] + uint32_t(stage * kStageBytes));
    } else {
      const int jb = j - CPA;
      const bool ok = unsigned(iy0[jb] + t.dy) < unsigned(a.h) && unsigned(ix0[jb] + t.dx) < unsigned(a.wd);
      lds_copy16(xd, t.dst + uint32_t(wave + NW * j) * 1024u,
                 ok ? uint32_t(pix[jb] + t.tap_off) : kOutOfRange);
    }
  };
  auto issue = [&](int stage) {
    const StageTap t = stage_tap(stage);
#pragma unroll
    for (int j = 0; j < CPW; ++j) copy(t, stage, j);
  };

  if (NCW > 0 && copier) {
    // copy wave: keep two stages in flight ahead of the MFMA waves
    issue(s_begin);
    if (s_begin + 1 < s_end) issue(s_begin + 1);
    for (int st = s_begin; st < s_end; ++st) {
      if (st + 1 < s_end)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CPW) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // stage st is visible to the MFMA waves, and they are done with stage
      // st - 1, whose buffer stage st + 2 overwrites
      __syncthreads();
      if (st + 2 < s_end) issue(st + 2);
    }
    return;
  }

  // Fragment read offsets inside a stage buffer, per k-step half h.
  int aoff[2][FN], boff[2][FM];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int ch = 4 * h + (lane >> 4);
#pragma unroll
    for (int i = 0; i < FN; ++i) aoff[h][i] = swz128x(wn * TNW + i * 16 + (lane & 15), ch);
#pragma unroll
    for (int j = 0; j < FM; ++j)
      boff[h][j] = BN * kStageBytes + swz128x(wm * TMW + j * 16 + (lane & 15), ch);
  }

  v4i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  if (NCW > 0) {
    // MFMA wave of a split workgroup: the copy waves fill the ring.  The
    // wave's fragments that lie wholly at or past m_end (the padding of a
    // last pixel tile: 120 of the 128 rows of the deep-K layer's fourth)
    // get no fragment reads and no MFMAs: the walk runs with the live
    // fragment count as a compile-time constant.
    const int row0 = tile_m + wm * TMW;
    const int live = m_end <= row0 ? 0 : min(FM, (m_end - row0 + 15) / 16);
    auto walk = [&](auto live_frags) {
      constexpr int F = decltype(live_frags)::value;
      for (int st = s_begin; st < s_end; ++st) {
        __syncthreads();
        const int8_t *buf = smem + ((st - s_begin) % kRing) * kTile;
        v4i af[2][FN], bf[2][F > 0 ? F : 1];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int i = 0; i < FN; ++i) af[h][i] = *reinterpret_cast<const v4i *>(buf + aoff[h][i]);
#pragma unroll
          for (int j = 0; j < F; ++j) bf[h][j] = *reinterpret_cast<const v4i *>(buf + boff[h][j]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < F; ++j) acc[i][j] = mfma16(af[h][i], bf[h][j], acc[i][j]);
      }
    };
    with_live_frags<0, FM>(live, walk);
  }
  if (NCW == 0) issue(s_begin);
  if (NCW == 0 && s_begin + 1 < s_end) issue(s_begin + 1);
  for (int st = s_begin; NCW == 0 && st < s_end; ++st) {
    // stage st has landed once only stage st + 1 (if any) is outstanding
    if (st + 1 < s_end)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CPW) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // every wave's copies of stage st are visible, and every wave is done
    // with stage st - 1, whose buffer the next issue overwrites
    __syncthreads();
    const bool more = st + 2 < s_end;
    const StageTap next = stage_tap(more ? st + 2 : st);
    const int8_t *buf = smem + ((st - s_begin) % kRing) * kTile;
    v4i af[2][FN], bf[2][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i) af[0][i] = *reinterpret_cast<const v4i *>(buf + aoff[0][i]);
#pragma unroll
    for (int j = 0; j < FM; ++j) bf[0][j] = *reinterpret_cast<const v4i *>(buf + boff[0][j]);
#pragma unroll
    for (int i = 0; i < FN; ++i) af[1][i] = *reinterpret_cast<const v4i *>(buf + aoff[1][i]);
#pragma unroll
    for (int j = 0; j < FM; ++j) bf[1][j] = *reinterpret_cast<const v4i *>(buf + boff[1][j]);
    // MFMAs in 2*FN groups of FM, with the copies of stage st + 2 spread
    // between the groups: a copy whose issue stalls (the buffer unit takes a
    // few in flight per wave) then holds back only a few queued MFMAs.
    constexpr int kGroups = 2 * FN;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const int h = g / FN, i = g % FN;
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(af[h][i], bf[h][j], acc[i][j]);
      if (more) {
#pragma unroll
        for (int c = (g * CPW + kGroups - 1) / kGroups; c < ((g + 1) * CPW + kGroups - 1) / kGroups; ++c)
          copy(next, st + 2, c);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Epilogue: lane holds channels oc0..oc0+3 of pixel px for each fragment.
  // The channel fragments of one pixel fragment are stored back to back
  // (i innermost), so the wave's 16-channel slices of a pixel row, 64 bytes
  // each, reach the L2 together and fill whole 128-byte lines; written
  // through (sector-aligned pitches) the layer then writes exactly its
  // output bytes.
  int32_t *out = a.y;
  if (kSplit) out = a.partial + size_t(blockIdx.y) * size_t(a.gemm_m) * size_t(a.gemm_n);
  const OutWindow ow = out_window(out, a.gemm_m, a.gemm_n, tile_m, a.m_step);
  const bool vec = (a.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 && ow.ok;
  v4i bias[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int oc0 = tile_n + wn * TNW + i * 16 + 4 * (lane >> 4);
    bias[i] = kSplit ? v4i{0, 0, 0, 0} : load_bias4(a.bias, a.gemm_n, oc0);
  }
  auto store_tile = [&](auto policy) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int px = tile_m + wm * TMW + j * 16 + (lane & 15);
      if (px >= m_end) continue;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int oc0 = tile_n + wn * TNW + i * 16 + 4 * (lane >> 4);
        const v4i v = add_wrap(acc[i][j], bias[i]);
        if (vec) {
          if (oc0 < a.gemm_n)
            store_out4<decltype(policy)::value>(
                ow.r, (uint32_t(px - tile_m) * uint32_t(a.gemm_n) + uint32_t(oc0)) * 4u, v);
        } else {
          int32_t *dst = out + size_t(px) * size_t(a.gemm_n) + oc0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (oc0 + e < a.gemm_n) store_out1(dst + e, v[e]);
        }
      }
    }
  };
  // Outputs beyond 128 MiB: fragment by fragment, evict-first.  Written
  // through, such outputs ran up to 1.75x slower (16x256x256x256 1x1: 220
  // -> 388 us; 268 MB and up all lost), while every output of the baseline
  // layers (0.8-51 MB) gains from it.
  auto store_tile_by_fragment = [&]() {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int oc0 = tile_n + wn * TNW + i * 16 + 4 * (lane >> 4);
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int px = tile_m + wm * TMW + j * 16 + (lane & 15);
        if (px >= m_end) continue;
        const v4i v = add_wrap(acc[i][j], bias[i]);
        if (vec) {
          if (oc0 < a.gemm_n)
            store_out4<kStoreStream>(
                ow.r, (uint32_t(px - tile_m) * uint32_t(a.gemm_n) + uint32_t(oc0)) * 4u, v);
        } else {
          int32_t *dst = out + size_t(px) * size_t(a.gemm_n) + oc0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (oc0 + e < a.gemm_n) store_out1(dst + e, v[e]);
        }
      }
    }
  };
  // Requantized int8 output: a lane's four channels of a pixel as one
  // 4-byte store (a pixel's 16-channel slice, 16 bytes, per four lanes;
  // ordinary stores, merged into lines in the L2).  Per 16-channel fragment
  // row, the odd-multiplier form (requant4_odd: four VALU operations per
  // value) where every channel of the wave's fragment row is in its domain
  // (a ballot over the active lanes), else the exact form (requant4, three
  // quarter-rate multiplies per value).  With int8 output, same box: the
  // 3x3 stride-2 128 -> 256-channel layer (config 3) 16.67-16.74 -> 15.73-
  // 15.76 us per launch, the dilated 256-channel one (config 5b) 25.64-25.69
  // -> 24.53-24.64.
  auto store_tile_requant = [&]() {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int oc0 = tile_n + wn * TNW + i * 16 + 4 * (lane >> 4);
      if (oc0 >= a.gemm_n) continue;
      const v4i m = *reinterpret_cast<const v4i *>(a.q_mult + oc0);
      const v4i sh = *reinterpret_cast<const v4i *>(a.q_shift + oc0);
      v4i mo, k, h;
      bool ok = true;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const RequantOdd o = requant_odd_params(m[e], sh[e], a.q_zp);
        ok = ok && o.ok;
        mo[e] = o.mo;
        k[e] = o.k;
        h[e] = o.sh;
      }
      if (__builtin_amdgcn_ballot_w64(!ok) == 0) {
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          const int px = tile_m + wm * TMW + j * 16 + (lane & 15);
          if (px >= m_end) continue;
          *reinterpret_cast<uint32_t *>(a.q_y + size_t(px) * size_t(a.gemm_n) + oc0) =
              requant4_odd(add_wrap(acc[i][j], bias[i]), mo, k, h);
        }
      } else {
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          const int px = tile_m + wm * TMW + j * 16 + (lane & 15);
          if (px >= m_end) continue;
          *reinterpret_cast<uint32_t *>(a.q_y + size_t(px) * size_t(a.gemm_n) + oc0) =
              requant4(add_wrap(acc[i][j], bias[i]), m, sh, a.q_zp);
        }
      }
    }
  };
  // one uniform branch for the whole epilogue
  if (!kSplit && a.q_y)
    store_tile_requant();
  else if (!kSplit && int64_t(a.gemm_m) * a.gemm_n * 4 > kStreamOutputBytes)
    store_tile_by_fragment();
  else if (sector_pitch(a.gemm_n))
    store_tile(std::integral_constant<int, kStoreThrough>{});
  else
    store_tile(std::integral_constant<int, 0>{});
}

template <int BM, int BN, int WM, int WN, int NCW = 0>
int launch_tile(const ConvArgs &a, int splits, hipStream_t stream) {
  const int tiles = int(((int64_t(a.gemm_m) + a.m_step - 1) / a.m_step) * ((a.gemm_n + BN - 1) / BN));
  const int stages = a.gemm_k / kStageBytes;
  const int ring = std::min(kRing, splits > 1 ? a.stages_per_split : stages);
  const size_t lds = size_t(ring) * size_t(BM + BN) * kStageBytes;
  auto kern = splits > 1 ? gemm_dma_kernel<BM, BN, WM, WN, true, NCW>
                         : gemm_dma_kernel<BM, BN, WM, WN, false, NCW>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) {
      set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
  }
  I8_LAUNCH(kern, dim3(unsigned(tiles), unsigned(splits)), dim3(64 * (WM * WN + NCW)),
                     lds, stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("pipelined gemm kernel launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

bool gemm_dma_tile_supported(int bm, int bn) {
  switch (bm * 1000 + bn) {
    case 128064: case 128128: case 256064: case 256128:
      return true;
    default:
      return false;
  }
}

int gemm_dma_copy_waves(const GemmPlan &p) {
  // Copy waves pay off once a workgroup has a steady state to overlap: with
  // two or three k-stages the MFMA waves mostly wait on the first copies
  // anyway, and the split roles only add a barrier hop per stage.
  // The planner picks 256 x 128 only for more than four k-stages.
  const int per_workgroup = p.splits > 1 ? p.stages_per_split : p.stages;
  if (p.bm == 256 && p.bn == 128) return 4;
  return p.bm == 128 && p.bn == 128 && per_workgroup >= 4 ? 4 : 0;
}

int launch_gemm_dma(const ConvArgs &args, const GemmPlan &p, int splits, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  ConvArgs a = args;
  a.m_step = p.m_step > 0 ? p.m_step : p.bm;
  // the kernel's assumptions, checked on the host: whole 128-byte stages in
  // one tap, a stage range per split, a tile it was built for, and LDS rows
  // the ring can hold
  const int stages = a.gemm_k / kStageBytes;
  if (a.c % kStageBytes != 0 || a.gemm_k % kStageBytes != 0 || stages < 1 ||
      (splits > 1 && (a.stages_per_split < 1 || int64_t(splits - 1) * a.stages_per_split >= stages)) ||
      !gemm_dma_tile_supported(p.bm, p.bn) || a.m_step % 16 != 0 || a.m_step > p.bm ||
      a.m_step < 16 ||
      size_t(kRing) * size_t(p.bm + p.bn) * kStageBytes > size_t(kLdsBudget)) {
    set_error("pipelined gemm plan out of range");
    return I8CONV_BAD_ARGUMENT;
  }
  // eight MFMA waves, two per SIMD (wave tiles 64 x 64, or 64 x 32 on the
  // narrower tiles), except the small 128 x 64 tile; plus four copy waves on
  // the wide tiles when the workgroup has k-stages enough
  const bool spec = gemm_dma_copy_waves(p) > 0;
  switch (p.bm * 1000 + p.bn) {
    case 128064: return launch_tile<128, 64, 2, 2>(a, splits, s);
    case 128128:
      return spec ? launch_tile<128, 128, 2, 4, 4>(a, splits, s) : launch_tile<128, 128, 2, 4>(a, splits, s);
    case 256064: return launch_tile<256, 64, 4, 2>(a, splits, s);
    case 256128: return launch_tile<256, 128, 4, 2, 4>(a, splits, s);
  }
  set_error("unsupported pipelined gemm tile");
  return I8CONV_BAD_ARGUMENT;
}

}  // namespace i8conv
