// Generic staged implicit GEMM on gfx950 INT8 MFMA, and its split-K form.
//
// Semantics follow generic_implicit_gemm.cuh:90-153 of the reference (GEMM
// view M = n*out_h*out_w pixels, N = k output channels, K = r*s*c with
// k = (fy*s + fx)*c + ci, bias added once, int32 result); the structure is
// new:
//   * the MFMA "A" operand is the filter (rows = output channels) and "B" is
//     the im2col view of the input (columns = pixels), so each lane ends with
//     four consecutive NHWK channels of one pixel -> 16-byte stores;
//   * 256-thread workgroups (4 x wave64), BM x BN tile, k staged 128 bytes at
//     a time through double-buffered, swizzled LDS; the next stage's global
//     loads are in flight while the current stage feeds the MFMAs;
//   * padding taps, rows m >= M, n >= N and k >= gemm_k are zero-filled by
//     the buffer unit (out-of-range offsets), not by branches;
//   * split-K: grid.y splits the stage range; each split writes raw int32
//     partial sums to a workspace and a second kernel adds them in split
//     order plus the bias (deterministic; integer addition is exact).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i add_wrap(v4i a, v4i b) {
  // int32 addition with two's-complement wrap, like the MFMA accumulator.
  return __builtin_bit_cast(v4i, __builtin_bit_cast(v4u, a) +
                                     __builtin_bit_cast(v4u, b));
}

template <int BM, int BN, int WM, bool kSplit>
__global__ __launch_bounds__(kThreads) void gemm_kernel(ConvArgs a) {
  constexpr int WN = 4 / WM;
  constexpr int TMW = BM / WM;  // pixels per wave
  constexpr int TNW = BN / WN;  // output channels per wave
  constexpr int FM = TMW / 16;
  constexpr int FN = TNW / 16;
  constexpr int PB = BM / 32;   // im2col rows staged per thread
  constexpr int PA = BN / 32;   // filter rows staged per thread
  constexpr int kTile = (BM + BN) * kStageBytes;
  static_assert(FM >= 1 && FN >= 1 && PA >= 1 && PB >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;

  const int tiles_n = (a.gemm_n + BN - 1) / BN;
  const int tile_m = int(blockIdx.x / tiles_n) * BM;
  const int tile_n = int(blockIdx.x % tiles_n) * BN;
  const int stages = (a.gemm_k + kStageBytes - 1) / kStageBytes;
  int stage_begin = 0;
  int stage_end = stages;
  if (kSplit) {
    stage_begin = int(blockIdx.y) * a.stages_per_split;
    stage_end = min(stages, stage_begin + a.stages_per_split);
  }

  const auto xr = make_rsrc(a.x, a.x_bytes);
  const auto wr = make_rsrc(a.w, a.w_bytes);

  // Staging assignment: thread -> 16-byte chunk (tid % 8) of rows
  // tid / 8 + 32 p.  The pixel decomposition is done once.
  const int chunk = tid & 7;
  const int row0 = tid >> 3;
  int pix_off[PB], iy0[PB], ix0[PB];
#pragma unroll
  for (int p = 0; p < PB; ++p) {
    const int m = tile_m + row0 + 32 * p;
    if (m < a.gemm_m) {
      const int b = int(fast_div(uint32_t(m), a.div_ohw));
      const int rem = m - b * a.out_h * a.out_w;
      const int oy = int(fast_div(uint32_t(rem), a.div_ow));
      const int ox = rem - oy * a.out_w;
      iy0[p] = oy * a.stride_h - a.pad_h;
      ix0[p] = ox * a.stride_w - a.pad_w;
      pix_off[p] = ((b * a.h + iy0[p]) * a.wd + ix0[p]) * a.c;
    } else {
      iy0[p] = -(1 << 29);  // every tap out of the image -> zeros
      ix0[p] = 0;
      pix_off[p] = 0;
    }
  }

  v4i ra[PA], rb[PB];
  auto load_stage = [&](int stage) {
    const int kk = stage * kStageBytes + chunk * 16;
    const bool kvalid = kk < a.gemm_k;
    int dy = -(1 << 29), dx = 0, tap_off = 0;
    if (kvalid) {
      const int tap = int(fast_div(uint32_t(kk), a.div_c));
      const int ci = kk - tap * a.c;
      const int fy = int(fast_div(uint32_t(tap), a.div_s));
      const int fx = tap - fy * a.s;
      dy = fy * a.dil_h;
      dx = fx * a.dil_w;
      tap_off = (dy * a.wd + dx) * a.c + ci;
    }
#pragma unroll
    for (int p = 0; p < PB; ++p) {
      const int iy = iy0[p] + dy;
      const int ix = ix0[p] + dx;
      const bool ok = unsigned(iy) < unsigned(a.h) && unsigned(ix) < unsigned(a.wd);
      rb[p] = load16(xr, ok ? uint32_t(pix_off[p] + tap_off) : kOutOfRange);
    }
#pragma unroll
    for (int p = 0; p < PA; ++p) {
      const int n = tile_n + row0 + 32 * p;
      const bool ok = kvalid && n < a.gemm_n;
      ra[p] = load16(wr, ok ? uint32_t(n * a.gemm_k + kk) : kOutOfRange);
    }
  };
  auto store_stage = [&](int buf) {
    int8_t *sa = smem + buf * kTile;
    int8_t *sb = sa + BN * kStageBytes;
#pragma unroll
    for (int p = 0; p < PA; ++p)
      *reinterpret_cast<v4i *>(sa + swz128(row0 + 32 * p, chunk)) = ra[p];
#pragma unroll
    for (int p = 0; p < PB; ++p)
      *reinterpret_cast<v4i *>(sb + swz128(row0 + 32 * p, chunk)) = rb[p];
  };

  v4i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  auto compute = [&](int buf, int stage) {
    const int8_t *sa = smem + buf * kTile;
    const int8_t *sb = sa + BN * kStageBytes;
#pragma unroll
    for (int ks = 0; ks < kStageBytes / 64; ++ks) {
      if (stage * kStageBytes + ks * 64 >= a.gemm_k) break;  // uniform
      const int ch = ks * 4 + (lane >> 4);
      v4i af[FN], bf[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i)
        af[i] = *reinterpret_cast<const v4i *>(
            sa + swz128(wn * TNW + i * 16 + (lane & 15), ch));
#pragma unroll
      for (int j = 0; j < FM; ++j)
        bf[j] = *reinterpret_cast<const v4i *>(
            sb + swz128(wm * TMW + j * 16 + (lane & 15), ch));
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
    }
  };

  load_stage(stage_begin);
  store_stage(0);
  __syncthreads();
  for (int st = stage_begin; st < stage_end; ++st) {
    const int buf = (st - stage_begin) & 1;
    const bool more = st + 1 < stage_end;
    if (more) load_stage(st + 1);
    compute(buf, st);
    if (more) store_stage(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds channels oc0..oc0+3 of pixel px for each fragment.
  int32_t *out = a.y;
  if (kSplit) out = a.partial + size_t(blockIdx.y) * size_t(a.gemm_m) * size_t(a.gemm_n);
  const OutWindow ow = out_window(out, a.gemm_m, a.gemm_n, tile_m, BM);
  const bool vec = (a.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 && ow.ok;
  // a pixel's channel fragments back to back, as in kernel_gemm_dma.hip
  v4i bias[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int oc0 = tile_n + wn * TNW + i * 16 + 4 * (lane >> 4);
    bias[i] = v4i{0, 0, 0, 0};
    if (!kSplit) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (oc0 + e < a.gemm_n) bias[i][e] = a.bias[oc0 + e];
    }
  }
  auto store_tile = [&](auto policy) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int px = tile_m + wm * TMW + j * 16 + (lane & 15);
      if (px >= a.gemm_m) continue;
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
            if (oc0 + e < a.gemm_n) dst[e] = v[e];
        }
      }
    }
  };
  if (sector_pitch(a.gemm_n))
    store_tile(std::integral_constant<int, kStoreThrough>{});
  else
    store_tile(std::integral_constant<int, 0>{});
}

// Second pass of split-K: y = bias + partial[0] + partial[1] + ... in split
// order.  Vector form: four consecutive channels per thread (N % 4 == 0).
// RQ: the sum requantized (requant4) and stored as four int8 values.
template <bool RQ>
__global__ __launch_bounds__(kThreads) void splitk_reduce_vec(
    const int32_t *__restrict__ partial, const int32_t *__restrict__ bias,
    int32_t *__restrict__ y, int n4, size_t total4, int splits,
    const int32_t *__restrict__ mult, const int32_t *__restrict__ shift, int32_t zp,
    uint32_t *__restrict__ q8) {
  // Each thread walks vec4 items q, q + G, ... (G threads in the grid); its
  // channel group q mod n4 is found once and then advanced by G mod n4,
  // so the loop has no 64-bit division.  The splits are added sixteen
  // loads at a time (all in flight together), still in split order.
  // The stores go through a window over the workgroup's kThreads items of
  // the pass (base qb, uniform), so 16-byte offsets stay small.
  const size_t grid = size_t(gridDim.x) * kThreads;
  const int step4 = int(grid % size_t(n4));
  int c4 = int((size_t(blockIdx.x) * kThreads + threadIdx.x) % size_t(n4));
  for (size_t qb = size_t(blockIdx.x) * kThreads; qb < total4; qb += grid) {
    const size_t q = qb + threadIdx.x;
    if (q < total4) {
      const v4i *src = reinterpret_cast<const v4i *>(partial) + q;
      v4i acc = reinterpret_cast<const v4i *>(bias)[c4];
      int sp = 0;
      for (; sp + 16 <= splits; sp += 16) {
        v4i t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = src[size_t(sp + u) * total4];
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = add_wrap(acc, t[u]);
      }
      for (; sp + 4 <= splits; sp += 4) {
        v4i t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = src[size_t(sp + u) * total4];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = add_wrap(acc, t[u]);
      }
      for (; sp < splits; ++sp) acc = add_wrap(acc, src[size_t(sp) * total4]);
      if constexpr (RQ) {
        q8[q] = requant4(acc, reinterpret_cast<const v4i *>(mult)[c4],
                         reinterpret_cast<const v4i *>(shift)[c4], zp);
        c4 += step4;
        if (c4 >= n4) c4 -= n4;
        continue;
      }
      const auto y_r = make_rsrc(reinterpret_cast<v4i *>(y) + qb,
                                 uint32_t(min(size_t(kThreads), total4 - qb)) * 16u);
      store_out4<kStoreThrough>(y_r, uint32_t(threadIdx.x) * 16u, acc);
    }
    c4 += step4;
    if (c4 >= n4) c4 -= n4;
  }
}

__global__ __launch_bounds__(kThreads) void splitk_reduce_scalar(
    const int32_t *__restrict__ partial, const int32_t *__restrict__ bias,
    int32_t *__restrict__ y, int gemm_n, size_t total, int splits) {
  for (size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += size_t(gridDim.x) * kThreads) {
    uint32_t acc = uint32_t(bias[i % size_t(gemm_n)]);
    for (int s = 0; s < splits; ++s) acc += uint32_t(partial[size_t(s) * total + i]);
    y[i] = int32_t(acc);
  }
}

template <int BM, int BN, int WM>
int launch_tile(const ConvArgs &a, int splits, hipStream_t stream) {
  const int tiles = ((a.gemm_m + BM - 1) / BM) * ((a.gemm_n + BN - 1) / BN);
  if (splits > 1) {
    I8_LAUNCH((gemm_kernel<BM, BN, WM, true>), dim3(tiles, splits),
                       dim3(kThreads), 0, stream, a);
  } else {
    I8_LAUNCH((gemm_kernel<BM, BN, WM, false>), dim3(tiles, 1),
                       dim3(kThreads), 0, stream, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("gemm kernel launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

int launch_any(const ConvArgs &a, const GemmPlan &p, int splits, hipStream_t s) {
  switch (p.bm * 1000 + p.bn) {
    case 64032: return launch_tile<64, 32, 2>(a, splits, s);
    case 64064: return launch_tile<64, 64, 2>(a, splits, s);
    case 64128: return launch_tile<64, 128, 1>(a, splits, s);
    case 128032: return launch_tile<128, 32, 4>(a, splits, s);
    case 128064: return launch_tile<128, 64, 2>(a, splits, s);
    case 128128: return launch_tile<128, 128, 2>(a, splits, s);
    case 256064: return launch_tile<256, 64, 4>(a, splits, s);
    case 256128: return launch_tile<256, 128, 2>(a, splits, s);
    default:
      set_error("unsupported gemm tile " + std::to_string(p.bm) + "x" + std::to_string(p.bn));
      return I8CONV_BAD_ARGUMENT;
  }
}

}  // namespace

int launch_gemm(const ConvArgs &a, const GemmPlan &p, void *stream) {
  ConvArgs args = a;
  args.partial = nullptr;
  args.splits = 1;
  args.stages_per_split = p.stages;
  if (p.pw && !args.q_y && pointwise_pointers_ok(args)) return launch_pointwise(args, nullptr, stream);
  if (args.q_y && !p.dma) {
    set_error("requantized GEMM output needs the pipelined kernel (C % 128 == 0)");
    return I8CONV_BAD_ARGUMENT;
  }
  if (p.dma) return launch_gemm_dma(args, p, 1, stream);
  return launch_any(args, p, 1, static_cast<hipStream_t>(stream));
}

int launch_splitk(const ConvArgs &a, const GemmPlan &p, void *workspace,
                  void *stream, const RequantArgs *rq) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  ConvArgs args = a;
  args.partial = static_cast<int32_t *>(workspace);
  args.splits = p.splits;
  args.stages_per_split = p.stages_per_split;
  const size_t total = size_t(a.gemm_m) * size_t(a.gemm_n);
  const bool vec = (a.gemm_n & 3) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(workspace) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.bias) & 15) == 0;
  // rejected before the first pass is enqueued, so that an error leaves
  // nothing queued
  if (rq && !vec) {
    set_error("split-K requantized reduce needs N % 4 == 0 and 16-byte aligned bias and workspace");
    return I8CONV_BAD_ARGUMENT;
  }
  int rc = p.deep  ? launch_deepk(args, p.deep_plan, workspace, stream)
           : p.dma ? launch_gemm_dma(args, p, p.splits, stream)
                   : launch_any(args, p, p.splits, s);
  if (rc != I8CONV_OK) return rc;
  const size_t work = vec ? total / 4 : total;
  size_t blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  if (blocks == 0) blocks = 1;
  if (rq) {
    I8_LAUNCH(splitk_reduce_vec<true>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                       args.partial, a.bias, nullptr, a.gemm_n / 4, total / 4, p.splits, rq->mult,
                       rq->shift, rq->zero_point, reinterpret_cast<uint32_t *>(rq->y));
  } else if (vec) {
    I8_LAUNCH(splitk_reduce_vec<false>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                       args.partial, a.bias, a.y, a.gemm_n / 4, total / 4, p.splits, nullptr,
                       nullptr, 0, nullptr);
  } else {
    I8_LAUNCH(splitk_reduce_scalar, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                       args.partial, a.bias, a.y, a.gemm_n, total, p.splits);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("split-K reduce launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace i8conv
