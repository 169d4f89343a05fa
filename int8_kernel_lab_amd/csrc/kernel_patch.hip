// Input-reuse kernels on gfx950 INT8 MFMA: the halo-tiled variant and the
// spatial-strip 3x3 specialization.
//
// Both compute a 2-D output tile (th rows x tw columns of one image) for
// bn = 64 * FN output channels.  The four waves split the output channels
// (16 * FN each) and all share one LDS-resident input region, because every
// input byte staged is read by all four waves while every filter byte is
// read by exactly one: the filter fragments therefore go straight from
// global memory (L2) into registers, one tap ahead of their use, and only
// the input goes through LDS.
//
//   halo  : one stage = one 64-channel group; the staged region is the whole
//           receptive field of the tile (ph x pw pixels, any stride and
//           dilation) and all r*s taps read it.
//   strip : one stage = (64-channel group, filter row fy); the staged region
//           is one input row per output row of the tile, tw + 2 pixels wide,
//           and the three horizontal taps read it at column offsets 0, 1, 2.
//           This is the role of spatial_strip.cuh:118-196 in the reference
//           (strip reused across filter columns), with a gfx950 tile that
//           covers whole output rows instead of 128 pixels of one row.
//
// Stages are double-buffered: the next stage's global loads are issued
// before the current stage's MFMAs.  Pixels outside the image are
// zero-filled by the buffer unit.
#include <hip/hip_runtime.h>

#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i add_wrap(v4i a, v4i b) {
  return __builtin_bit_cast(v4i, __builtin_bit_cast(v4u, a) +
                                     __builtin_bit_cast(v4u, b));
}

constexpr int kMaxFragsM = 8;  // at most 128 output pixels per tile

struct PatchArgs {
  int th, tw, ph, pw, stage_pixels;
  int tiles_y, tiles_x, tiles_n;
  int frags_m;
  FastDiv div_pw, div_tw;
};

template <int FN, int LPT, bool kStrip>
__global__ __launch_bounds__(kThreads) void patch_kernel(ConvArgs a, PatchArgs p) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const int stage_bytes = p.stage_pixels * 64;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  int bid = int(blockIdx.x);
  const int tn = bid % p.tiles_n;
  bid /= p.tiles_n;
  const int tx = bid % p.tiles_x;
  bid /= p.tiles_x;
  const int ty = bid % p.tiles_y;
  const int img = bid / p.tiles_y;
  const int oy0 = ty * p.th;
  const int ox0 = tx * p.tw;
  const int tile_n = tn * 64 * FN;

  const auto xr = make_rsrc(a.x, a.x_bytes);
  const auto wr = make_rsrc(a.w, a.w_bytes);

  const int groups = a.c >> 6;
  const int stages = kStrip ? groups * a.r : groups;

  // Origin of the staged region in input coordinates.
  const int iy_org = kStrip ? oy0 * a.stride_h - a.pad_h : oy0 * a.stride_h - a.pad_h;
  const int ix_org = ox0 * a.stride_w - a.pad_w;

  v4i stage_regs[LPT];
  auto load_stage = [&](int st) {
    int g = st, fy = 0;
    if (kStrip) {
      g = st / a.r;
      fy = st - g * a.r;
    }
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int q = tid + i * kThreads;
      const int pix = q >> 2;
      const int j = q & 3;
      uint32_t off = kOutOfRange;
      if (pix < p.stage_pixels) {
        const int py = int(fast_div(uint32_t(pix), p.div_pw));
        const int px = pix - py * p.pw;
        const int iy = kStrip ? iy_org + py * a.stride_h + fy * a.dil_h : iy_org + py;
        const int ix = ix_org + px;
        if (unsigned(iy) < unsigned(a.h) && unsigned(ix) < unsigned(a.wd))
          off = uint32_t(((img * a.h + iy) * a.wd + ix) * a.c + g * 64 + j * 16);
      }
      stage_regs[i] = load16(xr, off);
    }
  };
  auto store_stage = [&](int buf) {
    int8_t *dst = smem + buf * stage_bytes;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int q = tid + i * kThreads;
      const int pix = q >> 2;
      if (pix < p.stage_pixels)
        *reinterpret_cast<v4i *>(dst + swz64(pix, q & 3)) = stage_regs[i];
    }
  };

  // Per-fragment LDS pixel of tap (0, 0) for this lane's output pixel.
  int lbase[kMaxFragsM];
  const int tile_px = p.th * p.tw;
#pragma unroll
  for (int f = 0; f < kMaxFragsM; ++f) {
    int t = f * 16 + (lane & 15);
    if (t >= tile_px) t = 0;  // padded column: computed, never stored
    const int ly = int(fast_div(uint32_t(t), p.div_tw));
    const int lx = t - ly * p.tw;
    lbase[f] = kStrip ? ly * p.pw + lx : ly * a.stride_h * p.pw + lx * a.stride_w;
  }

  // Filter fragment addressing: lane row = output channel, 16 k-bytes of
  // k-block lane / 16 inside the 64-channel group.
  int w_row[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int oc = tile_n + wave * 16 * FN + i * 16 + (lane & 15);
    w_row[i] = oc < a.gemm_n ? oc * a.gemm_k + 16 * (lane >> 4) : -1;
  }
  auto load_filter = [&](v4i (&dst)[FN], int tap, int g) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
      dst[i] = load16(wr, w_row[i] >= 0 ? uint32_t(w_row[i] + tap * a.c + g * 64)
                                        : kOutOfRange);
  };

  v4i acc[FN][kMaxFragsM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int f = 0; f < kMaxFragsM; ++f) acc[i][f] = v4i{0, 0, 0, 0};

  const int chunk = lane >> 4;
  auto compute = [&](int buf, int st) {
    const int8_t *src = smem + buf * stage_bytes;
    int g = st, fy0 = 0, fy1 = a.r;
    if (kStrip) {
      g = st / a.r;
      fy0 = st - g * a.r;
      fy1 = fy0 + 1;
    }
    v4i af[FN], an[FN];
    load_filter(af, fy0 * a.s, g);
    for (int fy = fy0; fy < fy1; ++fy) {
      for (int fx = 0; fx < a.s; ++fx) {
        const int tap = fy * a.s + fx;
        // prefetch the next tap's filter fragments of this stage
        const bool next = fx + 1 < a.s || fy + 1 < fy1;
        if (next) load_filter(an, tap + 1, g);
        const int delta = kStrip ? fx : fy * a.dil_h * p.pw + fx * a.dil_w;
#pragma unroll
        for (int f = 0; f < kMaxFragsM; ++f) {
          if (f >= p.frags_m) break;  // uniform
          const v4i b = *reinterpret_cast<const v4i *>(src + swz64(lbase[f] + delta, chunk));
#pragma unroll
          for (int i = 0; i < FN; ++i) acc[i][f] = mfma16(af[i], b, acc[i][f]);
        }
        if (next) {
#pragma unroll
          for (int i = 0; i < FN; ++i) af[i] = an[i];
        }
      }
    }
  };

  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int st = 0; st < stages; ++st) {
    const int buf = st & 1;
    const bool more = st + 1 < stages;
    if (more) load_stage(st + 1);
    compute(buf, st);
    if (more) store_stage(buf ^ 1);
    __syncthreads();
  }

  // output window: the tile's output rows oy0 .. oy0 + th - 1 of image img
  const int64_t m_win = (int64_t(img) * a.out_h + oy0) * a.out_w;
  const OutWindow ow = out_window(a.y, a.gemm_m, a.gemm_n, m_win, int64_t(p.th) * a.out_w);
  const bool vec = (a.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && ow.ok;
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int oc0 = tile_n + wave * 16 * FN + i * 16 + 4 * (lane >> 4);
    v4i bv = v4i{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (oc0 + e < a.gemm_n) bv[e] = a.bias[oc0 + e];
#pragma unroll
    for (int f = 0; f < kMaxFragsM; ++f) {
      if (f >= p.frags_m) break;
      const int t = f * 16 + (lane & 15);
      if (t >= tile_px) continue;
      const int ly = int(fast_div(uint32_t(t), p.div_tw));
      const int lx = t - ly * p.tw;
      const int oy = oy0 + ly, ox = ox0 + lx;
      if (oy >= a.out_h || ox >= a.out_w) continue;
      const size_t m = size_t((img * a.out_h + oy) * a.out_w + ox);
      const v4i v = add_wrap(acc[i][f], bv);
      if (vec) {
        if (oc0 < a.gemm_n)
          store_out4<kStoreStream>(ow.r, (uint32_t(int64_t(m) - m_win) * uint32_t(a.gemm_n) + uint32_t(oc0)) * 4u, v);
      } else {
        int32_t *dst = a.y + m * size_t(a.gemm_n) + oc0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (oc0 + e < a.gemm_n) dst[e] = v[e];
      }
    }
  }
}

template <int FN, int LPT, bool kStrip>
int launch_t(const ConvArgs &a, const PatchArgs &pa, size_t blocks, size_t lds,
             hipStream_t s) {
  auto kern = patch_kernel<FN, LPT, kStrip>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void *>(kern),
        hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) {
      set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
  }
  I8_LAUNCH(kern, dim3(unsigned(blocks)), dim3(kThreads), lds, s, a, pa);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("patch kernel launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

int launch_patch(const ConvArgs &a, const PatchPlan &p, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  PatchArgs pa{};
  pa.th = p.th;
  pa.tw = p.tw;
  pa.ph = p.ph;
  pa.pw = p.pw;
  pa.stage_pixels = p.stage_pixels;
  pa.tiles_y = p.tiles_y;
  pa.tiles_x = p.tiles_x;
  pa.tiles_n = p.tiles_n;
  pa.frags_m = p.frags_m;
  pa.div_pw = make_fastdiv(uint32_t(p.pw));
  pa.div_tw = make_fastdiv(uint32_t(p.tw));
  const size_t blocks = size_t(a.n) * p.tiles_y * p.tiles_x * p.tiles_n;
  const size_t lds = size_t(2) * p.stage_pixels * 64;
  const int fn = p.bn / 64;
  const int lpt = p.loads_per_thread <= 4 ? 4 : (p.loads_per_thread <= 8 ? 8 : 12);
  if (p.loads_per_thread > 12 || p.frags_m > kMaxFragsM || (fn != 1 && fn != 2)) {
    set_error("patch plan out of range");
    return I8CONV_BAD_ARGUMENT;
  }
#define I8_PATCH_CASE(FN_, LPT_)                                            \
  if (fn == FN_ && lpt == LPT_)                                             \
    return p.strip ? launch_t<FN_, LPT_, true>(a, pa, blocks, lds, s)       \
                   : launch_t<FN_, LPT_, false>(a, pa, blocks, lds, s);
  I8_PATCH_CASE(1, 4)
  I8_PATCH_CASE(1, 8)
  I8_PATCH_CASE(1, 12)
  I8_PATCH_CASE(2, 4)
  I8_PATCH_CASE(2, 8)
  I8_PATCH_CASE(2, 12)
#undef I8_PATCH_CASE
  set_error("no patch kernel instance");
  return I8CONV_BAD_ARGUMENT;
}

}  // namespace i8conv
