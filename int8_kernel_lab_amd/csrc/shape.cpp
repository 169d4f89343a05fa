// Shape validation, tile planners and eligibility predicates (host only).
#include <limits.h>
#include <stdint.h>

#include <algorithm>
#include <string>

#include "i8conv_internal.hpp"

namespace i8conv {

// conv_shape.cuh:22-35.  out_h/out_w use the same C++ expression (integer
// division truncating toward zero) so that every shape the reference
// accepts derives to the same geometry.
int derive(const i8conv_shape &s, i8conv_geometry *g) {
  if (s.n < 1 || s.h < 1 || s.w < 1 || s.c < 1 || s.k < 1 || s.r < 1 ||
      s.s < 1 || s.pad_h < 0 || s.pad_w < 0 || s.stride_h < 1 ||
      s.stride_w < 1 || s.dilation_h < 1 || s.dilation_w < 1) {
    set_error("shape fields out of range (sizes, strides, dilations >= 1, pads >= 0)");
    return I8CONV_BAD_SHAPE;
  }
  if (s.c % 16 != 0) {
    set_error("input channels must be divisible by 16");
    return I8CONV_BAD_SHAPE;
  }
  const int64_t num_h = int64_t(s.h) + 2 * int64_t(s.pad_h) -
                        int64_t(s.dilation_h) * (s.r - 1) - 1;
  const int64_t num_w = int64_t(s.w) + 2 * int64_t(s.pad_w) -
                        int64_t(s.dilation_w) * (s.s - 1) - 1;
  const int64_t out_h = num_h / s.stride_h + 1;
  const int64_t out_w = num_w / s.stride_w + 1;
  if (out_h <= 0 || out_w <= 0) {
    set_error("output must be nonempty");
    return I8CONV_BAD_SHAPE;
  }
  const int64_t gemm_m = int64_t(s.n) * out_h * out_w;
  const int64_t gemm_k = int64_t(s.r) * s.s * s.c;
  const int64_t in_el = int64_t(s.n) * s.h * s.w * s.c;
  const int64_t f_el = int64_t(s.k) * gemm_k;
  const int64_t out_el = gemm_m * s.k;
  if (in_el > INT32_MAX || f_el > INT32_MAX || gemm_m > INT32_MAX ||
      gemm_k > INT32_MAX || out_el > (int64_t(1) << 40) || out_h > INT32_MAX ||
      out_w > INT32_MAX) {
    set_error("tensor too large (input/filter bytes and M must be < 2^31)");
    return I8CONV_BAD_SHAPE;
  }
  if (g) {
    g->out_h = int32_t(out_h);
    g->out_w = int32_t(out_w);
    g->gemm_m = gemm_m;
    g->gemm_n = s.k;
    g->gemm_k = int32_t(gemm_k);
    g->input_elements = in_el;
    g->filter_elements = f_el;
    g->output_elements = out_el;
  }
  return I8CONV_OK;
}

namespace {

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

// Workgroup tiles instantiated in kernel_gemm.hip (BM pixels x BN channels).
bool gemm_tile_supported(int bm, int bn) {
  switch (bm * 1000 + bn) {
    case 64032: case 64064: case 64128: case 128032: case 128064:
    case 128128: case 256064: case 256128:
      return true;
    default:
      return false;
  }
}

// The LDS-DMA pipelined kernel (kernel_gemm_dma.hip) needs every 128-byte
// k-stage inside one filter tap: c % 128 == 0.
static bool dma_eligible(const i8conv_shape &s) { return s.c % kStageBytes == 0; }

// Generic tile choice.  Pipelined kernel: 128 output channels per tile
// (64 when N <= 64), and 256 pixels when that still gives the grid about
// three quarters of the 256 compute units, else 128.  Short reductions (at
// most 4 stages: 1x1 layers) take 128 pixels regardless: they are bound by
// HBM, and the smaller LDS ring lets three workgroups share a compute unit
// (measured on a 1x1 C = 256 -> 64 layer: 20.0 us vs 25.1 us with 256).  Register-staged
// kernel: the smallest supported width covering N (32/64/128 columns, 128
// for wider layers); the pixel tile shrinks from 256 until the grid has
// enough workgroups to cover the 256 compute units.
// Pipelined kernel, tile step: when ceil(M / bm) * tiles_n workgroups (more
// than one per compute unit) leave a last round that covers only part of
// the 256 compute units, the layer waits on a few workgroups that run alone
// (a 1x1 C = 256 -> 64 layer: 1568 tiles of 128 pixels take 19.2 us, 1536
// take 17.8 us).  A tile that stores fewer pixel rows (a multiple of 16; its
// last rows are zero-filled by out-of-range copies) evens the rounds out:
// the step minimises ceil(tiles / 256) * (bn + step), ties to the larger
// step (config 4a: 1792 tiles storing 112 rows, 19.2 -> 18.8 us).  The
// zero-filled rows still pass through the copy path, so a grid of one round
// keeps whole tiles (config 3 with 208-row steps: 15.15 vs 15.07 us).
int gemm_dma_step(int64_t gemm_m, int64_t tiles_n, int bm, int bn) {
  int best = bm;
  const int64_t tiles = ceil_div(gemm_m, bm) * tiles_n;
  if (tiles <= 256) return best;
  int64_t best_cost = ceil_div(tiles, 256) * (bn + bm);
  for (int step = bm - 16; step > bm / 2; step -= 16) {
    const int64_t cost = ceil_div(ceil_div(gemm_m, step) * tiles_n, 256) * (bn + step);
    if (cost < best_cost) {
      best = step;
      best_cost = cost;
    }
  }
  return best;
}

// Pointwise streaming form: instances for C in {64, 128, 256, 512} and N in
// {32, 64, 128, 256}.  A wave holds a slice of the filter as MFMA A
// operands, at most 16384 bytes (64 VGPRs per lane): slices of
// min(N, 16384 / C) output channels, 2 to 8 of them where N * C > 16384.
bool pointwise_supported(int c, int n) {
  const bool cs = c == 64 || c == 128 || c == 256 || c == 512;
  const bool ns = n == 32 || n == 64 || n == 128 || n == 256;
  return cs && ns;
}

int pointwise_slices(int c, int n) {
  const int per = std::min(n, 16384 / c);
  return n / per;
}

bool pointwise_requant_supported(int c, int n) {
  if (!pointwise_supported(c, n)) return false;
  const int per = n / pointwise_slices(c, n);
  return per == 64 || per == 128;
}

// Two-wave workgroups of one fragment stream each, or one workgroup of SL
// waves per stream; at most kPwMaxWaves waves (fewer streams than
// fragments otherwise).
int pointwise_waves(int64_t gemm_m, int slices) {
  const int group = pw_group_waves(slices), streams_per_group = group / slices;
  const int64_t streams = std::min<int64_t>(ceil_div(gemm_m, 16), kPwMaxWaves / slices);
  return int(ceil_div(streams, streams_per_group) * group);
}

static bool pointwise_eligible(const i8conv_shape &s, const i8conv_geometry &g) {
  // 32-bit buffer offsets: input and output below 2 GiB, so that the
  // out-of-range offset 2^31 lies past both
  return s.r == 1 && s.s == 1 && s.stride_h == 1 && s.stride_w == 1 && s.pad_h == 0 &&
         s.pad_w == 0 && pointwise_supported(s.c, g.gemm_n) &&
         g.gemm_m * s.c < (int64_t(1) << 31) && g.gemm_m * g.gemm_n * 4 < (int64_t(1) << 31);
}

GemmPlan plan_generic(const i8conv_shape &s, const i8conv_geometry &g) {
  GemmPlan p;
  p.stages = int(ceil_div(g.gemm_k, kStageBytes));
  p.splits = 1;
  p.stages_per_split = p.stages;
  if (pointwise_eligible(s, g)) {
    p.pw = true;
    p.pw_waves = pointwise_waves(g.gemm_m, pointwise_slices(s.c, int(g.gemm_n)));
  }
  if (dma_eligible(s)) {
    p.dma = true;
    p.bn = g.gemm_n <= 64 ? 64 : 128;
    const int64_t tiles_n = ceil_div(g.gemm_n, p.bn);
    p.bm = p.stages > 4 && ceil_div(g.gemm_m, 256) * tiles_n >= 192 ? 256 : 128;
    p.m_step = gemm_dma_step(g.gemm_m, tiles_n, p.bm, p.bn);
    return p;
  }
  p.bn = g.gemm_n <= 32 ? 32 : (g.gemm_n <= 64 ? 64 : 128);
  const int64_t tiles_n = ceil_div(g.gemm_n, p.bn);
  p.bm = 64;
  for (int bm : {256, 128}) {
    if (!gemm_tile_supported(bm, p.bn)) continue;
    if (ceil_div(g.gemm_m, bm) * tiles_n >= 512) {
      p.bm = bm;
      break;
    }
  }
  if (!gemm_tile_supported(p.bm, p.bn)) p.bm = 128;
  return p;
}

// Split-K: a 128-pixel tile (64 for tiny M on the register-staged kernel),
// with the 128-byte k stages divided among enough splits to give about one
// workgroup per compute unit (pipelined kernel: its LDS ring allows one per
// unit) or two (register-staged).
GemmPlan plan_splitk(const i8conv_shape &s, const i8conv_geometry &g) {
  GemmPlan p;
  p.stages = int(ceil_div(g.gemm_k, kStageBytes));
  // 3x3 stride-1 layers whose output pixels all fit one workgroup's LDS
  // planes: the deep-channel kernel, one split per 128 input channels
  if (plan_deepk(s, g, &p.deep_plan)) {
    p.deep = true;
    p.dma = true;
    p.bm = int(g.gemm_m);
    p.bn = 32;
    p.splits = p.deep_plan.splits;
    p.stages_per_split = int(ceil_div(9 * 128, kStageBytes));
    return p;
  }
  p.dma = dma_eligible(s);
  if (p.dma) {
    p.bn = g.gemm_n <= 64 ? 64 : 128;
    p.bm = 128;
  } else {
    p.bn = g.gemm_n <= 32 ? 32 : (g.gemm_n <= 64 ? 64 : 128);
    p.bm = g.gemm_m <= 64 ? 64 : 128;
    if (!gemm_tile_supported(p.bm, p.bn)) p.bm = 128;
  }
  const int64_t tiles = ceil_div(g.gemm_m, p.bm) * ceil_div(g.gemm_n, p.bn);
  int64_t splits = ceil_div(p.dma ? 256 : 512, tiles);
  splits = std::max<int64_t>(2, std::min<int64_t>(splits, p.stages));
  p.stages_per_split = int(ceil_div(p.stages, splits));
  p.splits = int(ceil_div(p.stages, p.stages_per_split));
  return p;
}

size_t splitk_workspace_bytes(const i8conv_geometry &g, const GemmPlan &p) {
  return size_t(p.splits) * size_t(g.gemm_m) * size_t(g.gemm_n) * sizeof(int32_t);
}

namespace {

constexpr int kMaxTilePixels = 128;   // 8 MFMA column fragments
constexpr int kMaxStagePixels = 768;  // 12 staged 16-byte chunks per thread

enum class PatchMode { kStagedHalo, kStrip };

// Resident-halo plan (kernel_halo.hip).  The filter slice of a wave
// (16*fn channels x gemm_k bytes) must match an instantiated kernel, and
// every tap of every output pixel must land inside the zero-padded image
// (true unless out_h/out_w come from the truncating formula with a negative
// numerator).  Ranges: as few as fill the compute units once, more while
// the input rows of the longest range do not fit LDS.
bool plan_resident(const i8conv_shape &s, const i8conv_geometry &g, PatchPlan *p) {
  if (s.c % 64 != 0 || g.gemm_k % 64 != 0) return false;
  const int steps = g.gemm_k / 64;
  const int fn = (s.k > 64 && halo_instance_exists(2, steps)) ? 2 : 1;
  if (!halo_instance_exists(fn, steps)) return false;
  const int hp = s.h + 2 * s.pad_h;
  const int wp = s.w + 2 * s.pad_w;
  if (int64_t(g.out_h - 1) * s.stride_h + int64_t(s.r - 1) * s.dilation_h >= hp) return false;
  if (int64_t(g.out_w - 1) * s.stride_w + int64_t(s.s - 1) * s.dilation_w >= wp) return false;
  const int64_t total_frags = ceil_div(g.gemm_m, 16);
  const int tiles_n = int(ceil_div(s.k, 64 * fn));
  auto vrow = [&](int64_t m) {
    const int64_t b = m / (int64_t(g.out_h) * g.out_w);
    const int64_t oy = (m % (int64_t(g.out_h) * g.out_w)) / g.out_w;
    return b * hp + oy * s.stride_h;
  };
  const HaloRowLayout row = halo_row_layout(wp, s.c, kHaloPadUnits);
  if (row.row_bytes > kLdsBudget) return false;
  const int64_t first = std::max<int64_t>(1, std::min(total_frags, ceil_div(256, tiles_n)));
  const int64_t chunks = ceil_div(g.gemm_k, 128);
  for (int64_t ranges = first; ranges <= total_frags;
       ranges = std::min(total_frags, ranges * 5 / 4 + 1)) {
    // each workgroup re-reads the whole filter slice: beyond the first grid
    // that fills the compute units, keep at least four fragments per range
    if (ranges > first && total_frags / ranges < 4) break;
    int64_t max_rows = 0;
    for (int64_t r = 0; r < ranges; ++r) {
      const int64_t f0 = r * total_frags / ranges, f1 = (r + 1) * total_frags / ranges;
      if (f1 <= f0) continue;
      const int64_t m0 = f0 * 16, m1 = std::min<int64_t>(f1 * 16, g.gemm_m) - 1;
      const int64_t rows = vrow(m1) - vrow(m0) + int64_t(s.r - 1) * s.dilation_h + 1;
      max_rows = std::max(max_rows, rows);
    }
    const int64_t input_lds = kHaloBiasLds + max_rows * row.row_bytes;
    const int64_t slot = int64_t(halo_ring_slot_bytes(fn));
    const int64_t ring = input_lds >= kLdsBudget ? 0 :
        std::min<int64_t>({kHaloRing, chunks, (kLdsBudget - input_lds) / slot});
    if (ring >= 1 && ranges * tiles_n <= INT32_MAX) {
      p->ring = int(ring);
      p->resident = true;
      p->strip = false;
      p->bn = 64 * fn;
      p->tiles_n = tiles_n;
      p->ranges = int(ranges);
      p->rows = int(max_rows);
      p->frags_m = int(ceil_div(total_frags, ranges));
      p->th = p->tw = p->ph = p->pw = 0;
      p->tiles_y = p->tiles_x = 1;
      p->stage_pixels = int(max_rows * wp);
      return true;
    }
    if (ranges == total_frags) break;
  }
  return false;
}

// Row-streaming plan (kernel_row.hip): 3x3, stride 1, dilation 1, c % 64.
// Output rows of each image are cut into `blocks` near-equal blocks so the
// grid (n * blocks * tiles_n workgroups) covers the 256 compute units; a
// block's padded input rows (its rows plus two) must fit in LDS beside the
// filter ring.
bool plan_row(const i8conv_shape &s, const i8conv_geometry &g, PatchPlan *p) {
  if (!(s.r == 3 && s.s == 3 && s.stride_h == 1 && s.stride_w == 1 && s.dilation_h == 1 &&
        s.dilation_w == 1 && s.c % 64 == 0))
    return false;
  // the row kernels' geometry travels in packed preloaded argument words and
  // their grid is (channel tiles, row blocks, images)
  if (s.n >= 65536 || s.h >= 65536 || s.w >= 65536 || s.pad_h >= 256 || s.pad_w >= 256)
    return false;
  const int cg = s.c / 64;
  const int nfr = int(ceil_div(g.out_w, 16));
  const HaloRowLayout row = halo_row_layout(int64_t(s.w) + 2 * s.pad_w, s.c, kRowPadUnits);
  const int64_t chunks = ceil_div(g.gemm_k, 128);
  // For each channel slice width (16*fn channels per wave), the smallest
  // number of row blocks per image that gives every compute unit a
  // workgroup and fits in LDS.  Among the widths with a plan, keep the one
  // whose workgroup copies the fewest bytes (input rows + filter slice):
  // that copy is what the workgroup waits for before its MFMAs can run.
  bool found = false;
  int64_t best_bytes = 0;
  for (int fn : {2, 1}) {
    if (fn == 2 && s.k <= 64) continue;
    if (!row_instance_exists(fn, cg, nfr)) continue;
    const int tiles_n = int(ceil_div(s.k, 64 * fn));
    const int64_t slot = int64_t(halo_ring_slot_bytes(fn));
    int64_t blocks = std::min<int64_t>(g.out_h, std::max<int64_t>(1, ceil_div(256, int64_t(s.n) * tiles_n)));
    for (; blocks <= g.out_h; ++blocks) {
      const int64_t rows = ceil_div(g.out_h, blocks) + 2;
      const int64_t input_lds = kHaloBiasLds + rows * row.row_bytes;
      if (input_lds >= kLdsBudget) continue;
      const int64_t ring = std::min<int64_t>({kHaloRing, chunks, (kLdsBudget - input_lds) / slot});
      if (ring < 1) continue;
      if (int64_t(s.n) * blocks * tiles_n > INT32_MAX) break;
      const int64_t bytes = rows * row.row_bytes + int64_t(64) * fn * g.gemm_k;
      if (!found || bytes < best_bytes) {
        found = true;
        best_bytes = bytes;
        *p = PatchPlan{};
        p->row = true;
        p->bn = 64 * fn;
        p->tiles_n = tiles_n;
        p->ranges = int(blocks);
        p->rows = int(rows);
        p->ring = int(ring);
        p->frags_m = nfr;
        p->tiles_y = p->tiles_x = 1;
        p->stage_pixels = int(rows * (s.w + 2 * s.pad_w));
      }
      break;
    }
  }
  // 128 channels in 64-channel slices: the form with copy waves when it fits
  if (found && s.c == 128 && p->bn == 64 && rowpass_nfr(g.out_w) != 0 &&
      p->rows - 2 <= rowpass_max_rows(rowpass_nfr(g.out_w)) &&
      rowpass_lds_bytes(s.w + 2 * s.pad_w, p->rows - 2) <= size_t(kLdsBudget) &&
      g.output_elements * 4 <= INT32_MAX)
    p->streamed = true;
  return found;
}

bool finish_patch_plan(const i8conv_shape &s, const i8conv_geometry &g,
                       PatchMode mode, PatchPlan *p) {
  (void)mode;
  p->stage_pixels = p->ph * p->pw;
  if (p->stage_pixels > kMaxStagePixels) return false;
  if (size_t(2) * p->stage_pixels * 64 > size_t(kLdsBudget)) return false;
  p->tiles_y = int(ceil_div(g.out_h, p->th));
  p->tiles_x = int(ceil_div(g.out_w, p->tw));
  p->tiles_n = int(ceil_div(s.k, p->bn));
  p->frags_m = int(ceil_div(int64_t(p->th) * p->tw, 16));
  p->loads_per_thread = int(ceil_div(int64_t(p->stage_pixels) * 4, kThreads));
  const int64_t blocks = int64_t(s.n) * p->tiles_y * p->tiles_x * p->tiles_n;
  return blocks <= INT32_MAX;
}

// Tile search shared by halo and strip: the widest tile (whole output rows
// when out_w <= 128) whose staged region fits, preferring pixel counts that
// fill whole 16-column MFMA fragments.
bool search_patch_plan(const i8conv_shape &s, const i8conv_geometry &g,
                       PatchMode mode, int bn, PatchPlan *out) {
  PatchPlan best;
  bool found = false;
  double best_score = -1.0;
  for (int tw = std::min(g.out_w, kMaxTilePixels); tw >= 1; --tw) {
    // only full-width tiles, or widths that split the row evenly
    if (tw != g.out_w && g.out_w % tw != 0) continue;
    const int th_max = std::min(g.out_h, kMaxTilePixels / tw);
    for (int th = th_max; th >= 1; --th) {
      PatchPlan p;
      p.strip = mode == PatchMode::kStrip;
      p.th = th;
      p.tw = tw;
      p.bn = bn;
      if (p.strip) {
        p.ph = th;
        p.pw = tw + s.s - 1;
      } else {
        p.ph = (th - 1) * s.stride_h + (s.r - 1) * s.dilation_h + 1;
        p.pw = (tw - 1) * s.stride_w + (s.s - 1) * s.dilation_w + 1;
      }
      if (!finish_patch_plan(s, g, mode, &p)) continue;
      const int px = th * tw;
      // useful fraction of the MFMA columns the whole grid computes (edge
      // tiles included), times a mild preference for big tiles (less halo
      // re-read, fewer passes over the filter)
      const double fill = double(g.out_h) * g.out_w /
                          (double(p.tiles_y) * p.tiles_x * p.frags_m * 16);
      const double score = fill * (0.75 + 0.25 * double(px) / kMaxTilePixels);
      if (score > best_score + 1e-9) {
        best_score = score;
        best = p;
        found = true;
      }
      break;  // larger th is better for a given tw; stop at first fit
    }
  }
  if (found) *out = best;
  return found;
}

}  // namespace

// Halo-tiled predicate: 64-channel groups and a tile whose receptive field
// fits LDS.  Any filter size, stride and dilation.  3x3 layers whose halo of
// all channel groups fits LDS use the resident-halo kernel (input read once
// per tile, filter streamed); the others stage one channel group at a time.
bool plan_halo(const i8conv_shape &s, const i8conv_geometry &g, PatchPlan *p) {
  if (s.c % 64 != 0) return false;
  const int bn = s.k > 64 ? 128 : 64;
  if (plan_row(s, g, p) || plan_resident(s, g, p))
    return true;
  return search_patch_plan(s, g, PatchMode::kStagedHalo, bn, p);
}

// Spatial-strip predicate, re-derived from spatial_strip.cuh:11-15 for the
// gfx950 tile: 3x3 filter, horizontal stride and dilation 1 (the strip is
// reused across the three filter columns), C % 64 == 0 (one 64-channel MFMA
// k-block per stage).  The reference's K % 64 and out_w % 128 conditions are
// gone: the tile covers whole output rows (or an even split of a row) and
// the epilogue guards the channel tail.  Vertical stride/dilation and padding
// are free, as in the reference.
bool plan_strip(const i8conv_shape &s, const i8conv_geometry &g, PatchPlan *p) {
  if (!(s.r == 3 && s.s == 3 && s.stride_w == 1 && s.dilation_w == 1 &&
        s.c % 64 == 0))
    return false;
  return search_patch_plan(s, g, PatchMode::kStrip, s.k > 64 ? 128 : 64, p);
}

ConvArgs make_args(const i8conv_shape &s, const i8conv_geometry &g,
                   const int8_t *x, const int8_t *w, const int32_t *bias,
                   int32_t *y) {
  ConvArgs a{};
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.y = y;
  a.partial = nullptr;
  a.n = s.n;
  a.h = s.h;
  a.wd = s.w;
  a.c = s.c;
  a.k = s.k;
  a.r = s.r;
  a.s = s.s;
  a.pad_h = s.pad_h;
  a.pad_w = s.pad_w;
  a.stride_h = s.stride_h;
  a.stride_w = s.stride_w;
  a.dil_h = s.dilation_h;
  a.dil_w = s.dilation_w;
  a.out_h = g.out_h;
  a.out_w = g.out_w;
  a.gemm_m = int(g.gemm_m);
  a.gemm_n = g.gemm_n;
  a.gemm_k = g.gemm_k;
  a.x_bytes = uint32_t(g.input_elements);
  a.w_bytes = uint32_t(g.filter_elements);
  a.div_c = make_fastdiv(uint32_t(s.c));
  a.div_s = make_fastdiv(uint32_t(s.s));
  a.div_ow = make_fastdiv(uint32_t(g.out_w));
  a.div_ohw = make_fastdiv(uint32_t(int64_t(g.out_h) * g.out_w));
  a.stages_per_split = 0;
  a.splits = 1;
  a.m_step = 0;
  return a;
}

}  // namespace i8conv
