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

// Generic tile choice: the output-channel tile is the smallest supported
// width covering N (32/64/128 columns, 128 for wider layers); the pixel
// tile shrinks from 256 until the grid has enough workgroups to cover the
// 256 compute units.
GemmPlan plan_generic(const i8conv_geometry &g) {
  GemmPlan p;
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
  p.stages = int(ceil_div(g.gemm_k, kStageBytes));
  p.splits = 1;
  p.stages_per_split = p.stages;
  return p;
}

// Split-K: the generic tile, with the 128-byte k stages divided among
// enough splits to give about two workgroups per compute unit.
GemmPlan plan_splitk(const i8conv_geometry &g) {
  GemmPlan p;
  p.bn = g.gemm_n <= 32 ? 32 : (g.gemm_n <= 64 ? 64 : 128);
  p.bm = g.gemm_m <= 64 ? 64 : 128;
  if (!gemm_tile_supported(p.bm, p.bn)) p.bm = 128;
  p.stages = int(ceil_div(g.gemm_k, kStageBytes));
  const int64_t tiles = ceil_div(g.gemm_m, p.bm) * ceil_div(g.gemm_n, p.bn);
  int64_t splits = ceil_div(512, tiles);
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

bool finish_patch_plan(const i8conv_shape &s, const i8conv_geometry &g,
                       PatchPlan *p) {
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
                       bool strip, PatchPlan *out) {
  PatchPlan best;
  bool found = false;
  double best_score = -1.0;
  for (int tw = std::min(g.out_w, kMaxTilePixels); tw >= 1; --tw) {
    // only full-width tiles, or widths that split the row evenly
    if (tw != g.out_w && g.out_w % tw != 0) continue;
    const int th_max = std::min(g.out_h, kMaxTilePixels / tw);
    for (int th = th_max; th >= 1; --th) {
      PatchPlan p;
      p.strip = strip;
      p.th = th;
      p.tw = tw;
      p.bn = s.k > 64 ? 128 : 64;
      if (strip) {
        p.ph = th;
        p.pw = tw + s.s - 1;
      } else {
        p.ph = (th - 1) * s.stride_h + (s.r - 1) * s.dilation_h + 1;
        p.pw = (tw - 1) * s.stride_w + (s.s - 1) * s.dilation_w + 1;
      }
      if (!finish_patch_plan(s, g, &p)) continue;
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
// fits the LDS stage.  Any filter size, stride and dilation.
bool plan_halo(const i8conv_shape &s, const i8conv_geometry &g, PatchPlan *p) {
  if (s.c % 64 != 0) return false;
  return search_patch_plan(s, g, false, p);
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
  return search_patch_plan(s, g, true, p);
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
  return a;
}

}  // namespace i8conv
