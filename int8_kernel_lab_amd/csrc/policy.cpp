// Dispatch policy, kept outside the kernels (the reference's workflow,
// README.md:92-99: sweep, then encode the policy outside the kernels while
// eligibility stays an explicit predicate next to each kernel).
//
// The policy only ever returns an eligible kernel.  Its rules, in order,
// read off a sweep of the reference's 41-layer table on one MI355X:
//   1. the row-streaming 3x3 stride-1 kernel (a halo plan) whenever it has a
//      plan: it won every layer it covers (ResNet/Darknet 3x3 stages,
//      batched 56x56 and 28x28 layers, 14x14 C = 256);
//   2. split-K when the generic grid is tiny (at most 16 tiles) and the
//      reduction long: at least 16 stages of 128 k-bytes, or 8 for a 1x1
//      filter (deep 7x7 / 13x13 / 14x14 layers and stride-2 downsamplers at
//      batch 1: it won all of them; at 24 tiles and 18 stages the generic
//      GEMM won, 15.0 vs 15.7 us, and on a 32x32 3x3 layer of 9 stages the
//      halo kernel, 9.3 vs 11.0 us);
//   3. the pipelined generic GEMM (C % 128 == 0) when its grid has at least
//      128 tiles: large layers of any filter (it beat every halo/strip plan
//      from 28x28 x 32 images up to 256x256 x 16, stride 1 or 2, 3x3 or 5x5,
//      dilated or not);
//   4. otherwise an input-reuse kernel for a stride-1 spatial filter
//      (r*s > 1): halo when eligible, else strip (small dilated layers,
//      asymmetric 1x3/3x1, C = 64 layers wider than the row kernel's four
//      fragments); at stride 2 the generic GEMM beat the halo kernel on
//      every such layer (15.0 vs 18.0 us at 52x52, C = 256);
//   5. otherwise the generic implicit GEMM (1x1 layers, strided layers,
//      C % 64 != 0).
#include <cstring>
#include <mutex>

#include "i8conv_internal.hpp"

namespace i8conv {

namespace {
int dispatch_uncached(const i8conv_shape &s);

// The policy is a pure function of the shape, and its planners search
// (the resident-rows plan of a 64x64 dilated layer takes ~50 us of host
// time), so results are kept in a small direct-mapped cache: launches that
// go through the policy every call (the requantized launch, conv2d) then
// cost a lookup.
struct DispatchEntry {
  i8conv_shape shape;
  int id;
  bool used;
};
constexpr size_t kDispatchCache = 64;
std::mutex g_dispatch_mutex;
DispatchEntry g_dispatch_cache[kDispatchCache];

size_t shape_slot(const i8conv_shape &s) {
  const int *f = reinterpret_cast<const int *>(&s);
  uint32_t h = 2166136261u;  // FNV-1a over the 13 int fields
  for (size_t i = 0; i < sizeof(s) / sizeof(int); ++i) h = (h ^ uint32_t(f[i])) * 16777619u;
  return h % kDispatchCache;
}
}  // namespace

int dispatch(const i8conv_shape &s) {
  static_assert(sizeof(i8conv_shape) == 13 * sizeof(int), "shape fields are 13 ints");
  const size_t slot = shape_slot(s);
  {
    std::lock_guard<std::mutex> lock(g_dispatch_mutex);
    const DispatchEntry &e = g_dispatch_cache[slot];
    if (e.used && std::memcmp(&e.shape, &s, sizeof(s)) == 0) return e.id;
  }
  const int id = dispatch_uncached(s);
  std::lock_guard<std::mutex> lock(g_dispatch_mutex);
  g_dispatch_cache[slot] = DispatchEntry{s, id, true};
  return id;
}

namespace {
int dispatch_uncached(const i8conv_shape &s) {
  i8conv_geometry g;
  if (derive(s, &g) != I8CONV_OK) return -1;
  PatchPlan pp;
  const bool halo = plan_halo(s, g, &pp);
  if (halo && pp.row) return I8CONV_KERNEL_HALO;
  const GemmPlan gp = plan_generic(s, g);
  const int64_t tiles = ((g.gemm_m + gp.bm - 1) / gp.bm) *
                        ((int64_t(g.gemm_n) + gp.bn - 1) / gp.bn);
  const bool spatial = int64_t(s.r) * s.s > 1;
  if (tiles <= 16 && (gp.stages >= 16 || (!spatial && gp.stages >= 8)))
    return I8CONV_KERNEL_SPLITK;
  if (gp.dma && tiles >= 128) return I8CONV_KERNEL_GENERIC;
  if (spatial && s.stride_h == 1 && s.stride_w == 1) {
    if (halo) return I8CONV_KERNEL_HALO;
    if (plan_strip(s, g, &pp)) return I8CONV_KERNEL_STRIP;
  }
  return I8CONV_KERNEL_GENERIC;
}
}  // namespace

}  // namespace i8conv
