// Dispatch policy, kept outside the kernels (the reference's workflow,
// README.md:92-99: sweep, then encode the policy outside the kernels while
// eligibility stays an explicit predicate next to each kernel).
//
// The policy only ever returns an eligible kernel.  Its rules:
//   1. split-K when the generic grid cannot fill the chip (fewer than 128
//      workgroups) and the reduction is long (>= 16 stages of 128 k-bytes),
//      e.g. a 7x7 layer with C = 2048;
//   2. otherwise an input-reuse kernel for a spatial filter (r*s > 1):
//      halo when eligible, else strip;
//   3. otherwise the generic implicit GEMM (1x1 layers, C % 64 != 0).
#include "i8conv_internal.hpp"

namespace i8conv {

int dispatch(const i8conv_shape &s) {
  i8conv_geometry g;
  if (derive(s, &g) != I8CONV_OK) return -1;
  const GemmPlan gp = plan_generic(s, g);
  const int64_t tiles = ((g.gemm_m + gp.bm - 1) / gp.bm) *
                        ((int64_t(g.gemm_n) + gp.bn - 1) / gp.bn);
  if (tiles < 128 && gp.stages >= 16) return I8CONV_KERNEL_SPLITK;
  if (int64_t(s.r) * s.s > 1) {
    PatchPlan pp;
    if (plan_halo(s, g, &pp)) return I8CONV_KERNEL_HALO;
    if (plan_strip(s, g, &pp)) return I8CONV_KERNEL_STRIP;
  }
  return I8CONV_KERNEL_GENERIC;
}

}  // namespace i8conv
