// Host-side internals shared by the C ABI, the planners and the launchers.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>

#include "i8conv.h"
#include "i8conv_device.hpp"

#ifdef __HIPCC__
#include <hip/hip_ext.h>
#endif

#ifdef __HIPCC__
// Launches a kernel on the lab's conv path; kernels launched while the
// measurement loop has set launch_events() carry its events.
#define I8_LAUNCH(kern, grid, block, lds, stream, ...)                                    \
  do {                                                                                  \
    ::i8conv::LaunchEvents &ev_ = ::i8conv::launch_events();                            \
    if (ev_.start || ev_.stop) {                                                        \
      hipExtLaunchKernelGGL(kern, grid, block, lds, stream, ev_.start, ev_.stop, 0,       \
                            __VA_ARGS__);                                               \
      ev_.start = nullptr;                                                              \
    } else {                                                                            \
      hipLaunchKernelGGL(kern, grid, block, lds, stream, __VA_ARGS__);                  \
    }                                                                                   \
  } while (0)
#endif

namespace i8conv {

constexpr int kThreads = 256;      // 4 wave64 per workgroup
constexpr int kStageBytes = 128;   // k-bytes per LDS stage of the GEMM kernels
constexpr int kLdsBudget = 160 * 1024;

void set_error(const std::string &message);

// Validity + derived geometry (include/conv_shape.cuh:22-35).
int derive(const i8conv_shape &s, i8conv_geometry *g);

// ---- generic / split-K -----------------------------------------------------
// Workgroup tile of the staged implicit GEMM: BM output pixels x BN output
// channels, k staged 128 bytes at a time.
// Deep-channel split-K plan (kernel_deepk.hip): a workgroup per (128-channel
// input slice, 32-channel output tile) over all M pixels; planes and filter
// layout in LDS (16-byte units).
constexpr int kDeepMaxFrags = 8;  // 16-pixel fragments per MFMA wave (M <= 512)
// Planes: padded input pixel (b, row, col) at 16-byte unit b*I + row*S +
// col*kDeepUnits (8 data units, 2 zero).  S = 10 out_w and I = 10 out_h out_w
// modulo 32 units keep 16 consecutive output pixels 10 units apart modulo
// 512 bytes across row and image boundaries (conflict-free B fragment
// reads; tests/layout_check.cpp).
constexpr int kDeepUnits = 10;
inline int64_t deep_up_mod32(int64_t v, int64_t target) {
  const int64_t t = ((target % 32) + 32) % 32;
  return v + ((t - v % 32) + 32) % 32;
}
// The same on 32-bit values, for the device (|v|, |target| < 2^31).
I8_HD constexpr int deep_up_mod32_d(int v, int target) {
  return v + ((((target & 31) - (v & 31)) + 32) & 31);
}
inline int64_t deep_row_units(int64_t wp, int64_t out_w) {
  return deep_up_mod32(wp * kDeepUnits, 10 * out_w);
}
inline int64_t deep_image_units(int64_t hp, int64_t row_units, int64_t out_h, int64_t out_w) {
  return deep_up_mod32(hp * row_units, 10 * out_h * out_w);
}
constexpr int kDeepMaxLoadsPerWave = 24;  // 1 KB plane loads per copy wave (<= 768 pixels)
// Bytes of the chunk flags (filter, one per image) and the MFMA waves' halo
// flags, in whole 256-byte blocks (the planes follow them).
I8_HD constexpr int64_t deep_flags_bytes(int64_t n) { return ((16 * (2 + n) + 255) / 256) * 256; }
struct DeepPlan {
  int S = 0, I = 0;       // plane row / image strides
  int loads = 0;          // 1 KB plane loads (8 input pixels each)
  int frags = 0, nf = 0;  // fragments over M, per MFMA wave
  int splits = 0, tiles_n = 0;
  int flags_lds = 0, planes_lds = 0;
  size_t lds = 0;
};
bool plan_deepk(const i8conv_shape &s, const i8conv_geometry &g, DeepPlan *out);

struct GemmPlan {
  int bm = 0, bn = 0;
  int splits = 1;            // > 1 only for split-K
  int stages = 0;            // ceil(gemm_k / 128)
  int stages_per_split = 0;
  // pipelined kernel: pixel rows each tile stores (bm, or fewer to even out
  // the last round of workgroups; the tile's remaining rows are zeros)
  int m_step = 0;
  // c % 128 == 0: the LDS-DMA pipelined kernel (kernel_gemm_dma.hip), else
  // the register-staged one (kernel_gemm.hip)
  bool dma = false;
  // split-K only: the deep-channel kernel instead of the GEMM
  bool deep = false;
  DeepPlan deep_plan;
  // generic only: 1x1 stride-1 unpadded layer whose filter fits a wave's
  // registers, run by the pointwise streaming kernel (kernel_pointwise.hip)
  // when the four pointers are 16-byte aligned; the tile fields above then
  // describe the fallback GEMM for unaligned pointers
  bool pw = false;
  int pw_waves = 0;
};
bool gemm_tile_supported(int bm, int bn);
bool gemm_dma_tile_supported(int bm, int bn);
// copy-only waves the pipelined kernel adds to a workgroup of this plan (0:
// every wave copies and runs MFMAs)
int gemm_dma_copy_waves(const GemmPlan &p);
GemmPlan plan_generic(const i8conv_shape &s, const i8conv_geometry &g);
int gemm_dma_step(int64_t gemm_m, int64_t tiles_n, int bm, int bn);
GemmPlan plan_splitk(const i8conv_shape &s, const i8conv_geometry &g);
size_t splitk_workspace_bytes(const i8conv_geometry &g, const GemmPlan &p);

// ---- halo / strip ----------------------------------------------------------
// 2-D output tile (th rows x tw columns of one image) x bn output channels.
// halo : the whole input patch of one 64-channel group is staged in LDS and
//        reused by all r*s taps.
// strip: one input row per output row of the tile (filter row fy) is staged
//        per (channel group, fy) and reused by the s horizontal taps.
struct PatchPlan {
  int th = 0, tw = 0, bn = 0;
  int ph = 0, pw = 0;          // staged region (pixels) of one stage
  int stage_pixels = 0;        // ph * pw
  int tiles_y = 0, tiles_x = 0, tiles_n = 0;
  int frags_m = 0;             // ceil(th * tw / 16)
  int loads_per_thread = 0;    // 16-byte chunks each thread stages per stage
  bool strip = false;
  // halo only: flattened pixel ranges with their input rows of every channel
  // group resident in LDS and the filter slice in registers (kernel_halo.hip)
  bool resident = false;
  // halo, 3x3 stride 1: output-row blocks streamed row by row with the
  // taps formed in registers (kernel_row.hip); `ranges` = blocks per image
  bool row = false;
  // row-streaming, 128 channels: the form with copy waves (kernel_rowpass.hip)
  bool streamed = false;
  int ranges = 0;  // resident: pixel ranges per channel slice
  int rows = 0;    // resident: most padded input rows any range needs
  int ring = 0;    // resident: filter staging slots in LDS
};
bool plan_halo(const i8conv_shape &s, const i8conv_geometry &g, PatchPlan *p);
bool plan_strip(const i8conv_shape &s, const i8conv_geometry &g, PatchPlan *p);

// Dispatch policy (policy.cpp): an eligible kernel id, or -1 for a bad shape.
int dispatch(const i8conv_shape &s);

ConvArgs make_args(const i8conv_shape &s, const i8conv_geometry &g,
                   const int8_t *x, const int8_t *w, const int32_t *bias,
                   int32_t *y);

// Launchers (asynchronous; return an i8conv_status).
struct RequantArgs;
int launch_gemm(const ConvArgs &a, const GemmPlan &p, void *stream);
// rq: the reduce writes requantized int8 output instead of int32 (needs
// N % 4 == 0, 16-byte aligned bias, workspace, multipliers and shifts and a
// 4-byte aligned output)
int launch_splitk(const ConvArgs &a, const GemmPlan &p, void *workspace,
                  void *stream, const RequantArgs *rq = nullptr);
// kernel_gemm_dma.hip; splits > 1 writes partial sums to a.partial
int launch_gemm_dma(const ConvArgs &a, const GemmPlan &p, int splits, void *stream);
// kernel_pointwise.hip: C and N with an instance (C in {64, 128, 256,
// 512}, N in {32, 64, 128, 256}), the output-channel slices it splits N
// into (each of 16384 / C channels, at most N), the waves of a launch, its
// launch, and the pointer alignment it needs (16 bytes each)
constexpr int kPwMaxWaves = 1024;  // waves per launch, at most
// waves per workgroup: one per slice, two for one slice
constexpr int pw_group_waves(int slices) { return slices < 2 ? 2 : slices; }
bool pointwise_supported(int c, int n);
int pointwise_slices(int c, int n);
int pointwise_waves(int64_t gemm_m, int slices);
// rq: requantized int8 output instead of int32 (needs
// pointwise_requant_supported and 16-byte aligned mult, shift and output)
int launch_pointwise(const ConvArgs &a, const RequantArgs *rq, void *stream);
bool pointwise_pointers_ok(const ConvArgs &a);
// slices of 64 or 128 channels
bool pointwise_requant_supported(int c, int n);
int launch_patch(const ConvArgs &a, const PatchPlan &p, void *stream);
int launch_halo_resident(const ConvArgs &a, const PatchPlan &p, void *stream);
int launch_row(const ConvArgs &a, const PatchPlan &p, void *stream);
// Requantized int8 output (kernel_requant.hip): per output channel k,
// y = clamp(zero_point + round(acc * mult[k] / 2^shift[k]), -128, 127).
struct RequantArgs {
  const int32_t *mult;
  const int32_t *shift;
  int32_t zero_point;
  int8_t *y;  // NHWK int8
};
int launch_requant(const int32_t *acc, int64_t pixels, int32_t channels, const int32_t *mult,
                   const int32_t *shift, int32_t zero_point, int8_t *out, void *stream);
// kernel_layout.hip: batched [rows][cols] -> [cols][rows] of esize-byte
// elements (1 or 4), and NHWC <-> N, C/vect, H, W, vect packing.
int launch_transpose(const void *src, void *dst, int64_t batch, int rows, int cols, int esize,
                     void *stream);
int launch_pack_vect(const int8_t *src, int8_t *dst, int n, int h, int w, int c, int vect,
                     bool unpack, void *stream);
// q == nullptr: int32 output to a.y; else the requantized int8 output to
// q->y, computed in the kernel's epilogue (a.y unused)
int launch_rowpass(const ConvArgs &a, const PatchPlan &p, void *stream,
                   const RequantArgs *q = nullptr);
// kernel_rowpass.hip: fragments per output row of its instance for out_w
// (0: none), and its LDS bytes for wp padded columns and `rows` output rows
int rowpass_nfr(int out_w);
// ... and the most output rows per block it has an instance for
int rowpass_max_rows(int nfr);
size_t rowpass_lds_bytes(int wp, int rows);
// kernel_rowpass.hip: reads and clears the device word its waves set when a
// bounded wait gives up (synchronizes the device); *expired = 1 if it was set.
int rowpass_wait_expired(int *expired);
// capi.hip: polls each bounded chunk wait of the row kernel with copy waves
// and the deep-channel split-K makes before it gives up; read at launch
// (i8conv_set_wait_spin_limit; 2^20 by default)
int wait_spin_limit();
// capi.hip: events that the next kernel launches of this host thread carry
// (hipExtLaunchKernel), set only by the measurement loop: `start` is taken
// by the first kernel launched and cleared, `stop` by every kernel launched
// while it is set (the last one's end stands).  Both null otherwise.
#ifdef __HIPCC__
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
LaunchEvents &launch_events();
#endif
int launch_deepk(const ConvArgs &a, const DeepPlan &p, void *workspace, void *stream);
int deepk_wait_expired(int *expired);
// kernel_probe.hip: a store-only kernel (16-byte buffer stores, write-through
// or ordinary) over `bytes` of y (a multiple of 16, below 2^31) in the
// launch shape workgroups x threads with `lds` bytes of dynamic LDS.
int launch_store_floor(int32_t *y, size_t bytes, int workgroups, int threads, size_t lds,
                       bool write_through, void *stream);
// kernel_probe.hip: the LDS read probe, pattern 0..5 (linear, swz128,
// stride128, stride256, xor_rows, pitch80), `iters` 16-byte reads per lane; sink holds
// workgroups * threads int32.
int launch_lds_probe(int pattern, int32_t *sink, int workgroups, int threads, int iters,
                     void *stream);
// Whether kernel_row.hip has an instance for 16*fn channels per wave, cg
// 64-channel groups and nfr 16-column fragments per output row.
bool row_instance_exists(int fn, int cg, int nfr);
// Whether kernel_halo.hip has an instance for 16*fn channels per wave and
// `steps` 64-byte k-steps.
bool halo_instance_exists(int fn, int steps);
// kernel_halo.hip stages the filter through a ring of up to kHaloRing LDS
// slots of 64*fn rows x 128 bytes each, after the input rows.
constexpr int kHaloRing = 8;
// ... and keeps the bias of each wave's channels in the first kHaloBiasLds
// bytes (256 per wave), before the input rows.
constexpr int kHaloBiasLds = 1024;
inline size_t halo_ring_slot_bytes(int fn) { return size_t(64) * fn * 128; }
// LDS layout of one padded input row in kernel_halo.hip: wp pixels of
// `units` 16-byte units each (all c channels, then one pad unit), written by
// row_copies 1 KB copy instructions.  Rows are row_bytes apart, with
// row_bytes / 16 >= 64 * row_copies (a row's copies never spill into the
// next row) and row_bytes / 16 == row_units (mod 16), so the 16-byte bank
// groups keep cycling across a row boundary as they do inside a row.
struct HaloRowLayout {
  int64_t units, row_units, row_copies, row_bytes;
};
// Padding units after each pixel's c bytes: one for the halo kernel (an odd
// pitch, whose strided fragment reads stay spread over the banks), two for
// the row kernel (pitch c + 32: 2 x odd units for c % 64 == 0, which makes
// its stride-1 fragment reads conflict-free by gfx950's ds_read_b128 bank
// rule; with c + 16 they were 2-way conflicts).
constexpr int kHaloPadUnits = 1;
constexpr int kRowPadUnits = 2;
inline HaloRowLayout halo_row_layout(int64_t wp, int64_t c, int pad_units) {
  HaloRowLayout l;
  l.units = c / 16 + pad_units;
  l.row_units = wp * l.units;
  l.row_copies = (l.row_units + 63) / 64;
  const int64_t span = 64 * l.row_copies;
  l.row_bytes = 16 * (span + ((l.row_units - span) % 16 + 16) % 16);
  return l;
}

}  // namespace i8conv
