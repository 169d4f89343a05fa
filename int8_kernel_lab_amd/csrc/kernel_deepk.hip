// Deep-channel split-K kernel on gfx950 INT8 MFMA: 3x3 stride-1 layers with
// few output pixels and many input channels (the 7x7 and 14x14 stages at
// small batch: 392 pixels x 512 channels x k = 18432 on the 8x7x7x2048
// layer).  The pipelined GEMM's split-K form copies, per workgroup, a
// 128-pixel x 1152-byte im2col slice and a 128-channel x 1152-byte filter
// slice (295 KB) and reads the 9.4 MB filter once per pixel tile (four
// times).  Here a workgroup takes every output pixel of the layer at once:
//
// Work split.  Workgroup (split s, channel tile t): input channels
// [128 s, 128 s + 128) through all nine taps (k = 1152) for output channels
// [32 t, 32 t + 32) and all M output pixels; it writes that slice's int32
// partial sums, partial[s][m][oc]; splitk_reduce_vec (kernel_gemm.hip) then
// adds the splits in split order plus the bias.  Each filter byte is copied
// by exactly one workgroup; the input slice of split s (M pixels x 128
// bytes) is copied by the tiles_n workgroups of that split, which the
// XCD-aware order puts on one XCD (one L2).  Per workgroup on the
// 8x7x7x2048 layer: 36 KB of filter and 50 KB of input fetched.
//
// LDS.  [filter: 9 taps x 2 fragments x 16 channels x 128 bytes, swz128]
// [chunk flags][planes].  Planes: the slice's padded input, pixel (b, row,
// col) at unit b*I + row*S + col*10 (16-byte units; 8 data units, 2 zero);
// S = 10 out_w and I = 10 out_h out_w (mod 32 units) make 16 consecutive
// output pixels 10 units apart modulo 512 bytes even across row and image
// boundaries: with a B fragment read (lane l: pixel l % 16, unit l / 16 +
// 4 h) lanes 0..31 land on 32 distinct units and every four consecutive
// lanes on distinct units modulo 128 bytes, gfx950's conflict-free pattern
// for ds_read_b128 (only a fragment that runs past the last pixel, whose
// extra lanes read the last pixel again, conflicts).  The planes are copied
// as one run of 1 KB LDS-DMA copies over all images; padding pixels, pad
// units and rows outside the images come in as zeros (out-of-range
// offsets), and each pixel's 128-byte line is fetched whole by 8 lanes.
//
// Waves.  Four MFMA waves and four copy waves (copies stall the wave that
// issues them while the compute unit's memory pipeline is full).  The copy
// waves issue the filter (chunk 0), then the planes image by image (chunk
// k ends with the copy that holds image k - 1's last unit), each wave
// following its share of a chunk with a 4-byte LDS-DMA copy of a device word
// holding 1 into its flag of the chunk: a wave's loads land in issue order,
// so four set flags mean the chunk is in LDS.  The copy waves never wait.
// MFMA wave w keeps the slice's 32 x 1152-byte filter in VGPRs (144
// registers) and takes pixel fragments w, w + 4, ...: for each, once the
// chunk of its last pixel's image has landed, 18 B reads (9 taps x 2
// k-halves) feed 36 MFMAs into two accumulators (16 channels each), then
// 16-byte write-through stores of the fragment's partial sums (a pixel's 32
// channels are one 128-byte line).  The waits are bounded like the row
// kernel's; a give-up sets g_deepk_wait_expired (i8conv_wait_expired).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <type_traits>
#include <utility>

#include "halo_common.hpp"

namespace i8conv {

// Set by an MFMA wave whose bounded chunk wait gave up; read and cleared by
// deepk_wait_expired on the host.
__device__ __attribute__((aligned(4))) unsigned int g_deepk_wait_expired;

namespace {

constexpr int kDkUnits = kDeepUnits;          // 16-byte units per plane pixel
constexpr int kDkFilterBytes = 9 * 2 * 2048;  // taps x fragments x 16 rows x 128 B
constexpr int kDkMaxLoads = kDeepMaxLoadsPerWave;  // plane loads per copy wave

// The source word of every flag copy.
__device__ __attribute__((aligned(16))) int g_dk_one[4] = {1, 1, 1, 1};

// The arguments past the preloaded ones (deepk_kernel).
struct DeepArgs {
  int32_t *partial;
  uint32_t partial_bytes;
  int pad_h, pad_w;
  int out_w, gemm_m;
  int S, I;         // plane row / image strides, 16-byte units
  int hp, wp;       // padded rows and columns per image
  int frags;        // 16-pixel fragments over M
  int spin_limit;   // polls of about 64 cycles each per bounded wait (wait_spin_limit())
  FastDiv3 div_hpwp, div_wp, div_ohw, div_ow;
};

template <class F, size_t... J>
__device__ __forceinline__ void for_each_index(F &f, std::index_sequence<J...>) {
  (f(std::integral_constant<int, int(J)>{}), ...);
}

__device__ __forceinline__ bool flags_set(v4i f) {
  return __builtin_amdgcn_readfirstlane(f[0] & f[1] & f[2] & f[3]) != 0;
}

__device__ __forceinline__ void flag_wait(uint32_t addr, int spin_limit) {
  for (int spin = 0; spin < spin_limit; ++spin) {
    v4i v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    if (flags_set(v)) return;
    __builtin_amdgcn_s_sleep(1);
  }
  // the chunk never arrived: one vector store to global memory, which the
  // host finds set after the launch
  __hip_atomic_store(&g_deepk_wait_expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// DeepArgs, the kernel's last argument, read from the kernel-argument
// segment where it is called.  The segment pointer passes through an empty
// asm first, so the compiler cannot hoist the loads to the kernel's entry:
// there they would hold SGPRs that the copy waves' path reuses, and the copy
// waves would wait for them (~0.3 us) before their first copy.  The
// argument's offset: two 8-byte pointers and nine 4-byte words, rounded up
// to the struct's 8-byte alignment.
constexpr uint32_t kDeepArgsOffset = (2 * 8 + 9 * 4 + 7) / 8 * 8;
static_assert(alignof(DeepArgs) == 8, "DeepArgs offset assumes 8-byte alignment");
__device__ __forceinline__ DeepArgs deep_args() {
  uint64_t kp = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
  asm volatile("" : "+s"(kp));
  const auto *src =
      reinterpret_cast<const __attribute__((address_space(4))) uint32_t *>(kp + kDeepArgsOffset);
  static_assert(sizeof(DeepArgs) % 4 == 0, "argument block of whole words");
  uint32_t w[sizeof(DeepArgs) / 4];
#pragma unroll
  for (int i = 0; i < int(sizeof(DeepArgs) / 4); ++i) w[i] = src[i];
  DeepArgs d;
  __builtin_memcpy(&d, w, sizeof(d));
  return d;
}

// The kernel's leading arguments arrive preloaded in SGPRs (this file is
// built with -amdgpu-kernarg-preload-count=11: eleven arguments, thirteen
// words): the input and filter base pointers, the input channels, the
// output channels, the images, h | wd << 16, pad_h | pad_w << 8 and the
// dividers by h*wd and wd (multiplier; add | shift << 1), which is all
// the copy waves use: the split and channel tile of the workgroup, the
// filter rows, the input pixels and their places in the planes.  The rest
// of the arguments (DeepArgs, the MFMA waves' set-up) are loaded from the
// kernel-argument segment, a cold scalar round trip of ~0.3 us after a
// launch enqueued on a stream, while the first copies land.
template <int NF>
__global__ __launch_bounds__(2 * kThreads, 1) void deepk_kernel(
    const int8_t *x_pre, const int8_t *w_pre, uint32_t c_pre, uint32_t gemm_n_pre,
    uint32_t n_pre, uint32_t hw_pre, uint32_t pads_pre, uint32_t div_hw_mul,
    uint32_t div_hw_as, uint32_t div_w_mul, uint32_t div_w_as, DeepArgs p_arg) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  (void)p_arg;  // read through deep_args() on the MFMA waves' path only

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = int(c_pre), gemm_n = int(gemm_n_pre), n = int(n_pre);
  const int h = int(hw_pre & 0xffffu), wd = int(hw_pre >> 16);
  const int pad_h = int(pads_pre & 0xffu), pad_w = int(pads_pre >> 8);
  const int gemm_k = 9 * c;
  const int tiles_n = (gemm_n + 31) >> 5;
  const int grid = (c >> 7) * tiles_n;
  // consecutive work items are one split's channel tiles; with the XCD
  // order (grids of a multiple of 8 workgroups: workgroup i runs on XCD
  // i mod 8) they run on one XCD and share its L2 copy of the input slice
  const int per_xcd = (grid & 7) == 0 ? grid >> 3 : 0;
  const int bid = int(blockIdx.x);
  const int item = per_xcd ? (bid & 7) * per_xcd + (bid >> 3) : bid;
  const int split = int(uint32_t(item) / uint32_t(tiles_n));
  const int tn = item - split * tiles_n;
  const uint32_t base = lds_addr(smem);
  const uint32_t flags = base + uint32_t(kDkFilterBytes);
  const int nchunks = 1 + n;
  // flags of chunk k at flags + 16 k (one word per copy wave); then the
  // MFMA waves' halo flags
  const uint32_t halo_flags = flags + 16u * uint32_t(nchunks);
  const uint32_t planes = base + uint32_t(kDkFilterBytes + deep_flags_bytes(n));

  if (wave_id == 0) {
    // every flag starts at zero before any flag write can land
    for (int k = lane; k <= nchunks; k += 64)
      asm volatile("ds_write_b128 %0, %1" ::"v"(flags + 16u * uint32_t(k)), "v"(v4i{0, 0, 0, 0})
                   : "memory");
  }
  // The workgroup barrier orders wave 0's flag writes before every flag
  // write and flag read; it waits for LDS operations only.  The copy waves
  // pass it once their filter copies are issued: those may land at any
  // time, the flags only after it.
  auto barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  if (wave_id >= 4) {
    const int cw = wave_id - 4;
    const v4u wdesc = make_desc(w_pre, uint32_t(gemm_n) * uint32_t(gemm_k));
    const v4u one = make_desc(g_dk_one, 16u);
    auto signal = [&](int k) {
      if (lane == 0) lds_copy4(one, flags + 16u * uint32_t(k) + 4u * uint32_t(cw), 0u);
    };
    // chunk 0, the filter: copy j = (tap, fragment a, half) holds rows
    // 8 half .. + 7 of block tap*2 + a; lane -> row 8 half + lane / 8,
    // physical chunk lane % 8 (the logical chunk swz128 puts there)
    const int frow = lane >> 3;
    const int fchunk0 = lane & 7;
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const int j = cw + 4 * i;
      const int blk = j >> 1, half = j & 1;
      const int t = blk >> 1, a = blk & 1;
      const int row = 8 * half + frow;
      const int oc = tn * 32 + 16 * a + row;
      const uint32_t off =
          oc < gemm_n ? uint32_t(oc) * uint32_t(gemm_k) +
                            uint32_t(t * c + split * 128 + 16 * swz128_chunk(row, fchunk0))
                      : kOutOfRange;
      lds_copy16(wdesc, base + uint32_t(blk * 2048 + half * 1024), off);
    }
    // the filter's flag right behind it: a wave's loads land in issue order
    barrier();
    signal(0);
    // chunks 1..n, the planes: load i (8 input pixels, lane -> pixel
    // 8 i + lane / 8, 16-byte unit lane % 8: whole 128-byte lines) goes
    // global -> VGPRs -> its place in the padded planes; this wave takes
    // i = cw, cw + 4, ..., issues them all, then writes each as it lands
    // and sets its flag of chunk k once it has written every one of its
    // loads that holds a pixel of image k - 1 (LDS writes of a wave land in
    // order, so the flag lands after them)
    const uint32_t col0 = uint32_t(split * 128);
    const int hw = h * wd;
    const int npix = n * hw;
    const auto xr = make_rsrc(x_pre, uint32_t(npix) * uint32_t(c));
    const int loads = (npix + 7) >> 3;
    const int nload = loads > cw ? (loads - cw + 3) / 4 : 0;  // <= kDkMaxLoads
    const int u = lane & 7;
    const FastDiv3 div_hw{div_hw_mul, div_hw_as & 1u, div_hw_as >> 1};
    const FastDiv3 div_w{div_w_mul, div_w_as & 1u, div_w_as >> 1};
    // plane strides (deep_row_units, deep_image_units)
    const int out_h = h + 2 * pad_h - 2, out_w = wd + 2 * pad_w - 2;
    const int S = deep_up_mod32_d((wd + 2 * pad_w) * kDkUnits, 10 * out_w);
    const int I = deep_up_mod32_d((h + 2 * pad_h) * S, 10 * out_h * out_w);
    // Exactly kDkMaxLoads loads per wave, those past the wave's share out of
    // range (no memory access): the wait for load j is then the constant
    // vmcnt(kDkMaxLoads - 1 - j).  (A run-time vmcnt needs a switch per wait;
    // 24 of them made the kernel larger than the instruction cache.)
    v4i data[kDkMaxLoads];
#pragma unroll
    for (int j = 0; j < kDkMaxLoads; ++j) {
      const int pix = 8 * (cw + 4 * j) + (lane >> 3);
      data[j] = load16(xr, j < nload && pix < npix
                               ? uint32_t(pix) * uint32_t(c) + col0 + 16u * uint32_t(u)
                               : kOutOfRange);
    }
    auto signal_ds = [&](int k) {
      if (lane == 0)
        asm volatile("ds_write_b32 %0, %1" ::"v"(flags + 16u * uint32_t(k) + 4u * uint32_t(cw)),
                     "v"(1)
                     : "memory");
    };
    // last load holding a pixel of image k - 1
    auto last_load = [&](int k) { return (k * hw - 1) >> 3; };
    int kdone = 1;
    while (kdone <= n && last_load(kdone) < cw) signal_ds(kdone++);
    auto step = [&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if (j >= nload) return;
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDkMaxLoads - 1 - j) : "memory");
      const int pix = 8 * (cw + 4 * j) + (lane >> 3);
      if (pix < npix) {
        const int b = int(fast_div(uint32_t(pix), div_hw));
        const int rem = pix - b * hw;
        const int iy = int(fast_div(uint32_t(rem), div_w));
        const int ix = rem - iy * wd;
        const uint32_t unit =
            uint32_t(b * I + (iy + pad_h) * S + (ix + pad_w) * kDkUnits + u);
        *reinterpret_cast<__attribute__((address_space(3))) v4i *>(size_t(planes + 16u * unit)) =
            data[j];
      }
      const int next = cw + 4 * (j + 1);
      while (kdone <= n && last_load(kdone) < next) signal_ds(kdone++);
    };
    for_each_index(step, std::make_index_sequence<kDkMaxLoads>{});
    while (kdone <= n) signal_ds(kdone++);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    return;
  }

  // the remaining arguments, in one batch, after the barrier (which then
  // waits for wave 0's flag writes only)
  barrier();
  const DeepArgs p = deep_args();
  pin_sgprs(p);
  // MFMA wave: zero the halo pixels of the planes (the padding rows and
  // columns every tap may read; units 0..7), a quarter each, then flag it
  const int wv = wave_id;
  {
    const int hpwp = p.hp * p.wp;
    for (int j = lane + 64 * wv; j < n * hpwp; j += 256) {
      const int b = int(fast_div(uint32_t(j), p.div_hpwp));
      const int r = j - b * hpwp;
      const int prow = int(fast_div(uint32_t(r), p.div_wp));
      const int pcol = r - prow * p.wp;
      const bool inside = unsigned(prow - p.pad_h) < unsigned(h) &&
                          unsigned(pcol - p.pad_w) < unsigned(wd);
      if (!inside) {
        auto *z = reinterpret_cast<__attribute__((address_space(3))) v4i *>(
            size_t(planes + 16u * uint32_t(b * p.I + prow * p.S + pcol * kDkUnits)));
#pragma unroll
        for (int e = 0; e < 8; ++e) z[e] = v4i{0, 0, 0, 0};
      }
    }
    if (lane == 0)
      asm volatile("s_waitcnt lgkmcnt(0)\n\tds_write_b32 %0, %1" ::"v"(halo_flags + 4u * uint32_t(wv)),
                   "v"(1)
                   : "memory");
  }
  flag_wait(halo_flags, p.spin_limit);
  // the slice's filter into VGPRs
  flag_wait(flags, p.spin_limit);
  v4i A[9][2][2];
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int hk = 0; hk < 2; ++hk)
#pragma unroll
      for (int a = 0; a < 2; ++a)
        A[t][hk][a] = *reinterpret_cast<const v4i *>(
            smem + (t * 2 + a) * 2048 + swz128(lane & 15, 4 * hk + (lane >> 4)));

  const auto pr = make_rsrc(p.partial, p.partial_bytes);
  const int ohw = p.gemm_m / n;
  // B fragment base address of fragment f for this lane; lanes past the
  // last pixel read the last pixel again (never stored)
  auto frag_addr = [&](int f) {
    const int mc = min(16 * f + (lane & 15), p.gemm_m - 1);
    const int b = int(fast_div(uint32_t(mc), p.div_ohw));
    const int rem = mc - b * ohw;
    const int oy = int(fast_div(uint32_t(rem), p.div_ow));
    const int ox = rem - oy * p.out_w;
    return planes + 16u * uint32_t(b * p.I + oy * p.S + ox * kDkUnits + (lane >> 4));
  };
  auto bread = [&](uint32_t addr, int t, int hk) {
    const uint32_t tap = 16u * uint32_t((t / 3) * p.S + (t % 3) * kDkUnits + 4 * hk);
    return *reinterpret_cast<const __attribute__((address_space(3))) v4i *>(size_t(addr + tap));
  };
  // Stores of whole 128-byte lines (a pixel's 32 channels): lane (g, px)
  // = (lane / 16, lane % 16) holds channels 4 g .. + 3 of pixel px in acc0
  // and 16 + 4 g .. in acc1; rotating acc1 by 8 lanes within each row of 16
  // pairs each pixel's two halves, so one store writes pixels 0..7 of the
  // fragment whole and the other pixels 8..15 (two 64-byte halves of a line
  // from two write-through stores went out as two partial writes).
  const uint32_t sbase = uint32_t(split) * uint32_t(p.gemm_m);
  auto store_frag = [&](int f, v4i acc0, v4i acc1) {
    v4i r;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      r[e] = __builtin_amdgcn_update_dpp(0, acc1[e], 0x128, 0xf, 0xf, false);  // row_ror:8
    const int g = lane >> 4, px = lane & 15;
    const bool lo = px < 8;
    const v4i da = lo ? acc0 : r, db = lo ? r : acc0;
    const int ma = 16 * f + (lo ? px : px - 8), mb = 16 * f + (lo ? px + 8 : px);
    const int oca = tn * 32 + (lo ? 4 * g : 16 + 4 * g), ocb = tn * 32 + (lo ? 16 + 4 * g : 4 * g);
    if (ma < p.gemm_m && oca < gemm_n)
      store_out4<kStoreThrough>(pr, ((sbase + uint32_t(ma)) * uint32_t(gemm_n) + uint32_t(oca)) * 4u, da);
    if (mb < p.gemm_m && ocb < gemm_n)
      store_out4<kStoreThrough>(pr, ((sbase + uint32_t(mb)) * uint32_t(gemm_n) + uint32_t(ocb)) * 4u, db);
  };
  // One fragment at a time, four accumulator chains (channel fragment a x
  // k-half hk), B fragments two taps ahead of the MFMAs that use them; the
  // partial sums of the two k-halves are added at the end (int32 addition
  // wraps, so the sum is exact).  Measured: ~40 cycles per MFMA in this
  // loop against 16 in the row kernel's walk, with two, four or eight
  // chains and with the B reads replaced by registers; taking two
  // fragments at a time (each filter operand feeding two consecutive
  // MFMAs) gave ~32 cycles per MFMA but started later, 13.5 against
  // 12.8 us per layer.
#pragma unroll 1
  for (int i = 0; i < NF; ++i) {
    const int f = wv + 4 * i;
    if (f >= p.frags) break;
    const uint32_t addr = frag_addr(f);
    // the chunk of the image of the fragment's last pixel (every unit the
    // fragment reads is in that image or an earlier one)
    const int last = min(16 * f + 15, p.gemm_m - 1);
    const int need = int(fast_div(uint32_t(last), p.div_ohw)) + 1;
    flag_wait(flags + 16u * uint32_t(need), p.spin_limit);
    v4i acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int hk = 0; hk < 2; ++hk) acc[a][hk] = v4i{0, 0, 0, 0};
    v4i bq[3][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int hk = 0; hk < 2; ++hk) bq[t][hk] = bread(addr, t, hk);
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      if (t + 2 < 9) {
        bq[(t + 2) % 3][0] = bread(addr, t + 2, 0);
        bq[(t + 2) % 3][1] = bread(addr, t + 2, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int hk = 0; hk < 2; ++hk)
#pragma unroll
        for (int a = 0; a < 2; ++a) acc[a][hk] = mfma16(A[t][hk][a], bq[t % 3][hk], acc[a][hk]);
      __builtin_amdgcn_sched_barrier(0);
    }
    store_frag(f, add_wrap4(acc[0][0], acc[0][1]), add_wrap4(acc[1][0], acc[1][1]));
  }
}

}  // namespace

bool plan_deepk(const i8conv_shape &s, const i8conv_geometry &g, DeepPlan *out) {
  if (s.r != 3 || s.s != 3 || s.stride_h != 1 || s.stride_w != 1 || s.dilation_h != 1 ||
      s.dilation_w != 1 || s.c % 128 != 0 || s.c < 256 || g.gemm_n % 4 != 0 ||
      s.h >= 65536 || s.w >= 65536 || s.pad_h >= 256 || s.pad_w >= 256)
    return false;  // (h | w << 16 and pad_h | pad_w << 8 are preloaded argument words)
  const int64_t hp = int64_t(s.h) + 2 * s.pad_h, wp = int64_t(s.w) + 2 * s.pad_w;
  if (g.out_h != hp - 2 || g.out_w != wp - 2 || g.out_h < 1 || g.out_w < 1) return false;
  const int64_t frags = (g.gemm_m + 15) / 16;
  const int64_t nf = (frags + 3) / 4;
  if (nf > kDeepMaxFrags) return false;
  const int64_t S = deep_row_units(wp, g.out_w);
  const int64_t I = deep_image_units(hp, S, g.out_h, g.out_w);
  const int64_t units = int64_t(s.n) * I;
  const int64_t loads = (int64_t(s.n) * s.h * s.w + 7) / 8;
  if ((loads + 3) / 4 > kDkMaxLoads) return false;
  // chunk flags (filter, one per image) and the MFMA waves' halo flags
  const int64_t flags_bytes = deep_flags_bytes(s.n);
  const int64_t lds = kDkFilterBytes + flags_bytes + units * 16;
  if (lds > kLdsBudget) return false;
  const int64_t splits = s.c / 128, tiles_n = (g.gemm_n + 31) / 32;
  if (splits * tiles_n > INT32_MAX || splits * g.gemm_m * g.gemm_n * 4 > INT32_MAX) return false;
  DeepPlan p;
  p.S = int(S);
  p.I = int(I);
  p.loads = int(loads);
  p.frags = int(frags);
  p.nf = int(nf);
  p.splits = int(splits);
  p.tiles_n = int(tiles_n);
  p.flags_lds = kDkFilterBytes;
  p.planes_lds = int(kDkFilterBytes + flags_bytes);
  p.lds = size_t(lds);
  if (out) *out = p;
  return true;
}

int launch_deepk(const ConvArgs &a, const DeepPlan &p, void *workspace, void *stream) {
  const FastDiv3 div_hw = make_fastdiv3(uint32_t(a.h * a.wd));
  const FastDiv3 div_w = make_fastdiv3(uint32_t(a.wd));
  if (a.h >= 65536 || a.wd >= 65536 || a.c % 128 != 0 || a.pad_h < 0 || a.pad_h >= 256 ||
      a.pad_w < 0 || a.pad_w >= 256 || p.S != deep_up_mod32_d((a.wd + 2 * a.pad_w) * kDkUnits, 10 * a.out_w) ||
      p.I != deep_up_mod32_d((a.h + 2 * a.pad_h) * p.S, 10 * a.out_h * a.out_w) ||
      int64_t(a.c / 128) * ((a.gemm_n + 31) / 32) != int64_t(p.splits) * p.tiles_n ||
      p.planes_lds != kDkFilterBytes + deep_flags_bytes(a.n) ||
      (int64_t(a.n) * a.h * a.wd + 7) / 8 != p.loads) {
    set_error("deep-channel split-K: plan and shape disagree");
    return I8CONV_BAD_ARGUMENT;
  }
  DeepArgs h{};
  h.partial = static_cast<int32_t *>(workspace);
  h.spin_limit = wait_spin_limit();
  h.partial_bytes = uint32_t(int64_t(p.splits) * a.gemm_m * a.gemm_n * 4);
  h.pad_h = a.pad_h;
  h.pad_w = a.pad_w;
  h.out_w = a.out_w;
  h.gemm_m = a.gemm_m;
  h.S = p.S;
  h.I = p.I;
  h.hp = a.h + 2 * a.pad_h;
  h.wp = a.wd + 2 * a.pad_w;
  h.frags = p.frags;
  const int64_t grid = int64_t(p.splits) * p.tiles_n;
  h.div_hpwp = make_fastdiv3(uint32_t(h.hp * h.wp));
  h.div_wp = make_fastdiv3(uint32_t(h.wp));
  h.div_ohw = make_fastdiv3(uint32_t(a.out_h * a.out_w));
  h.div_ow = make_fastdiv3(uint32_t(a.out_w));
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto run = [&](auto kern) {
    if (p.lds > 64 * 1024) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               int(p.lds));
      if (e != hipSuccess) {
        set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
        return I8CONV_HIP_ERROR;
      }
    }
    I8_LAUNCH(kern, dim3(unsigned(grid)), dim3(2 * kThreads), p.lds, s, a.x, a.w,
                       uint32_t(a.c), uint32_t(a.gemm_n), uint32_t(a.n),
                       uint32_t(a.h) | uint32_t(a.wd) << 16,
                       uint32_t(a.pad_h) | uint32_t(a.pad_w) << 8, div_hw.mul,
                       div_hw.add | div_hw.shift << 1, div_w.mul, div_w.add | div_w.shift << 1, h);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      set_error(std::string("deep-channel split-K launch: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
    return I8CONV_OK;
  };
  switch (p.nf) {
    case 1: return run(deepk_kernel<1>);
    case 2: return run(deepk_kernel<2>);
    case 3: return run(deepk_kernel<3>);
    case 4: return run(deepk_kernel<4>);
    case 5: return run(deepk_kernel<5>);
    case 6: return run(deepk_kernel<6>);
    case 7: return run(deepk_kernel<7>);
    case 8: return run(deepk_kernel<8>);
    default: break;
  }
  set_error("no deep-channel split-K instance for this plan");
  return I8CONV_BAD_ARGUMENT;
}

int deepk_wait_expired(int *expired) {
  void *word = nullptr;
  hipError_t e = hipGetSymbolAddress(&word, HIP_SYMBOL(g_deepk_wait_expired));
  if (e != hipSuccess) {
    set_error(std::string("hipGetSymbolAddress(g_deepk_wait_expired): ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  unsigned int v = 0;
  e = hipMemcpy(&v, word, sizeof(v), hipMemcpyDeviceToHost);
  if (e == hipSuccess && v != 0) {
    const unsigned int zero = 0;
    e = hipMemcpy(word, &zero, sizeof(zero), hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    set_error(std::string("reading g_deepk_wait_expired: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  *expired = v != 0 ? 1 : 0;
  return I8CONV_OK;
}

}  // namespace i8conv
