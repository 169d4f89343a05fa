// Row-streaming 3x3 kernel on gfx950 INT8 MFMA: the halo-tiled variant for
// stride-1, dilation-1 3x3 layers, built so that each input byte staged in
// LDS is read once per channel group instead of once per tap.
//
// Work split.  A workgroup takes a block of consecutive output rows of one
// image (and one 64*FN-channel slice of K); its padded input rows (the block
// plus two) are copied into LDS once, as in kernel_halo.hip.  Output rows are
// cut into ceil(out_w / 16) fragments of 16 consecutive columns (NFR per row;
// lanes past out_w are computed and dropped).
//
// Reuse.  The B fragment of tap (fy, fx) for output pixels (oy, x0..x0+15)
// is input row oy + fy, columns x0 + fx .. x0 + fx + 15, and it is the same
// fragment for the three output rows oy = ir - fy that input row ir feeds.
// So the kernel walks the input rows once: for input row ir and channel
// group cg it reads the 3 * NFR fragments at column offsets fx = 0, 1, 2 (one
// LDS read each) and feeds each one to the output rows ir, ir - 1, ir - 2
// (taps fy = 0, 1, 2), FN MFMAs per row, whose accumulators rotate through
// three register sets: when input row ir is done, output row ir - 2 is
// complete and is stored at once, so stores are spread over the whole
// kernel.  Each B read feeds 3 * FN MFMAs (FN in a per-tap walk): about
// 1024 / (3 * FN) LDS bytes per 16-cycle MFMA per SIMD, a third of the LDS
// read rate, so the MFMAs are no longer fed at LDS speed.  (Forming the
// fx = 1, 2 fragments from the fx = 0 ones with DPP lane moves would save
// LDS reads the kernel does not need to save; the VALU moves contend with
// the MFMA issue of the single wave per SIMD and measured slower.)
//
// Filter.  Each wave keeps its 16*FN channels x 9*c bytes in VGPRs for the
// whole workgroup (stationary A).  It streams in through the same per-wave
// LDS ring as in kernel_halo.hip, in k order (fy-major), and the first three
// input rows only need taps fy <= ir, so the fetch overlaps their MFMAs.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "halo_common.hpp"

namespace i8conv {
namespace {

// The arguments of the walk and the stores (the copies' come preloaded:
// see row_kernel).
struct RowArgs {
  int32_t *y;
  int n, out_h, out_w, gemm_n;
  int row_bytes;    // LDS bytes between consecutive rows
};

// RowArgs, the kernel's last argument, read from the kernel-argument segment
// where it is called.  The segment pointer passes through an empty asm, so
// the compiler cannot hoist the loads to the kernel's entry, where they would
// hold SGPRs that the copy code reuses and make it wait for them (~0.3 us)
// before its first copy.  The offset: three 8-byte pointers and five 4-byte
// words, rounded up to the struct's 8-byte alignment.
constexpr uint32_t kRowArgsOffset = (3 * 8 + 5 * 4 + 7) / 8 * 8;
static_assert(alignof(RowArgs) == 8, "RowArgs offset assumes 8-byte alignment");
__device__ __forceinline__ RowArgs row_args() {
  uint64_t kp = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
  asm volatile("" : "+s"(kp));
  const auto *src =
      reinterpret_cast<const __attribute__((address_space(4))) uint32_t *>(kp + kRowArgsOffset);
  static_assert(sizeof(RowArgs) % 4 == 0, "argument block of whole words");
  uint32_t w[sizeof(RowArgs) / 4];
#pragma unroll
  for (int i = 0; i < int(sizeof(RowArgs) / 4); ++i) w[i] = src[i];
  RowArgs r;
  __builtin_memcpy(&r, w, sizeof(r));
  return r;
}

// Padded input rows vr0 .. vr0 + nrows - 1 (image-major: row hp of image b
// is row 0 of image b + 1) into LDS, 1 KB LDS-DMA copies dealt round-robin
// to the four waves, as copy_input_rows (halo_common.hpp) but with the
// pixel's 16-byte units a compile-time count (c = 64 CG) and no run-time
// dividers: a wave's copies q = wave, wave + 4, ... walk the (row, copy)
// pairs in order, and a row past the image's last (vr0's image b, at most
// hp rows later) is the next image's.
template <int CG>
__device__ __forceinline__ void copy_rows_pre(v4u xd, uint32_t lds0, int b, int oy0, int nrows,
                                              int wave, int lane, int row_copies, int row_bytes,
                                              int hp, int n, int h, int wd, int pad_h,
                                              int pad_w) {
  constexpr int kC = 64 * CG;
  constexpr int kUnits = kC / 16 + kRowPadUnits;
  int rr = 0, j = wave;
  while (j >= row_copies) {
    j -= row_copies;
    ++rr;
  }
  for (; rr < nrows;) {
    const int pr = oy0 + rr;
    const int bb = b + (pr >= hp ? 1 : 0);
    const int iy = pr - (pr >= hp ? hp : 0) - pad_h;
    const bool row_ok = bb < n && unsigned(iy) < unsigned(h);
    // modulo 2^32: exact wherever it is used (the sum below is in [0, 2^31))
    const uint32_t row_off = uint32_t((bb * h + iy) * wd - pad_w) * uint32_t(kC);
    const int slot = j * 64 + lane;
    const int pix = slot / kUnits;
    const int u = slot - pix * kUnits;
    const bool ok = row_ok && u < (kC >> 4) && unsigned(pix - pad_w) < unsigned(wd);
    const uint32_t off = ok ? row_off + uint32_t(pix * kC + 16 * u) : kOutOfRange;
    lds_copy16(xd, lds0 + rr * row_bytes + j * 1024, off);
    j += 4;
    while (j >= row_copies) {
      j -= row_copies;
      ++rr;
    }
  }
}

template <int FN, int CG, int NFR>
struct RowState {
  static constexpr int kSteps = 9 * CG;
  v4i wf[kSteps][FN];       // stationary filter fragments, k-step t = (fy*3 + fx)*CG + cg
  v4i acc[3][NFR][FN];      // output rows ir, ir - 1, ir - 2 rotate through these
  int colofs[3][NFR];       // LDS offset of this lane's column + fx / k-block in a row
};

// Input row ir (K == ir % 3, compile time, fixes the accumulator roles):
// the fragments of every channel group at the three column offsets fx, and
// the filter rows fy in MASK (bit fy; compile time, so the MFMAs of a row
// form one straight-line block).  Each fragment feeds the output rows
// ir - fy of every fy in MASK, FN MFMAs each.  With kCheck, a filter row
// also needs 0 <= ir - fy < rows_out at run time (blocks of fewer than two
// rows, whose first and last rows overlap).
//
// `frag` holds the fragments of (ir, channel group 0) on entry and those of
// (ir + 1, channel group 0) on return: each group's reads are issued before
// the MFMAs of the previous one, so with one wave per SIMD the LDS latency
// is hidden behind MFMAs instead of stalling them.  The last input row (only
// filter row 2 left: MASK 4, or 7 in a one-row block) reads row 0 again.
template <int FN, int CG, int NFR, int kPolicy, int K, int MASK, bool kCheck>
__device__ __forceinline__ void row_step(const RowArgs &p, RowState<FN, CG, NFR> &st,
                                         v4i (&frag)[3][NFR], const int8_t *rows,
                                         const int8_t *bias_lds, int ir, int rows_out,
                                         int m_row0, int tile_n, int wave, int lane) {
  constexpr int s0 = K, s1 = (K + 2) % 3, s2 = (K + 1) % 3;  // sets of rows ir, ir-1, ir-2
  if (MASK & 1) {  // output row ir starts here
#pragma unroll
    for (int j = 0; j < NFR; ++j)
#pragma unroll
      for (int i = 0; i < FN; ++i) st.acc[s0][j][i] = v4i{0, 0, 0, 0};
  }
  const bool v0 = (MASK & 1) && (!kCheck || ir < rows_out);
  const bool v1 = (MASK & 2) && (!kCheck || (ir >= 1 && ir - 1 < rows_out));
  const bool v2 = (MASK & 4) && (!kCheck || (ir >= 2 && ir - 2 < rows_out));
  const int8_t *row = rows + ir * p.row_bytes;
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    v4i cur[3][NFR];
#pragma unroll
    for (int fx = 0; fx < 3; ++fx)
#pragma unroll
      for (int j = 0; j < NFR; ++j) cur[fx][j] = frag[fx][j];
    constexpr bool kLast = MASK == 4 || (kCheck && MASK == 7);
    const int8_t *next = cg + 1 < CG ? row + (cg + 1) * 64 : kLast ? rows : row + p.row_bytes;
#pragma unroll
    for (int fx = 0; fx < 3; ++fx)
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        frag[fx][j] = *reinterpret_cast<const v4i *>(next + st.colofs[fx][j]);
    // keep the reads here: the scheduler would otherwise sink them to their use
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int fx = 0; fx < 3; ++fx) {
      if ((MASK & 1) && (!kCheck || v0)) {
#pragma unroll
        for (int j = 0; j < NFR; ++j)
#pragma unroll
          for (int i = 0; i < FN; ++i)
            st.acc[s0][j][i] = mfma16(st.wf[(0 + fx) * CG + cg][i], cur[fx][j], st.acc[s0][j][i]);
      }
      if ((MASK & 2) && (!kCheck || v1)) {
#pragma unroll
        for (int j = 0; j < NFR; ++j)
#pragma unroll
          for (int i = 0; i < FN; ++i)
            st.acc[s1][j][i] = mfma16(st.wf[(3 + fx) * CG + cg][i], cur[fx][j], st.acc[s1][j][i]);
      }
      if ((MASK & 4) && (!kCheck || v2)) {
#pragma unroll
        for (int j = 0; j < NFR; ++j)
#pragma unroll
          for (int i = 0; i < FN; ++i)
            st.acc[s2][j][i] = mfma16(st.wf[(6 + fx) * CG + cg][i], cur[fx][j], st.acc[s2][j][i]);
      }
    }
  }
  if (!(MASK & 4) || (kCheck && !v2)) return;
  // output row ir - 2 is complete: bias + stores
  v4i bv[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i)
    bv[i] = *reinterpret_cast<const v4i *>(bias_lds + (i * 16 + 4 * (lane >> 4)) * 4);
  const int m_row = m_row0 + (ir - 2) * p.out_w;
  // output window: this output row's out_w pixels
  const OutWindow ow = out_window(p.y, int64_t(p.n) * p.out_h * p.out_w, p.gemm_n, m_row, p.out_w);
  const bool vec = (p.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && ow.ok;
#pragma unroll
  for (int j = 0; j < NFR; ++j) {
    const int col = 16 * j + (lane & 15);
    if (col >= p.out_w) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int oc0 = tile_n + wave * 16 * FN + i * 16 + 4 * (lane >> 4);
      const v4i v = add_wrap4(st.acc[s2][j][i], bv[i]);
      if (vec) {
        if (oc0 < p.gemm_n)
          store_out4<kPolicy>(ow.r, (uint32_t(col) * uint32_t(p.gemm_n) + uint32_t(oc0)) * 4u, v);
      } else {
        int32_t *dst = p.y + size_t(m_row + col) * size_t(p.gemm_n) + oc0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (oc0 + e < p.gemm_n) store_out1(dst + e, v[e]);
      }
    }
  }
}

// Takes ring chunks [C0, C1) (chunk c = k-steps 2c, 2c + 1) into st.wf.
template <int FN, int CG, int NFR, int C0, int C1>
__device__ __forceinline__ void take_chunks(FilterRing<FN, 9 * CG> &ring,
                                            RowState<FN, CG, NFR> &st) {
#pragma unroll
  for (int c = C0; c < C1; ++c) ring.take(c, st.wf);
}

// kPolicy: the output store policy, write-through where the pixel pitch is
// sector-aligned (sector_pitch), else ordinary.
// The leading arguments arrive preloaded in SGPRs (this file is built with
// -amdgpu-kernarg-preload-count=8: eight arguments, eleven words): the
// input, filter and bias pointers, the images, h | wd << 16, pad_h | pad_w
// << 8 | blocks << 16 (row blocks per image), the output channels and ring |
// rows << 8 (filter ring slots, LDS input rows), from which every copy is
// derived; RowArgs follows for the walk.  The grid is (channel tiles, row
// blocks, images).
template <int FN, int CG, int NFR, int kPolicy>
__global__ __launch_bounds__(kThreads, 1) void row_kernel(
    const int8_t *x_pre, const int8_t *w_pre, const int32_t *bias_pre, uint32_t n_pre,
    uint32_t hw_pre, uint32_t pads_pre, uint32_t gemm_n_pre, uint32_t ring_pre, RowArgs p_arg) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  (void)p_arg;  // read through row_args() once the copies are issued
  constexpr int kSteps = 9 * CG;
  constexpr int kChunks = (kSteps + 1) / 2;
  constexpr int kC = 64 * CG;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // bit 31 of n_pre: the grid groups images by XCD (below)
  const bool by_xcd = (n_pre >> 31) != 0;
  const int n = int(n_pre & 0xffffu);
  const int h = int(hw_pre & 0xffffu), wd = int(hw_pre >> 16);
  const int pad_h = int(pads_pre & 0xffu), pad_w = int((pads_pre >> 8) & 0xffu);
  const int blocks = int(pads_pre >> 16);
  const int gemm_n = int(gemm_n_pre);
  const int ring_slots = int(ring_pre & 0xffu), rows_lds = int(ring_pre >> 8);
  const int hp = h + 2 * pad_h, wp = wd + 2 * pad_w;
  const int out_h = hp - 2;
  // the LDS row layout (halo_row_layout with kRowPadUnits)
  constexpr int kUnits = kC / 16 + kRowPadUnits;
  const int row_units = wp * kUnits;
  const int row_copies = (row_units + 63) >> 6;
  const int row_bytes = 16 * (64 * row_copies + (((row_units - 64 * row_copies) % 16) + 16) % 16);

  // grid: (channel tiles, row blocks, images), or with by_xcd (n % 8 == 0)
  // (8 x channel tiles, row blocks, images / 8) with blockIdx.x = x + 8 tn
  // and image 8 blockIdx.z + x: workgroup i of a launch runs on XCD i mod 8
  // = x, so every workgroup of an image runs on one XCD, whose L2 fetches
  // the image's rows from HBM once for all of them.
  const int tn = by_xcd ? int(blockIdx.x >> 3) : int(blockIdx.x);
  const int q = int(blockIdx.y);
  const int b = by_xcd ? int(8 * blockIdx.z + (blockIdx.x & 7)) : int(blockIdx.z);
  // out_h < 2^16 and q < blocks <= out_h: the products fit in 32 bits
  const int oy0 = int(uint32_t(q * out_h) / uint32_t(blocks));
  const int rows_out = int(uint32_t((q + 1) * out_h) / uint32_t(blocks)) - oy0;
  const int tile_n = tn * 64 * FN;

  const int8_t *bias_lds = smem + wave * 256;
  stage_bias<FN>(bias_pre, gemm_n, tile_n + wave * 16 * FN, bias_lds, lane);

  // padded input rows oy0 .. oy0 + rows_out + 1 of image b
  const int8_t *rows = smem + kHaloBiasLds;
  copy_rows_pre<CG>(make_desc(x_pre, uint32_t(n) * uint32_t(h) * uint32_t(wd) * uint32_t(kC)),
                    lds_addr(rows), b, oy0, rows_out + 2, wave, lane, row_copies, row_bytes, hp,
                    n, h, wd, pad_h, pad_w);

  FilterRing<FN, kSteps> ring;
  ring.wd = make_desc(w_pre, uint32_t(gemm_n) * uint32_t(9 * kC));
  ring.ptr = rows + rows_lds * row_bytes;
  ring.lds = lds_addr(ring.ptr);
  ring.slots = ring_slots;
  ring.cur = 0;
  ring.wave = wave;
  ring.lane = lane;
  ring.init(tile_n, gemm_n, 9 * kC);
  // A wave whose output channels all lie past N (the last waves of a slice
  // when N is not a multiple of 64 FN: K = 36 keeps three of four) issues
  // only its share of the input-row copies.  It skips its filter stream and
  // its walk: it waits for its row copies and joins the barrier that
  // publishes the input rows (taking chunk 0, the other waves join it), then
  // ends.  Each wave copies and reads only its own filter rows, so nothing
  // else reads what it leaves out.  (16x28x28x64, K = 36: 4.137-4.138 ->
  // 4.069-4.073 us per launch, same box; a quarter fewer MFMAs issued.)
  if (tile_n + wave * 16 * FN >= gemm_n) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    return;
  }
  for (int c = 0; c < ring.slots && c < kChunks; ++c) ring.issue(c, c);

  const RowArgs p = row_args();
  pin_sgprs(p);
  RowState<FN, CG, NFR> st;
#pragma unroll
  for (int fx = 0; fx < 3; ++fx)
#pragma unroll
    for (int j = 0; j < NFR; ++j) {
      // columns past the padded row (read only for dropped lanes) are clamped
      const int col = min(16 * j + (lane & 15) + fx, wp - 1);
      st.colofs[fx][j] = col * (kC + 16 * kRowPadUnits) + 16 * (lane >> 4);
    }
  const int m_row0 = (b * out_h + oy0) * p.out_w;

  // Input row ir feeds output rows ir - fy (fy = 0, 1, 2) that exist:
  // row 0 only fy = 0, row 1 fy <= 1, rows 2 .. rows_out - 1 all three, row
  // rows_out fy >= 1 and row rows_out + 1 only fy = 2.  The first rows need
  // only the filter rows fy <= ir, so the chunks holding taps fy = 0 (k-steps
  // [0, 3*CG)), fy = 1 and fy = 2 are taken just before rows 0, 1 and 2;
  // taking chunk 0 also publishes the input rows (its barrier).
  constexpr int kC1 = (3 * CG + 1) / 2, kC2 = (6 * CG + 1) / 2;
#define I8_ROW(K, MASK, CHECK, IR)                                                         \
  row_step<FN, CG, NFR, kPolicy, K, MASK, CHECK>(p, st, frag, rows, bias_lds, IR, rows_out, m_row0, \
                                        tile_n, wave, lane)
  take_chunks<FN, CG, NFR, 0, kC1>(ring, st);
  v4i frag[3][NFR];
#pragma unroll
  for (int fx = 0; fx < 3; ++fx)
#pragma unroll
    for (int j = 0; j < NFR; ++j)
      frag[fx][j] = *reinterpret_cast<const v4i *>(rows + st.colofs[fx][j]);
  if (rows_out < 2) {
    // one output row: input rows 0, 1, 2 with run-time checks
    I8_ROW(0, 1, true, 0);
    take_chunks<FN, CG, NFR, kC1, kC2>(ring, st);
    I8_ROW(1, 3, true, 1);
    take_chunks<FN, CG, NFR, kC2, kChunks>(ring, st);
    I8_ROW(2, 7, true, 2);
    return;
  }
  I8_ROW(0, 1, false, 0);
  take_chunks<FN, CG, NFR, kC1, kC2>(ring, st);
  I8_ROW(1, 3, false, 1);
  take_chunks<FN, CG, NFR, kC2, kChunks>(ring, st);
  int ir = 2;
  for (; ir + 2 < rows_out; ir += 3) {
    I8_ROW(2, 7, false, ir);
    I8_ROW(0, 7, false, ir + 1);
    I8_ROW(1, 7, false, ir + 2);
  }
  // 0 to 2 full rows left, then the two rows that only finish earlier ones
  switch (rows_out - ir) {
    case 2:
      I8_ROW(2, 7, false, ir);
      I8_ROW(0, 7, false, ir + 1);
      I8_ROW(1, 6, false, ir + 2);
      I8_ROW(2, 4, false, ir + 3);
      break;
    case 1:
      I8_ROW(2, 7, false, ir);
      I8_ROW(0, 6, false, ir + 1);
      I8_ROW(1, 4, false, ir + 2);
      break;
    default:
      I8_ROW(2, 6, false, ir);
      I8_ROW(0, 4, false, ir + 1);
      break;
  }
#undef I8_ROW
}

// The preloaded leading arguments of row_kernel.
struct RowPre {
  const int8_t *x;
  const int8_t *w;
  const int32_t *bias;
  uint32_t n, hw, pads, gemm_n, ring;
};

template <int FN, int CG, int NFR>
int launch_t(const RowPre &a, const RowArgs &h, dim3 grid, size_t lds, hipStream_t s) {
  auto kern = (h.gemm_n & 7) == 0 ? row_kernel<FN, CG, NFR, kStoreThrough>
                                  : row_kernel<FN, CG, NFR, 0>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(lds));
    if (e != hipSuccess) {
      set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
  }
  I8_LAUNCH(kern, grid, dim3(kThreads), lds, s, a.x, a.w, a.bias, a.n, a.hw, a.pads,
                     a.gemm_n, a.ring, h);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("row kernel launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

bool row_instance_exists(int fn, int cg, int nfr) {
  // (the register budget of 512 per lane caps cg * nfr: the filter slice is
  // 9 * cg * fn fragments and each input row holds 3 * nfr of them twice)
  if (nfr < 1 || nfr > 4 || fn * nfr > 4) return false;
  return (fn == 2 && (cg == 1 || cg == 2)) ||
         (fn == 1 && (cg == 1 || cg == 2 || (cg == 4 && nfr <= 2)));
}

int launch_row(const ConvArgs &a, const PatchPlan &p, void *stream) {
  const int fn = p.bn / 64;
  const int cg = a.c / 64;
  const int nfr = (a.out_w + 15) / 16;
  const HaloRowLayout row = halo_row_layout(a.wd + 2 * a.pad_w, a.c, kRowPadUnits);
  const size_t lds = size_t(kHaloBiasLds) + size_t(p.rows) * size_t(row.row_bytes) +
                     size_t(p.ring) * halo_ring_slot_bytes(fn);
  if (a.r != 3 || a.s != 3 || a.stride_h != 1 || a.stride_w != 1 || a.dil_h != 1 ||
      a.dil_w != 1 || a.c % 64 != 0 || !row_instance_exists(fn, cg, nfr) ||
      lds > size_t(kLdsBudget) || p.ranges < 1 || p.rows < 3 || p.ring < 1 ||
      p.ring > kHaloRing || a.wd + 2 * a.pad_w != a.out_w + 2) {
    set_error("row plan out of range");
    return I8CONV_BAD_ARGUMENT;
  }
  if (a.h >= 65536 || a.wd >= 65536 || a.pad_h < 0 || a.pad_h >= 256 || a.pad_w < 0 ||
      a.pad_w >= 256 || p.ranges >= 65536 || a.n >= 65536 || p.ring >= 256 ||
      int64_t(p.rows) >= (int64_t(1) << 24) || a.out_h != a.h + 2 * a.pad_h - 2) {
    set_error("row plan: geometry beyond the packed kernel arguments");
    return I8CONV_BAD_ARGUMENT;
  }
  RowPre pre;
  pre.x = a.x;
  pre.w = a.w;
  pre.bias = a.bias;
  // n % 8 == 0: the grid groups each image's workgroups on one XCD
  const bool by_xcd = a.n % 8 == 0;
  pre.n = uint32_t(a.n) | (by_xcd ? 0x80000000u : 0u);
  pre.hw = uint32_t(a.h) | uint32_t(a.wd) << 16;
  pre.pads = uint32_t(a.pad_h) | uint32_t(a.pad_w) << 8 | uint32_t(p.ranges) << 16;
  pre.gemm_n = uint32_t(a.gemm_n);
  pre.ring = uint32_t(p.ring) | uint32_t(p.rows) << 8;
  RowArgs h{};
  h.y = a.y;
  h.n = a.n;
  h.out_h = a.out_h;
  h.out_w = a.out_w;
  h.gemm_n = a.gemm_n;
  h.row_bytes = int(row.row_bytes);
  const dim3 grid = by_xcd ? dim3(8 * unsigned(p.tiles_n), unsigned(p.ranges), unsigned(a.n / 8))
                           : dim3(unsigned(p.tiles_n), unsigned(p.ranges), unsigned(a.n));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define I8_ROW_CASE(FN, CG, NFR) \
  if (fn == FN && cg == CG && nfr == NFR) return launch_t<FN, CG, NFR>(pre, h, grid, lds, s);
  I8_ROW_CASE(2, 1, 1) I8_ROW_CASE(2, 1, 2) I8_ROW_CASE(2, 2, 1) I8_ROW_CASE(2, 2, 2)
  I8_ROW_CASE(1, 1, 1) I8_ROW_CASE(1, 1, 2) I8_ROW_CASE(1, 1, 3) I8_ROW_CASE(1, 1, 4)
  I8_ROW_CASE(1, 2, 1) I8_ROW_CASE(1, 2, 2) I8_ROW_CASE(1, 2, 3) I8_ROW_CASE(1, 2, 4)
  I8_ROW_CASE(1, 4, 1) I8_ROW_CASE(1, 4, 2)
#undef I8_ROW_CASE
  set_error("no row-kernel instance for this plan");
  return I8CONV_BAD_ARGUMENT;
}

}  // namespace i8conv
