// Two-pass row-streaming 3x3 kernel for 128-channel layers on gfx950 INT8
// MFMA: the row-streaming halo kernel (kernel_row.hip) reorganised so that
// its MFMAs start after half of the workgroup's copies instead of all of
// them.
//
// Why.  A row-streaming workgroup copies its padded input rows and its
// filter slice (16 output channels x 9 x 128 bytes per wave) into LDS
// before most of its MFMAs can run: from the second input row on, every
// row needs all nine taps.  At kernel start the L2s are cold and all 256
// compute units copy at once, so that copy (about 120 KB per workgroup on
// a 28x28x128 layer) is the longest single phase of the kernel.
//
// How.  Both operands are split by 64-channel group (cg = 0, 1) and copied
// group by group: first the group-0 half of every input row and of the
// filter, then the group-1 halves.  Pass 0 walks the input rows with the
// group-0 data only and accumulates every output row of the block in
// registers (R rows x NFR fragments); pass 1 repeats the walk with group 1
// and completes output row ir - 2 at input row ir, which is stored one
// input row later.
// Pass 0 needs half of the bytes, and the group-1 copies land while it runs.
//
// Layouts.  Input: one LDS plane per (group, padded row): wp pixels x 80
// bytes (the group's 64 channels, then 16 bytes of padding), so the 16
// pixels of a fragment hit 16 distinct 16-byte bank groups (pitch 5 units).
// Filter: per wave, 18 1 KB halves (group-major, then tap): 16 output
// channels x 64 bytes in the swz64 layout, copied with the swizzle applied
// at the source.  Each wave copies and reads only its own filter rows.
//
// Reuse and MFMAs are as in kernel_row.hip: the fragment of input row ir at
// column offset fx feeds output rows ir - fy for fy = 0, 1, 2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>

#include "halo_common.hpp"

namespace i8conv {
namespace {

constexpr int kGroups = 2;      // 64-channel groups: c == 128
constexpr int kUnits = 5;       // 16-byte units per pixel in a plane (4 data + 1 pad)
constexpr int kTaps = 9;
constexpr int kHalves = kTaps * kGroups;  // 1 KB filter halves per wave

// Everything the kernel reads; loaded into SGPRs in one batch.
struct PassArgs {
  const int8_t *x;
  const int8_t *w;
  const int32_t *bias;
  int32_t *y;
  uint32_t x_bytes, w_bytes;
  uint32_t y_bytes;  // output bytes (< 2^31: checked at launch)
  int n, h, wd, c, pad_h, pad_w;
  int out_h, out_w, gemm_n, gemm_k;
  int hp, wp;        // padded rows per image, padded columns
  int plane_copies;  // 1 KB copies per plane: ceil(wp * 5 / 64)
  int rows_in;       // input rows per block: R + 2
  int blocks, tiles_n;
  FastDiv3 div_plane_copies, div_hp, div_blocks, div_tiles_n;
};

template <int R, int NFR>
struct PassState {
  v4i wf[kTaps];           // this wave's 16 channels, one group, all taps (t = fy*3 + fx)
  v4i acc[R][NFR];         // output rows of the block
  v4i frag[3][NFR];        // fragments of the next input row (column offsets 0, 1, 2)
  int colofs[3][NFR];      // LDS offset of this lane's column + fx / k-block in a plane
  const int8_t *planes;    // group-0 planes, then group-1 planes
  int plane_bytes;
  // Output, vector path: a buffer resource over y, this lane's byte offset
  // of output row 0 per fragment (out of range where the column or the
  // channels fall outside the layer: the store is dropped, no branch), and
  // the byte stride between output rows (a scalar offset per row).
  __amdgpu_buffer_rsrc_t yr;
  uint32_t voff[NFR];
  uint32_t row_stride;

  __device__ __forceinline__ void load_row(const int8_t *plane) {
#pragma unroll
    for (int fx = 0; fx < 3; ++fx)
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        frag[fx][j] = *reinterpret_cast<const v4i *>(plane + colofs[fx][j]);
  }

  // Input row IR of group G: MFMAs into output rows IR - fy (compile-time
  // valid ones); in pass 1, output row IR - 2 is then complete and stored.
  template <int G, int IR>
  __device__ __forceinline__ void step(const PassArgs &p, bool vec, int rows_out, int m_row0,
                                       int oc0, int lane) {
    v4i cur[3][NFR];
#pragma unroll
    for (int fx = 0; fx < 3; ++fx)
#pragma unroll
      for (int j = 0; j < NFR; ++j) cur[fx][j] = frag[fx][j];
    if (IR + 1 < R + 2) {
      load_row(planes + (G * p.rows_in + IR + 1) * plane_bytes);
      // keep the reads here: the scheduler would otherwise sink them to their use
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int fx = 0; fx < 3; ++fx) {
#pragma unroll
      for (int fy = 0; fy < 3; ++fy) {
        const int o = IR - fy;  // a constant once the loops are unrolled
        if (o >= 0 && o < R) {
#pragma unroll
          for (int j = 0; j < NFR; ++j) acc[o][j] = mfma16(wf[fy * 3 + fx], cur[fx][j], acc[o][j]);
        }
      }
    }
    // Output row IR - 2 is complete after this row's MFMAs; it is stored one
    // row later, so that its accumulators are read long after the MFMAs that
    // wrote them (reading them right away would stall the wave until those
    // MFMAs drained, every row).
    if (G == kGroups - 1 && IR >= 3)
      store_row<(IR >= 3 ? IR - 3 : 0)>(p, vec, rows_out, m_row0, oc0, lane);
  }

  // Output row O: the accumulators already hold bias + dot products.  N % 4
  // == 0 (and a 16-byte aligned output): one 16-byte buffer store per
  // fragment (write-through, kStoreThrough) at a scalar row offset, no
  // address arithmetic; otherwise element stores.
  template <int O>
  __device__ __forceinline__ void store_row(const PassArgs &p, bool vec, int rows_out, int m_row0,
                                            int oc0, int lane) {
    if (O >= rows_out) return;
    if (vec) {
#pragma unroll
      for (int j = 0; j < NFR; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(acc[O][j], yr, voff[j], O * row_stride,
                                               kStoreThrough);
      return;
    }
    const int m_row = m_row0 + O * p.out_w;
#pragma unroll
    for (int j = 0; j < NFR; ++j) {
      const int col = 16 * j + (lane & 15);
      if (col >= p.out_w) continue;
      int32_t *dst = p.y + size_t(m_row + col) * size_t(p.gemm_n) + oc0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (oc0 + e < p.gemm_n) store_out1(dst + e, acc[O][j][e]);
    }
  }

  template <int G, size_t... I>
  __device__ __forceinline__ void pass(const PassArgs &p, bool vec, int rows_out, int m_row0,
                                       int oc0, int lane, std::index_sequence<I...>) {
    (step<G, int(I)>(p, vec, rows_out, m_row0, oc0, lane), ...);
  }
};

// Cross-wave signals in LDS: a wave adds 1 to a counter once its copies
// have landed (its own vmcnt says so: LDS-DMA data is in LDS when the count
// drops), and a consumer polls the counter.  The wait is bounded: after
// kSpinLimit polls (far beyond any real copy time) it gives up, so every
// wave always reaches the end of the kernel.
constexpr int kSpinLimit = 1 << 20;

__device__ __forceinline__ void flag_add(uint32_t addr) {
  asm volatile("ds_add_u32 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(addr), "v"(1) : "memory");
}

__device__ __forceinline__ void flag_wait(uint32_t addr, int target) {
  for (int spin = 0; spin < kSpinLimit; ++spin) {
    int v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    if (__builtin_amdgcn_readfirstlane(v) >= target) return;
    __builtin_amdgcn_s_sleep(1);
  }
}

// Eight waves: waves 0-3 run the MFMAs (16 output channels each), waves 4-7
// only copy the group-1 half of the operands.  A wave that is issuing copies
// stalls while the compute unit's memory pipeline is full (all 256 compute
// units copy at once at kernel start), so the MFMA waves issue only the
// group-0 copies and the copy waves issue the group-1 copies after them:
// pass 0 starts as soon as group 0 has landed, while group 1 is still
// arriving.  Signals: flag 0 counts MFMA waves whose group-0 copies have
// landed, flag 1 copy waves whose group-1 copies have landed.
template <int R, int NFR>
__global__ __launch_bounds__(2 * kThreads, 1) void rowpass_kernel(PassArgs p_arg) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const PassArgs p = p_arg;
  pin_sgprs(p);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool copier = wave_id >= 4;
  // the MFMA wave this wave is (or copies the group-1 filter rows for)
  const int wave = wave_id & 3;

  const int rest = int(fast_div(blockIdx.x, p.div_tiles_n));
  const int tn = int(blockIdx.x) - rest * p.tiles_n;
  const int b = int(fast_div(uint32_t(rest), p.div_blocks));
  const int q = rest - b * p.blocks;
  const int oy0 = int((int64_t(q) * p.out_h) / p.blocks);
  const int rows_out = int((int64_t(q + 1) * p.out_h) / p.blocks) - oy0;  // <= R
  const int tile_n = tn * 64;

  // LDS: [bias, 256 B per wave][planes: group 0 rows, group 1 rows]
  //      [ring: 18 KB per wave][flags]
  const int8_t *bias_lds = smem + wave * 256;
  PassState<R, NFR> st;
  st.planes = smem + kHaloBiasLds;
  st.plane_bytes = p.plane_copies * 1024;
  const int8_t *ring = st.planes + kGroups * p.rows_in * st.plane_bytes;
  const uint32_t flags = lds_addr(ring) + uint32_t(4 * kHalves * 1024);
  const v4u xd = make_desc(p.x, p.x_bytes);
  const v4u wd = make_desc(p.w, p.w_bytes);
  const uint32_t planes_lds = lds_addr(st.planes);

  // Copies of the group-G plane of every input row, every fourth one from
  // copy number `wave`: copy qq covers units [64j, 64j + 64) of row rr's
  // plane; unit u of pixel pix is slot pix*5 + u (u == 4: padding, left out
  // of range -> zeros).
  const int plane_total = p.rows_in * p.plane_copies;
  auto copy_planes = [&](int g) {
    for (int qq = wave; qq < plane_total; qq += 4) {
      const int rr = int(fast_div(uint32_t(qq), p.div_plane_copies));
      const int j = qq - rr * p.plane_copies;
      const int vr = b * p.hp + oy0 + rr;
      const int bb = int(fast_div(uint32_t(vr), p.div_hp));
      const int iy = vr - bb * p.hp - p.pad_h;
      const bool row_ok = bb < p.n && unsigned(iy) < unsigned(p.h);
      // modulo 2^32: exact wherever it is used (the sum below is in [0, 2^31))
      const uint32_t row_off = uint32_t((bb * p.h + iy) * p.wd - p.pad_w) * uint32_t(p.c) + uint32_t(64 * g);
      const int slot = j * 64 + lane;
      const int pix = slot / kUnits;
      const int u = slot - pix * kUnits;
      const bool ok = row_ok && u < kUnits - 1 && unsigned(pix - p.pad_w) < unsigned(p.wd);
      const uint32_t off = ok ? row_off + uint32_t(pix * p.c + 16 * u) : kOutOfRange;
      lds_copy16(xd, planes_lds + uint32_t((g * p.rows_in + rr) * st.plane_bytes + j * 1024), off);
    }
  };
  // Filter halves of group G for MFMA wave `wave`: lane -> filter row
  // 16*wave + lane/4 and 16-byte chunk lane%4, holding the chunk swz64 puts
  // in that slot.
  const int frow = lane >> 2;
  const int fchunk = swz64_chunk(frow, lane & 3);
  const int oc_copy = tile_n + wave * 16 + frow;
  const uint32_t fbase = oc_copy < p.gemm_n
                             ? uint32_t(oc_copy) * uint32_t(p.gemm_k) + uint32_t(16 * fchunk)
                             : kOutOfRange;
  const uint32_t ring_lds = lds_addr(ring) + uint32_t(wave * kHalves * 1024);
  auto copy_filter = [&](int g) {
#pragma unroll
    for (int t = 0; t < kTaps; ++t)
      lds_copy16(wd, ring_lds + uint32_t((g * kTaps + t) * 1024),
                 fbase + uint32_t(t * 128 + g * 64));
  };

  if (copier) {
    __syncthreads();  // the MFMA waves have issued the group-0 copies
    copy_planes(1);
    copy_filter(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) flag_add(flags + 4);
    return;
  }

  if (wave == 0 && lane == 0) {
    // both flags start at zero; published by the barrier below, before any add
    asm volatile("ds_write_b64 %0, %1" ::"v"(flags), "v"(uint64_t(0)) : "memory");
  }
  stage_bias<1>(p.bias, p.gemm_n, tile_n + wave * 16, bias_lds, lane);
  copy_planes(0);
  copy_filter(0);
  __syncthreads();

  auto take_filter = [&](int g) {
    const int8_t *src = ring + (wave * kHalves + g * kTaps) * 1024;
#pragma unroll
    for (int t = 0; t < kTaps; ++t)
      st.wf[t] = *reinterpret_cast<const v4i *>(src + t * 1024 + swz64(lane & 15, lane >> 4));
  };
#pragma unroll
  for (int fx = 0; fx < 3; ++fx)
#pragma unroll
    for (int j = 0; j < NFR; ++j) {
      // columns past the padded row (read only for dropped lanes) are clamped
      const int col = min(16 * j + (lane & 15) + fx, p.wp - 1);
      st.colofs[fx][j] = col * (16 * kUnits) + 16 * (lane >> 4);
    }
  const int m_row0 = (b * p.out_h + oy0) * p.out_w;
  const int oc0 = tile_n + wave * 16 + 4 * (lane >> 4);
  const bool vec = (p.gemm_n & 3) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0;
  st.yr = make_rsrc(p.y, p.y_bytes);
  st.row_stride = uint32_t(p.out_w) * uint32_t(p.gemm_n) * 4u;
#pragma unroll
  for (int j = 0; j < NFR; ++j) {
    const int col = 16 * j + (lane & 15);
    st.voff[j] = col < p.out_w && oc0 < p.gemm_n
                     ? (uint32_t(m_row0 + col) * uint32_t(p.gemm_n) + uint32_t(oc0)) * 4u
                     : kOutOfRange;
  }

  // Pass 0 once the bias and every wave's group-0 planes and filter halves
  // have landed.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (lane == 0) flag_add(flags);
  flag_wait(flags, 4);
  take_filter(0);
  st.load_row(st.planes);
  // the accumulators start at the bias (the oracle adds the bias first)
  const v4i bv = *reinterpret_cast<const v4i *>(bias_lds + 16 * (lane >> 4));
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NFR; ++j) st.acc[r][j] = bv;
  st.template pass<0>(p, vec, rows_out, m_row0, oc0, lane, std::make_index_sequence<R + 2>{});
  // Pass 1 once the copy waves' group-1 copies have landed (no store has
  // been issued yet).
  flag_wait(flags + 4, 4);
  take_filter(1);
  st.load_row(st.planes + p.rows_in * st.plane_bytes);
  st.template pass<1>(p, vec, rows_out, m_row0, oc0, lane, std::make_index_sequence<R + 2>{});
  st.template store_row<R - 1>(p, vec, rows_out, m_row0, oc0, lane);
}

template <int R, int NFR>
int launch_t(const PassArgs &h, size_t blocks, size_t lds, hipStream_t s) {
  auto kern = rowpass_kernel<R, NFR>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(lds));
    if (e != hipSuccess) {
      set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
  }
  hipLaunchKernelGGL(kern, dim3(unsigned(blocks)), dim3(2 * kThreads), lds, s, h);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("two-pass row kernel launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

// Instances: R = 1..8 output rows per block with NFR = 1 or 2 fragments per
// output row (out_w <= 16, 32), R = 1..4 with NFR = 4 (out_w <= 64): an MFMA
// wave has 256 VGPRs when the workgroup runs eight waves, and R x NFR
// accumulators beyond 32 fragments would spill.
int rowpass_nfr(int out_w) {
  const int f = (out_w + 15) / 16;
  return f <= 2 ? f : (f <= 4 ? 4 : 0);
}

int rowpass_max_rows(int nfr) { return nfr == 4 ? 4 : 8; }

size_t rowpass_lds_bytes(int wp, int rows) {
  const size_t plane_copies = (size_t(wp) * kUnits + 63) / 64;
  return size_t(kHaloBiasLds) + size_t(kGroups) * size_t(rows + 2) * plane_copies * 1024 +
         size_t(4) * kHalves * 1024 + 16;
}

int launch_rowpass(const ConvArgs &a, const PatchPlan &p, void *stream) {
  const int R = p.rows - 2;
  const int nfr = rowpass_nfr(a.out_w);
  const int wp = a.wd + 2 * a.pad_w;
  const size_t lds = rowpass_lds_bytes(wp, R);
  if (a.r != 3 || a.s != 3 || a.stride_h != 1 || a.stride_w != 1 || a.dil_h != 1 ||
      a.dil_w != 1 || a.c != 64 * kGroups || R < 1 || nfr == 0 || R > rowpass_max_rows(nfr) ||
      p.bn != 64 ||
      lds > size_t(kLdsBudget) || p.ranges < 1 || wp != a.out_w + 2 ||
      int64_t(a.out_h) > int64_t(p.ranges) * R ||
      int64_t(a.gemm_m) * a.gemm_n * 4 > int64_t(INT32_MAX)) {
    set_error("two-pass row plan out of range");
    return I8CONV_BAD_ARGUMENT;
  }
  PassArgs h{};
  h.x = a.x;
  h.w = a.w;
  h.bias = a.bias;
  h.y = a.y;
  h.x_bytes = a.x_bytes;
  h.w_bytes = a.w_bytes;
  h.y_bytes = uint32_t(int64_t(a.gemm_m) * a.gemm_n * 4);
  h.n = a.n;
  h.h = a.h;
  h.wd = a.wd;
  h.c = a.c;
  h.pad_h = a.pad_h;
  h.pad_w = a.pad_w;
  h.out_h = a.out_h;
  h.out_w = a.out_w;
  h.gemm_n = a.gemm_n;
  h.gemm_k = a.gemm_k;
  h.hp = a.h + 2 * a.pad_h;
  h.wp = wp;
  h.plane_copies = (wp * kUnits + 63) / 64;
  h.rows_in = R + 2;
  h.blocks = p.ranges;
  h.tiles_n = p.tiles_n;
  h.div_plane_copies = make_fastdiv3(uint32_t(h.plane_copies));
  h.div_hp = make_fastdiv3(uint32_t(h.hp));
  h.div_blocks = make_fastdiv3(uint32_t(h.blocks));
  h.div_tiles_n = make_fastdiv3(uint32_t(h.tiles_n));
  const size_t grid = size_t(a.n) * size_t(p.ranges) * size_t(p.tiles_n);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define I8_PASS_CASE(RR)                                                   \
  if (R == RR) {                                                           \
    if (nfr == 1) return launch_t<RR, 1>(h, grid, lds, s);                 \
    if (nfr == 2) return launch_t<RR, 2>(h, grid, lds, s);                 \
    if constexpr (RR <= 4) return launch_t<RR, 4>(h, grid, lds, s);        \
  }
  I8_PASS_CASE(1) I8_PASS_CASE(2) I8_PASS_CASE(3) I8_PASS_CASE(4)
  I8_PASS_CASE(5) I8_PASS_CASE(6) I8_PASS_CASE(7) I8_PASS_CASE(8)
#undef I8_PASS_CASE
  set_error("no two-pass row-kernel instance for this plan");
  return I8CONV_BAD_ARGUMENT;
}

}  // namespace i8conv
