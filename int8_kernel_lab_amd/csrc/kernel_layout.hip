// Layout transforms around the convolution (the step before and after the
// path; the reference does its packing on the host, src/cudnn_lab.cu:7-18):
//   * batched transpose [rows][cols] -> [cols][rows] of 1- or 4-byte
//     elements: NCHW <-> NHWC int8 activations, NHWK -> NKHW int32 output;
//   * channel-vector packing NHWC (or KRSC) -> N, C/V, H, W, V and back,
//     the layout of the reference's cuDNN INT8x32 path (V = 32).
// All are HBM-bound byte movement.
//
// Tiled transposes (16-byte rows on both sides: rows * esize and cols *
// esize multiples of 16, 16-byte aligned bases): one workgroup per 128 x
// 128-byte tile (bytes: two tiles side by side where the source rows hold
// 256 bytes or more), read as whole 128-byte source row pieces (8 lanes x 16
// bytes), staged in LDS and written as whole 128-byte rows of the transposed
// matrix.  With one side short instead (any length), the short-row and
// short-column forms below run; otherwise an element-per-thread form.
//
// Bytes: each lane takes 16 rows x 4 columns of the tile, reads them as 16
// dwords (4 columns of a row each), turns every 4 x 4 byte block around with
// two levels of v_perm_b32 and stores four 16-byte pieces, one per column: 4
// LDS reads per 16 output bytes.
//
// Byte tile row i sits at dword 32 i + 8 (i / 16): rows start on 16-byte
// boundaries, so the read phase writes whole 16-byte pieces with 32
// consecutive lanes on 32 distinct 16-byte units; and for one row offset the
// 64 lanes of a wave in the write phase (8 row groups 16 rows apart x 8
// consecutive dwords) fall in 64 distinct banks (16 x 32 + 8 = 520 = 8 mod 64).
//
// Packing: one thread per 16-byte piece of the NHWC tensor; V % 16 == 0 and
// C % V == 0, so a piece never straddles a channel vector; reads and writes
// are 16 bytes per lane, pixels consecutive across lanes on both sides.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

constexpr int kTileRowBytes = 128;
constexpr int kLdsPitch = 132;

__device__ __forceinline__ int byte_tile_row(int i) { return 32 * i + 8 * (i >> 4); }

// 4 x 4 byte transpose: a[k] holds row k's bytes of columns 0..3; o[c]
// gets column c's bytes of rows 0..3.  v_perm_b32(s0, s1, sel): byte n of
// the result is byte sel.n of {s0:s1}, s1 supplying bytes 0-3.
__device__ __forceinline__ void transpose4x4(const uint32_t (&a)[4], uint32_t (&o)[4]) {
  const uint32_t lo01 = __builtin_amdgcn_perm(a[1], a[0], 0x05010400u);  // a0.0 a1.0 a0.1 a1.1
  const uint32_t hi01 = __builtin_amdgcn_perm(a[1], a[0], 0x07030602u);  // a0.2 a1.2 a0.3 a1.3
  const uint32_t lo23 = __builtin_amdgcn_perm(a[3], a[2], 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(a[3], a[2], 0x07030602u);
  o[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);  // a0.0 a1.0 a2.0 a3.0
  o[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);  // a0.1 a1.1 a2.1 a3.1
  o[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

template <int kSub>
__global__ __launch_bounds__(kThreads) void transpose_bytes_tiled(const int8_t *src, int8_t *dst,
                                                                  int rows, int cols, int tiles_r,
                                                                  int tiles_c) {
  constexpr int T = kTileRowBytes;
  constexpr int kTileDw = 32 * T + 8 * (T / 16);  // one 128 x 128 tile
  __shared__ __align__(16) uint32_t tile[kSub * kTileDw];
  const int per_mat = tiles_r * tiles_c;
  const int mat = int(blockIdx.x) / per_mat;
  const int t = int(blockIdx.x) - mat * per_mat;
  const int tr = t / tiles_c;
  const int tc = t - tr * tiles_c;
  const size_t mat_bytes = size_t(rows) * size_t(cols);  // < 2^31: checked at launch
  const auto sr = make_rsrc(src + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const auto dr = make_rsrc(dst + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const int r0 = tr * T, c0 = tc * T * kSub;
  // read: tile row i = source row r0 + i, bytes [c0, c0 + 128 kSub); piece
  // pc of the row goes to tile pc / 8
  for (int idx = threadIdx.x; idx < T * 8 * kSub; idx += kThreads) {
    const int i = idx / (8 * kSub), pc = idx % (8 * kSub);
    const uint32_t cb = uint32_t(c0 + pc * 16);
    const bool ok = r0 + i < rows && cb < uint32_t(cols);
    *reinterpret_cast<v4i *>(&tile[(pc >> 3) * kTileDw + byte_tile_row(i) + 4 * (pc & 7)]) =
        load16(sr, ok ? uint32_t(r0 + i) * uint32_t(cols) + cb : kOutOfRange);
  }
  __syncthreads();
  // write: lane (column group cg, row group rg) -> columns 4 cg .. + 3 of
  // each tile, rows r0 + 16 rg .. + 15; the 8 row groups of a column are 8
  // consecutive lanes, so each output row gets 128 contiguous bytes
  const int cg = threadIdx.x >> 3, rg = threadIdx.x & 7;
  const int i0 = 16 * rg;
  if (r0 + i0 >= rows) return;  // rows % 16 == 0: a row group is whole or absent
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    uint32_t out[4][4];  // [column][4-row group]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t a[4], o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] = tile[sub * kTileDw + byte_tile_row(i0 + 4 * q + k) + cg];
      transpose4x4(a, o);
#pragma unroll
      for (int c = 0; c < 4; ++c) out[c][q] = o[c];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int col = c0 + T * sub + 4 * cg + c;
      if (col >= cols) continue;
      const v4i v{int32_t(out[c][0]), int32_t(out[c][1]), int32_t(out[c][2]), int32_t(out[c][3])};
      __builtin_amdgcn_raw_buffer_store_b128(v, dr, uint32_t(col) * uint32_t(rows) + uint32_t(r0 + i0),
                                             0, kStoreThrough);
    }
  }
}

// Dwords: the tile has a 132-byte pitch (33 dwords: the 32 rows of one
// column fall in distinct banks); each lane gathers 4 rows of one column.
__global__ __launch_bounds__(kThreads) void transpose_dwords_tiled(const int8_t *src, int8_t *dst,
                                                                   int rows, int cols, int tiles_r,
                                                                   int tiles_c) {
  constexpr int T = kTileRowBytes / 4;  // tile side in dwords
  __shared__ uint32_t tile[T * kLdsPitch / 4];
  const int per_mat = tiles_r * tiles_c;
  const int mat = int(blockIdx.x) / per_mat;
  const int t = int(blockIdx.x) - mat * per_mat;
  const int tr = t / tiles_c;
  const int tc = t - tr * tiles_c;
  const size_t mat_bytes = size_t(rows) * size_t(cols) * 4;  // < 2^31: checked at launch
  const auto sr = make_rsrc(src + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const auto dr = make_rsrc(dst + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const int r0 = tr * T, c0 = tc * T;
  const uint32_t row_bytes = uint32_t(cols) * 4;
  // read: tile row i = source row r0 + i, bytes [c0*4, c0*4 + 128)
  for (int idx = threadIdx.x; idx < T * 8; idx += kThreads) {
    const int i = idx >> 3, piece = idx & 7;
    const uint32_t cb = uint32_t(c0 * 4 + piece * 16);
    const bool ok = r0 + i < rows && cb < row_bytes;
    const v4i v = load16(sr, ok ? uint32_t(r0 + i) * row_bytes + cb : kOutOfRange);
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[(i * kLdsPitch + piece * 16) / 4 + e] = uint32_t(v[e]);
  }
  __syncthreads();
  // write: output row j = column c0 + j, bytes [r0*4, r0*4 + 128): the lane
  // gathers tile rows i0 .. i0 + 3 of column j (rows % 4 == 0: the 4 rows are
  // all inside the matrix or all outside)
  const uint32_t out_row_bytes = uint32_t(rows) * 4;
  for (int idx = threadIdx.x; idx < T * 8; idx += kThreads) {
    const int j = idx >> 3, piece = idx & 7;
    const int i0 = piece * 4;
    const int c = c0 + j;
    if (c >= cols || r0 + i0 >= rows) continue;
    v4i v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = int32_t(tile[((i0 + e) * kLdsPitch) / 4 + j]);
    __builtin_amdgcn_raw_buffer_store_b128(v, dr, uint32_t(c) * out_row_bytes + uint32_t(r0 + i0) * 4,
                                           0, 0);
  }
}

// Transposes with one short side (any length), the other side's bytes a
// multiple of 16: the short side makes a workgroup's share of one tensor a
// single contiguous byte range, copied as 16-byte pieces; the other tensor
// is read or written as 16-byte pieces of its rows.  Elements change place
// in LDS (ES-byte LDS accesses).  Used when the tiled form cannot run
// (e.g. H x W = 7 x 7 or 14 x 14).
constexpr int kShortLds = 32768;

// Source rows short (cols elements, cols * ES <= kShortLds / 16) and
// rows * ES % 16 == 0: the workgroup takes source rows [r0, r0 + R) (R % 16
// == 0), one contiguous range, and writes R elements of each output row j.
template <int ES>
__global__ __launch_bounds__(kThreads) void transpose_short_rows(const int8_t *src, int8_t *dst,
                                                                 int rows, int cols, int R,
                                                                 int tiles) {
  __shared__ __align__(16) int8_t buf[kShortLds];
  const int mat = int(blockIdx.x) / tiles;
  const int t = int(blockIdx.x) - mat * tiles;
  const size_t mat_bytes = size_t(rows) * size_t(cols) * ES;  // < 2^31: checked at launch
  const auto sr = make_rsrc(src + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const auto dr = make_rsrc(dst + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const int r0 = t * R;
  const int rn = min(R, rows - r0);                     // rn * ES % 16 == 0
  const uint32_t base = uint32_t(r0) * uint32_t(cols) * ES;  // 16-byte aligned: R % 16 == 0
  const uint32_t span = uint32_t(rn) * uint32_t(cols) * ES;  // <= kShortLds, % 16 == 0
  for (uint32_t q = threadIdx.x; q < span / 16; q += kThreads)
    *reinterpret_cast<v4i *>(buf + 16 * q) = load16(sr, base + 16 * q);
  __syncthreads();
  // output row j, piece p: elements r0 + kPer p .. + kPer - 1 of column j;
  // the pieces of one output row are consecutive lanes
  constexpr int kPer = 16 / ES;
  const int pieces = rn / kPer;
  for (int idx = threadIdx.x; idx < cols * pieces; idx += kThreads) {
    const int j = idx / pieces, p = idx - j * pieces;
    v4i v;
    if constexpr (ES == 1) {
      const uint8_t *b = reinterpret_cast<const uint8_t *>(buf) + (16 * p) * cols + j;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) word |= uint32_t(b[(4 * e + k) * cols]) << (8 * k);
        v[e] = int32_t(word);
      }
    } else {
      const int32_t *b = reinterpret_cast<const int32_t *>(buf) + (4 * p) * cols + j;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = b[e * cols];
    }
    __builtin_amdgcn_raw_buffer_store_b128(
        v, dr, (uint32_t(j) * uint32_t(rows) + uint32_t(r0 + kPer * p)) * ES, 0, kStoreThrough);
  }
}

// Output rows short (rows elements, rows * ES <= kShortLds / 16) and
// cols * ES % 16 == 0: the workgroup takes source columns [c0, c0 + W) (W * ES
// % 16 == 0), whose output is one contiguous range: it reads 16-byte pieces
// of every source row, puts each element at its output place in LDS and
// copies LDS out as 16-byte pieces.
template <int ES>
__global__ __launch_bounds__(kThreads) void transpose_short_cols(const int8_t *src, int8_t *dst,
                                                                 int rows, int cols, int W,
                                                                 int tiles) {
  __shared__ __align__(16) int8_t buf[kShortLds];
  const int mat = int(blockIdx.x) / tiles;
  const int t = int(blockIdx.x) - mat * tiles;
  const size_t mat_bytes = size_t(rows) * size_t(cols) * ES;  // < 2^31: checked at launch
  const auto sr = make_rsrc(src + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const auto dr = make_rsrc(dst + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const int c0 = t * W;
  const int cn = min(W, cols - c0);  // cn * ES % 16 == 0
  constexpr int kPer = 16 / ES;
  const int pieces = cn / kPer;  // per source row
  for (int idx = threadIdx.x; idx < rows * pieces; idx += kThreads) {
    const int r = idx / pieces, q = idx - r * pieces;
    const v4i v = load16(sr, (uint32_t(r) * uint32_t(cols) + uint32_t(c0 + kPer * q)) * ES);
    // element c0 + kPer q + e -> output element (kPer q + e) * rows + r
    if constexpr (ES == 1) {
      uint8_t *b = reinterpret_cast<uint8_t *>(buf) + (16 * q) * rows + r;
#pragma unroll
      for (int e = 0; e < 16; ++e) b[e * rows] = uint8_t(uint32_t(v[e >> 2]) >> (8 * (e & 3)));
    } else {
      int32_t *b = reinterpret_cast<int32_t *>(buf) + (4 * q) * rows + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) b[e * rows] = v[e];
    }
  }
  __syncthreads();
  const uint32_t base = uint32_t(c0) * uint32_t(rows) * ES;  // 16-byte aligned: W * ES % 16 == 0
  const uint32_t span = uint32_t(cn) * uint32_t(rows) * ES;  // <= kShortLds, % 16 == 0
  for (uint32_t q = threadIdx.x; q < span / 16; q += kThreads)
    __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const v4i *>(buf + 16 * q), dr,
                                           base + 16 * q, 0, kStoreThrough);
}

template <class E>
__global__ __launch_bounds__(kThreads) void transpose_elements(const E *src, E *dst, int rows,
                                                               int cols, int64_t total) {
  for (int64_t q = int64_t(blockIdx.x) * kThreads + threadIdx.x; q < total;
       q += int64_t(gridDim.x) * kThreads) {
    const int64_t per = int64_t(rows) * cols;
    const int64_t mat = q / per;
    const int64_t rc = q - mat * per;
    const int64_t r = rc / cols, c = rc - (rc / cols) * cols;
    dst[mat * per + c * rows + r] = src[q];
  }
}

// Piece q of the NHWC tensor (16 bytes): pixel q / (C/16), channel byte
// 16 * (q % (C/16)); its place in the packed tensor is
// V * (p + HW * (g + (C/V) * n)) + o  with c = g*V + o, pixel = n*HW + p.
__global__ __launch_bounds__(kThreads) void pack_vect(const int8_t *src, int8_t *dst,
                                                      FastDiv3 div_pieces, FastDiv3 div_hw,
                                                      int pieces, int hw, int vect, int groups,
                                                      uint32_t total, uint32_t bytes, int unpack) {
  const auto sr = make_rsrc(src, bytes);
  const auto dr = make_rsrc(dst, bytes);
  for (uint32_t q = blockIdx.x * kThreads + threadIdx.x; q < total; q += gridDim.x * kThreads) {
    const uint32_t pix = fast_div(q, div_pieces);
    const uint32_t cb = (q - pix * uint32_t(pieces)) * 16u;
    const uint32_t n = fast_div(pix, div_hw);
    const uint32_t p = pix - n * uint32_t(hw);
    const uint32_t g = cb / uint32_t(vect), o = cb - g * uint32_t(vect);
    const uint32_t packed = uint32_t(vect) * (p + uint32_t(hw) * (g + uint32_t(groups) * n)) + o;
    const uint32_t plain = q * 16u;
    const v4i v = load16(sr, unpack ? packed : plain);
    __builtin_amdgcn_raw_buffer_store_b128(v, dr, unpack ? plain : packed, 0, 0);
  }
}

int launch_status(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

int launch_transpose(const void *src, void *dst, int64_t batch, int rows, int cols, int esize,
                     void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t total = batch * int64_t(rows) * cols;
  if (total == 0) return I8CONV_OK;
  const bool aligned16 = (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  const bool rows16 = (int64_t(rows) * esize) % 16 == 0;
  const bool cols16 = (int64_t(cols) * esize) % 16 == 0;
  const auto *in = static_cast<const int8_t *>(src);
  auto *out = static_cast<int8_t *>(dst);
  if (aligned16 && rows16 && cols16) {
    const int T = kTileRowBytes / esize;
    const int tiles_r = (rows + T - 1) / T;
    if (esize == 1) {
      // two 128-column tiles per workgroup (256-byte source row pieces)
      // where the source rows are long enough to fill them
      const int sub = cols >= 2 * T ? 2 : 1;
      const int tiles_c = (cols + sub * T - 1) / (sub * T);
      const int64_t blocks = batch * tiles_r * tiles_c;  // < 2^31: checked by the caller
      if (sub == 2)
        hipLaunchKernelGGL(transpose_bytes_tiled<2>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                           in, out, rows, cols, tiles_r, tiles_c);
      else
        hipLaunchKernelGGL(transpose_bytes_tiled<1>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                           in, out, rows, cols, tiles_r, tiles_c);
    } else {
      const int tiles_c = (cols + T - 1) / T;
      const int64_t blocks = batch * tiles_r * tiles_c;
      hipLaunchKernelGGL(transpose_dwords_tiled, dim3(unsigned(blocks)), dim3(kThreads), 0, s, in,
                         out, rows, cols, tiles_r, tiles_c);
    }
    return launch_status("transpose launch");
  }
  if (aligned16 && rows16 && int64_t(cols) * esize * 16 <= kShortLds) {
    const int R = int(std::min<int64_t>(128, kShortLds / (int64_t(cols) * esize) / 16 * 16));
    const int tiles = (rows + R - 1) / R;
    const int64_t blocks = batch * tiles;
    if (esize == 1)
      hipLaunchKernelGGL(transpose_short_rows<1>, dim3(unsigned(blocks)), dim3(kThreads), 0, s, in,
                         out, rows, cols, R, tiles);
    else
      hipLaunchKernelGGL(transpose_short_rows<4>, dim3(unsigned(blocks)), dim3(kThreads), 0, s, in,
                         out, rows, cols, R, tiles);
    return launch_status("transpose launch");
  }
  if (aligned16 && cols16 && int64_t(rows) * esize * 16 <= kShortLds) {
    const int wb = int(std::min<int64_t>(kTileRowBytes, kShortLds / (int64_t(rows) * esize) / 16 * 16));
    const int W = wb / esize;
    const int tiles = (cols + W - 1) / W;
    const int64_t blocks = batch * tiles;
    if (esize == 1)
      hipLaunchKernelGGL(transpose_short_cols<1>, dim3(unsigned(blocks)), dim3(kThreads), 0, s, in,
                         out, rows, cols, W, tiles);
    else
      hipLaunchKernelGGL(transpose_short_cols<4>, dim3(unsigned(blocks)), dim3(kThreads), 0, s, in,
                         out, rows, cols, W, tiles);
    return launch_status("transpose launch");
  }
  const unsigned blocks = unsigned(std::min<int64_t>((total + kThreads - 1) / kThreads, 1 << 20));
  if (esize == 1)
    hipLaunchKernelGGL(transpose_elements<int8_t>, dim3(blocks), dim3(kThreads), 0, s,
                       static_cast<const int8_t *>(src), static_cast<int8_t *>(dst), rows, cols,
                       total);
  else
    hipLaunchKernelGGL(transpose_elements<int32_t>, dim3(blocks), dim3(kThreads), 0, s,
                       static_cast<const int32_t *>(src), static_cast<int32_t *>(dst), rows, cols,
                       total);
  return launch_status("transpose launch");
}

int launch_pack_vect(const int8_t *src, int8_t *dst, int n, int h, int w, int c, int vect,
                     bool unpack, void *stream) {
  const int64_t bytes = int64_t(n) * h * w * c;
  if (bytes == 0) return I8CONV_OK;
  const int pieces = c / 16;
  const uint32_t total = uint32_t(bytes / 16);
  const unsigned blocks = unsigned(std::min<int64_t>((total + kThreads - 1) / kThreads, 1 << 20));
  hipLaunchKernelGGL(pack_vect, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     src, dst, make_fastdiv3(uint32_t(pieces)), make_fastdiv3(uint32_t(h * w)),
                     pieces, h * w, vect, c / vect, total, uint32_t(bytes), unpack ? 1 : 0);
  return launch_status("pack_vect_c launch");
}

}  // namespace i8conv
