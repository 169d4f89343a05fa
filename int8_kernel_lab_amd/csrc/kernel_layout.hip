// Layout transforms around the convolution (the step before and after the
// path; the reference does its packing on the host, src/cudnn_lab.cu:7-18):
//   * batched transpose [rows][cols] -> [cols][rows] of 1- or 4-byte
//     elements: NCHW <-> NHWC int8 activations, NHWK -> NKHW int32 output;
//   * channel-vector packing NHWC (or KRSC) -> N, C/V, H, W, V and back,
//     the layout of the reference's cuDNN INT8x32 path (V = 32).
// All are HBM-bound byte movement.
//
// Transpose: one workgroup per T x T tile (T * esize = 128 bytes), read as
// whole 128-byte rows (8 lanes x 16 bytes), staged in LDS with a 132-byte
// pitch (33 dwords: the T rows of one column fall in distinct banks), and
// written as whole 128-byte rows of the transposed matrix, each lane
// gathering 16 bytes of one column.  Needs 16-byte rows on both sides
// (rows * esize and cols * esize multiples of 16) and 16-byte aligned
// bases; otherwise an element-per-thread form runs.
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

template <int ES>
__global__ __launch_bounds__(kThreads) void transpose_tiled(const int8_t *src, int8_t *dst,
                                                            int rows, int cols, int tiles_r,
                                                            int tiles_c) {
  constexpr int T = kTileRowBytes / ES;  // tile side in elements
  __shared__ uint32_t tile[T * kLdsPitch / 4];
  const int per_mat = tiles_r * tiles_c;
  const int mat = int(blockIdx.x) / per_mat;
  const int t = int(blockIdx.x) - mat * per_mat;
  const int tr = t / tiles_c;
  const int tc = t - tr * tiles_c;
  const size_t mat_bytes = size_t(rows) * size_t(cols) * ES;  // < 2^31: checked at launch
  const auto sr = make_rsrc(src + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const auto dr = make_rsrc(dst + size_t(mat) * mat_bytes, uint32_t(mat_bytes));
  const int r0 = tr * T, c0 = tc * T;
  const uint32_t row_bytes = uint32_t(cols) * ES;
  // read: tile row i = source row r0 + i, bytes [c0*ES, c0*ES + 128)
  for (int idx = threadIdx.x; idx < T * 8; idx += kThreads) {
    const int i = idx >> 3, piece = idx & 7;
    const uint32_t cb = uint32_t(c0 * ES + piece * 16);
    const bool ok = r0 + i < rows && cb < row_bytes;
    const v4i v = load16(sr, ok ? uint32_t(r0 + i) * row_bytes + cb : kOutOfRange);
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[(i * kLdsPitch + piece * 16) / 4 + e] = uint32_t(v[e]);
  }
  __syncthreads();
  // write: output row j = column c0 + j, bytes [r0*ES, r0*ES + 128): lane
  // gathers the 16 / ES tile rows i0 .. of column j
  const uint8_t *tb = reinterpret_cast<const uint8_t *>(tile);
  const uint32_t out_row_bytes = uint32_t(rows) * ES;
  for (int idx = threadIdx.x; idx < T * 8; idx += kThreads) {
    const int j = idx >> 3, piece = idx & 7;
    constexpr int kPer = 16 / ES;
    const int i0 = piece * kPer;
    const int c = c0 + j;
    if (c >= cols) continue;
    v4i v;
    if constexpr (ES == 1) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) word |= uint32_t(tb[(i0 + 4 * e + k) * kLdsPitch + j]) << (8 * k);
        v[e] = int32_t(word);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = int32_t(tile[((i0 + e) * kLdsPitch) / 4 + j]);
    }
    const int valid = min(kPer, rows - (r0 + i0));
    if (valid <= 0) continue;
    const uint32_t off = uint32_t(c) * out_row_bytes + uint32_t((r0 + i0) * ES);
    if (valid == kPer) {
      __builtin_amdgcn_raw_buffer_store_b128(v, dr, off, 0, 0);
    } else {
      // a tile row past the end of the matrix: element stores of the valid part
      for (int k = 0; k < valid * ES; ++k)
        __builtin_amdgcn_raw_buffer_store_b8(uint8_t(uint32_t(v[k / 4]) >> (8 * (k % 4))), dr,
                                             off + uint32_t(k), 0, 0);
    }
  }
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
  const bool tiled = (int64_t(rows) * esize) % 16 == 0 && (int64_t(cols) * esize) % 16 == 0 &&
                     (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  if (tiled) {
    const int T = kTileRowBytes / esize;
    const int tiles_r = (rows + T - 1) / T, tiles_c = (cols + T - 1) / T;
    const int64_t blocks = batch * tiles_r * tiles_c;  // < 2^31: checked by the caller
    if (esize == 1)
      hipLaunchKernelGGL(transpose_tiled<1>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                         static_cast<const int8_t *>(src), static_cast<int8_t *>(dst), rows, cols,
                         tiles_r, tiles_c);
    else
      hipLaunchKernelGGL(transpose_tiled<4>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                         static_cast<const int8_t *>(src), static_cast<int8_t *>(dst), rows, cols,
                         tiles_r, tiles_c);
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
