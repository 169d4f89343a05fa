// Pointwise streaming kernel on gfx950 INT8 MFMA: 1x1, stride-1, unpadded
// layers (output pixel m reads input pixel m), the generic GEMM's form for
// them when the whole filter fits a wave's registers.  Such layers are a
// plain [M x C] x [C x N] product with a short reduction (C <= 512) and are
// bound by HBM: 2 bytes in + N * 4 bytes out per pixel and channel pair
// (config 4a, 64 x 56 x 56 x 256 -> 64: 51 MB read, 51 MB written).  The
// tiled GEMM stages pixel tiles and the filter through LDS and keeps a
// workgroup's tile in flight at a time; here no LDS is used at all:
//
//  * each wave loads the N x C filter once into VGPRs as MFMA A operands
//    (lane l: output channel 16 a + l % 16, bytes 64 ks + 16 (l / 16) of
//    its row), N * C / 1024 registers (64 for 64 x 256); where N * C >
//    16384 the output channels split into SL slices of 16384 / C channels,
//    one per wave of a workgroup, and the SL waves of a workgroup walk the
//    same fragments (the input of a fragment is fetched from HBM once and
//    read by the other slices from the compute unit's L1 or the L2);
//  * the wave walks 16-pixel fragments f = wave, wave + waves, ...; a
//    fragment's B operands come straight from global memory (lane l: pixel
//    16 f + l % 16, the same 16 bytes of each 64-byte k-step), so the 64
//    lanes of one load read four whole 64-byte halves of 16 pixel rows and
//    the fragment as a whole reads its pixels' rows exactly once;
//  * D fragments are in flight per wave (about 16 KB of loads), issued D
//    fragments ahead of the MFMAs that consume them;
//  * accumulators start from the bias; N / 16 x C / 64 MFMAs per fragment;
//  * stores pair output-channel fragments (2j, 2j + 1) across the two
//    halves of each 16-lane row with a DPP rotate by 8 lanes, so that one
//    16-byte store per lane writes 8 pixels x 32 channels, a whole 128-byte
//    line per pixel, write-through (outputs above 128 MiB: evict-first).
//
// Launch shape (measured on config 4a, 64 x 56 x 56 x 256 -> 64): two-wave
// workgroups, at most 1024 waves (16.4 us per launch; four-wave workgroups
// over the same 1024 waves 18.0 us, 256 waves 17.4-19.6 us, eight waves per
// workgroup 18.7 us); with slices, SL-wave workgroups (two for SL = 1),
// at most 1024 waves in all.  Fragments past the last pixel read zeros (their
// buffer offsets lie beyond the input) and their stores are dropped by the
// output buffer's range check.
#include <hip/hip_runtime.h>

#include <string>

#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

__device__ __forceinline__ v4i pw_mfma(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// NA = 16-channel fragments per slice (even), KS = C / 64 k-steps, SL
// slices (N = 16 NA SL), D fragments in flight, POL the store cache policy.
template <int NA, int KS, int SL, int D, int POL>
__global__ __launch_bounds__(64 * pw_group_waves(SL)) void pointwise_kernel(
    const int8_t *__restrict__ x, const int8_t *__restrict__ w,
    const int32_t *__restrict__ bias, int32_t *__restrict__ y, int gemm_m, int nfrag) {
  constexpr uint32_t kC = 64 * KS, kNs = 16 * NA, kN = kNs * SL;
  constexpr int kGroupWaves = pw_group_waves(SL), kStreams = kGroupWaves / SL;
  const int lane = threadIdx.x & 63;
  const int in_group = threadIdx.x >> 6;
  const uint32_t oc0 = kNs * uint32_t(in_group % SL);  // this wave's slice
  const int wave = blockIdx.x * kStreams + in_group / SL;  // fragment stream
  const int waves = gridDim.x * kStreams;
  const auto xr = make_rsrc(x, uint32_t(gemm_m) * kC);
  const auto wr = make_rsrc(w, kN * kC);
  const auto br = make_rsrc(bias, kN * 4u);
  const auto yr = make_rsrc(y, uint32_t(gemm_m) * kN * 4u);
  const int px = lane & 15, g = lane >> 4;

  v4i A[NA][KS];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      A[a][ks] = load16(wr, (oc0 + uint32_t(16 * a + px)) * kC + 64u * ks + 16u * g);
  v4i b4[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) b4[a] = load16(br, (oc0 + uint32_t(16 * a + 4 * g)) * 4u);

  const uint32_t boff = uint32_t(px) * kC + 16u * g;
  v4i B[D][KS];
  auto load = [&](int slot, int f) {
    const uint32_t base = f < nfrag ? uint32_t(f) * 16u * kC + boff : kOutOfRange;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) B[slot][ks] = load16(xr, base + 64u * ks);
  };
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, wave + d * waves);

  const bool lo = px < 8;
  for (int f0 = wave; f0 < nfrag; f0 += D * waves) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int f = f0 + d * waves;
      if (f >= nfrag) break;
      v4i acc[NA];
#pragma unroll
      for (int a = 0; a < NA; ++a) acc[a] = b4[a];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int a = 0; a < NA; ++a) acc[a] = pw_mfma(A[a][ks], B[d][ks], acc[a]);
      load(d, f + D * waves);
      // Lanes 0-7 of row g store their own pixel's channels 32 j + 4 g and
      // the rotated-in pixel px + 8's channels 32 j + 16 + 4 g; lanes 8-15
      // the mirror image: each store instruction covers 8 pixels x 128
      // bytes.
#pragma unroll
      for (int j = 0; j < NA / 2; ++j) {
        v4i r;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          r[e] = __builtin_amdgcn_update_dpp(0, acc[2 * j + 1][e], 0x128, 0xf, 0xf, false);
        const v4i da = lo ? acc[2 * j] : r, db = lo ? r : acc[2 * j];
        const uint32_t pa = 16u * f + (lo ? px : px - 8), pb = 16u * f + (lo ? px + 8 : px);
        const uint32_t ca = oc0 + 32u * j + (lo ? 4 * g : 16 + 4 * g);
        const uint32_t cb = oc0 + 32u * j + (lo ? 16 + 4 * g : 4 * g);
        __builtin_amdgcn_raw_buffer_store_b128(da, yr, (pa * kN + ca) * 4u, 0, POL);
        __builtin_amdgcn_raw_buffer_store_b128(db, yr, (pb * kN + cb) * 4u, 0, POL);
      }
    }
  }
}

constexpr int pw_depth(int ks) { return ks >= 4 ? (16 / ks < 2 ? 2 : 16 / ks) : 8; }

template <int NA, int KS, int SL>
int launch_pw(const ConvArgs &a, hipStream_t stream) {
  const int nfrag = int((int64_t(a.gemm_m) + 15) / 16);
  const int waves = pointwise_waves(a.gemm_m, SL);
  const dim3 grid(unsigned(waves / pw_group_waves(SL))), block(64 * pw_group_waves(SL));
  if (int64_t(a.gemm_m) * a.gemm_n * 4 > kStreamOutputBytes)
    hipLaunchKernelGGL((pointwise_kernel<NA, KS, SL, pw_depth(KS), kStoreStream>), grid, block,
                       0, stream, a.x, a.w, a.bias, a.y, a.gemm_m, nfrag);
  else
    hipLaunchKernelGGL((pointwise_kernel<NA, KS, SL, pw_depth(KS), kStoreThrough>), grid, block,
                       0, stream, a.x, a.w, a.bias, a.y, a.gemm_m, nfrag);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("pointwise kernel launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

bool pointwise_pointers_ok(const ConvArgs &a) {
  auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return al(a.x) && al(a.w) && al(a.bias) && al(a.y);
}

int launch_pointwise(const ConvArgs &a, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!pointwise_supported(a.c, a.gemm_n)) {
    set_error("pointwise kernel: unsupported C = " + std::to_string(a.c) +
              ", N = " + std::to_string(a.gemm_n));
    return I8CONV_BAD_ARGUMENT;
  }
  // C / 64 and N / 32 as one key; slices where N * C > 16384
  switch ((a.c / 64) * 100 + a.gemm_n / 32) {
    case 101: return launch_pw<2, 1, 1>(a, s);
    case 102: return launch_pw<4, 1, 1>(a, s);
    case 104: return launch_pw<8, 1, 1>(a, s);
    case 108: return launch_pw<16, 1, 1>(a, s);
    case 201: return launch_pw<2, 2, 1>(a, s);
    case 202: return launch_pw<4, 2, 1>(a, s);
    case 204: return launch_pw<8, 2, 1>(a, s);
    case 208: return launch_pw<8, 2, 2>(a, s);
    case 401: return launch_pw<2, 4, 1>(a, s);
    case 402: return launch_pw<4, 4, 1>(a, s);
    case 404: return launch_pw<4, 4, 2>(a, s);
    case 408: return launch_pw<4, 4, 4>(a, s);
    case 801: return launch_pw<2, 8, 1>(a, s);
    case 802: return launch_pw<2, 8, 2>(a, s);
    case 804: return launch_pw<2, 8, 4>(a, s);
    case 808: return launch_pw<2, 8, 8>(a, s);
    default: break;
  }
  set_error("pointwise kernel: no instance for C = " + std::to_string(a.c) +
            ", N = " + std::to_string(a.gemm_n));
  return I8CONV_BAD_ARGUMENT;
}

}  // namespace i8conv
