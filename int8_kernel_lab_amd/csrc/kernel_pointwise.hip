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
// Requantized int8 output (RQ): the same walk with the requantization of
// kernel_requant.hip (requant4) applied to the accumulators, the filter
// slice's multipliers and shifts held in VGPRs; a wave whose channels all
// allow it takes the short form (one 32-bit high multiply per value; the
// exact form's 64-bit product made the epilogue, not HBM, the limit).  A
// slice needs 64 or 128 channels: one or two groups of four channel
// fragments.  Lane (px, g) holds, for each group, four dwords of channels
// 16 a + 4 g (a = 0..3); two permlane32 and two permlane16 swaps among the
// lanes px, px + 16, px + 32, px + 48 transpose them so that the lane holds
// the 16 contiguous bytes of channels 16 g .. 16 g + 15, one 16-byte store
// per lane and group.  Two groups are paired by the DPP rotate as above (8
// pixels x 128 bytes per store, write-through); a 64-channel slice writes
// 16 pixels x 64 bytes per store, whole lines when the layer has 64
// channels (write-through), half lines otherwise (ordinary stores, merged
// in the L2).
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

// requant1_short (i8conv_device.hpp) with am = |mult| and shx = (shift - 32)
// | sign bit of mult, so that two registers per channel carry the constants:
// shifts take the low five bits of shx (sh is 1..30), hh = 2^(sh - 1) is
// formed on the fly, and the sign of acc xor mult is that of acc xor shx.
// Four channels packed as int8 like requant4_odd (i8conv_device.hpp).
__device__ __forceinline__ uint32_t pw_requant4_short(v4i acc, v4i am, v4i shx, int32_t zp) {
  int32_t y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t a = acc[e] < 0 ? 0u - uint32_t(acc[e]) : uint32_t(acc[e]);
    const uint32_t sh = uint32_t(shx[e]) & 31u;
    const uint32_t r = (__umulhi(a, uint32_t(am[e])) + (1u << (sh - 1u))) >> sh;
    const uint32_t sg = uint32_t((acc[e] ^ shx[e]) >> 31);
    const int32_t v = int32_t((r ^ sg) - sg) + zp;
    y[e] = v < -128 ? -128 : (v > 127 ? 127 : v);
  }
  const uint32_t lo = __builtin_amdgcn_perm(uint32_t(y[1]), uint32_t(y[0]), 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(uint32_t(y[3]), uint32_t(y[2]), 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// NA = 16-channel fragments per slice (even), KS = C / 64 k-steps, SL
// slices (N = 16 NA SL), D fragments in flight, POL the store cache policy.
template <int NA, int KS, int SL, int D, int POL, bool RQ>
__global__ __launch_bounds__(64 * pw_group_waves(SL)) void pointwise_kernel(
    const int8_t *__restrict__ x, const int8_t *__restrict__ w,
    const int32_t *__restrict__ bias, int32_t *__restrict__ y, int gemm_m, int nfrag,
    const int32_t *__restrict__ mult, const int32_t *__restrict__ shift, int32_t zp,
    int8_t *__restrict__ q) {
  static_assert(!RQ || (NA % 4 == 0 && NA <= 8), "requantized slices: 64 or 128 channels");
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
  const auto yr = make_rsrc(RQ ? static_cast<void *>(q) : static_cast<void *>(y),
                            uint32_t(gemm_m) * kN * (RQ ? 1u : 4u));
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
  v4i m4[RQ ? NA : 1], s4[RQ ? NA : 1], h4[RQ ? NA : 1];
  // The requantization's form, a uniform choice per wave: the odd-
  // multiplier form (requant4_odd: m4, s4 and h4 then hold mo, k and sh)
  // when every channel of the wave's slice is in its domain, four VALU
  // operations per value; else the short form (requant1_short) when every
  // channel has shift >= 33 and |zp| <= 2^30 (m4 and s4 then hold am and
  // shx: pw_requant4_short), about a dozen; else the exact form (requant4).
  bool qodd = false, qshort = false;
  if constexpr (RQ) {
    const auto mr = make_rsrc(mult, kN * 4u), sr = make_rsrc(shift, kN * 4u);
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      m4[a] = load16(mr, (oc0 + uint32_t(16 * a + 4 * g)) * 4u);
      s4[a] = load16(sr, (oc0 + uint32_t(16 * a + 4 * g)) * 4u);
    }
    v4i mo4[NA], k4[NA];
    bool okodd = true;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const RequantOdd o = requant_odd_params(m4[a][e], s4[a][e], zp);
        okodd = okodd && o.ok;
        mo4[a][e] = o.mo;
        k4[a][e] = o.k;
        h4[a][e] = o.sh;
      }
    qodd = __builtin_amdgcn_ballot_w64(!okodd) == 0;
    if (qodd) {
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        m4[a] = mo4[a];
        s4[a] = k4[a];
      }
    }
    bool ok = !qodd && requant_short_zp_ok(zp);
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int e = 0; e < 4; ++e) ok = ok && requant_short_ok(s4[a][e]);
    qshort = __builtin_amdgcn_ballot_w64(!ok) == 0;
    if (qshort) {
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t m = m4[a][e];
          m4[a][e] = int32_t(requant_short_am(m));
          s4[a][e] = int32_t(requant_short_sh(s4[a][e]) | (uint32_t(m) & 0x80000000u));
        }
    }
  }

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
      if constexpr (RQ) {
        // per group of four fragments: requantize, transpose across the
        // four lanes of a pixel, then one 16-byte vector per lane
        constexpr int kGroups = NA / 4;
        v4i t[kGroups];
#pragma unroll
        for (int h = 0; h < kGroups; ++h) {
          uint32_t dq[4];
          if (qodd) {
#pragma unroll
            for (int a = 0; a < 4; ++a)
              dq[a] = requant4_odd(acc[4 * h + a], m4[4 * h + a], s4[4 * h + a], h4[4 * h + a]);
          } else if (qshort) {
#pragma unroll
            for (int a = 0; a < 4; ++a)
              dq[a] = pw_requant4_short(acc[4 * h + a], m4[4 * h + a], s4[4 * h + a], zp);
          } else {
#pragma unroll
            for (int a = 0; a < 4; ++a)
              dq[a] = requant4(acc[4 * h + a], m4[4 * h + a], s4[4 * h + a], zp);
          }
          // 4 x 4 transpose over (row g, dword a) with gfx950's lane swaps:
          // permlane32_swap(X, Y) exchanges X's rows 2-3 with Y's rows 0-1,
          // permlane16_swap(X, Y) X's odd rows with Y's even rows (lane
          // layout checked on the device); afterwards dword j of row g
          // holds row j's dword g
          const auto x02 = __builtin_amdgcn_permlane32_swap(dq[0], dq[2], false, false);
          const auto x13 = __builtin_amdgcn_permlane32_swap(dq[1], dq[3], false, false);
          const auto y01 = __builtin_amdgcn_permlane16_swap(x02[0], x13[0], false, false);
          const auto y23 = __builtin_amdgcn_permlane16_swap(x02[1], x13[1], false, false);
          t[h][0] = int(y01[0]);
          t[h][1] = int(y01[1]);
          t[h][2] = int(y23[0]);
          t[h][3] = int(y23[1]);
        }
        // lane (px, g) holds pixel 16 f + px, channels oc0 + 64 h + 16 g ...
        if constexpr (kGroups == 1) {
          const uint32_t p = 16u * f + px;
          __builtin_amdgcn_raw_buffer_store_b128(t[0], yr, p * kN + oc0 + 16u * g, 0, POL);
        } else {
#pragma unroll
          for (int j = 0; j < kGroups / 2; ++j) {
            v4i r;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              r[e] = __builtin_amdgcn_update_dpp(0, t[2 * j + 1][e], 0x128, 0xf, 0xf, false);
            const v4i da = lo ? t[2 * j] : r, db = lo ? r : t[2 * j];
            const uint32_t pa = 16u * f + (lo ? px : px - 8), pb = 16u * f + (lo ? px + 8 : px);
            const uint32_t ca = oc0 + 128u * j + (lo ? 16 * g : 64 + 16 * g);
            const uint32_t cb = oc0 + 128u * j + (lo ? 64 + 16 * g : 16 * g);
            __builtin_amdgcn_raw_buffer_store_b128(da, yr, pa * kN + ca, 0, POL);
            __builtin_amdgcn_raw_buffer_store_b128(db, yr, pb * kN + cb, 0, POL);
          }
        }
        continue;
      }
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
int launch_pw(const ConvArgs &a, const RequantArgs *rq, hipStream_t stream) {
  const int nfrag = int((int64_t(a.gemm_m) + 15) / 16);
  const int waves = pointwise_waves(a.gemm_m, SL);
  const dim3 grid(unsigned(waves / pw_group_waves(SL))), block(64 * pw_group_waves(SL));
  if (rq) {
    // whole 128-byte lines per store: paired groups, or one group of a
    // 64-channel layer; else ordinary stores (merged in the L2)
    constexpr bool kWhole = NA > 4 || SL == 1;
    constexpr int kBig = kWhole ? kStoreStream : 0, kSmall = kWhole ? kStoreThrough : 0;
    // about 8 KB of loads in flight per wave (8 / KS fragments, at least 2):
    // on config 4a 16.6-16.8 us per launch against 16.8-17.0 with 16 KB and
    // 18.7 with 32 KB; twice the waves (two per SIMD) 19.4-21.1 us
    constexpr int kD = KS >= 4 ? 2 : 8 / KS;
    if constexpr (NA % 4 == 0 && NA <= 8) {
      if (int64_t(a.gemm_m) * a.gemm_n > kStreamOutputBytes)
        I8_LAUNCH((pointwise_kernel<NA, KS, SL, kD, kBig, true>), grid, block,
                           0, stream, a.x, a.w, a.bias, nullptr, a.gemm_m, nfrag, rq->mult,
                           rq->shift, rq->zero_point, rq->y);
      else
        I8_LAUNCH((pointwise_kernel<NA, KS, SL, kD, kSmall, true>), grid,
                           block, 0, stream, a.x, a.w, a.bias, nullptr, a.gemm_m, nfrag, rq->mult,
                           rq->shift, rq->zero_point, rq->y);
    } else {
      set_error("pointwise kernel: no requantizing instance for C = " + std::to_string(a.c) +
                ", N = " + std::to_string(a.gemm_n));
      return I8CONV_BAD_ARGUMENT;
    }
  } else if (int64_t(a.gemm_m) * a.gemm_n * 4 > kStreamOutputBytes) {
    I8_LAUNCH((pointwise_kernel<NA, KS, SL, pw_depth(KS), kStoreStream, false>), grid,
                       block, 0, stream, a.x, a.w, a.bias, a.y, a.gemm_m, nfrag, nullptr, nullptr,
                       0, nullptr);
  } else {
    I8_LAUNCH((pointwise_kernel<NA, KS, SL, pw_depth(KS), kStoreThrough, false>), grid,
                       block, 0, stream, a.x, a.w, a.bias, a.y, a.gemm_m, nfrag, nullptr, nullptr,
                       0, nullptr);
  }
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

int launch_pointwise(const ConvArgs &a, const RequantArgs *rq, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (rq && !pointwise_requant_supported(a.c, a.gemm_n)) {
    set_error("pointwise kernel: no requantizing form for C = " + std::to_string(a.c) +
              ", N = " + std::to_string(a.gemm_n));
    return I8CONV_BAD_ARGUMENT;
  }
  if (!pointwise_supported(a.c, a.gemm_n)) {
    set_error("pointwise kernel: unsupported C = " + std::to_string(a.c) +
              ", N = " + std::to_string(a.gemm_n));
    return I8CONV_BAD_ARGUMENT;
  }
  // C / 64 and N / 32 as one key; slices where N * C > 16384
  switch ((a.c / 64) * 100 + a.gemm_n / 32) {
    case 101: return launch_pw<2, 1, 1>(a, rq, s);
    case 102: return launch_pw<4, 1, 1>(a, rq, s);
    case 104: return launch_pw<8, 1, 1>(a, rq, s);
    case 108: return launch_pw<16, 1, 1>(a, rq, s);
    case 201: return launch_pw<2, 2, 1>(a, rq, s);
    case 202: return launch_pw<4, 2, 1>(a, rq, s);
    case 204: return launch_pw<8, 2, 1>(a, rq, s);
    case 208: return launch_pw<8, 2, 2>(a, rq, s);
    case 401: return launch_pw<2, 4, 1>(a, rq, s);
    case 402: return launch_pw<4, 4, 1>(a, rq, s);
    case 404: return launch_pw<4, 4, 2>(a, rq, s);
    case 408: return launch_pw<4, 4, 4>(a, rq, s);
    case 801: return launch_pw<2, 8, 1>(a, rq, s);
    case 802: return launch_pw<2, 8, 2>(a, rq, s);
    case 804: return launch_pw<2, 8, 4>(a, rq, s);
    case 808: return launch_pw<2, 8, 8>(a, rq, s);
    default: break;
  }
  set_error("pointwise kernel: no instance for C = " + std::to_string(a.c) +
            ", N = " + std::to_string(a.gemm_n));
  return I8CONV_BAD_ARGUMENT;
}

}  // namespace i8conv
