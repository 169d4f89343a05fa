// Probes that calibrate what the convolution kernels are measured against.
//
// Store-floor probe: a kernel that only writes, in the launch shape of the
// row kernels (workgroups x threads, the same dynamic LDS allocation) and
// with their output instruction (16-byte buffer stores, write-through or
// ordinary).  Its time per launch is the floor under any convolution whose
// output is that many bytes in that launch shape: no loads, no MFMAs.  With
// zero bytes it is an empty kernel of the shape, the dispatch floor.
//
// Unit u (16 bytes) holds the int32 value u in its four lanes, so a caller
// can check that every replay wrote every byte.
//
// LDS probe: ds_read_b128 in a fixed per-lane pattern, the control for the
// LDS bank-conflict counters (SQ_LDS_BANK_CONFLICT against
// SQ_LDS_IDX_ACTIVE).  The LDS has 64 banks of 4 bytes, so a 16-byte read
// covers one of sixteen 4-bank groups modulo 256 bytes:
//   0 linear    lane l at 16 * l: each 16 lanes cover all sixteen groups
//   1 swz128    lane l at swz128(l % 16, l / 16): a fragment read of the
//               row kernels' filter ring (conflict-free)
//   2 stride128 lane l at 128 * l: two groups per 16 lanes (8-way)
//   3 stride256 lane l at 256 * l: one group per 16 lanes (16-way)
//   4 xor_rows  lane l at swz128x(l % 16, l / 16), the pipelined GEMM's
//               layout: 16 distinct groups per 16 lanes, yet 2-way on
//               gfx950 (its 32-lane condition)
//   5 pitch80   lane l at 80 * (l % 16) + 16 * (l / 16): a 5-unit pixel
//               pitch, 2-way on gfx950 likewise
// Iteration i reads at pattern + 16384 * (i % 4) in 64 KB of LDS filled
// with unit u = (u, ~u, 3u, u ^ 0x55); each lane stores the four-way XOR of
// the XOR of everything it read (sink[global thread id]).
#include <hip/hip_runtime.h>

#include <string>

#include "i8conv_device.hpp"
#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

template <bool kThrough>
__global__ void store_floor_kernel(int32_t *y, uint32_t units, uint32_t slice) {
  // the dynamic LDS is allocated (occupancy and dispatch as for the row
  // kernels) and never touched
  const uint32_t first = blockIdx.x * slice;
  const uint32_t last = min(first + slice, units);
  const auto r = make_rsrc(y, units * 16u);
  for (uint32_t u = first + threadIdx.x; u < last; u += blockDim.x) {
    const int32_t v = int32_t(u);
    __builtin_amdgcn_raw_buffer_store_b128(v4i{v, v, v, v}, r, u * 16u, 0,
                                           kThrough ? kStoreThrough : 0);
  }
}

template <bool kThrough>
int launch_t(int32_t *y, uint32_t units, int workgroups, int threads, size_t lds,
             hipStream_t s) {
  auto kern = store_floor_kernel<kThrough>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(lds));
    if (e != hipSuccess) {
      set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      return I8CONV_HIP_ERROR;
    }
  }
  const uint32_t slice = (units + uint32_t(workgroups) - 1) / uint32_t(workgroups);
  I8_LAUNCH(kern, dim3(unsigned(workgroups)), dim3(unsigned(threads)), lds, s, y, units,
                     slice);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("store floor, launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

constexpr int kProbeLds = 65536;

template <int kPattern>
__global__ __launch_bounds__(1024) void lds_probe_kernel(int32_t *sink, int iters) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  v4i *units = reinterpret_cast<v4i *>(smem);
  for (int u = threadIdx.x; u < kProbeLds / 16; u += blockDim.x)
    units[u] = v4i{u, ~u, 3 * u, u ^ 0x55};
  __syncthreads();
  const int lane = threadIdx.x & 63;
  uint32_t base;
  if constexpr (kPattern == 0)
    base = 16u * uint32_t(lane);
  else if constexpr (kPattern == 1)
    base = uint32_t(swz128(lane & 15, lane >> 4));
  else if constexpr (kPattern == 2)
    base = 128u * uint32_t(lane);
  else if constexpr (kPattern == 3)
    base = 256u * uint32_t(lane);
  else if constexpr (kPattern == 4) {
    base = uint32_t(swz128x(lane & 15, lane >> 4));
  } else
    base = uint32_t(80 * (lane & 15) + 16 * (lane >> 4));
  v4i acc = v4i{0, 0, 0, 0};
  // each offset is made opaque to the compiler, so that every iteration
  // reads LDS (the reads are otherwise loop-invariant and would be hoisted
  // out of the loop); eight reads in flight per wave
  auto read = [&](int i) {
    uint32_t off = base + 16384u * uint32_t(i & 3);
    asm volatile("" : "+v"(off));
    return *reinterpret_cast<const v4i *>(smem + off);
  };
  int i = 0;
  for (; i + 8 <= iters; i += 8) {
    v4i r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = read(i + u);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= r[u];
  }
  for (; i < iters; ++i) acc ^= read(i);
  sink[blockIdx.x * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

template <int kPattern>
int launch_lds_t(int32_t *sink, int workgroups, int threads, int iters, hipStream_t s) {
  auto kern = lds_probe_kernel<kPattern>;
  const hipError_t a = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kProbeLds);
  if (a != hipSuccess) {
    set_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(a));
    return I8CONV_HIP_ERROR;
  }
  I8_LAUNCH(kern, dim3(unsigned(workgroups)), dim3(unsigned(threads)), kProbeLds, s,
                     sink, iters);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("lds probe, launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

int launch_lds_probe(int pattern, int32_t *sink, int workgroups, int threads, int iters,
                     void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (pattern) {
    case 0: return launch_lds_t<0>(sink, workgroups, threads, iters, s);
    case 1: return launch_lds_t<1>(sink, workgroups, threads, iters, s);
    case 2: return launch_lds_t<2>(sink, workgroups, threads, iters, s);
    case 3: return launch_lds_t<3>(sink, workgroups, threads, iters, s);
    case 4: return launch_lds_t<4>(sink, workgroups, threads, iters, s);
    case 5: return launch_lds_t<5>(sink, workgroups, threads, iters, s);
    default: set_error("lds probe: pattern must be 0..5"); return I8CONV_BAD_ARGUMENT;
  }
}

int launch_store_floor(int32_t *y, size_t bytes, int workgroups, int threads, size_t lds,
                       bool write_through, void *stream) {
  const uint32_t units = uint32_t(bytes / 16);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return write_through ? launch_t<true>(y, units, workgroups, threads, lds, s)
                       : launch_t<false>(y, units, workgroups, threads, lds, s);
}

}  // namespace i8conv
