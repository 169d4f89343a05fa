// Store-floor probe: a kernel that only writes, in the launch shape of the
// row kernels (workgroups x threads, the same dynamic LDS allocation) and
// with their output instruction (16-byte buffer stores, write-through or
// ordinary).  Its time per launch is the floor under any convolution whose
// output is that many bytes in that launch shape: no loads, no MFMAs.  With
// zero bytes it is an empty kernel of the shape, the dispatch floor.
//
// Unit u (16 bytes) holds the int32 value u in its four lanes, so a caller
// can check that every replay wrote every byte.
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
  hipLaunchKernelGGL(kern, dim3(unsigned(workgroups)), dim3(unsigned(threads)), lds, s, y, units,
                     slice);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("store floor, launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace

int launch_store_floor(int32_t *y, size_t bytes, int workgroups, int threads, size_t lds,
                       bool write_through, void *stream) {
  const uint32_t units = uint32_t(bytes / 16);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return write_through ? launch_t<true>(y, units, workgroups, threads, lds, s)
                       : launch_t<false>(y, units, workgroups, threads, lds, s);
}

}  // namespace i8conv
