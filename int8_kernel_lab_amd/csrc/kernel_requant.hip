// Requantization of an int32 NHWK tensor to int8 (the step after the
// convolution; no counterpart in the reference, whose vendor comparison
// writes INT8 output, README.md:89-90): per output channel k,
//   y = clamp(zero_point + round(acc * mult[k] / 2^shift[k]), -128, 127)
// (requant1 in i8conv_device.hpp).  An HBM-bound elementwise pass: each
// thread reads 16 bytes of int32 (four channels of one pixel) and writes
// their four int8 values as one dword; a scalar form covers N % 4 != 0.
// The row kernel with copy waves applies the same function in its epilogue
// instead (kernel_rowpass.hip); every other kernel's output goes through
// this pass.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "i8conv_internal.hpp"

namespace i8conv {
namespace {

__global__ __launch_bounds__(kThreads) void requant_vec(const int32_t *__restrict__ acc,
                                                        const int32_t *__restrict__ mult,
                                                        const int32_t *__restrict__ shift,
                                                        int32_t zp, uint32_t *__restrict__ out,
                                                        int n4, size_t total4) {
  const size_t grid = size_t(gridDim.x) * kThreads;
  const int step4 = int(grid % size_t(n4));
  size_t q = size_t(blockIdx.x) * kThreads + threadIdx.x;
  int c4 = int(q % size_t(n4));  // channel group of item q, advanced without division
  for (; q < total4; q += grid) {
    const v4i a = reinterpret_cast<const v4i *>(acc)[q];
    const v4i m = reinterpret_cast<const v4i *>(mult)[c4];
    const v4i s = reinterpret_cast<const v4i *>(shift)[c4];
    out[q] = requant4(a, m, s, zp);
    c4 += step4;
    if (c4 >= n4) c4 -= n4;
  }
}

__global__ __launch_bounds__(kThreads) void requant_scalar(const int32_t *__restrict__ acc,
                                                           const int32_t *__restrict__ mult,
                                                           const int32_t *__restrict__ shift,
                                                           int32_t zp, int8_t *__restrict__ out,
                                                           int channels, size_t total) {
  for (size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += size_t(gridDim.x) * kThreads) {
    const int k = int(i % size_t(channels));
    out[i] = int8_t(requant1(acc[i], mult[k], shift[k], zp));
  }
}

}  // namespace

int launch_requant(const int32_t *acc, int64_t pixels, int32_t channels, const int32_t *mult,
                   const int32_t *shift, int32_t zero_point, int8_t *out, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t total = size_t(pixels) * size_t(channels);
  if (total == 0) return I8CONV_OK;
  const bool vec = channels % 4 == 0 && (reinterpret_cast<uintptr_t>(acc) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(mult) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(shift) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 3) == 0;
  const size_t items = vec ? total / 4 : total;
  // one item per thread (many independent loads in flight); the loop in
  // the kernels only repeats for tensors beyond 2^28 items
  const unsigned blocks = unsigned(std::min<size_t>((items + kThreads - 1) / kThreads, 1u << 20));
  if (vec)
    I8_LAUNCH(requant_vec, dim3(blocks), dim3(kThreads), 0, s, acc, mult, shift,
                       zero_point, reinterpret_cast<uint32_t *>(out), channels / 4, items);
  else
    I8_LAUNCH(requant_scalar, dim3(blocks), dim3(kThreads), 0, s, acc, mult, shift,
                       zero_point, out, channels, total);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("requant launch: ") + hipGetErrorString(e));
    return I8CONV_HIP_ERROR;
  }
  return I8CONV_OK;
}

}  // namespace i8conv
