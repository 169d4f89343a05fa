// vendor_lab: the vendor library's INT8 convolution timed beside this lab's
// dispatched kernel on one case, the counterpart of the reference's cuDNN
// comparison (src/cudnn_lab.cu, include/cudnn_legacy.cuh, README.md:76-90;
// sweep.py:44-56 adds its columns).  On MI355X the vendor library is MIOpen.
//
// Contract of the comparison.  Same layer and same seeded data as conv_lab.
// MIOpen: NHWC int8 input, KYXC (= KRSC) int8 filter, NHWC int32 output,
// alpha = 1, beta = 0, no bias; its fastest forward algorithm is chosen by
// miopenFindConvolutionForwardAlgorithm (exhaustive search) outside the
// timed region.  The dispatched kernel runs the same layer with a zero bias,
// so both write the plain int32 convolution; the two outputs are compared
// element for element (vendor_correct).  Timing is conv_lab's: warmup, then
// the median of per-launch event pairs, plus the mean of back-to-back
// launches.  Performance only: the lab's path adds the bias in the same
// kernel, MIOpen's would need a second pass.
//
// Prints one CSV row (header with --csv); exits 0 also when MIOpen has no
// algorithm for the layer (vendor_ms = -1, contract says why), nonzero on a
// HIP/ABI error.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>
#include <miopen/miopen.h>

#include "i8conv.h"
#include "workload_table.hpp"

namespace {

using i8conv_host::exe_dir;
using i8conv_host::fail;
using i8conv_host::load_case;

void check(int status, const char *what) {
  if (status != I8CONV_OK) {
    std::cerr << what << ": " << i8conv_status_string(status) << " ("
              << i8conv_last_error() << ")\n";
    std::exit(EXIT_FAILURE);
  }
}

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

struct Options {
  std::string config, name;
  bool csv = false, header = true;
  int warmup = 20, iterations = 101;
  uint64_t seed = 20260925;  // the reference's seed (conv_lab.cu:149)
};

Options parse(int argc, char **argv) {
  Options o;
  o.config = exe_dir() + "/workloads/baseline.csv";
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto value = [&]() -> std::string {
      if (i + 1 >= argc) fail("missing value for " + a);
      return argv[++i];
    };
    if (a == "--config") o.config = value();
    else if (a == "--case") o.name = value();
    else if (a == "--csv") o.csv = true;
    else if (a == "--no-header") o.header = false;
    else if (a == "--warmup") o.warmup = std::stoi(value());
    else if (a == "--iterations") o.iterations = std::stoi(value());
    else if (a == "--seed") o.seed = std::stoull(value());
    else fail("usage: vendor_lab --case NAME [--config FILE] [--csv] [--no-header] "
              "[--warmup N] [--iterations N] [--seed N]");
  }
  if (o.name.empty() || o.warmup < 0 || o.iterations <= 0) fail("vendor_lab: bad options");
  return o;
}

const char *algo_name(miopenConvFwdAlgorithm_t a) {
  switch (a) {
    case miopenConvolutionFwdAlgoGEMM: return "gemm";
    case miopenConvolutionFwdAlgoDirect: return "direct";
    case miopenConvolutionFwdAlgoFFT: return "fft";
    case miopenConvolutionFwdAlgoWinograd: return "winograd";
    case miopenConvolutionFwdAlgoImplicitGEMM: return "implicit_gemm";
    default: return "other";
  }
}

}  // namespace

int main(int argc, char **argv) {
  const Options opt = parse(argc, argv);
  const i8conv_shape s = load_case(opt.config, opt.name);
  i8conv_geometry g;
  check(i8conv_derive(&s, &g), "derive");

  // the same data as conv_lab (input, then filter, from one stream); zero bias
  uint64_t state = opt.seed;
  std::vector<int8_t> x(size_t(g.input_elements)), w(size_t(g.filter_elements));
  i8conv_fill_int8(x.data(), x.size(), -128, 127, &state);
  i8conv_fill_int8(w.data(), w.size(), -128, 127, &state);
  const std::vector<int32_t> bias(size_t(g.gemm_n), 0);

  void *dx = nullptr, *dw = nullptr, *db = nullptr, *dy = nullptr, *dv = nullptr, *ws = nullptr;
  const size_t ybytes = size_t(g.output_elements) * 4;
  check(i8conv_device_alloc(&dx, x.size()), "alloc input");
  check(i8conv_device_alloc(&dw, w.size()), "alloc filter");
  check(i8conv_device_alloc(&db, bias.size() * 4), "alloc bias");
  check(i8conv_device_alloc(&dy, ybytes), "alloc output");
  check(i8conv_device_alloc(&dv, ybytes), "alloc vendor output");
  check(i8conv_copy_to_device(dx, x.data(), x.size()), "copy input");
  check(i8conv_copy_to_device(dw, w.data(), w.size()), "copy filter");
  check(i8conv_copy_to_device(db, bias.data(), bias.size() * 4), "copy bias");

  // ---- this lab: the dispatched kernel ----
  const int id = i8conv_dispatch(&s);
  if (id < 0) fail("no dispatched kernel");
  const size_t lab_ws = i8conv_workspace_bytes(id, &s);
  void *lws = nullptr;
  if (lab_ws) check(i8conv_device_alloc(&lws, lab_ws), "alloc workspace");
  check(i8conv_launch(id, &s, static_cast<int8_t *>(dx), static_cast<int8_t *>(dw),
                      static_cast<int32_t *>(db), static_cast<int32_t *>(dy), lws, lab_ws, nullptr),
        "launch");
  check(i8conv_synchronize(), "synchronize");
  float lab_med = 0, lab_batched = 0;
  check(i8conv_measure(id, &s, static_cast<int8_t *>(dx), static_cast<int8_t *>(dw),
                       static_cast<int32_t *>(db), static_cast<int32_t *>(dy), lws, lab_ws, nullptr,
                       opt.warmup, opt.iterations, &lab_med, &lab_batched),
        "measure");

  // ---- MIOpen ----
  std::string contract = "miopen int8 NHWC x KYXC -> int32 NHWC, alpha 1 beta 0, no bias";
  float v_med = -1, v_batched = -1;
  int v_correct = -1;
  std::string v_algo = "-";
  miopenHandle_t h = nullptr;
  miopenTensorDescriptor_t xd = nullptr, wd = nullptr, yd = nullptr;
  miopenConvolutionDescriptor_t cd = nullptr;
  hipStream_t stream = nullptr;
  hip_check(hipStreamCreate(&stream), "hipStreamCreate");
  bool ok = miopenCreateWithStream(&h, stream) == miopenStatusSuccess &&
            miopenCreateTensorDescriptor(&xd) == miopenStatusSuccess &&
            miopenCreateTensorDescriptor(&wd) == miopenStatusSuccess &&
            miopenCreateTensorDescriptor(&yd) == miopenStatusSuccess &&
            miopenCreateConvolutionDescriptor(&cd) == miopenStatusSuccess;
  if (!ok) fail("MIOpen handle/descriptor creation failed");
  const int xl[4] = {s.n, s.c, s.h, s.w};
  const int wl[4] = {s.k, s.c, s.r, s.s};
  const int yl[4] = {s.n, s.k, g.out_h, g.out_w};
  miopenStatus_t st = miopenSetNdTensorDescriptorWithLayout(xd, miopenInt8, miopenTensorNHWC, xl, 4);
  if (st == miopenStatusSuccess)
    st = miopenSetNdTensorDescriptorWithLayout(wd, miopenInt8, miopenTensorNHWC, wl, 4);
  if (st == miopenStatusSuccess)
    st = miopenSetNdTensorDescriptorWithLayout(yd, miopenInt32, miopenTensorNHWC, yl, 4);
  if (st == miopenStatusSuccess)
    st = miopenInitConvolutionDescriptor(cd, miopenConvolution, s.pad_h, s.pad_w, s.stride_h,
                                         s.stride_w, s.dilation_h, s.dilation_w);
  size_t ws_bytes = 0;
  if (st == miopenStatusSuccess)
    st = miopenConvolutionForwardGetWorkSpaceSize(h, wd, xd, cd, yd, &ws_bytes);
  if (st == miopenStatusSuccess && ws_bytes) hip_check(hipMalloc(&ws, ws_bytes), "hipMalloc ws");
  miopenConvAlgoPerf_t perf[8];
  int found = 0;
  if (st == miopenStatusSuccess)
    st = miopenFindConvolutionForwardAlgorithm(h, xd, dx, wd, dw, cd, yd, dv, 8, &found, perf, ws,
                                               ws_bytes, true);
  if (st != miopenStatusSuccess || found == 0) {
    contract += std::string("; unsupported: ") + miopenGetErrorString(st);
  } else {
    const miopenConvFwdAlgorithm_t algo = perf[0].fwd_algo;
    v_algo = algo_name(algo);
    const float alpha = 1.0f, beta = 0.0f;
    auto run = [&]() {
      return miopenConvolutionForward(h, &alpha, xd, dx, wd, dw, cd, algo, &beta, yd, dv, ws,
                                      ws_bytes);
    };
    hip_check(hipMemsetAsync(dv, 0xA5, ybytes, stream), "poison");
    if (run() != miopenStatusSuccess) fail("miopenConvolutionForward failed");
    hip_check(hipStreamSynchronize(stream), "sync");
    // correctness: element for element against the dispatched kernel
    std::vector<int32_t> a(size_t(g.output_elements)), b(size_t(g.output_elements));
    check(i8conv_copy_to_host(a.data(), dy, ybytes), "copy lab output");
    hip_check(hipMemcpy(b.data(), dv, ybytes, hipMemcpyDeviceToHost), "copy vendor output");
    v_correct = a == b ? 1 : 0;
    for (int i = 0; i < opt.warmup; ++i) run();
    hip_check(hipStreamSynchronize(stream), "sync");
    hipEvent_t e0, e1;
    hip_check(hipEventCreate(&e0), "event");
    hip_check(hipEventCreate(&e1), "event");
    std::vector<float> t;
    for (int i = 0; i < opt.iterations; ++i) {
      hip_check(hipEventRecord(e0, stream), "record");
      run();
      hip_check(hipEventRecord(e1, stream), "record");
      hip_check(hipEventSynchronize(e1), "sync");
      float ms = 0;
      hip_check(hipEventElapsedTime(&ms, e0, e1), "elapsed");
      t.push_back(ms);
    }
    std::sort(t.begin(), t.end());
    v_med = t[t.size() / 2];
    hip_check(hipEventRecord(e0, stream), "record");
    for (int i = 0; i < opt.iterations; ++i) run();
    hip_check(hipEventRecord(e1, stream), "record");
    hip_check(hipEventSynchronize(e1), "sync");
    float total = 0;
    hip_check(hipEventElapsedTime(&total, e0, e1), "elapsed");
    v_batched = total / float(opt.iterations);
    hip_check(hipEventDestroy(e0), "event");
    hip_check(hipEventDestroy(e1), "event");
  }

  std::ostringstream row;
  row << opt.name << ',' << s.n << ',' << s.h << ',' << s.w << ',' << s.c << ',' << s.k << ','
      << s.r << ',' << s.s << ',' << s.pad_h << ',' << s.pad_w << ',' << s.stride_h << ','
      << s.stride_w << ',' << s.dilation_h << ',' << s.dilation_w << ',' << i8conv_kernel_name(id)
      << ',' << lab_med << ',' << lab_batched << ",miopen," << v_algo << ',' << v_med << ','
      << v_batched << ',' << (v_med > 0 ? v_med / lab_med : -1.0f) << ',' << v_correct << ",\""
      << contract << "\"";
  if (opt.csv) {
    if (opt.header)
      std::cout << "case,n,h,w,c,k,r,s,pad_h,pad_w,stride_h,stride_w,dilation_h,dilation_w,"
                   "dispatch,dispatch_ms,dispatch_batched_ms,vendor,vendor_algo,vendor_ms,"
                   "vendor_batched_ms,vendor_over_dispatch,vendor_correct,comparison_contract\n";
    std::cout << row.str() << '\n';
  } else {
    std::cout << opt.name << ": dispatch " << i8conv_kernel_name(id) << " " << lab_med * 1e3
              << " us; miopen " << v_algo << " " << v_med * 1e3 << " us (x"
              << (v_med > 0 ? v_med / lab_med : -1.0f) << "), correct " << v_correct << "; "
              << contract << '\n';
  }
  if (ws) hip_check(hipFree(ws), "free");
  miopenDestroyConvolutionDescriptor(cd);
  miopenDestroyTensorDescriptor(yd);
  miopenDestroyTensorDescriptor(wd);
  miopenDestroyTensorDescriptor(xd);
  miopenDestroy(h);
  hip_check(hipStreamDestroy(stream), "stream");
  for (void *p : {dx, dw, db, dy, dv, lws})
    if (p) check(i8conv_device_free(p), "free");
  return v_correct == 0 ? 1 : 0;
}
