// conv_lab: host driver of the INT8 convolution lab (the counterpart of the
// reference's src/conv_lab.cu).  It reads one case from a workload CSV at run
// time (the reference compiled one case per binary, gen_case.py + Makefile),
// generates seeded data, and for every selected candidate kernel:
//   poison the output -> launch -> check EVERY output element against a CPU
//   INT32 direct convolution -> only if correct, time it (warmup + median of
//   per-launch event pairs, conv_lab.cu:88-110, plus a batched figure).
// It then prints the reference's CSV row (conv_lab.cu:223-230) with extra
// columns appended, and exits 0 iff every candidate run was correct and a
// winner exists (conv_lab.cu:241).
//
// All GPU work goes through the C ABI in i8conv.h; this file is plain C++.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

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

// ---- options (conv_lab.cu:112-145, extended) ------------------------------

struct Options {
  std::string strategy = "both";  // generic|strip|halo|splitk|both|all|dispatch
  bool csv = false;
  bool header = true;
  int warmup = 20;
  int iterations = 101;
  std::string config;  // workload CSV
  std::string name = "cfg1_smoke";
  std::string range = "baseline";  // baseline: int8 full range; reference: U[-4,4]
  uint64_t seed = 20260925;
  int threads = 0;  // CPU check threads, 0 = all
};

[[noreturn]] void usage() {
  std::cerr << "usage: conv_lab [--strategy generic|strip|halo|splitk|both|all|dispatch] "
               "[--csv] [--no-header] [--warmup N] [--iterations N] [--config FILE] "
               "[--case NAME] [--range baseline|reference] [--seed N] [--threads N]\n";
  std::exit(EXIT_FAILURE);
}

Options parse_options(int argc, char **argv) {
  Options o;
  o.config = exe_dir() + "/workloads/baseline.csv";
  for (int i = 1; i < argc; ++i) {
    const std::string arg = argv[i];
    if (arg == "--csv") {
      o.csv = true;
    } else if (arg == "--no-header") {
      o.header = false;
    } else if ((arg == "--strategy" || arg == "--warmup" || arg == "--iterations" ||
                arg == "--config" || arg == "--case" || arg == "--range" ||
                arg == "--seed" || arg == "--threads") &&
               i + 1 < argc) {
      const std::string v = argv[++i];
      try {
        if (arg == "--strategy") o.strategy = v;
        if (arg == "--warmup") o.warmup = std::stoi(v);
        if (arg == "--iterations") o.iterations = std::stoi(v);
        if (arg == "--config") o.config = v;
        if (arg == "--case") o.name = v;
        if (arg == "--range") o.range = v;
        if (arg == "--seed") o.seed = std::stoull(v);
        if (arg == "--threads") o.threads = std::stoi(v);
      } catch (const std::exception &) {
        usage();
      }
    } else {
      usage();
    }
  }
  static const char *kStrategies[] = {"generic", "strip", "halo", "splitk",
                                      "both", "all", "dispatch"};
  bool known = false;
  for (const char *s : kStrategies) known = known || o.strategy == s;
  if (!known || o.warmup < 0 || o.iterations <= 0 || o.threads < 0 ||
      (o.range != "baseline" && o.range != "reference")) {
    std::cerr << "invalid benchmark options\n";
    std::exit(EXIT_FAILURE);
  }
  return o;
}

// ---- CPU INT32 check --------------------------------------------------------
// bias + sum over valid taps (fy, fx) and channels of x*w, int32 with wrap,
// for every output element (the semantics of conv_lab.cu:39-66), split over
// output pixels across threads.
void cpu_conv(const i8conv_shape &s, const i8conv_geometry &g,
              const std::vector<int8_t> &x, const std::vector<int8_t> &w,
              const std::vector<int32_t> &bias, std::vector<int32_t> &out,
              int threads) {
  auto work = [&](int64_t m0, int64_t m1) {
    std::vector<uint32_t> acc(size_t(s.k));
    for (int64_t m = m0; m < m1; ++m) {
      const int ox = int(m % g.out_w);
      const int oy = int((m / g.out_w) % g.out_h);
      const int b = int(m / (int64_t(g.out_w) * g.out_h));
      for (int j = 0; j < s.k; ++j) acc[size_t(j)] = uint32_t(bias[size_t(j)]);
      for (int fy = 0; fy < s.r; ++fy) {
        const int iy = oy * s.stride_h + fy * s.dilation_h - s.pad_h;
        if (iy < 0 || iy >= s.h) continue;
        for (int fx = 0; fx < s.s; ++fx) {
          const int ix = ox * s.stride_w + fx * s.dilation_w - s.pad_w;
          if (ix < 0 || ix >= s.w) continue;
          const int8_t *xp = &x[((size_t(b) * s.h + iy) * s.w + ix) * s.c];
          for (int j = 0; j < s.k; ++j) {
            const int8_t *wp = &w[((size_t(j) * s.r + fy) * s.s + fx) * s.c];
            int32_t dot = 0;
            for (int ci = 0; ci < s.c; ++ci) dot += int32_t(xp[ci]) * int32_t(wp[ci]);
            acc[size_t(j)] += uint32_t(dot);
          }
        }
      }
      for (int j = 0; j < s.k; ++j) out[size_t(m) * s.k + j] = int32_t(acc[size_t(j)]);
    }
  };
  const int64_t m = g.gemm_m;
  const int t = int(std::max<int64_t>(1, std::min<int64_t>(threads, m)));
  std::vector<std::thread> pool;
  for (int i = 0; i < t; ++i) pool.emplace_back(work, m * i / t, m * (i + 1) / t);
  for (auto &th : pool) th.join();
}

// Full comparison (the reference sampled 2048 outputs, conv_lab.cu:72-77).
bool validate(const std::vector<int32_t> &expected, const std::vector<int32_t> &got,
              const char *label) {
  for (size_t i = 0; i < expected.size(); ++i) {
    if (expected[i] != got[i]) {
      std::cerr << label << " mismatch at output " << i << ": expected " << expected[i]
                << ", got " << got[i] << '\n';
      return false;
    }
  }
  return true;
}

struct Result {
  bool eligible = false;
  bool ran = false;
  bool correct = true;
  float ms = -1.f;
  float batched_ms = -1.f;
};

std::string fmt(float v) {
  std::ostringstream o;
  o << v;
  return o.str();
}

}  // namespace

int main(int argc, char **argv) {
  const Options opt = parse_options(argc, argv);
  const i8conv_shape shape = load_case(opt.config, opt.name);
  i8conv_geometry g;
  check(i8conv_derive(&shape, &g), "shape");

  // Data: input, then filter, then bias from one seeded stream.
  uint64_t state = opt.seed;
  std::vector<int8_t> x(size_t(g.input_elements)), w(size_t(g.filter_elements));
  std::vector<int32_t> bias(size_t(shape.k));
  const bool ref_range = opt.range == "reference";
  i8conv_fill_int8(x.data(), x.size(), ref_range ? -4 : -128, ref_range ? 4 : 127, &state);
  i8conv_fill_int8(w.data(), w.size(), ref_range ? -4 : -128, ref_range ? 4 : 127, &state);
  i8conv_fill_int32(bias.data(), bias.size(), ref_range ? -31 : -(1 << 20),
                    ref_range ? 31 : (1 << 20), &state);

  const int threads = opt.threads ? opt.threads
                                  : int(std::max(1u, std::thread::hardware_concurrency()));
  std::vector<int32_t> expected(size_t(g.output_elements));
  const auto t0 = std::chrono::steady_clock::now();
  cpu_conv(shape, g, x, w, bias, expected, threads);
  const double cpu_ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();

  void *d_x = nullptr, *d_w = nullptr, *d_b = nullptr, *d_y = nullptr, *d_ws = nullptr;
  check(i8conv_device_alloc(&d_x, x.size()), "alloc input");
  check(i8conv_device_alloc(&d_w, w.size()), "alloc filter");
  check(i8conv_device_alloc(&d_b, bias.size() * 4), "alloc bias");
  check(i8conv_device_alloc(&d_y, expected.size() * 4), "alloc output");
  check(i8conv_copy_to_device(d_x, x.data(), x.size()), "copy input");
  check(i8conv_copy_to_device(d_w, w.data(), w.size()), "copy filter");
  check(i8conv_copy_to_device(d_b, bias.data(), bias.size() * 4), "copy bias");
  size_t ws_bytes = 0;
  for (int id = 0; id < i8conv_kernel_count(); ++id)
    ws_bytes = std::max(ws_bytes, i8conv_workspace_bytes(id, &shape));
  if (ws_bytes) check(i8conv_device_alloc(&d_ws, ws_bytes), "alloc workspace");

  const int dispatched = i8conv_dispatch(&shape);
  std::vector<int> run;
  const std::string &st = opt.strategy;
  for (int id = 0; id < i8conv_kernel_count(); ++id) {
    const std::string name = i8conv_kernel_name(id);
    const bool pick = st == "all" || st == name ||
                      (st == "both" && (name == "generic" || name == "strip")) ||
                      (st == "dispatch" && id == dispatched);
    if (pick) run.push_back(id);
  }

  const size_t kernel_count = size_t(i8conv_kernel_count());
  std::vector<Result> res(kernel_count);
  std::vector<int32_t> got(expected.size());
  for (int id = 0; id < i8conv_kernel_count(); ++id)
    res[size_t(id)].eligible = i8conv_eligible(id, &shape) != 0;
  for (int id : run) {
    Result &r = res[size_t(id)];
    if (!r.eligible) continue;
    const char *name = i8conv_kernel_name(id);
    r.ran = true;
    // Poison so a kernel that skips stores cannot pass on stale output.
    check(i8conv_device_fill(d_y, 0xA5, expected.size() * 4), "poison output");
    check(i8conv_launch(id, &shape, static_cast<int8_t *>(d_x), static_cast<int8_t *>(d_w),
                        static_cast<int32_t *>(d_b), static_cast<int32_t *>(d_y), d_ws,
                        ws_bytes, nullptr),
          name);
    check(i8conv_synchronize(), name);
    check(i8conv_copy_to_host(got.data(), d_y, got.size() * 4), "copy output");
    r.correct = validate(expected, got, name);
    // a bounded wait that gave up means data the kernel read had not landed
    int expired = 0;
    check(i8conv_wait_expired(&expired), name);
    if (expired) {
      std::cerr << name << ": a bounded wait inside the kernel gave up\n";
      r.correct = false;
    }
    if (r.correct) {
      check(i8conv_measure(id, &shape, static_cast<int8_t *>(d_x), static_cast<int8_t *>(d_w),
                           static_cast<int32_t *>(d_b), static_cast<int32_t *>(d_y), d_ws,
                           ws_bytes, nullptr, opt.warmup, opt.iterations, &r.ms,
                           &r.batched_ms),
            name);
      check(i8conv_wait_expired(&expired), name);
      if (expired) {
        std::cerr << name << ": a bounded wait gave up during the timed launches\n";
        r.correct = false;
        r.ms = -1.0f;
      }
    }
  }

  int winner = -1;
  for (int id : run) {
    const Result &r = res[size_t(id)];
    if (r.ms >= 0 && (winner < 0 || r.ms < res[size_t(winner)].ms)) winner = id;
  }
  bool all_correct = true;
  for (int id : run) all_correct = all_correct && res[size_t(id)].correct;

  const double ops = 2.0 * double(g.gemm_m) * double(g.gemm_n) * double(g.gemm_k);
  const double bytes = double(g.input_elements) + double(g.filter_elements) +
                       4.0 * double(shape.k) + 4.0 * double(g.output_elements);
  int cus = 0, clock_khz = 0;
  char arch[64] = {0};
  check(i8conv_device_info(&cus, &clock_khz, arch, sizeof(arch)), "device info");
  const double best_ms = winner >= 0 ? res[size_t(winner)].ms : -1.0;
  const double tops = best_ms > 0 ? ops / (best_ms * 1e-3) / 1e12 : -1.0;
  const double peak_tops = 5000.0;  // MI355X dense INT8 MFMA, published
  const double gbps = best_ms > 0 ? bytes / (best_ms * 1e-3) / 1e9 : -1.0;
  const double hbm_gbps = 8000.0;   // MI355X HBM3E, published

  char plan_buf[256] = {0};
  if (dispatched >= 0) i8conv_describe(dispatched, &shape, plan_buf, sizeof(plan_buf));
  std::string plan(plan_buf);
  std::replace(plan.begin(), plan.end(), ',', ';');  // keep the CSV row flat
  const Result &gr = res[I8CONV_KERNEL_GENERIC];
  const Result &sr = res[I8CONV_KERNEL_STRIP];
  const Result &hr = res[I8CONV_KERNEL_HALO];
  const Result &kr = res[I8CONV_KERNEL_SPLITK];
  const char *wname = winner >= 0 ? i8conv_kernel_name(winner) : "none";
  if (opt.csv) {
    if (opt.header)
      std::cout << "case,n,h,w,c,k,r,s,out_h,out_w,eligible_strip,generic_ms,"
                   "strip_ms,winner,generic_correct,strip_correct,"
                   "pad_h,pad_w,stride_h,stride_w,dilation_h,dilation_w,"
                   "eligible_halo,halo_ms,halo_correct,eligible_splitk,splitk_ms,"
                   "splitk_correct,dispatch,winner_batched_ms,tops,pct_int8_peak,gbps,"
                   "pct_hbm,cpu_check_ms,cpu_threads,device,cus,dispatch_plan\n";
    std::cout << opt.name << ',' << shape.n << ',' << shape.h << ',' << shape.w << ','
              << shape.c << ',' << shape.k << ',' << shape.r << ',' << shape.s << ','
              << g.out_h << ',' << g.out_w << ',' << (sr.eligible ? 1 : 0) << ','
              << fmt(gr.ms) << ',' << fmt(sr.ms) << ',' << wname << ','
              << (gr.correct ? 1 : 0) << ',' << (sr.correct ? 1 : 0) << ','
              << shape.pad_h << ',' << shape.pad_w << ',' << shape.stride_h << ','
              << shape.stride_w << ',' << shape.dilation_h << ',' << shape.dilation_w << ','
              << (hr.eligible ? 1 : 0) << ',' << fmt(hr.ms) << ',' << (hr.correct ? 1 : 0)
              << ',' << (kr.eligible ? 1 : 0) << ',' << fmt(kr.ms) << ','
              << (kr.correct ? 1 : 0) << ','
              << (dispatched >= 0 ? i8conv_kernel_name(dispatched) : "none") << ','
              << fmt(winner >= 0 ? res[size_t(winner)].batched_ms : -1.f) << ','
              << std::setprecision(6) << tops << ',' << (tops > 0 ? 100.0 * tops / peak_tops : -1.0)
              << ',' << gbps << ',' << (gbps > 0 ? 100.0 * gbps / hbm_gbps : -1.0) << ','
              << cpu_ms << ',' << threads << ',' << arch << ',' << cus << ',' << plan << '\n';
  } else {
    std::cout << opt.name << ":";
    for (int id : run) {
      const Result &r = res[size_t(id)];
      std::cout << ' ' << i8conv_kernel_name(id) << ' ';
      if (!r.eligible) std::cout << "ineligible";
      else if (r.ms >= 0) std::cout << std::fixed << std::setprecision(4) << r.ms << " ms";
      else std::cout << "failed";
      std::cout << ',';
    }
    std::cout << " winner " << wname;
    if (tops > 0)
      std::cout << std::fixed << std::setprecision(1) << " (" << tops << " TOPS, "
                << 100.0 * tops / peak_tops << "% of INT8 peak, " << gbps << " GB/s)";
    std::cout << '\n';
  }

  i8conv_device_free(d_ws);
  i8conv_device_free(d_y);
  i8conv_device_free(d_b);
  i8conv_device_free(d_w);
  i8conv_device_free(d_x);
  return all_correct && winner >= 0 ? 0 : 1;
}
