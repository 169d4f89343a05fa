// The C ABI: registry, eligibility, launch, and the thin HIP runtime layer
// the host driver uses (allocation, copies, events).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "i8conv_internal.hpp"

namespace i8conv {

namespace {
thread_local std::string g_last_error;

const char *const kNames[I8CONV_KERNEL_COUNT] = {"generic", "strip", "halo", "splitk"};

int hip_fail(const char *what, hipError_t e) {
  set_error(std::string(what) + ": " + hipGetErrorString(e));
  return I8CONV_HIP_ERROR;
}

bool aligned(const void *p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// Clock stamps of measure_graph_loop's stamped region.  stamps[0] counts
// the stamped graph replays that have started; replay i's start time goes to
// stamps[2 + 2 i], its end time to stamps[3 + 2 i] (i < cap; later replays
// are not recorded).  The time is the device's constant-rate clock
// (hipDeviceAttributeWallClockRate), read when the kernel's wave runs, that
// is once the graph's previous node has finished.  One lane, vector atomics
// and stores.
__global__ void clock_stamp_kernel(unsigned long long *stamps, int cap, int end) {
  if (threadIdx.x != 0) return;
  const unsigned long long t = __builtin_amdgcn_s_memrealtime();
  const unsigned long long i = end ? atomicAdd(stamps, 0ull) - 1ull : atomicAdd(stamps, 1ull);
  if (i < static_cast<unsigned long long>(cap)) stamps[2 + 2 * i + (end ? 1 : 0)] = t;
}
// measure() of conv_lab.cu:88-110 around any launch: `warmup` launches,
// then `iterations` back-to-back launches between one event pair on
// `stream` (mean per launch: the timed steps are enqueued right behind the
// warmup, with no synchronization between), then `iterations` launches each
// bracketed by its own event pair and synchronized (median per launch).
template <class Launch>
int measure_loop(Launch launch, void *stream, int warmup, int iterations, float *median_ms,
                 float *batched_ms) {
  if (warmup < 0 || iterations <= 0 || !median_ms) {
    set_error("measure needs warmup >= 0, iterations > 0 and an output");
    return I8CONV_BAD_ARGUMENT;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int i = 0; i < warmup; ++i) {
    const int rc = launch();
    if (rc != I8CONV_OK) return rc;
  }
  hipError_t e = hipSuccess;
  // without the batched figure the warmup is synchronized here; with it,
  // the batched launches are enqueued right behind the warmup (the GPU
  // does not idle before them) and synchronized after
  if (!batched_ms && (e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail("warmup", e);
  hipEvent_t start, stop;
  if ((e = hipEventCreate(&start)) != hipSuccess) return hip_fail("hipEventCreate", e);
  if ((e = hipEventCreate(&stop)) != hipSuccess) {
    (void)hipEventDestroy(start);
    return hip_fail("hipEventCreate", e);
  }
  int rc = I8CONV_OK;
  if (batched_ms) {
    float ms = 0.f;
    if ((e = hipEventRecord(start, s)) != hipSuccess) rc = hip_fail("hipEventRecord", e);
    for (int i = 0; i < iterations && rc == I8CONV_OK; ++i) rc = launch();
    if (rc == I8CONV_OK && (e = hipEventRecord(stop, s)) != hipSuccess) rc = hip_fail("hipEventRecord", e);
    if (rc == I8CONV_OK && (e = hipEventSynchronize(stop)) != hipSuccess) rc = hip_fail("hipEventSynchronize", e);
    if (rc == I8CONV_OK && (e = hipEventElapsedTime(&ms, start, stop)) != hipSuccess) rc = hip_fail("hipEventElapsedTime", e);
    if (rc == I8CONV_OK) *batched_ms = ms / float(iterations);
  }
  std::vector<float> samples;
  samples.reserve(size_t(iterations));
  for (int i = 0; i < iterations && rc == I8CONV_OK; ++i) {
    float ms = 0.f;
    if ((e = hipEventRecord(start, s)) != hipSuccess) { rc = hip_fail("hipEventRecord", e); break; }
    if ((rc = launch()) != I8CONV_OK) break;
    if ((e = hipEventRecord(stop, s)) != hipSuccess) { rc = hip_fail("hipEventRecord", e); break; }
    if ((e = hipEventSynchronize(stop)) != hipSuccess) { rc = hip_fail("hipEventSynchronize", e); break; }
    if ((e = hipEventElapsedTime(&ms, start, stop)) != hipSuccess) { rc = hip_fail("hipEventElapsedTime", e); break; }
    samples.push_back(ms);
  }
  if (rc == I8CONV_OK) {
    std::sort(samples.begin(), samples.end());
    *median_ms = samples[samples.size() / 2];
  }
  // teardown: a failure here cannot change the measured result
  (void)hipEventDestroy(start);
  (void)hipEventDestroy(stop);
  return rc;
}

// Back-to-back launches replayed from HIP graphs on a stream of its own
// (default priority), the steps documented at i8conv_measure_graph.  The
// warmup ends in a tail of replays that the host does not wait for, and
// both timed regions are enqueued behind it: the timed launches run on a
// GPU that has not idled since the warmup (an idle of some hundred
// microseconds while the host synchronizes, poisons the output and records
// events let the first launches after it run ~10 % slower on 28x28x128,
// which weighed on short runs).  Each graph replay starts some microseconds
// after the previous one ends (28x28x128: ~8 us), so the event-timed region
// holds one such gap per replay; event records captured into a graph would
// keep it out, but HIP cannot time them (hipEventElapsedTime fails on
// them), hence the stamped figure beside it.  launch(stream) enqueues one
// launch.
template <class Launch>
int measure_graph_loop(Launch launch, void *output, size_t out_bytes, int warmup,
                       double min_warmup_ms, int iterations, int launches_per_graph,
                       int poison_byte, i8conv_graph_timing *timing) {
  const int per_graph = std::min(launches_per_graph, iterations);
  const int full_replays = iterations / per_graph;
  const int remainder = iterations - full_replays * per_graph;
  const int replays = full_replays + (remainder > 0 ? 1 : 0);
  *timing = i8conv_graph_timing{};

  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);  // default priority
  if (e != hipSuccess) return hip_fail("hipStreamCreateWithFlags", e);
  // graphs: [0] main, [1] remainder, [2] stamped main, [3] stamped remainder
  hipGraph_t graphs[4] = {nullptr, nullptr, nullptr, nullptr};
  hipGraphExec_t execs[4] = {nullptr, nullptr, nullptr, nullptr};
  hipEvent_t start = nullptr, stop = nullptr, sstart = nullptr, sstop = nullptr;
  hipEvent_t kstart = nullptr, kstop = nullptr;
  // fills the output with the poison byte, enqueued on the stream (a fill
  // kernel outside any graph), so that a check after the stream region
  // sees only what its launches wrote
  auto poison = [&]() {
    if (poison_byte < 0 || out_bytes == 0) return int(I8CONV_OK);
    const hipError_t pe = hipMemsetAsync(output, poison_byte, out_bytes, s);
    return pe == hipSuccess ? int(I8CONV_OK) : hip_fail("poison", pe);
  };
  // stamped replays: one record each (start, end)
  const int stamp_cap = replays;
  const size_t stamp_bytes = sizeof(unsigned long long) * size_t(2 + 2 * stamp_cap);
  unsigned long long *stamps = nullptr;
  // captures `count` launches (kernel nodes only) into graphs[slot]; the
  // stamped slots (2, 3) between a start and an end clock-stamp kernel
  auto capture = [&](int slot, int count) {
    const bool stamped = slot >= 2;
    hipError_t ce = hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed);
    if (ce != hipSuccess) return hip_fail("hipStreamBeginCapture", ce);
    int crc = I8CONV_OK;
    auto stamp = [&](int end) {
      if (!stamped || crc != I8CONV_OK) return;
      hipLaunchKernelGGL(clock_stamp_kernel, dim3(1), dim3(64), 0, s, stamps, stamp_cap, end);
      const hipError_t le = hipGetLastError();
      if (le != hipSuccess) crc = hip_fail("clock stamp launch", le);
    };
    stamp(0);
    for (int i = 0; i < count && crc == I8CONV_OK; ++i) crc = launch(s);
    stamp(1);
    // end the capture whatever happened inside it
    ce = hipStreamEndCapture(s, &graphs[slot]);
    if (crc == I8CONV_OK && ce != hipSuccess) crc = hip_fail("hipStreamEndCapture", ce);
    if (crc == I8CONV_OK &&
        (ce = hipGraphInstantiate(&execs[slot], graphs[slot], nullptr, nullptr, 0)) != hipSuccess)
      crc = hip_fail("hipGraphInstantiate", ce);
    return crc;
  };
  // enqueues the K timed launches from graph slots base (main) and base + 1
  auto replay_all = [&](int base) {
    for (int i = 0; i < full_replays; ++i)
      if (const hipError_t ge = hipGraphLaunch(execs[base], s); ge != hipSuccess)
        return hip_fail("hipGraphLaunch", ge);
    if (remainder > 0)
      if (const hipError_t ge = hipGraphLaunch(execs[base + 1], s); ge != hipSuccess)
        return hip_fail("hipGraphLaunch", ge);
    return int(I8CONV_OK);
  };
  int dev = 0, rate_khz = 0;
  // one launch outside the graphs (checks the arguments, sets any function
  // attribute the kernel needs), then the captures
  int rc = launch(s);
  if (rc == I8CONV_OK && (e = hipStreamSynchronize(s)) != hipSuccess) rc = hip_fail("launch", e);
  if (rc == I8CONV_OK && (e = hipGetDevice(&dev)) != hipSuccess) rc = hip_fail("hipGetDevice", e);
  if (rc == I8CONV_OK &&
      (e = hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev)) != hipSuccess)
    rc = hip_fail("hipDeviceGetAttribute(WallClockRate)", e);
  if (rc == I8CONV_OK && rate_khz <= 0) {
    set_error("measure_graph: the device reports no wall-clock rate");
    rc = I8CONV_HIP_ERROR;
  }
  if (rc == I8CONV_OK && (e = hipMalloc(reinterpret_cast<void **>(&stamps), stamp_bytes)) != hipSuccess)
    rc = hip_fail("hipMalloc(stamps)", e);
  if (rc == I8CONV_OK && (e = hipEventCreate(&start)) != hipSuccess) rc = hip_fail("hipEventCreate", e);
  if (rc == I8CONV_OK && (e = hipEventCreate(&stop)) != hipSuccess) rc = hip_fail("hipEventCreate", e);
  if (rc == I8CONV_OK && (e = hipEventCreate(&sstart)) != hipSuccess) rc = hip_fail("hipEventCreate", e);
  if (rc == I8CONV_OK && (e = hipEventCreate(&kstart)) != hipSuccess) rc = hip_fail("hipEventCreate", e);
  if (rc == I8CONV_OK && (e = hipEventCreate(&kstop)) != hipSuccess) rc = hip_fail("hipEventCreate", e);
  if (rc == I8CONV_OK && (e = hipEventCreate(&sstop)) != hipSuccess) rc = hip_fail("hipEventCreate", e);
  if (rc == I8CONV_OK) rc = capture(0, per_graph);
  if (rc == I8CONV_OK && remainder > 0) rc = capture(1, remainder);
  if (rc == I8CONV_OK) rc = capture(2, per_graph);
  if (rc == I8CONV_OK && remainder > 0) rc = capture(3, remainder);
  // warmup: replays of the main graph until at least `warmup` launches have
  // run and at least min_warmup_ms of wall time has passed (back-to-back
  // launches need some tens of ms to bring the clocks to their steady
  // state); batches of replays between host checks, doubling up to 64
  int warm_launches = 0;
  double warm_ms = 0.0, batch_ms = 0.0;
  int last_batch = 1;
  const auto t0 = std::chrono::steady_clock::now();
  for (int batch = 1; rc == I8CONV_OK && (warm_launches < warmup || warm_ms < min_warmup_ms);) {
    const auto b0 = std::chrono::steady_clock::now();
    for (int i = 0; i < batch && rc == I8CONV_OK; ++i)
      if ((e = hipGraphLaunch(execs[0], s)) != hipSuccess) rc = hip_fail("hipGraphLaunch", e);
    if (rc == I8CONV_OK && (e = hipStreamSynchronize(s)) != hipSuccess) rc = hip_fail("warmup", e);
    const auto b1 = std::chrono::steady_clock::now();
    warm_launches += batch * per_graph;
    warm_ms = std::chrono::duration<double, std::milli>(b1 - t0).count();
    batch_ms = std::chrono::duration<double, std::milli>(b1 - b0).count();
    last_batch = batch;
    batch = std::min(2 * batch, 64);
  }
  // The tail: about kTailMs of main-graph replays (by the last batch's
  // rate, at least one and at most 4096), not waited for; everything after
  // it is enqueued while it runs, so the GPU goes from warm launches
  // straight into the timed ones.
  constexpr double kTailMs = 5.0;
  const double ms_per_replay = batch_ms / double(last_batch);
  const int tail = ms_per_replay > 0.0
                       ? int(std::min(4096.0, std::max(1.0, std::ceil(kTailMs / ms_per_replay))))
                       : 1;
  for (int i = 0; i < tail && rc == I8CONV_OK; ++i)
    if ((e = hipGraphLaunch(execs[0], s)) != hipSuccess) rc = hip_fail("hipGraphLaunch", e);
  if (rc == I8CONV_OK) warm_launches += tail * per_graph;
  // stamped region: the stamp records cleared on the stream, then the K
  // launches from the stamped graphs
  if (rc == I8CONV_OK && (e = hipMemsetAsync(stamps, 0, stamp_bytes, s)) != hipSuccess)
    rc = hip_fail("hipMemsetAsync(stamps)", e);
  if (rc == I8CONV_OK) rc = replay_all(2);
  // event-timed graph region: exactly `iterations` launches from the main
  // and remainder graphs between one pair of events
  if (rc == I8CONV_OK && (e = hipEventRecord(start, s)) != hipSuccess) rc = hip_fail("hipEventRecord", e);
  if (rc == I8CONV_OK) rc = replay_all(0);
  if (rc == I8CONV_OK && (e = hipEventRecord(stop, s)) != hipSuccess) rc = hip_fail("hipEventRecord", e);
  // stream region: the output poisoned, then the K launches enqueued one by
  // one on the stream (no graph) between one pair of events; they are
  // enqueued while the tail still runs, so the GPU does not wait for the
  // host, and the output then holds only what they wrote
  if (rc == I8CONV_OK) rc = poison();
  if (rc == I8CONV_OK && (e = hipEventRecord(sstart, s)) != hipSuccess) rc = hip_fail("hipEventRecord", e);
  // the first launch's first kernel also carries kstart, the last launch's
  // kernels kstop: the launches timed by their own start and end
  // timestamps, without the event packets around them
  {
    LaunchEvents &ev = launch_events();
    ev.start = kstart;
    for (int i = 0; i < iterations && rc == I8CONV_OK; ++i) {
      if (i == iterations - 1) ev.stop = kstop;
      rc = launch(s);
    }
    ev = LaunchEvents{};
  }
  if (rc == I8CONV_OK && (e = hipEventRecord(sstop, s)) != hipSuccess) rc = hip_fail("hipEventRecord", e);
  if (rc == I8CONV_OK && (e = hipStreamSynchronize(s)) != hipSuccess) rc = hip_fail("hipStreamSynchronize", e);
  float ms = 0.f, sms = 0.f, kms = 0.f;
  if (rc == I8CONV_OK && (e = hipEventElapsedTime(&ms, start, stop)) != hipSuccess)
    rc = hip_fail("hipEventElapsedTime", e);
  if (rc == I8CONV_OK && (e = hipEventElapsedTime(&sms, sstart, sstop)) != hipSuccess)
    rc = hip_fail("hipEventElapsedTime", e);
  if (rc == I8CONV_OK && (e = hipEventElapsedTime(&kms, kstart, kstop)) != hipSuccess)
    rc = hip_fail("hipEventElapsedTime(kernel events)", e);
  std::vector<unsigned long long> host(size_t(2 + 2 * stamp_cap), 0ull);
  if (rc == I8CONV_OK &&
      (e = hipMemcpy(host.data(), stamps, stamp_bytes, hipMemcpyDeviceToHost)) != hipSuccess)
    rc = hip_fail("hipMemcpy(stamps)", e);
  if (rc == I8CONV_OK) {
    const int last = replays - 1;
    const unsigned long long t0s = host[2], t1s = host[3 + 2 * last];
    if (host[0] != static_cast<unsigned long long>(replays) || t1s <= t0s) {
      set_error("measure_graph: clock stamps out of order");
      rc = I8CONV_HIP_ERROR;
    } else {
      timing->mean_ms = ms / float(iterations);
      timing->launches_per_graph = per_graph;
      timing->full_replays = full_replays;
      timing->remainder_launches = remainder;
      timing->warmup_launches = warm_launches;
      timing->warmup_ms = float(warm_ms);
      timing->stamped_ms = float(double(t1s - t0s) / (double(rate_khz) * double(iterations)));
      timing->stream_ms = sms / float(iterations);
      timing->kernel_ms = kms / float(iterations);
    }
  }
  // teardown: drain the stream first; a failure here cannot change the result
  (void)hipStreamSynchronize(s);
  if (stamps) (void)hipFree(stamps);
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  if (sstart) (void)hipEventDestroy(sstart);
  if (kstart) (void)hipEventDestroy(kstart);
  if (kstop) (void)hipEventDestroy(kstop);
  if (sstop) (void)hipEventDestroy(sstop);
  for (int i = 0; i < 4; ++i) {
    if (execs[i]) (void)hipGraphExecDestroy(execs[i]);
    if (graphs[i]) (void)hipGraphDestroy(graphs[i]);
  }
  (void)hipStreamDestroy(s);
  return rc;
}
}  // namespace

// Scratch of i8conv_launch_noalloc: a file-scope device array of
// kScratchBytes, one copy per GPU (each GPU the library runs on holds it
// until the process ends).  Host code never passes `scratch` itself to a
// kernel (on the host the name is a stand-in, not a device address): it
// uses the address hipGetSymbolAddress returns on each device, kept per
// device in g_scratch_ptr.
constexpr size_t kScratchBytes = size_t(16) << 20;
constexpr int kScratchDevices = 64;
__device__ __attribute__((aligned(256))) int32_t scratch[kScratchBytes / sizeof(int32_t)];

namespace {
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kScratchDevices] = {};

// The current device's copy of `scratch`, looked up once per device (with
// that device current) and then reused.
int scratch_for_current_device(void **ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail("hipGetDevice", e);
  if (dev < 0 || dev >= kScratchDevices) {
    set_error("launch_noalloc: device index " + std::to_string(dev) + " beyond the " +
              std::to_string(kScratchDevices) + " devices the scratch table covers");
    return I8CONV_BAD_ARGUMENT;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail("hipGetSymbolAddress(scratch)", e);
    if (!p) {
      set_error("hipGetSymbolAddress(scratch) returned a null address");
      return I8CONV_HIP_ERROR;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return I8CONV_OK;
}
}  // namespace

void set_error(const std::string &message) { g_last_error = message; }

namespace {
constexpr int kDefaultSpinLimit = 1 << 20;
std::atomic<int> g_spin_limit{kDefaultSpinLimit};
}  // namespace
int wait_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

LaunchEvents &launch_events() {
  static thread_local LaunchEvents events;
  return events;
}

}  // namespace i8conv

using namespace i8conv;

extern "C" {

int i8conv_derive(const i8conv_shape *shape, i8conv_geometry *geometry) {
  if (!shape) {
    set_error("null shape");
    return I8CONV_BAD_ARGUMENT;
  }
  return derive(*shape, geometry);
}

int i8conv_kernel_count(void) { return I8CONV_KERNEL_COUNT; }

const char *i8conv_kernel_name(int id) {
  return (id >= 0 && id < I8CONV_KERNEL_COUNT) ? kNames[id] : nullptr;
}

int i8conv_kernel_id(const char *name) {
  if (!name) return -1;
  for (int i = 0; i < I8CONV_KERNEL_COUNT; ++i)
    if (std::string(name) == kNames[i]) return i;
  return -1;
}

int i8conv_eligible(int id, const i8conv_shape *shape) {
  if (!shape) return 0;
  i8conv_geometry g;
  if (derive(*shape, &g) != I8CONV_OK) return 0;
  PatchPlan pp;
  switch (id) {
    case I8CONV_KERNEL_GENERIC: return 1;
    case I8CONV_KERNEL_STRIP: return plan_strip(*shape, g, &pp) ? 1 : 0;
    case I8CONV_KERNEL_HALO: return plan_halo(*shape, g, &pp) ? 1 : 0;
    case I8CONV_KERNEL_SPLITK: return plan_generic(*shape, g).stages >= 2 ? 1 : 0;
    default: return 0;
  }
}

size_t i8conv_workspace_bytes(int id, const i8conv_shape *shape) {
  if (id != I8CONV_KERNEL_SPLITK || !i8conv_eligible(id, shape)) return 0;
  i8conv_geometry g;
  derive(*shape, &g);
  return splitk_workspace_bytes(g, plan_splitk(*shape, g));
}

int i8conv_describe(int id, const i8conv_shape *shape, char *buf, size_t len) {
  if (!shape || !buf || len == 0) return I8CONV_BAD_ARGUMENT;
  buf[0] = '\0';
  if (id < 0 || id >= I8CONV_KERNEL_COUNT) return I8CONV_UNKNOWN_KERNEL;
  i8conv_geometry g;
  const int rc = derive(*shape, &g);
  if (rc != I8CONV_OK) return rc;
  if (!i8conv_eligible(id, shape)) return I8CONV_INELIGIBLE;
  std::string d;
  auto tiles = [](int64_t a, int64_t b) { return std::to_string((a + b - 1) / b); };
  if (id == I8CONV_KERNEL_GENERIC || id == I8CONV_KERNEL_SPLITK) {
    const GemmPlan p = id == I8CONV_KERNEL_GENERIC ? plan_generic(*shape, g) : plan_splitk(*shape, g);
    if (p.deep)
      d = std::string(kNames[id]) + " deep-channel: all " + std::to_string(g.gemm_m) +
          "px x 32oc per workgroup, grid " + std::to_string(p.deep_plan.tiles_n) + "x" +
          std::to_string(p.splits) + " splits of 128 channels, " +
          std::to_string(p.deep_plan.lds / 1024) + " KB LDS, ordered reduce";
    else
    d = std::string(kNames[id]) +
        (p.pw ? " pointwise streaming: filter in registers, 16px fragments x " +
                    std::to_string(g.gemm_n) + "oc" +
                    (pointwise_slices(shape->c, int(g.gemm_n)) > 1
                         ? " in " + std::to_string(pointwise_slices(shape->c, int(g.gemm_n))) +
                               " slices"
                         : std::string()) +
                    ", " + std::to_string(p.pw_waves) +
                    " waves; unaligned pointers:"
              : "") +
        (p.dma ? " pipelined" : " register-staged") + " tile " +
        std::to_string(p.bm) + "px x " + std::to_string(p.bn) + "oc" +
        (p.m_step > 0 && p.m_step < p.bm ? " (" + std::to_string(p.m_step) + "px stored)" : "") +
        ", grid " + tiles(g.gemm_m, p.m_step > 0 ? p.m_step : p.bm) + "x" +
        tiles(g.gemm_n, p.bn) + (p.splits > 1 ? "x" + std::to_string(p.splits) + " splits" : "") +
        ", " + std::to_string(p.stages) + " k-stages" +
        (p.dma && gemm_dma_copy_waves(p) > 0 ? ", " + std::to_string(gemm_dma_copy_waves(p)) + " copy waves" : "");
  } else {
    PatchPlan p;
    if (id == I8CONV_KERNEL_STRIP) plan_strip(*shape, g, &p);
    else plan_halo(*shape, g, &p);
    if (p.row) {
      const size_t row_bytes =
          size_t(halo_row_layout(shape->w + 2 * shape->pad_w, shape->c, kRowPadUnits).row_bytes);
      const std::string lds =
          p.streamed ? std::to_string(rowpass_lds_bytes(shape->w + 2 * shape->pad_w, p.rows - 2) / 1024) +
                        " KB"
                  : std::to_string((kHaloBiasLds + size_t(p.rows) * row_bytes) / 1024) + "+" +
                        std::to_string(p.ring * halo_ring_slot_bytes(p.bn / 64) / 1024) + " KB";
      d = std::string(kNames[id]) + (p.streamed ? " row-streaming with copy waves: " : " row-streaming: ") +
          std::to_string(p.ranges) + " row blocks/image of <=" + std::to_string(p.rows - 2) +
          " rows x " + std::to_string(p.bn) + "oc, " + std::to_string(p.frags_m) +
          " frags/row, LDS " + lds + ", grid " +
          std::to_string(int64_t(shape->n) * p.ranges * p.tiles_n);
    } else if (p.resident) {
      d = std::string(kNames[id]) + " resident rows: " + std::to_string(p.ranges) +
          " pixel ranges of <=" + std::to_string(p.frags_m * 16) + "px x " +
          std::to_string(p.bn) + "oc, LDS " +
          std::to_string((kHaloBiasLds + size_t(p.rows) *
                         size_t(halo_row_layout(shape->w + 2 * shape->pad_w, shape->c, kHaloPadUnits).row_bytes)) /
                         1024) + "+" +
          std::to_string(p.ring * halo_ring_slot_bytes(p.bn / 64) / 1024) + " KB, grid " +
          std::to_string(int64_t(p.ranges) * p.tiles_n);
    } else {
      d = std::string(kNames[id]) + " tile " + std::to_string(p.th) + "x" +
          std::to_string(p.tw) + "px x " + std::to_string(p.bn) + "oc, staged " +
          std::to_string(p.ph) + "x" + std::to_string(p.pw) + "px, grid " +
          std::to_string(int64_t(shape->n) * p.tiles_y * p.tiles_x * p.tiles_n);
    }
  }
  const size_t n = std::min(len - 1, d.size());
  d.copy(buf, n);
  buf[n] = '\0';
  return I8CONV_OK;
}

int i8conv_dispatch(const i8conv_shape *shape) {
  if (!shape) return -1;
  return dispatch(*shape);
}

size_t i8conv_dispatch_workspace_bytes(const i8conv_shape *shape) {
  const int id = i8conv_dispatch(shape);
  return id < 0 ? 0 : i8conv_workspace_bytes(id, shape);
}

int i8conv_launch(int id, const i8conv_shape *shape, const int8_t *input,
                  const int8_t *filter, const int32_t *bias, int32_t *output,
                  void *workspace, size_t workspace_bytes, void *stream) {
  if (id < 0 || id >= I8CONV_KERNEL_COUNT) {
    set_error("unknown kernel id " + std::to_string(id));
    return I8CONV_UNKNOWN_KERNEL;
  }
  if (!shape) {
    set_error("null shape");
    return I8CONV_BAD_ARGUMENT;
  }
  i8conv_geometry g;
  const int rc = derive(*shape, &g);
  if (rc != I8CONV_OK) return rc;
  if (!input || !filter || !bias || !output) {
    set_error("null tensor pointer");
    return I8CONV_BAD_ARGUMENT;
  }
  if (!aligned(input, 16) || !aligned(filter, 16) || !aligned(bias, 4) ||
      !aligned(output, 4)) {
    set_error("input/filter must be 16-byte aligned, bias/output 4-byte aligned");
    return I8CONV_BAD_ARGUMENT;
  }
  const ConvArgs args = make_args(*shape, g, input, filter, bias, output);
  switch (id) {
    case I8CONV_KERNEL_GENERIC:
      return launch_gemm(args, plan_generic(*shape, g), stream);
    case I8CONV_KERNEL_STRIP:
    case I8CONV_KERNEL_HALO: {
      PatchPlan pp;
      const bool ok = id == I8CONV_KERNEL_STRIP ? plan_strip(*shape, g, &pp)
                                                : plan_halo(*shape, g, &pp);
      if (!ok) {
        set_error(std::string(kNames[id]) + " is not eligible for this shape");
        return I8CONV_INELIGIBLE;
      }
      return pp.row ? (pp.streamed ? launch_rowpass(args, pp, stream) : launch_row(args, pp, stream))
             : pp.resident ? launch_halo_resident(args, pp, stream)
                           : launch_patch(args, pp, stream);
    }
    case I8CONV_KERNEL_SPLITK: {
      if (!i8conv_eligible(id, shape)) {
        set_error("splitk needs at least two 128-byte k stages");
        return I8CONV_INELIGIBLE;
      }
      const GemmPlan p = plan_splitk(*shape, g);
      const size_t need = splitk_workspace_bytes(g, p);
      if (!workspace || workspace_bytes < need || !aligned(workspace, 16)) {
        set_error("splitk needs a 16-byte aligned workspace of " +
                  std::to_string(need) + " bytes");
        return I8CONV_WORKSPACE_TOO_SMALL;
      }
      return launch_splitk(args, p, workspace, stream);
    }
  }
  return I8CONV_UNKNOWN_KERNEL;
}

int i8conv_launch_generic(const i8conv_shape *shape, const int8_t *input,
                          const int8_t *filter, const int32_t *bias,
                          int32_t *output, void *stream) {
  return i8conv_launch(I8CONV_KERNEL_GENERIC, shape, input, filter, bias,
                       output, nullptr, 0, stream);
}

int i8conv_launch_spatial_strip(const i8conv_shape *shape, const int8_t *input,
                                const int8_t *filter, const int32_t *bias,
                                int32_t *output, void *stream) {
  return i8conv_launch(I8CONV_KERNEL_STRIP, shape, input, filter, bias, output,
                       nullptr, 0, stream);
}

int i8conv_spatial_strip_eligible(const i8conv_shape *shape) {
  return i8conv_eligible(I8CONV_KERNEL_STRIP, shape);
}

int i8conv_launch_dispatched(const i8conv_shape *shape, const int8_t *input,
                             const int8_t *filter, const int32_t *bias,
                             int32_t *output, void *workspace,
                             size_t workspace_bytes, void *stream) {
  const int id = i8conv_dispatch(shape);
  if (id < 0) {
    if (shape) derive(*shape, nullptr);  // records the reason
    return I8CONV_BAD_SHAPE;
  }
  return i8conv_launch(id, shape, input, filter, bias, output, workspace,
                       workspace_bytes, stream);
}

int i8conv_launch_noalloc(int id, const i8conv_shape *shape, const int8_t *input,
                          const int8_t *filter, const int32_t *bias, int32_t *output,
                          void *stream) {
  // 0 for kernels without a workspace, and for an unknown id, a bad shape
  // or an ineligible one: i8conv_launch then reports those
  const size_t need = i8conv_workspace_bytes(id, shape);
  if (need > kScratchBytes) {
    set_error("launch_noalloc: " + std::string(i8conv_kernel_name(id)) + " needs " +
              std::to_string(need) + " bytes of scratch for this shape; the library's static "
              "scratch holds " + std::to_string(kScratchBytes) +
              " (pass a workspace to i8conv_launch instead)");
    return I8CONV_WORKSPACE_TOO_SMALL;
  }
  void *ws = nullptr;
  if (need > 0) {
    if (const int rc = scratch_for_current_device(&ws); rc != I8CONV_OK) return rc;
  }
  return i8conv_launch(id, shape, input, filter, bias, output, ws, need, stream);
}

// ---- requantized int8 output -------------------------------------------------

namespace {
// Where the dispatched kernel for a shape requantizes: in its own epilogue
// (the row kernel with copy waves; the pointwise streaming form with a
// requantizing instance; split-K's second pass; the pipelined GEMM's
// epilogue), or not at all (the convolution into an int32 workspace, then
// a requantizing pass).
enum RequantRoute { kRqUnfused, kRqRow, kRqPointwise, kRqSplitK, kRqGemm };

RequantRoute requant_route(const i8conv_shape &s, const i8conv_geometry &g) {
  const int id = dispatch(s);
  PatchPlan pp;
  if (id == I8CONV_KERNEL_HALO && plan_halo(s, g, &pp) && pp.row && pp.streamed) return kRqRow;
  if (id == I8CONV_KERNEL_GENERIC && plan_generic(s, g).pw &&
      pointwise_requant_supported(s.c, int(g.gemm_n)))
    return kRqPointwise;
  if (id == I8CONV_KERNEL_SPLITK && g.gemm_n % 4 == 0) return kRqSplitK;
  if (id == I8CONV_KERNEL_GENERIC && g.gemm_n % 4 == 0 && plan_generic(s, g).dma) return kRqGemm;
  return kRqUnfused;
}

// The pointer alignment a fused route's epilogue needs (16-byte vector
// loads of bias, mult and shift; the pointwise form's 16-byte stores).
// Without it the launch goes the unfused way.
bool requant_route_aligned(RequantRoute r, const int32_t *bias, const int32_t *mult,
                           const int32_t *shift, const int8_t *output) {
  switch (r) {
    case kRqRow: return true;  // the row kernel falls back to element stores itself
    case kRqPointwise:
      return aligned(bias, 16) && aligned(mult, 16) && aligned(shift, 16) && aligned(output, 16);
    case kRqSplitK:
      return aligned(bias, 16) && aligned(mult, 16) && aligned(shift, 16) && aligned(output, 4);
    case kRqGemm: return aligned(mult, 16) && aligned(shift, 16) && aligned(output, 4);
    default: return false;
  }
}
size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
}  // namespace

int i8conv_requantize(const int32_t *acc, int64_t pixels, int32_t channels,
                      const int32_t *mult, const int32_t *shift, int32_t zero_point,
                      int8_t *output, void *stream) {
  if (pixels < 0 || channels <= 0) {
    set_error("requantize: pixels must be >= 0 and channels > 0");
    return I8CONV_BAD_ARGUMENT;
  }
  if (pixels > 0 && (!acc || !mult || !shift || !output)) {
    set_error("requantize: null tensor pointer");
    return I8CONV_BAD_ARGUMENT;
  }
  if (!aligned(acc, 4) || !aligned(mult, 4) || !aligned(shift, 4)) {
    set_error("requantize: acc, mult and shift must be 4-byte aligned");
    return I8CONV_BAD_ARGUMENT;
  }
  return launch_requant(acc, pixels, channels, mult, shift, zero_point, output, stream);
}

int i8conv_requant_fused(const i8conv_shape *shape) {
  if (!shape) return 0;
  i8conv_geometry g;
  if (derive(*shape, &g) != I8CONV_OK) return 0;
  return requant_route(*shape, g) != kRqUnfused ? 1 : 0;
}

size_t i8conv_requant_workspace_bytes(const i8conv_shape *shape) {
  if (!shape) return 0;
  i8conv_geometry g;
  if (derive(*shape, &g) != I8CONV_OK) return 0;
  // fused: the dispatched kernel's own workspace (split-K's partial sums;
  // nothing for the others)
  if (requant_route(*shape, g) != kRqUnfused) return i8conv_dispatch_workspace_bytes(shape);
  return align256(size_t(g.output_elements) * 4) + i8conv_dispatch_workspace_bytes(shape);
}

int i8conv_launch_requant(const i8conv_shape *shape, const int8_t *input, const int8_t *filter,
                          const int32_t *bias, const int32_t *mult, const int32_t *shift,
                          int32_t zero_point, int8_t *output, void *workspace,
                          size_t workspace_bytes, void *stream) {
  if (!shape) {
    set_error("null shape");
    return I8CONV_BAD_ARGUMENT;
  }
  i8conv_geometry g;
  const int rc = derive(*shape, &g);
  if (rc != I8CONV_OK) return rc;
  if (!input || !filter || !bias || !mult || !shift || !output) {
    set_error("null tensor pointer");
    return I8CONV_BAD_ARGUMENT;
  }
  if (!aligned(input, 16) || !aligned(filter, 16) || !aligned(bias, 4) || !aligned(mult, 4) ||
      !aligned(shift, 4)) {
    set_error("input/filter must be 16-byte aligned, bias/mult/shift 4-byte aligned");
    return I8CONV_BAD_ARGUMENT;
  }
  const int id = dispatch(*shape);
  const RequantRoute route = requant_route(*shape, g);
  if (route != kRqUnfused && requant_route_aligned(route, bias, mult, shift, output)) {
    ConvArgs args = make_args(*shape, g, input, filter, bias, nullptr);
    const RequantArgs q{mult, shift, zero_point, output};
    switch (route) {
      case kRqRow: {
        // the output is < 2 GiB (the plan checks it)
        PatchPlan pp;
        plan_halo(*shape, g, &pp);
        return launch_rowpass(args, pp, stream, &q);
      }
      case kRqPointwise:
        // the pointwise form's eligibility keeps the output < 2 GiB
        return launch_pointwise(args, &q, stream);
      case kRqSplitK: {
        // split-K's second pass requantizes as it adds the splits: only the
        // partial sums need the workspace
        const size_t need = i8conv_workspace_bytes(I8CONV_KERNEL_SPLITK, shape);
        if (!workspace || workspace_bytes < need || !aligned(workspace, 256)) {
          set_error("requantized split-K launch needs a 256-byte aligned workspace of " +
                    std::to_string(need) + " bytes");
          return I8CONV_WORKSPACE_TOO_SMALL;
        }
        return launch_splitk(args, plan_splitk(*shape, g), workspace, stream, &q);
      }
      default:
        // the pipelined GEMM's epilogue requantizes: no workspace
        args.q_mult = mult;
        args.q_shift = shift;
        args.q_zp = zero_point;
        args.q_y = output;
        return launch_gemm(args, plan_generic(*shape, g), stream);
    }
  }
  const size_t acc_bytes = align256(size_t(g.output_elements) * 4);
  const size_t need = acc_bytes + i8conv_workspace_bytes(id, shape);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256)) {
    set_error("requantized launch needs a 256-byte aligned workspace of " + std::to_string(need) +
              " bytes" +
              (route != kRqUnfused
                   ? std::string(" (or bias, mult, shift and output 16-byte aligned)")
                   : std::string()));
    return I8CONV_WORKSPACE_TOO_SMALL;
  }
  int32_t *acc = static_cast<int32_t *>(workspace);
  void *conv_ws = static_cast<char *>(workspace) + acc_bytes;
  const int r = i8conv_launch(id, shape, input, filter, bias, acc, conv_ws,
                              workspace_bytes - acc_bytes, stream);
  if (r != I8CONV_OK) return r;
  return launch_requant(acc, g.gemm_m, g.gemm_n, mult, shift, zero_point, output, stream);
}

// ---- layout transforms -------------------------------------------------------

namespace {
int check_layout(const void *src, const void *dst, int64_t elements, int esize,
                 std::initializer_list<int> dims) {
  for (int d : dims)
    if (d < 0) {
      set_error("layout: negative dimension");
      return I8CONV_BAD_ARGUMENT;
    }
  if (elements * esize >= (int64_t(1) << 31)) {
    set_error("layout: tensors must be below 2^31 bytes");
    return I8CONV_BAD_ARGUMENT;
  }
  if (elements > 0 && (!src || !dst || src == dst)) {
    set_error("layout: null or aliasing tensor pointers");
    return I8CONV_BAD_ARGUMENT;
  }
  if (!aligned(src, esize) || !aligned(dst, esize)) {
    set_error("layout: tensors must be aligned to their element size");
    return I8CONV_BAD_ARGUMENT;
  }
  return I8CONV_OK;
}
}  // namespace

int i8conv_nchw_to_nhwc(const int8_t *src, int8_t *dst, int n, int c, int h, int w,
                        void *stream) {
  const int rc = check_layout(src, dst, int64_t(n) * c * h * w, 1, {n, c, h, w});
  if (rc != I8CONV_OK) return rc;
  return launch_transpose(src, dst, n, c, h * w, 1, stream);
}

int i8conv_nhwc_to_nchw(const int8_t *src, int8_t *dst, int n, int h, int w, int c,
                        void *stream) {
  const int rc = check_layout(src, dst, int64_t(n) * c * h * w, 1, {n, c, h, w});
  if (rc != I8CONV_OK) return rc;
  return launch_transpose(src, dst, n, h * w, c, 1, stream);
}

int i8conv_nhwk_to_nkhw(const int32_t *src, int32_t *dst, int n, int h, int w, int k,
                        void *stream) {
  const int rc = check_layout(src, dst, int64_t(n) * k * h * w, 4, {n, k, h, w});
  if (rc != I8CONV_OK) return rc;
  return launch_transpose(src, dst, n, h * w, k, 4, stream);
}

namespace {
int pack_common(const int8_t *src, int8_t *dst, int n, int h, int w, int c, int vect,
                bool unpack, void *stream) {
  const int rc = check_layout(src, dst, int64_t(n) * c * h * w, 1, {n, h, w, c});
  if (rc != I8CONV_OK) return rc;
  if (vect <= 0 || vect % 16 != 0 || c % vect != 0 || !aligned(src, 16) || !aligned(dst, 16)) {
    set_error("pack_vect_c needs vect % 16 == 0, c % vect == 0 and 16-byte aligned tensors");
    return I8CONV_BAD_ARGUMENT;
  }
  return launch_pack_vect(src, dst, n, h, w, c, vect, unpack, stream);
}
}  // namespace

int i8conv_pack_vect_c(const int8_t *src, int8_t *dst, int n, int h, int w, int c, int vect,
                       void *stream) {
  return pack_common(src, dst, n, h, w, c, vect, false, stream);
}

int i8conv_unpack_vect_c(const int8_t *src, int8_t *dst, int n, int h, int w, int c, int vect,
                         void *stream) {
  return pack_common(src, dst, n, h, w, c, vect, true, stream);
}

// ---- runtime layer -------------------------------------------------------

int i8conv_device_count(int *count) {
  if (!count) return I8CONV_BAD_ARGUMENT;
  const hipError_t e = hipGetDeviceCount(count);
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipGetDeviceCount", e);
}

int i8conv_set_device(int device) {
  const hipError_t e = hipSetDevice(device);
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipSetDevice", e);
}

int i8conv_device_alloc(void **ptr, size_t bytes) {
  if (!ptr) return I8CONV_BAD_ARGUMENT;
  *ptr = nullptr;
  const hipError_t e = hipMalloc(ptr, bytes ? bytes : 1);
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipMalloc", e);
}

int i8conv_device_free(void *ptr) {
  if (!ptr) return I8CONV_OK;
  const hipError_t e = hipFree(ptr);
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipFree", e);
}

int i8conv_copy_to_device(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return I8CONV_OK;
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipMemcpy H2D", e);
}

int i8conv_copy_to_host(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return I8CONV_OK;
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipMemcpy D2H", e);
}

int i8conv_device_fill(void *ptr, int value, size_t bytes) {
  if (bytes == 0) return I8CONV_OK;
  hipError_t e = hipMemset(ptr, value, bytes);
  if (e != hipSuccess) return hip_fail("hipMemset", e);
  e = hipDeviceSynchronize();
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipDeviceSynchronize", e);
}

int i8conv_synchronize(void) {
  const hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipDeviceSynchronize", e);
}

int i8conv_stream_create(void **stream) {
  if (!stream) return I8CONV_BAD_ARGUMENT;
  hipStream_t s = nullptr;
  const hipError_t e = hipStreamCreate(&s);  // default priority
  *stream = s;
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipStreamCreate", e);
}

int i8conv_stream_destroy(void *stream) {
  if (!stream) return I8CONV_OK;
  const hipError_t e = hipStreamDestroy(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? I8CONV_OK : hip_fail("hipStreamDestroy", e);
}

int i8conv_set_wait_spin_limit(int polls) {
  if (polls < 0) {
    set_error("set_wait_spin_limit needs polls >= 0");
    return I8CONV_BAD_ARGUMENT;
  }
  g_spin_limit.store(polls, std::memory_order_relaxed);
  return I8CONV_OK;
}

int i8conv_wait_spin_limit(void) { return wait_spin_limit(); }

int i8conv_wait_expired(int *expired) {
  if (!expired) {
    set_error("wait_expired needs an output");
    return I8CONV_BAD_ARGUMENT;
  }
  int row = 0, deep = 0;
  int rc = rowpass_wait_expired(&row);
  if (rc == I8CONV_OK) rc = deepk_wait_expired(&deep);
  if (rc != I8CONV_OK) return rc;
  *expired = row | deep;
  return I8CONV_OK;
}

int i8conv_device_info(int *compute_units, int *clock_khz, char *arch_name,
                       size_t name_len) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail("hipGetDevice", e);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return hip_fail("hipGetDeviceProperties", e);
  if (compute_units) *compute_units = prop.multiProcessorCount;
  if (clock_khz) *clock_khz = prop.clockRate;
  if (arch_name && name_len) {
    const std::string n(prop.gcnArchName);
    const size_t len = std::min(name_len - 1, n.size());
    n.copy(arch_name, len);
    arch_name[len] = '\0';
  }
  return I8CONV_OK;
}

int i8conv_measure(int id, const i8conv_shape *shape, const int8_t *input,
                   const int8_t *filter, const int32_t *bias, int32_t *output,
                   void *workspace, size_t workspace_bytes, void *stream,
                   int warmup, int iterations, float *median_ms,
                   float *batched_ms) {
  return measure_loop(
      [&]() {
        return i8conv_launch(id, shape, input, filter, bias, output, workspace,
                             workspace_bytes, stream);
      },
      stream, warmup, iterations, median_ms, batched_ms);
}

int i8conv_measure_graph(int id, const i8conv_shape *shape, const int8_t *input,
                         const int8_t *filter, const int32_t *bias, int32_t *output,
                         void *workspace, size_t workspace_bytes, int warmup,
                         double min_warmup_ms, int iterations, int launches_per_graph,
                         int poison_byte, i8conv_graph_timing *timing) {
  if (warmup < 0 || !(min_warmup_ms >= 0.0) || iterations <= 0 || launches_per_graph <= 0 ||
      poison_byte > 255 || !timing) {
    set_error("measure_graph needs warmup >= 0, min_warmup_ms >= 0, iterations > 0, "
              "launches_per_graph > 0, poison_byte < 256 and a timing record");
    return I8CONV_BAD_ARGUMENT;
  }
  i8conv_geometry g{};
  if (const int rc = i8conv_derive(shape, &g); rc != I8CONV_OK) return rc;
  return measure_graph_loop(
      [&](hipStream_t s) {
        return i8conv_launch(id, shape, input, filter, bias, output, workspace, workspace_bytes,
                             s);
      },
      output, size_t(g.output_elements) * sizeof(int32_t), warmup, min_warmup_ms, iterations,
      launches_per_graph, poison_byte, timing);
}

int i8conv_measure_store_floor(int32_t *output, size_t bytes, int workgroups,
                               int threads_per_workgroup, size_t lds_bytes, int write_through,
                               int warmup, double min_warmup_ms, int iterations,
                               int launches_per_graph, i8conv_graph_timing *timing) {
  if (!output || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(output) & 15) != 0 ||
      bytes >= (size_t(1) << 31) || workgroups <= 0 || threads_per_workgroup <= 0 ||
      threads_per_workgroup > 1024 || threads_per_workgroup % 64 != 0 ||
      lds_bytes > size_t(kLdsBudget) || warmup < 0 || !(min_warmup_ms >= 0.0) ||
      iterations <= 0 || launches_per_graph <= 0 || !timing) {
    set_error("measure_store_floor needs a 16-byte aligned output, bytes a multiple of 16 below "
              "2^31, workgroups > 0, 64..1024 threads in whole waves, lds_bytes within the LDS "
              "budget, warmup >= 0, min_warmup_ms >= 0, iterations and launches_per_graph > 0 "
              "and a timing record");
    return I8CONV_BAD_ARGUMENT;
  }
  // a first launch sets the LDS attribute the shape may need
  return measure_graph_loop(
      [&](hipStream_t s) {
        return launch_store_floor(output, bytes, workgroups, threads_per_workgroup, lds_bytes,
                                  write_through != 0, s);
      },
      output, bytes, warmup, min_warmup_ms, iterations, launches_per_graph, 0x5A, timing);
}

int i8conv_measure_lds_probe(int pattern, int32_t *sink, int workgroups,
                             int threads_per_workgroup, int iterations_per_lane, int warmup,
                             double min_warmup_ms, int iterations, int launches_per_graph,
                             i8conv_graph_timing *timing) {
  if (!sink || (reinterpret_cast<uintptr_t>(sink) & 3) != 0 || pattern < 0 || pattern > 5 ||
      workgroups <= 0 || workgroups > (1 << 20) || threads_per_workgroup <= 0 ||
      threads_per_workgroup > 1024 || threads_per_workgroup % 64 != 0 ||
      iterations_per_lane <= 0 || warmup < 0 || !(min_warmup_ms >= 0.0) || iterations <= 0 ||
      launches_per_graph <= 0 || !timing) {
    set_error("measure_lds_probe needs a 4-byte aligned sink, pattern 0..5, 1..2^20 "
              "workgroups of 64..1024 threads in whole waves, iterations_per_lane > 0, warmup "
              ">= 0, min_warmup_ms >= 0, iterations and launches_per_graph > 0 and a timing "
              "record");
    return I8CONV_BAD_ARGUMENT;
  }
  const size_t sink_bytes = size_t(workgroups) * size_t(threads_per_workgroup) * 4;
  return measure_graph_loop(
      [&](hipStream_t s) {
        return launch_lds_probe(pattern, sink, workgroups, threads_per_workgroup,
                                iterations_per_lane, s);
      },
      sink, sink_bytes, warmup, min_warmup_ms, iterations, launches_per_graph, 0x5A, timing);
}

int i8conv_measure_requant(const i8conv_shape *shape, const int8_t *input, const int8_t *filter,
                           const int32_t *bias, const int32_t *mult, const int32_t *shift,
                           int32_t zero_point, int8_t *output, void *workspace,
                           size_t workspace_bytes, void *stream, int warmup, int iterations,
                           float *median_ms, float *batched_ms) {
  return measure_loop(
      [&]() {
        return i8conv_launch_requant(shape, input, filter, bias, mult, shift, zero_point, output,
                                     workspace, workspace_bytes, stream);
      },
      stream, warmup, iterations, median_ms, batched_ms);
}

const char *i8conv_status_string(int status) {
  switch (status) {
    case I8CONV_OK: return "ok";
    case I8CONV_INELIGIBLE: return "ineligible";
    case I8CONV_BAD_SHAPE: return "bad shape";
    case I8CONV_BAD_ARGUMENT: return "bad argument";
    case I8CONV_WORKSPACE_TOO_SMALL: return "workspace too small";
    case I8CONV_HIP_ERROR: return "hip error";
    case I8CONV_UNKNOWN_KERNEL: return "unknown kernel";
    default: return "unknown status";
  }
}

const char *i8conv_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"
