/*
 * i8conv.h - C ABI of the MI355X (gfx950) INT8 implicit-GEMM convolution lab.
 *
 * Contract (same as the reference's launchers):
 *   input  x    : NHWC int8          n*h*w*c bytes
 *   filter w    : KRSC int8          k*r*s*c bytes
 *   bias   b    : K int32            k values
 *   output y    : NHWK int32         n*out_h*out_w*k values
 *   y[m][j] = b[j] + sum over valid taps (fy, fx) and channels ci of
 *             x[batch][iy][ix][ci] * w[j][fy][fx][ci]      (int32, exact)
 * Every in-range output element is overwritten (beta = 0).  Taps that fall
 * outside the image contribute nothing (zero padding).
 *
 * Conventions of this ABI:
 *   - plain C types only; `stream` is a hipStream_t passed as void* (NULL is
 *     the default stream);
 *   - device pointers come from the caller (or from i8conv_device_alloc); the
 *     launch entry points allocate nothing;
 *   - input and filter base addresses must be 16-byte aligned, output and bias
 *     4-byte aligned (16-byte for the vector epilogue, checked at launch);
 *   - every function returns an i8conv_status (never exits the process);
 *     i8conv_last_error() describes the most recent failure on this thread.
 *
 * Reference interfaces replaced (file:line in pthodima/int8_kernel_lab):
 *   ConvShape<...>                include/conv_shape.cuh:5-36
 *   launch_generic<Shape>         include/generic_implicit_gemm.cuh:155-165
 *   launch_generic_sm80<Shape>    include/generic_implicit_gemm.cuh:229-238
 *   launch_spatial_strip<Shape>   include/spatial_strip.cuh:289-301
 *   kSpatialStripEligible<Shape>  include/spatial_strip.cuh:11-15
 *   DeviceBuffer<T>               src/conv_lab.cu:24-37
 *   measure(launch, warmup, it)   src/conv_lab.cu:88-110
 * The halo-tiled and split-K entries have no reference counterpart (the
 * reference names neither); they follow the same launcher contract.
 */
#ifndef I8CONV_H
#define I8CONV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Runtime shape descriptor: the 13 template parameters of ConvShape
 * (include/conv_shape.cuh:5-21), same names and meaning. */
typedef struct i8conv_shape {
  int32_t n, h, w, c, k, r, s;
  int32_t pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w;
} i8conv_shape;

/* Derived geometry (include/conv_shape.cuh:22-32). */
typedef struct i8conv_geometry {
  int32_t out_h, out_w;
  int64_t gemm_m; /* n * out_h * out_w */
  int32_t gemm_n; /* k */
  int32_t gemm_k; /* r * s * c */
  int64_t input_elements, filter_elements, output_elements;
} i8conv_geometry;

typedef enum i8conv_status {
  I8CONV_OK = 0,
  I8CONV_INELIGIBLE = 1,       /* kernel's predicate rejects the shape */
  I8CONV_BAD_SHAPE = 2,        /* shape violates conv_shape.cuh:34-35 or limits */
  I8CONV_BAD_ARGUMENT = 3,     /* null/misaligned pointer, bad count, ... */
  I8CONV_WORKSPACE_TOO_SMALL = 4,
  I8CONV_HIP_ERROR = 5,        /* a HIP runtime call failed */
  I8CONV_UNKNOWN_KERNEL = 6
} i8conv_status;

/* Kernel ids of the candidate family. */
enum {
  I8CONV_KERNEL_GENERIC = 0, /* staged implicit GEMM, any shape with c%16==0 */
  I8CONV_KERNEL_STRIP = 1,   /* 3x3 horizontal-stride-1 spatial strip */
  I8CONV_KERNEL_HALO = 2,    /* 2-D output tile with LDS-resident input halo */
  I8CONV_KERNEL_SPLITK = 3,  /* split reduction + deterministic second pass */
  I8CONV_KERNEL_COUNT = 4
};

/* ---- shape ------------------------------------------------------------- */

/* Fills *geometry.  I8CONV_BAD_SHAPE when c%16 != 0, the output is empty, a
 * field is out of range (n,h,w,c,k,r,s,stride,dilation >= 1, pad >= 0), or a
 * tensor exceeds 2^31-1 bytes.  Replaces conv_shape.cuh:22-35. */
int i8conv_derive(const i8conv_shape *shape, i8conv_geometry *geometry);

/* ---- kernel registry (host only, no GPU needed) ------------------------ */

int i8conv_kernel_count(void);
/* Name of kernel `id` ("generic", "strip", "halo", "splitk"), NULL if unknown. */
const char *i8conv_kernel_name(int id);
/* Id of a kernel by name, or -1. */
int i8conv_kernel_id(const char *name);
/* 1 if kernel `id` can run `shape`, else 0 (also 0 for a bad shape or id).
 * The strip predicate replaces kSpatialStripEligible (spatial_strip.cuh:11-15),
 * re-derived for the gfx950 tile. */
int i8conv_eligible(int id, const i8conv_shape *shape);
/* Device workspace a launch of `id` on `shape` needs, in bytes (0 for all
 * kernels but split-K).  0 also for an ineligible shape. */
size_t i8conv_workspace_bytes(int id, const i8conv_shape *shape);
/* Writes a one-line description of the tile plan kernel `id` would use for
 * `shape` (variant, tile, grid) into buf (NUL-terminated, at most len
 * bytes).  I8CONV_INELIGIBLE / I8CONV_BAD_SHAPE when there is none.  No
 * reference counterpart: it reports the launch geometry for logs and CSVs. */
int i8conv_describe(int id, const i8conv_shape *shape, char *buf, size_t len);

/* ---- dispatch policy (kept outside the kernels) ------------------------ */

/* Kernel id the policy picks for `shape` (always an eligible one), or -1 for
 * a bad shape.  Implements the "encode the policy outside the kernels" step
 * of the reference's workflow (README.md:92-99). */
int i8conv_dispatch(const i8conv_shape *shape);
/* Workspace the dispatched kernel needs. */
size_t i8conv_dispatch_workspace_bytes(const i8conv_shape *shape);

/* ---- launch (asynchronous on `stream`) --------------------------------- */

/* Launches kernel `id`.  `workspace` may be NULL when workspace_bytes is 0.
 * Returns I8CONV_INELIGIBLE for a shape the predicate rejects (the reference
 * made that a compile error, spatial_strip.cuh:202-203), I8CONV_HIP_ERROR if
 * the launch fails.  Allocates nothing. */
int i8conv_launch(int id, const i8conv_shape *shape, const int8_t *input,
                  const int8_t *filter, const int32_t *bias, int32_t *output,
                  void *workspace, size_t workspace_bytes, void *stream);

/* launch_generic<Shape> (generic_implicit_gemm.cuh:155-165) and its sm80
 * twin (:229-238): one gfx950 kernel replaces both. */
int i8conv_launch_generic(const i8conv_shape *shape, const int8_t *input,
                          const int8_t *filter, const int32_t *bias,
                          int32_t *output, void *stream);
/* launch_spatial_strip<Shape> (spatial_strip.cuh:289-301). */
int i8conv_launch_spatial_strip(const i8conv_shape *shape, const int8_t *input,
                                const int8_t *filter, const int32_t *bias,
                                int32_t *output, void *stream);
/* kSpatialStripEligible<Shape> (spatial_strip.cuh:11-15), re-derived. */
int i8conv_spatial_strip_eligible(const i8conv_shape *shape);
/* Launches whatever i8conv_dispatch picks. */
int i8conv_launch_dispatched(const i8conv_shape *shape, const int8_t *input,
                             const int8_t *filter, const int32_t *bias,
                             int32_t *output, void *workspace,
                             size_t workspace_bytes, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): i8conv_launch with the workspace taken
 * from the library's own static device scratch instead of an argument.
 * The scratch is a file-scope device array of 16 MiB (16777216 bytes), one
 * copy per GPU, held until the process ends; its device address is looked
 * up on a device's first call.  A kernel/shape whose workspace exceeds 16
 * MiB is rejected with I8CONV_WORKSPACE_TOO_SMALL (use i8conv_launch with a
 * caller workspace).  Calls no hipMalloc/hipFree or allocating routine.
 * Every call on a GPU shares that GPU's scratch, which keeps the last
 * call's contents (split-K rewrites every partial sum it reads, so nothing
 * has to start at zero): calls that overlap in time on one GPU (on
 * different streams or host threads) race on it; calls on one stream are
 * ordered and safe. */
int i8conv_launch_noalloc(int id, const i8conv_shape *shape, const int8_t *input,
                          const int8_t *filter, const int32_t *bias,
                          int32_t *output, void *stream);

/* ---- requantized int8 output (the step after the path) ---------------- */

/* No counterpart in the reference: its vendor comparison writes INT8 output
 * (README.md:89-90, cudnn_legacy.cuh:40-41) but it has no requantizing code.
 * The lab's definition, per output channel k:
 *   y = clamp(zero_point + round(acc * mult[k] / 2^shift[k]), -128, 127)
 * with acc the int32 convolution (bias included), shift[k] clamped to
 * [0, 62], the product exact in int64 and ties rounded away from zero.
 * mult and shift are device arrays of K int32; the output is NHWK int8. */

/* Requantizes an int32 [pixels][channels] tensor into int8 (asynchronous). */
int i8conv_requantize(const int32_t *acc, int64_t pixels, int32_t channels,
                      const int32_t *mult, const int32_t *shift,
                      int32_t zero_point, int8_t *output, void *stream);
/* 1 when the dispatched kernel for `shape` requantizes in its own epilogue
 * (no int32 tensor is written), 0 when the convolution goes through an
 * int32 workspace and a requantizing pass.  Fused: the row kernel with
 * copy waves; the generic kernel's pointwise streaming form (1x1 stride-1
 * unpadded layers with output-channel slices of 64 or 128), when bias,
 * mult, shift and output are 16-byte aligned; split-K's second pass (N % 4
 * == 0), when bias, mult and shift are 16-byte aligned; the pipelined GEMM's
 * epilogue (N % 4 == 0), when mult and shift are 16-byte aligned.  With
 * other pointers the launch takes the unfused way, whose workspace is the
 * int32 output plus the kernel's own. */
int i8conv_requant_fused(const i8conv_shape *shape);
/* Workspace i8conv_launch_requant needs: the dispatched kernel's own (split-K's
 * partial sums; nothing for the other kernels), plus the int32 output
 * (256-byte aligned) when the requantization is not fused. */
size_t i8conv_requant_workspace_bytes(const i8conv_shape *shape);
/* The dispatched convolution with int8 output: fused epilogue or
 * convolution into the workspace + requantizing pass.  Allocates nothing. */
int i8conv_launch_requant(const i8conv_shape *shape, const int8_t *input,
                          const int8_t *filter, const int32_t *bias,
                          const int32_t *mult, const int32_t *shift,
                          int32_t zero_point, int8_t *output, void *workspace,
                          size_t workspace_bytes, void *stream);
/* i8conv_measure (below) around i8conv_launch_requant. */
int i8conv_measure_requant(const i8conv_shape *shape, const int8_t *input,
                           const int8_t *filter, const int32_t *bias,
                           const int32_t *mult, const int32_t *shift,
                           int32_t zero_point, int8_t *output, void *workspace,
                           size_t workspace_bytes, void *stream, int warmup,
                           int iterations, float *median_ms, float *batched_ms);

/* ---- layout transforms (the step before and after the path) ------------ */

/* Asynchronous on `stream`; no workspace; tensors below 2^31 bytes.
 * NCHW -> NHWC int8 (activations in NCHW order into the kernels' layout). */
int i8conv_nchw_to_nhwc(const int8_t *src, int8_t *dst, int n, int c, int h,
                        int w, void *stream);
/* NHWC -> NCHW int8. */
int i8conv_nhwc_to_nchw(const int8_t *src, int8_t *dst, int n, int h, int w,
                        int c, void *stream);
/* NHWK -> NKHW int32 (the convolution's output in channel-major order). */
int i8conv_nhwk_to_nkhw(const int32_t *src, int32_t *dst, int n, int h, int w,
                        int k, void *stream);
/* pack_x / pack_w of the reference's cuDNN comparison (src/cudnn_lab.cu:7-18)
 * on the GPU: NHWC (or KRSC: n = k, h = r, w = s) -> N, C/vect, H, W, vect,
 * p[(c % V) + V*(w + W*(h + H*(c/V + C/V*n)))] = x[((n*H + h)*W + w)*C + c];
 * vect % 16 == 0 and c % vect == 0 (the reference uses vect = 32). */
int i8conv_pack_vect_c(const int8_t *src, int8_t *dst, int n, int h, int w,
                       int c, int vect, void *stream);
/* The inverse of i8conv_pack_vect_c. */
int i8conv_unpack_vect_c(const int8_t *src, int8_t *dst, int n, int h, int w,
                         int c, int vect, void *stream);

/* ---- thin HIP runtime layer used by the host driver -------------------- */

/* DeviceBuffer (conv_lab.cu:24-37) as C calls. */
int i8conv_device_count(int *count);
int i8conv_set_device(int device);
int i8conv_device_alloc(void **ptr, size_t bytes);
int i8conv_device_free(void *ptr);
int i8conv_copy_to_device(void *dst, const void *src, size_t bytes);
int i8conv_copy_to_host(void *dst, const void *src, size_t bytes);
/* Fills `bytes` of device memory with the byte `value` (poisoning before a
 * correctness run). */
int i8conv_device_fill(void *ptr, int value, size_t bytes);
int i8conv_synchronize(void);
int i8conv_stream_create(void **stream);
int i8conv_stream_destroy(void *stream);

/* No counterpart in the reference.  The row kernel with copy waves (the
 * halo kernel's form for 128-channel 3x3 layers) makes its compute waves
 * wait for copy waves through LDS counters; each wait is bounded (about
 * 2^20 polls, tens of ms) so that every wave ends, and a wave whose wait
 * runs out sets a device word.  This call synchronizes the current device,
 * reads that word into *expired (1: some launch since the last call gave up
 * waiting, and its output must be treated as wrong; 0: none did) and
 * clears it. */
int i8conv_wait_expired(int *expired);

/* No counterpart in the reference: a test hook for the give-up path above.
 * Sets the polls each bounded wait makes before it gives up, for launches
 * enqueued from then on (the value is read at launch, so a captured graph
 * keeps the limit of its capture).  Default 2^20 (some tens of ms); 0 makes
 * every wait give up at once: every wave still runs to its end, the output
 * is then wrong and i8conv_wait_expired reports it.  polls < 0 is rejected.
 * Process-wide, not per thread. */
int i8conv_set_wait_spin_limit(int polls);
/* The current limit (i8conv_set_wait_spin_limit). */
int i8conv_wait_spin_limit(void);

/* Device facts for roofline reporting: compute units, peak engine clock in
 * kHz, gcnArchName (at most `name_len` bytes incl. NUL). */
int i8conv_device_info(int *compute_units, int *clock_khz, char *arch_name,
                       size_t name_len);

/* Result of i8conv_measure_graph. */
typedef struct i8conv_graph_timing {
  float mean_ms;          /* graph region: elapsed / iterations */
  int launches_per_graph; /* launches in the main graph */
  int full_replays;       /* replays of the main graph in the timed region */
  int remainder_launches; /* launches of the remainder graph (0: none) */
  int warmup_launches;    /* launches replayed before the timed region */
  float warmup_ms;        /* host wall time of the warmup */
  /* (end stamp of the last timed graph - start stamp of the first) /
   * iterations, from the device's constant-rate clock read by a one-wave
   * kernel captured at the start and at the end of each graph: the timed
   * launches plus one dispatch, without the gap before the first replay
   * starts running */
  float stamped_ms;
  /* the same K launches enqueued one by one on the stream (no graph),
   * between one pair of events, after the poison fill that follows the
   * graph region: elapsed / iterations */
  float stream_ms;
  /* the same K stream launches timed by events the launches themselves
   * carry (hipExtLaunchKernel: the first kernel's start to the last
   * kernel's end), without the two event packets around them:
   * elapsed / iterations */
  float kernel_ms;
} i8conv_graph_timing;

/* No counterpart in the reference, which times launches one by one
 * (conv_lab.cu:88-110).  Back-to-back launches replayed from HIP graphs, on
 * a stream of its own (default priority):
 *   1. one launch outside any graph, synchronized;
 *   2. graphs of L = min(launches_per_graph, iterations) i8conv_launch
 *      calls are captured (kernel nodes only), plus a remainder graph of
 *      iterations % L launches when that is nonzero: a plain pair and a
 *      stamped pair, whose graphs begin and end with a one-wave kernel
 *      that reads the device's constant-rate clock;
 *   3. warmup: main-graph replays, in batches the host waits for, until at
 *      least `warmup` launches have run and at least min_warmup_ms of host
 *      wall time has passed;
 *   4. a tail of about 5 ms of main-graph replays that the host does not
 *      wait for; steps 5-7 are enqueued behind it, so the GPU goes from
 *      warm launches into the timed ones without idling;
 *   5. stamped region: the K launches from the stamped graphs; stamped_ms
 *      runs from the first graph's start stamp to the last one's end stamp
 *      (the launches plus one stamp dispatch, without the gap before each
 *      graph replay begins to run);
 *   6. event-timed graph region: iterations / L main-graph replays plus the
 *      remainder graph, exactly `iterations` launches, between one pair of
 *      events recorded on the stream (mean_ms).  Each graph replay begins
 *      with a gap of some microseconds after the previous one, which the
 *      region holds once per replay: a larger L spreads it over more
 *      launches;
 *   7. when poison_byte >= 0, the output is filled with that byte (a fill on
 *      the stream, outside any graph); then the stream region: the K
 *      launches enqueued one by one on the stream (no graph) between one
 *      pair of events (stream_ms).  The first of them also carries a start
 *      event and the last a stop event of its own (hipExtLaunchKernel),
 *      whose interval, from the first kernel's start to the last one's end,
 *      gives kernel_ms.  They are enqueued while the tail still runs, so the
 *      GPU does not wait for the host, and the output then holds only what
 *      they wrote.
 * Fills *timing.  Synchronous. */
int i8conv_measure_graph(int id, const i8conv_shape *shape, const int8_t *input,
                         const int8_t *filter, const int32_t *bias, int32_t *output,
                         void *workspace, size_t workspace_bytes, int warmup,
                         double min_warmup_ms, int iterations,
                         int launches_per_graph, int poison_byte,
                         i8conv_graph_timing *timing);

/* No counterpart in the reference: the store floor of a launch shape.  A
 * kernel that only writes `bytes` of `output` (16-byte aligned, a multiple
 * of 16 below 2^31) with 16-byte buffer stores, write-through when
 * write_through != 0 (the row kernels' output policy) else ordinary, in
 * `workgroups` x threads_per_workgroup (whole waves, at most 1024) with
 * lds_bytes of dynamic LDS allocated and unused; timed as
 * i8conv_measure_graph times a convolution (poison byte 0x5A).  16-byte
 * unit u of the output ends up holding the int32 value u four times.
 * bytes == 0 times an empty kernel of the launch shape (the dispatch
 * floor).  Synchronous. */
int i8conv_measure_store_floor(int32_t *output, size_t bytes, int workgroups,
                               int threads_per_workgroup, size_t lds_bytes,
                               int write_through, int warmup,
                               double min_warmup_ms, int iterations,
                               int launches_per_graph,
                               i8conv_graph_timing *timing);

/* No counterpart in the reference: the control for the LDS bank-conflict
 * counters.  A kernel whose lanes only read LDS with ds_read_b128, 16 bytes
 * at a fixed per-lane pattern: 0 linear (lane l at 16*l: conflict-free), 1
 * a fragment read of the swz128 layout (the row kernels' filter ring), 2 a
 * 128-byte lane stride (two 4-bank groups per 16 lanes), 3 a 256-byte
 * stride (one group: the most conflicting read there is), 4 a fragment read
 * of the swz128x layout (the pipelined GEMM's) and 5 an 80-byte pixel pitch
 * (both 2-way on gfx950 although each 16 lanes cover all sixteen 4-bank
 * groups); `iterations` reads per lane over 64 KB of
 * LDS, in `workgroups` x threads_per_workgroup (whole waves, at most 1024).
 * Timed as i8conv_measure_graph times a convolution, with `sink`
 * (workgroups * threads_per_workgroup int32, poison byte 0x5A) as its
 * output: thread t stores the four-way XOR of the XOR of its reads, a
 * value the caller can recompute.  Synchronous. */
int i8conv_measure_lds_probe(int pattern, int32_t *sink, int workgroups,
                             int threads_per_workgroup, int iterations_per_lane,
                             int warmup, double min_warmup_ms, int iterations,
                             int launches_per_graph,
                             i8conv_graph_timing *timing);

/* measure() (conv_lab.cu:88-110): `warmup` launches, synchronize; when
 * batched_ms is non-NULL, `iterations` back-to-back launches between one
 * event pair on `stream` (mean per launch, right after the warmup); then
 * `iterations` launches each bracketed by its own event pair and
 * synchronized; *median_ms is their median (it includes per-launch event
 * overhead). */
int i8conv_measure(int id, const i8conv_shape *shape, const int8_t *input,
                   const int8_t *filter, const int32_t *bias, int32_t *output,
                   void *workspace, size_t workspace_bytes, void *stream,
                   int warmup, int iterations, float *median_ms,
                   float *batched_ms);

/* ---- errors and synthetic data ----------------------------------------- */

const char *i8conv_status_string(int status);
/* Text of the most recent failure on the calling thread ("" if none). */
const char *i8conv_last_error(void);

/* Seeded synthetic data (host memory).  SplitMix64 (Steele, Lea, Flood,
 * "Fast splittable pseudorandom number generators", OOPSLA 2014) advanced
 * from `*state`; value i = lo + (next() mod (hi - lo + 1)).  `*state` is
 * updated so that successive calls continue one stream (input, then filter,
 * then bias). */
void i8conv_fill_int8(int8_t *dst, size_t count, int lo, int hi,
                      uint64_t *state);
void i8conv_fill_int32(int32_t *dst, size_t count, int32_t lo, int32_t hi,
                       uint64_t *state);

#ifdef __cplusplus
}
#endif

#endif /* I8CONV_H */
