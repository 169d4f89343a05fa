/*
 * conv_oracle.c - CPU oracle of the INT8 convolution lab.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker / the timed CPU baseline.  The product (libi8conv.so, conv_lab)
 * never links or calls it.
 *
 * A plain restatement of the reference's CPU INT32 oracle and of the pieces
 * of its contract that the oracle needs (pthodima/int8_kernel_lab):
 *   oracle_derive            include/conv_shape.cuh:22-35
 *   oracle_reference_value   src/conv_lab.cu:39-66
 *   oracle_conv              reference_value over every output index
 *   oracle_validate_sampled  src/conv_lab.cu:68-86 (sampling rule)
 *   oracle_strip_eligible_reference  include/spatial_strip.cuh:11-15
 *   oracle_pack_vect_c       src/cudnn_lab.cu:7-18 (pack_x / pack_w: NHWC or
 *                            KRSC -> channel vectors of `vect`, the layout
 *                            of cuDNN's INT8x32 path) and its inverse
 *   oracle_transpose         batched [rows][cols] -> [cols][rows] of 1- or
 *                            4-byte elements (NCHW <-> NHWC, NHWK -> NKHW)
 *   oracle_requantize        the lab's int32 -> int8 requantization (no
 *                            reference code: the reference's vendor path
 *                            writes INT8, README.md:89-90; see below)
 * Accumulation is int32 with two's-complement wrap (done in uint32 so that
 * wrap is defined C), the same as the reference's int32 `sum += x * w` for
 * every input that does not overflow and the same as the MFMA accumulator.
 *
 * Pinning (tests/test_oracle.py): torch.nn.functional.conv2d in float64
 * fixtures (exact: |acc| < 2^53), brute-force sums on tiny shapes, and
 * invariants (zero input, one-hot filter, linearity, padding-only taps).
 */
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#ifndef ORACLE_CFLAGS
#define ORACLE_CFLAGS "unknown"
#endif

/* Compiler and flags this library was built with (reported beside CPU
 * timings of the oracle). */
const char *oracle_build_info(void) {
#if defined(__VERSION__)
  return "cc " __VERSION__ ", " ORACLE_CFLAGS;
#else
  return "cc (unknown version), " ORACLE_CFLAGS;
#endif
}

typedef struct oracle_shape {
  int32_t n, h, w, c, k, r, s;
  int32_t pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w;
} oracle_shape;

typedef struct oracle_geometry {
  int32_t out_h, out_w;
  int64_t gemm_m;
  int32_t gemm_n, gemm_k;
  int64_t input_elements, filter_elements, output_elements;
} oracle_geometry;

/* conv_shape.cuh:22-35: same expressions (C integer division truncates
 * toward zero, as in the reference's constexpr int arithmetic) and the same
 * two static_asserts (c % 16 == 0, nonempty output).  Returns 0 on success,
 * 1 when an assert would fire. */
int oracle_derive(const oracle_shape *s, oracle_geometry *g) {
  const int32_t out_h =
      (s->h + 2 * s->pad_h - s->dilation_h * (s->r - 1) - 1) / s->stride_h + 1;
  const int32_t out_w =
      (s->w + 2 * s->pad_w - s->dilation_w * (s->s - 1) - 1) / s->stride_w + 1;
  if (s->c % 16 != 0) return 1;
  if (!(out_h > 0 && out_w > 0)) return 1;
  g->out_h = out_h;
  g->out_w = out_w;
  g->gemm_m = (int64_t)s->n * out_h * out_w;
  g->gemm_n = s->k;
  g->gemm_k = s->r * s->s * s->c;
  g->input_elements = (int64_t)s->n * s->h * s->w * s->c;
  g->filter_elements = (int64_t)s->k * s->r * s->s * s->c;
  g->output_elements = g->gemm_m * g->gemm_n;
  return 0;
}

/* conv_lab.cu:39-66: decode channel = idx % k, then ox, oy, batch; start at
 * bias[channel]; loop fy -> fx -> c, skipping taps outside the image. */
int32_t oracle_reference_value(const oracle_shape *S, const int8_t *input,
                               const int8_t *filter, const int32_t *bias,
                               int64_t output_index) {
  oracle_geometry g;
  oracle_derive(S, &g);
  const int channel = (int)(output_index % S->k);
  const int64_t m = output_index / S->k;
  const int ox = (int)(m % g.out_w);
  const int oy = (int)((m / g.out_w) % g.out_h);
  const int batch = (int)(m / ((int64_t)g.out_h * g.out_w));
  uint32_t sum = (uint32_t)bias[channel];
  for (int fy = 0; fy < S->r; ++fy) {
    const int iy = oy * S->stride_h + fy * S->dilation_h - S->pad_h;
    if (iy < 0 || iy >= S->h) continue;
    for (int fx = 0; fx < S->s; ++fx) {
      const int ix = ox * S->stride_w + fx * S->dilation_w - S->pad_w;
      if (ix < 0 || ix >= S->w) continue;
      const int8_t *xp = input + (((int64_t)batch * S->h + iy) * S->w + ix) * S->c;
      const int8_t *wp = filter + (((int64_t)channel * S->r + fy) * S->s + fx) * S->c;
      int32_t dot = 0; /* |dot| <= c * 2^14 < 2^31 for c < 2^17 */
      for (int c = 0; c < S->c; ++c) dot += (int32_t)xp[c] * (int32_t)wp[c];
      sum += (uint32_t)dot;
    }
  }
  return (int32_t)sum;
}

typedef struct {
  const oracle_shape *s;
  const int8_t *x;
  const int8_t *w;
  const int32_t *b;
  int32_t *out;
  int64_t begin, end;
} oracle_job;

static void *oracle_worker(void *arg) {
  const oracle_job *j = (const oracle_job *)arg;
  for (int64_t i = j->begin; i < j->end; ++i)
    j->out[i] = oracle_reference_value(j->s, j->x, j->w, j->b, i);
  return NULL;
}

/* Every output element, split statically over `threads` POSIX threads (in
 * contiguous ranges of output indices).  Returns 0, or 1 for a bad shape. */
int oracle_conv(const oracle_shape *s, const int8_t *input, const int8_t *filter,
                const int32_t *bias, int32_t *output, int threads) {
  oracle_geometry g;
  if (oracle_derive(s, &g)) return 1;
  const int64_t total = g.output_elements;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t tid[256];
  int spawned[256];
  oracle_job jobs[256];
  for (int t = 0; t < threads; ++t) {
    jobs[t].s = s;
    jobs[t].x = input;
    jobs[t].w = filter;
    jobs[t].b = bias;
    jobs[t].out = output;
    jobs[t].begin = total * t / threads;
    jobs[t].end = total * (t + 1) / threads;
    spawned[t] = t < threads - 1 &&
                 pthread_create(&tid[t], NULL, oracle_worker, &jobs[t]) == 0;
    if (!spawned[t]) oracle_worker(&jobs[t]); /* last range, or a failed spawn */
  }
  for (int t = 0; t < threads; ++t)
    if (spawned[t]) pthread_join(tid[t], NULL);
  return 0;
}

/* conv_lab.cu:68-86: full comparison when output_elements <= 65536, else
 * 2048 samples at index sample * output_elements / 2048.  Returns the first
 * mismatching index, or -1 when every sampled output matches. */
int64_t oracle_validate_sampled(const oracle_shape *s, const int8_t *input,
                                const int8_t *filter, const int32_t *bias,
                                const int32_t *output) {
  oracle_geometry g;
  if (oracle_derive(s, &g)) return 0;
  const int64_t total = g.output_elements;
  const int64_t samples = total <= 65536 ? total : 2048;
  for (int64_t k = 0; k < samples; ++k) {
    const int64_t idx = samples == total ? k : k * total / samples;
    if (output[idx] != oracle_reference_value(s, input, filter, bias, idx)) return idx;
  }
  return -1;
}

/* spatial_strip.cuh:11-15, the reference's own strip predicate. */
int oracle_strip_eligible_reference(const oracle_shape *s) {
  oracle_geometry g;
  if (oracle_derive(s, &g)) return 0;
  return s->r == 3 && s->s == 3 && s->stride_w == 1 && s->dilation_w == 1 &&
         s->c % 64 == 0 && s->k % 64 == 0 && g.out_w % 128 == 0;
}

/*
 * Requantization of the int32 output to int8, per output channel k:
 *   y = clamp(zero_point + round(acc * mult[k] / 2^shift[k]), -128, 127)
 * with shift[k] clamped to [0, 62], the product exact in int64 (|acc| and
 * |mult| are at most 2^31, so |p| <= 2^62), and round() rounding ties away
 * from zero.  The lab's own definition (the reference has no requantizing
 * code; its cuDNN comparison writes INT8 output, README.md:89-90).  Parity
 * is pinned by an exact rational computation in tests/test_requant.py.
 * acc and out are [pixels][channels] (NHWK).
 */
static int64_t requant_round(int64_t p, int s) {
  if (s == 0) return p;
  const int64_t half = (int64_t)1 << (s - 1);
  return p >= 0 ? (p + half) >> s : -((-p + half) >> s);
}

void oracle_requantize(const int32_t *acc, int64_t pixels, int32_t channels,
                       const int32_t *mult, const int32_t *shift, int32_t zero_point,
                       int8_t *out) {
  for (int64_t m = 0; m < pixels; ++m) {
    for (int32_t k = 0; k < channels; ++k) {
      const int s = shift[k] < 0 ? 0 : (shift[k] > 62 ? 62 : shift[k]);
      const int64_t p = (int64_t)acc[m * channels + k] * (int64_t)mult[k];
      int64_t q = requant_round(p, s) + (int64_t)zero_point;
      if (q < -128) q = -128;
      if (q > 127) q = 127;
      out[m * channels + k] = (int8_t)q;
    }
  }
}

/*
 * src/cudnn_lab.cu:7-18 (pack_x; pack_w is the same map over k, r, s, c):
 *   p[(c % V) + V*(w + W*(h + H*(c / V + (C / V)*n)))] = x[((n*H + h)*W + w)*C + c]
 * with V = vect (32 in the reference).  unpack != 0 applies the inverse.
 */
void oracle_pack_vect_c(const int8_t *src, int8_t *dst, int32_t n_, int32_t h_, int32_t w_,
                        int32_t c_, int32_t vect, int unpack) {
  const int64_t groups = c_ / vect;
  for (int64_t n = 0; n < n_; ++n)
    for (int64_t c = 0; c < c_; ++c)
      for (int64_t h = 0; h < h_; ++h)
        for (int64_t w = 0; w < w_; ++w) {
          const int64_t packed = (c % vect) + vect * (w + w_ * (h + h_ * (c / vect + groups * n)));
          const int64_t plain = ((n * h_ + h) * w_ + w) * c_ + c;
          if (unpack) dst[plain] = src[packed];
          else dst[packed] = src[plain];
        }
}

/* Batched transpose: batch matrices of [rows][cols] elements of `esize`
 * bytes (1 or 4) -> [cols][rows]. */
void oracle_transpose(const void *src, void *dst, int64_t batch, int64_t rows, int64_t cols,
                      int esize) {
  const char *s = (const char *)src;
  char *d = (char *)dst;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t r = 0; r < rows; ++r)
      for (int64_t c = 0; c < cols; ++c)
        for (int e = 0; e < esize; ++e)
          d[((b * cols + c) * rows + r) * esize + e] = s[((b * rows + r) * cols + c) * esize + e];
}
