/*
 * oracle.c — TEST INFRASTRUCTURE, NOT PART OF THE PRODUCT: the CPU restatement of pyodide-llm's int8/int6 forward
 * path in the reference's float32 order. Loaded only by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg (as the parity reference / the timed CPU baseline). Built with -ffp-contract=off: no fused multiply-adds,
 * every float32 operation rounded on its own as WebAssembly's f32 arithmetic is.
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *   or_quantize, or_quantize6, or_pack6/unpack6 : golden vectors written by the reference's own quantize(),
 *       quantize6(), pack6() (tests/golden/make_golden.py) and the layout closed form of tests/test_int6.py:16-26;
 *   or_quantize_x  : bias 0 equal to quantize() bytes (tests/smoke.mjs:285-289), extremes, the closed form;
 *   or_matmul_*    : the LCG known-answer tests of tests/forward-check.mjs:119-276 (lane sums, closed forms,
 *       q6r == q8r on widened values, power-of-two scales equal to exact float64 sums);
 *   or_attention   : tests/attention-check.mjs (far-leading scores, float64 expectation within 1e-3), and float64
 *       softmax-attention within a tolerance on random inputs;
 *   or_fexp/vexp   : within 2 ulp of exp() over the range, and exact at integer powers of two;
 *   or_to_f16/from_f16 : NumPy astype(float16) / astype(float32) over all finite halves;
 *   or_rmsnorm, or_rope, or_swiglu : float64 expectations within a few ulp, and the tables against the reference's
 *       rope_tables() golden vectors;
 *   or_places      : golden plans written by the reference's external_tensors();
 *   or_model_run   : blocks equal one-at-a-time to the bit (tests/forward-check.mjs:438-452), and the reference's
 *       NumPy forward on a tiny model (golden logits) within the int8 line of tests/test_quantize.py:81-90;
 *   or_penalize, or_sample : the reference's sampler tests restated (tests/test_sample.py: the drawn set is the
 *       float64 top-p set, a peaked distribution, a low temperature, the penalty's values and window, logits that
 *       are not finite), and the draws of a float64 restatement of NumPy's Llama.sample
 *       (public/llama2_numpy.py:1529-1563) away from its boundaries (tests/smoke.mjs:176-272 holds the kernel to it).
 */
#include "oracle.h"

#include <math.h>
#include <stddef.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define GS 32

/* ------------------------------------------------------------------------------------------------ synthetic data */

/* splitmix64's finalizer (Steele, Lea, Flood 2014): a bijective 64-bit mixer */
uint64_t or_mix64(uint64_t z) {
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}

/* sigma / the standard deviation of a sum of four uniform 16-bit integers, sqrt(4 * (65536^2 - 1) / 12), as one
 * float32: the factor every synthetic value is multiplied by (host and device take the same float) */
float or_synth_factor(double sigma) { return (float)(sigma / sqrt(4.0 * (65536.0 * 65536.0 - 1.0) / 12.0)); }

/* value `index` of stream `stream`: the four 16-bit quarters of a hash summed and centred (an Irwin-Hall(4) variate:
 * mean 0, variance 1 after the factor), times factor. Integer arithmetic and one float32 multiply: bit-identical on
 * every machine. */
float or_synth_value(uint64_t seed, int32_t stream, uint64_t index, float factor) {
  uint64_t key = or_mix64(seed * 0x9E3779B97F4A7C15ull ^ ((uint64_t)(uint32_t)stream * 0xD1B54A32D192ED03ull));
  uint64_t r = or_mix64(key + index * 0x9E3779B97F4A7C15ull);
  int32_t s = (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) + (int32_t)(r >> 48);
  return (float)(s - 131070) * factor;
}

void or_synth_fill(float *out, uint64_t n, uint64_t seed, int32_t stream, uint64_t first, double sigma) {
  float factor = or_synth_factor(sigma);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; i++) out[i] = or_synth_value(seed, stream, first + (uint64_t)i, factor);
}

/* ------------------------------------------------------------------------------------------------ weight formats */

/* public/llama2_convert.py:25-29 group_size */
int32_t or_group_size(int32_t row_length) {
  int32_t size = 32;
  while (row_length % size) size /= 2;
  return size;
}

/* public/llama2_convert.py:125-130 quantize(): scale = f32(max|x| / 127), inverse = f32(1 / scale) (0 where the
 * scale is 0), q = rint(x * inverse) as int8. count values, groups of `group`. */
void or_quantize(int8_t *q, float *scales, const float *x, int64_t count, int32_t group) {
  int64_t groups = count / group;
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < groups; g++) {
    const float *v = x + g * group;
    float amax = 0.0f;
    for (int32_t i = 0; i < group; i++) {
      float a = fabsf(v[i]);
      if (a > amax) amax = a;
    }
    float scale = amax / 127.0f;
    float inverse = scale > 0 ? 1.0f / scale : 0.0f;
    scales[g] = scale;
    for (int32_t i = 0; i < group; i++) q[g * group + i] = (int8_t)rintf(v[i] * inverse);
  }
}

/* public/llama2_numpy.py:695-702 quantize6(): scale = f32(max|x| / 31), v = clip(rint(x / scale), -32, 31), stored
 * as the int8 4v and the scale f32(scale / 4). */
void or_quantize6(int8_t *q, float *scales, const float *x, int64_t groups) {
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < groups; g++) {
    const float *v = x + g * GS;
    float amax = 0.0f;
    for (int32_t i = 0; i < GS; i++) {
      float a = fabsf(v[i]);
      if (a > amax) amax = a;
    }
    float scale = amax / 31.0f;
    float inverse = scale > 0 ? 1.0f / scale : 0.0f;
    for (int32_t i = 0; i < GS; i++) {
      float r = rintf(v[i] * inverse);
      if (r < -32.0f) r = -32.0f;
      if (r > 31.0f) r = 31.0f;
      q[g * GS + i] = (int8_t)((int32_t)r * 4);
    }
    scales[g] = scale / 4.0f;
  }
}

/* public/llama2_numpy.py:678-684 pack6(): the low four of the six bits of values j and j+16 in byte j (0..15), the
 * top two bits of values k, k+8, k+16, k+24 in byte 16+k at bits 0, 2, 4, 6 */
void or_pack6(uint8_t *out, const int8_t *q, int64_t groups) {
  for (int64_t g = 0; g < groups; g++) {
    uint8_t b[GS];
    for (int32_t j = 0; j < GS; j++) b[j] = (uint8_t)(((uint8_t)q[g * GS + j] >> 2) & 63);
    uint8_t *o = out + g * 24;
    for (int32_t j = 0; j < 16; j++) o[j] = (uint8_t)((b[j] & 15) | ((b[j + 16] & 15) << 4));
    for (int32_t k = 0; k < 8; k++)
      o[16 + k] = (uint8_t)((b[k] >> 4) | ((b[k + 8] >> 4) << 2) | ((b[k + 16] >> 4) << 4) | ((b[k + 24] >> 4) << 6));
  }
}

/* kernels/six.ts:16-31 and public/forward.js:680-683 (weightAt): value j of a group of 24 bytes */
void or_unpack6(int8_t *out, const uint8_t *packed, int64_t groups) {
  for (int64_t g = 0; g < groups; g++) {
    const uint8_t *b = packed + g * 24;
    for (int32_t j = 0; j < GS; j++) {
      int32_t low = j < 16 ? (b[j] & 15) : (b[j - 16] >> 4);
      int32_t top = (b[16 + (j % 8)] >> (2 * (j / 8))) & 3;
      out[g * GS + j] = (int8_t)(uint8_t)((low | (top << 4)) << 2);
    }
  }
}

/* ------------------------------------------------------------------------------------------------ float helpers */

/* i32.trunc_sat_f32_s (WebAssembly): NaN to 0, out of range to the nearest end */
static inline int32_t trunc_sat(float f) {
  if (f != f) return 0;
  if (f >= 2147483648.0f) return 2147483647;
  if (f < -2147483648.0f) return (-2147483647 - 1);
  return (int32_t)f;
}
static inline int32_t sat16(int32_t v) { return v > 32767 ? 32767 : v < -32768 ? -32768 : v; }
static inline int32_t sat8(int32_t v) { return v > 127 ? 127 : v < -128 ? -128 : v; }
/* f32x4.max: NaN if either is NaN, else the larger (+0 above -0) */
static inline float wmax(float a, float b) {
  if (a != a || b != b) return a + b;
  if (a == b) return signbit(a) ? b : a;
  return a > b ? a : b;
}
static inline float wmin(float a, float b) {
  if (a != a || b != b) return a + b;
  if (a == b) return signbit(a) ? a : b;
  return a < b ? a : b;
}
static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* kernels/kernel.ts:15-29 fexp: the table-free Cephes expf (S. L. Moshier's Cephes math library) */
float or_fexp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) x = 88.0f;
  float k = rintf(x * 1.44269504088896341f);
  float r = x - k * 0.693359375f - k * -2.12194440e-4f;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  float e = p * (r * r) + r + 1.0f;
  return e * bits_f32((uint32_t)((int32_t)k + 127) << 23);
}

/* kernels/kernel.ts:33-45 vexp: fexp with x clamped to [-87, 88] (below -87 it gives exp(-87), not 0) */
static inline float vexp1(float x) {
  x = wmin(wmax(x, -87.0f), 88.0f);
  float k = rintf(x * 1.44269504088896341f);
  float r = (x - k * 0.693359375f) - k * -2.12194440e-4f;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  float e = (p * (r * r) + r) + 1.0f;
  return e * bits_f32((uint32_t)(trunc_sat(k) + 127) << 23);
}
void or_vexp(float *x, int32_t n) {
  for (int32_t i = 0; i < n; i++) x[i] = vexp1(x[i]);
}

/* ------------------------------------------------------------------------------------------------ quantize_x */

/* kernels/kernel.ts:129-156: per group of 32, amax by lane maxima then scalar compares (groupMax, :71-81),
 * scale = f32(amax / qmax), inv = scale > 0 ? f32(1 / scale) : 0, q = narrow(trunc_sat(nearest(x * inv)) + bias) */
void or_quantize_x(int8_t *xq, float *xs, const float *x, int32_t n, int32_t bias) {
  const float qmax = bias == 0 ? 127.0f : 63.0f;
  for (int32_t g = 0; g < n; g += GS) {
    const float *p = x + g;
    float lane[4];
    for (int32_t l = 0; l < 4; l++) {
      /* the tree of kernels/kernel.ts:73-74 over the eight vectors, lane l */
      float a[8];
      for (int32_t v = 0; v < 8; v++) a[v] = fabsf(p[4 * v + l]);
      lane[l] = wmax(wmax(wmax(a[0], a[1]), wmax(a[2], a[3])), wmax(wmax(a[4], a[5]), wmax(a[6], a[7])));
    }
    float amax = lane[0];
    if (lane[1] > amax) amax = lane[1];
    if (lane[2] > amax) amax = lane[2];
    if (lane[3] > amax) amax = lane[3];
    float scale = amax / qmax;
    xs[g / GS] = scale;
    float inv = scale > 0 ? 1.0f / scale : 0.0f;
    for (int32_t i = 0; i < GS; i++) {
      int32_t t = (int32_t)((uint32_t)trunc_sat(rintf(p[i] * inv)) + (uint32_t)bias); /* i32x4.add wraps */
      xq[g + i] = (int8_t)sat8(sat16(t));
    }
  }
}

/* ------------------------------------------------------------------------------------------------ matmuls */

static inline int32_t dot32(const int8_t *w, const int8_t *x) {
  int32_t s = 0;
  for (int32_t i = 0; i < GS; i++) s += (int32_t)w[i] * (int32_t)x[i];
  return s;
}

/* the activations with the bias of 64 taken out: dot(w, q - 64) is dot(w, q) + int8_sums' correction -64 * sum(w)
 * (kernels/kernel_relaxed.ts:47-55, kernels/kernel.ts:204-212), the same integer */
static void centred(int8_t *xc, const int8_t *xq, int32_t k) {
  for (int32_t i = 0; i < k; i++) xc[i] = (int8_t)(xq[i] - 64);
}

/* the float32 order of kernels/kernel_relaxed.ts:34-67 over a row's exact group sums S_g: lane g % 4 for the groups
 * in fours, the lanes added in order, then the groups past the fours one at a time */
static float relaxed_row(const int32_t *S, const float *ws, const float *xs, int32_t ng) {
  const int32_t ng4 = ng & ~3;
  float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int32_t g = 0;
  for (; g < ng4; g++) {
    float scale = ws[g] * xs[g];
    l[g & 3] = l[g & 3] + (float)S[g] * scale;
  }
  float sum = l[0] + l[1] + l[2] + l[3];
  for (; g < ng; g++) sum = sum + (float)S[g] * (ws[g] * xs[g]);
  return sum;
}

/* kernels/kernel_relaxed.ts:34-67 matmul_q8r: rows r0..r1 of int8 w [rows][k], scales ws [rows][k/32] */
void or_matmul_q8r(float *y, const int8_t *xq, const float *xs, const int8_t *w, const float *ws, int32_t k,
                   int32_t r0, int32_t r1) {
  const int32_t ng = k / GS;
  int8_t *xc = (int8_t *)malloc((size_t)k);
  centred(xc, xq, k);
#pragma omp parallel for schedule(dynamic, 16) if (r1 - r0 >= 256)
  for (int32_t r = r0; r < r1; r++) {
    int32_t S[1024];
    int32_t *s = ng <= 1024 ? S : (int32_t *)malloc(sizeof(int32_t) * (size_t)ng);
    const int8_t *row = w + (int64_t)r * k;
    for (int32_t g = 0; g < ng; g++) s[g] = dot32(row + g * GS, xc + g * GS);
    y[r] = relaxed_row(s, ws + (int64_t)r * ng, xs, ng);
    if (s != S) free(s);
  }
  free(xc);
}

/* the four lanes of kernels/kernel.ts:222-229 dot32: lane k holds products 2k, 2k+1, 2k+8, 2k+9 of each half */
static inline void lanes32(int32_t *lane, const int8_t *w, const int8_t *x) {
  for (int32_t k = 0; k < 4; k++) {
    int32_t s = 0;
    for (int32_t h = 0; h < 32; h += 16) {
      s += (int32_t)w[h + 2 * k] * x[h + 2 * k] + (int32_t)w[h + 2 * k + 1] * x[h + 2 * k + 1] +
           (int32_t)w[h + 2 * k + 8] * x[h + 2 * k + 8] + (int32_t)w[h + 2 * k + 9] * x[h + 2 * k + 9];
    }
    lane[k] = s;
  }
}

/* the float32 order of kernels/kernel.ts:231-258 matmul_q8: every group's four lanes each scaled by the group's
 * scale and added into its own accumulator, the four added in order at the end (hsum, :10-12) */
static float plain_row(const int32_t *L, const float *ws, const float *xs, int32_t ng) {
  float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int32_t g = 0; g < ng; g++) {
    float s = ws[g] * xs[g];
    for (int32_t k = 0; k < 4; k++) f[k] = f[k] + (float)L[4 * g + k] * s;
  }
  return f[0] + f[1] + f[2] + f[3];
}

void or_matmul_q8(float *y, const int8_t *xq, const float *xs, const int8_t *w, const float *ws, int32_t k,
                  int32_t r0, int32_t r1) {
  const int32_t ng = k / GS;
#pragma omp parallel for schedule(dynamic, 16) if (r1 - r0 >= 256)
  for (int32_t r = r0; r < r1; r++) {
    int32_t *L = (int32_t *)malloc(sizeof(int32_t) * 4 * (size_t)ng);
    const int8_t *row = w + (int64_t)r * k;
    for (int32_t g = 0; g < ng; g++) lanes32(L + 4 * g, row + g * GS, xq + g * GS);
    y[r] = plain_row(L, ws + (int64_t)r * ng, xs, ng);
    free(L);
  }
}

/* kernels/kernel_relaxed.ts:195-218 matmul_q6r: matmul_q8r on the widened int6 groups (24 bytes each) */
void or_matmul_q6r(float *y, const int8_t *xq, const float *xs, const uint8_t *w, const float *ws, int32_t k,
                   int32_t r0, int32_t r1) {
  const int32_t ng = k / GS;
  int8_t *xc = (int8_t *)malloc((size_t)k);
  centred(xc, xq, k);
#pragma omp parallel for schedule(dynamic, 16) if (r1 - r0 >= 256)
  for (int32_t r = r0; r < r1; r++) {
    int8_t *wide = (int8_t *)malloc((size_t)k);
    int32_t *s = (int32_t *)malloc(sizeof(int32_t) * (size_t)ng);
    or_unpack6(wide, w + (int64_t)r * ng * 24, ng);
    for (int32_t g = 0; g < ng; g++) s[g] = dot32(wide + g * GS, xc + g * GS);
    y[r] = relaxed_row(s, ws + (int64_t)r * ng, xs, ng);
    free(s);
    free(wide);
  }
  free(xc);
}

/* kernels/kernel.ts:261-278 matmul_q6: matmul_q8 on the widened int6 groups */
void or_matmul_q6(float *y, const int8_t *xq, const float *xs, const uint8_t *w, const float *ws, int32_t k,
                  int32_t r0, int32_t r1) {
  const int32_t ng = k / GS;
#pragma omp parallel for schedule(dynamic, 16) if (r1 - r0 >= 256)
  for (int32_t r = r0; r < r1; r++) {
    int8_t *wide = (int8_t *)malloc((size_t)k);
    int32_t *L = (int32_t *)malloc(sizeof(int32_t) * 4 * (size_t)ng);
    or_unpack6(wide, w + (int64_t)r * ng * 24, ng);
    for (int32_t g = 0; g < ng; g++) lanes32(L + 4 * g, wide + g * GS, xq + g * GS);
    y[r] = plain_row(L, ws + (int64_t)r * ng, xs, ng);
    free(L);
    free(wide);
  }
}

/* the exact integers the matmuls scale: bias 64, one a group, dot(w, q - 64); bias 0, the four lanes of a group */
void or_group_sums(int32_t *s, const int8_t *xq, const void *w, int32_t rows, int32_t k, int32_t bias, int32_t six) {
  const int32_t ng = k / GS;
  int8_t *xc = (int8_t *)malloc((size_t)k);
  if (bias) centred(xc, xq, k);
  else memcpy(xc, xq, (size_t)k);
  int8_t *wide = (int8_t *)malloc((size_t)k);
  for (int32_t r = 0; r < rows; r++) {
    const int8_t *row;
    if (six) {
      or_unpack6(wide, (const uint8_t *)w + (int64_t)r * ng * 24, ng);
      row = wide;
    } else {
      row = (const int8_t *)w + (int64_t)r * k;
    }
    for (int32_t g = 0; g < ng; g++) {
      if (bias) s[(int64_t)r * ng + g] = dot32(row + g * GS, xc + g * GS);
      else lanes32(s + ((int64_t)r * ng + g) * 4, row + g * GS, xc + g * GS);
    }
  }
  free(wide);
  free(xc);
}

/* m tokens ([m][k] activations, [m][k/32] scales) against every row: y [m][rows]; matmul_q8r_tile
 * (kernels/kernel_relaxed.ts:164-183) is matmul_q8r per token to the bit, so this is the one-token kernel per token */
void or_matmul(float *y, const int8_t *xq, const float *xs, const void *w, const float *ws, int32_t m, int32_t rows,
               int32_t k, int32_t bias, int32_t six) {
  for (int32_t t = 0; t < m; t++) {
    const int8_t *xt = xq + (int64_t)t * k;
    const float *st = xs + (int64_t)t * (k / GS);
    float *yt = y + (int64_t)t * rows;
    if (six) {
      if (bias) or_matmul_q6r(yt, xt, st, (const uint8_t *)w, ws, k, 0, rows);
      else or_matmul_q6(yt, xt, st, (const uint8_t *)w, ws, k, 0, rows);
    } else {
      if (bias) or_matmul_q8r(yt, xt, st, (const int8_t *)w, ws, k, 0, rows);
      else or_matmul_q8(yt, xt, st, (const int8_t *)w, ws, k, 0, rows);
    }
  }
}

/* ------------------------------------------------------------------------------------------------ elementwise */

/* kernels/kernel.ts:330-342 rmsnorm: squares in four lanes over n & ~3, hsum ((l0+l1)+l2)+l3, the tail in order,
 * s = 1 / sqrt(ss / n + eps), out = w * (s * x) */
void or_rmsnorm(float *out, const float *x, const float *w, int32_t n, float eps) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int32_t n4 = n & ~3;
  int32_t j = 0;
  for (; j < n4; j += 4)
    for (int32_t l = 0; l < 4; l++) acc[l] = acc[l] + x[j + l] * x[j + l];
  float ss = acc[0] + acc[1] + acc[2] + acc[3];
  for (; j < n; j++) ss = ss + x[j] * x[j];
  const float s = 1.0f / sqrtf(ss / (float)n + eps);
  for (j = 0; j < n; j++) out[j] = w[j] * (s * x[j]);
}

/* kernels/kernel.ts:344-357 rope: pairs (v[2i], v[2i+1]) of every head turned by cos/sin of the position's row */
void or_rope(float *v, const float *fcr, const float *fci, int32_t nh, int32_t hs, int32_t rot) {
  const int32_t turned = rot > 0 && rot < hs ? rot : hs;
  for (int32_t h = 0; h < nh; h++) {
    float *base = v + h * hs;
    for (int32_t i = 0; i < turned; i += 2) {
      const float c = fcr[i >> 1], s = fci[i >> 1];
      const float v0 = base[i], v1 = base[i + 1];
      base[i] = v0 * c - v1 * s;
      base[i + 1] = v0 * s + v1 * c;
    }
  }
}

/* kernels/kernel.ts:570-599 to_f16: float32 to float16, round to nearest even; 65536 and above (and NaN) to inf */
void or_to_f16(uint16_t *out, const float *x, int32_t n) {
  for (int32_t i = 0; i < n; i++) {
    const uint32_t bits = f32_bits(x[i]);
    const uint32_t sign = (bits >> 16) & 0x8000;
    const int32_t exponent = (int32_t)((bits >> 23) & 0xff) - 112;
    uint32_t mantissa = bits & 0x7fffff;
    uint32_t result;
    if (exponent >= 31) {
      result = sign | 0x7c00;
    } else if (exponent <= 0) {
      if (exponent < -10) {
        result = sign;
      } else {
        mantissa |= 0x800000;
        const uint32_t shift = (uint32_t)(14 - exponent);
        const uint32_t rest = mantissa & ((1u << shift) - 1), middle = 1u << (shift - 1);
        uint32_t value = mantissa >> shift;
        if (rest > middle || (rest == middle && (value & 1))) value++;
        result = sign | value;
      }
    } else {
      const uint32_t rest = mantissa & 0x1fff;
      uint32_t value = ((uint32_t)exponent << 10) | (mantissa >> 13);
      if (rest > 0x1000 || (rest == 0x1000 && (value & 1))) value++;
      result = sign | value;
    }
    out[i] = (uint16_t)result;
  }
}

/* kernels/kernel.ts:383-392 halves4/half: the half's bits sign-extended, shifted by 13, masked with 0x8fffffff, times
 * 2^112: exact for every finite half (an infinity reads back as 65536) */
static inline float half_to_f32(uint16_t h) {
  const int32_t bits = ((int32_t)(int16_t)h << 13) & (int32_t)0x8fffffff;
  return bits_f32((uint32_t)bits) * 5.192296858534828e33f;
}
void or_from_f16(float *out, const uint16_t *x, int32_t n) {
  for (int32_t i = 0; i < n; i++) out[i] = half_to_f32(x[i]);
}

/* public/forward.js:593-597 halfToFloat, what keysAndValues() reads a float16 cache with: exact for every finite half,
 * and unlike the kernels' half() an infinity stays infinite and a NaN is NaN */
static float half_to_float(uint16_t h) {
  const uint32_t exponent = (h >> 10) & 0x1f, fraction = h & 0x3ff;
  if (exponent == 31) return fraction ? NAN : ((h & 0x8000) ? -INFINITY : INFINITY);
  return half_to_f32(h);
}

/* kernels/kernel.ts:654-667 swiglu: v / (1 + vexp(-v)) * h3 (the scalar tail's fexp gives the same bits: where the
 * two differ, 1 + exp(x) is 1 either way) */
void or_swiglu(float *out, const float *h1, const float *h3, int32_t n) {
  for (int32_t j = 0; j < n; j++) {
    const float v = h1[j];
    out[j] = v / (1.0f + vexp1(-v)) * h3[j];
  }
}

/* kernels/kernel.ts:610-634 layernorm: the sum of x in four lanes over n & ~3, hsum ((l0+l1)+l2)+l3, the tail in
 * order, mean = total / n; the same for (x - mean)^2; s = 1 / sqrt(ss / n + 1e-5); out = w * (s * (x - mean)) + b */
void or_layernorm(float *out, const float *x, const float *w, const float *b, int32_t n) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int32_t n4 = n & ~3;
  int32_t j = 0;
  for (; j < n4; j += 4)
    for (int32_t l = 0; l < 4; l++) acc[l] = acc[l] + x[j + l];
  float total = acc[0] + acc[1] + acc[2] + acc[3];
  for (; j < n; j++) total = total + x[j];
  const float mean = total / (float)n;
  float sq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (j = 0; j < n4; j += 4)
    for (int32_t l = 0; l < 4; l++) {
      const float d = x[j + l] - mean;
      sq[l] = sq[l] + d * d;
    }
  float ss = sq[0] + sq[1] + sq[2] + sq[3];
  for (; j < n; j++) {
    const float d = x[j] - mean;
    ss = ss + d * d;
  }
  const float s = 1.0f / sqrtf(ss / (float)n + 1e-5f);
  for (j = 0; j < n; j++) out[j] = w[j] * (s * (x[j] - mean)) + b[j];
}

/* kernels/kernel.ts:636-652 gelu (GPT-2's gelu_new) with the bias first: v = x + b, inner = c * (v + 0.044715 v v v),
 * out = v / (1 + vexp(-2 inner)) (the scalar tail's fexp gives the same bits, as in or_swiglu) */
void or_gelu(float *out, const float *x, const float *b, int32_t n) {
  for (int32_t j = 0; j < n; j++) {
    const float v = x[j] + b[j];
    const float inner = 0.7978845608028654f * (v + ((0.044715f * v) * v) * v);
    out[j] = v / (1.0f + vexp1(-2.0f * inner));
  }
}

/* kernels/kernel.ts:671-689 add_columns: y[j] += a[c] * rows[c][j] for c = 0, 1, ... in order, each product rounded */
void or_add_columns(float *y, const float *rows, const float *a, int32_t count, int32_t n) {
  for (int32_t j = 0; j < n; j++) {
    float acc = y[j];
    for (int32_t c = 0; c < count; c++) acc = acc + a[c] * rows[(int64_t)c * n + j];
    y[j] = acc;
  }
}

/* kernels/kernel.ts:691-693 */
void or_add(float *x, const float *y, int32_t n) {
  for (int32_t j = 0; j < n; j++) x[j] = x[j] + y[j];
}

/* kernels/kernel.ts:695-699: the first index of the largest */
int32_t or_argmax(const float *x, int32_t n) {
  int32_t mi = 0;
  float mv = x[0];
  for (int32_t j = 1; j < n; j++)
    if (x[j] > mv) {
      mv = x[j];
      mi = j;
    }
  return mi;
}

/* ------------------------------------------------------------------------------------------------ sampling */

/* kernels/kernel.ts:705-719 penalize: each distinct token of tokens[0..count) once (a later repeat is skipped),
 * value > 0 ? value / penalty : value * penalty */
void or_penalize(float *logits, const int32_t *tokens, int32_t count, float penalty) {
  for (int32_t i = 0; i < count; i++) {
    int32_t seen = 0;
    for (int32_t j = 0; j < i; j++)
      if (tokens[j] == tokens[i]) {
        seen = 1;
        break;
      }
    if (seen) continue;
    const float v = logits[tokens[i]];
    logits[tokens[i]] = v > 0 ? v / penalty : v * penalty;
  }
}

static const float *sort_probs;  /* the nucleus sort's keys (qsort has no context argument) */
static const int32_t *sort_index;
static int nucleus_order(const void *a, const void *b) {
  const int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
  if (sort_probs[x] != sort_probs[y]) return sort_probs[x] > sort_probs[y] ? -1 : 1;
  return sort_index[x] < sort_index[y] ? -1 : (sort_index[x] > sort_index[y] ? 1 : 0);
}

/* kernels/kernel.ts:803-868 sample, with largest (:423-445) and the nucleus of sortNucleus/intoNucleus (:729-787):
 *   best = the largest logit (a NaN anywhere gives NaN); -1 unless it is finite;
 *   nucleus = 0 < topp < 1; floor = nucleus ? best - temperature * 16.118095 : -FLT_MAX;
 *   kept, in index order: (v - best, i) for every v >= floor;
 *   p = vexp((v - best) * f32(1 / temperature)) for the first 4 * floor(count / 4), fexp((v - best) / temperature)
 *     for the rest; total = the float64 sum in that order, top = the largest p;
 *   nucleus: cutoff = min((1 - topp) / max(count - 1, 1) * total, top) (float64); the kept p >= cutoff sorted from
 *     the most probable, their float64 running sum up to the first >= topp * total (the last taken, the mass);
 *   the first token whose running float64 sum passes random * mass, else the last.
 * Equal probabilities in the nucleus go in index order: kernel.ts's quicksort takes them in no set order (either is
 * its distribution, public/shaders.js:3290-3292), and public/shaders.js's sampleLikeCpu takes index order.
 * probs and index: scratch of n each; order: scratch of n ints. */
int32_t or_sample(const float *logits, int32_t n, float temperature, float topp, double random, float *probs,
                  int32_t *index, int32_t *order) {
  float best = logits[0];
  for (int32_t i = 0; i < n; i++) best = wmax(best, logits[i]);
  if (!isfinite(best)) return -1;
  const int nucleus = topp > 0 && topp < 1;
  const float floor_ = nucleus ? best - temperature * 16.118095f : -3.4028234663852886e38f;
  int32_t count = 0;
  for (int32_t i = 0; i < n; i++)
    if (logits[i] >= floor_) {
      probs[count] = logits[i] - best;
      index[count] = i;
      count++;
    }
  const float inverse = 1.0f / temperature;
  const int32_t simd = count & ~3;
  for (int32_t k = 0; k < count; k++) probs[k] = k < simd ? vexp1(probs[k] * inverse) : or_fexp(probs[k] / temperature);
  double total = 0;
  float top = 0;
  for (int32_t k = 0; k < count; k++) {
    total += probs[k];
    top = fmaxf(top, probs[k]);
  }
  int32_t last = count - 1;
  double mass = total;
  for (int32_t k = 0; k < count; k++) order[k] = k;
  if (nucleus) {
    const double ceiling = (1.0 - (double)topp) / (double)(count > 1 ? count - 1 : 1) * total;
    const double cutoff = ceiling < (double)top ? ceiling : (double)top;
    int32_t likely = 0;
    for (int32_t k = 0; k < count; k++)
      if ((double)probs[k] >= cutoff) order[likely++] = k;
    sort_probs = probs;
    sort_index = index;
    qsort(order, (size_t)likely, sizeof(int32_t), nucleus_order);
    const double limit = (double)topp * total;
    double sum = 0;
    last = likely - 1;
    for (int32_t k = 0; k < likely; k++) {
      sum += probs[order[k]];
      if (sum >= limit) {
        last = k;
        break;
      }
    }
    mass = sum;
  }
  const double target = random * mass;
  double cumulative = 0;
  for (int32_t k = 0; k <= last; k++) {
    cumulative += probs[order[k]];
    if (cumulative > target) return index[order[k]];
  }
  return index[order[last]];
}

/* ------------------------------------------------------------------------------------------------ attention */

static inline float kv_at(const void *c, int64_t i, int32_t half) {
  return half ? half_to_f32(((const uint16_t *)c)[i]) : ((const float *)c)[i];
}

/* kernels/kernel.ts:448-566 attentionOf: heads h0..h1 of token at position pos over the cache rows 0..pos
 * ([pos][nkv*hs], f32 or f16); att holds nh*(pos+1) scores. */
void or_attention(float *out, const float *q, const void *kc, const void *vc, float *att, int32_t pos, int32_t nh,
                  int32_t nkv, int32_t hs, int32_t h0, int32_t h1, int32_t half) {
  const int32_t kvDim = nkv * hs, kvMul = nh / nkv, hs4 = hs & ~3;
  const int32_t count = pos + 1, count4 = count & ~3;
  const float isq = 1.0f / sqrtf((float)hs);
  /* 1. scores: four lanes over j < hs4, reduced (l0+l2)+(l1+l3) (sums4/sum4, :406-414), the tail added, times isq */
  for (int32_t h = h0; h < h1; h++) {
    const float *qh = q + h * hs;
    for (int32_t t = 0; t < count; t++) {
      const int64_t kt = (int64_t)t * kvDim + (h / kvMul) * hs;
      float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      int32_t j = 0;
      for (; j < hs4; j += 4)
        for (int32_t l = 0; l < 4; l++) a[l] = a[l] + qh[j + l] * kv_at(kc, kt + j + l, half);
      float sc = (a[0] + a[2]) + (a[1] + a[3]);
      for (; j < hs; j++) sc = sc + qh[j] * kv_at(kc, kt + j, half);
      att[h * count + t] = sc * isq;
    }
  }
  /* 2. softmax: the largest (order-free), vexp over the fours and fexp past them, the sums in four lanes then in
   * order, times f32(1 / sum) */
  for (int32_t h = h0; h < h1; h++) {
    float *scores = att + h * count;
    float mx = -3.4028234663852886e38f;
    for (int32_t t = 0; t < count; t++) mx = wmax(mx, scores[t]);
    float sums[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int32_t t = 0;
    for (; t < count4; t += 4)
      for (int32_t l = 0; l < 4; l++) {
        const float e = vexp1(scores[t + l] - mx);
        scores[t + l] = e;
        sums[l] = sums[l] + e;
      }
    float sum = sums[0] + sums[1] + sums[2] + sums[3];
    for (; t < count; t++) {
      const float e = or_fexp(scores[t] - mx);
      scores[t] = e;
      sum = sum + e;
    }
    const float inv = 1.0f / sum;
    for (t = 0; t < count; t++) scores[t] = scores[t] * inv;
  }
  /* 3. the weighted values: four positions a step, (w0 v0 + w1 v1) + (w2 v2 + w3 v3) added to out; then the positions
   * past the fours one at a time */
  for (int32_t j = h0 * hs; j < h1 * hs; j++) out[j] = 0.0f;
  int32_t t = 0;
  for (; t < count4; t += 4) {
    for (int32_t h = h0; h < h1; h++) {
      const float *wt = att + h * count + t;
      float *oh = out + h * hs;
      const int64_t v0 = (int64_t)t * kvDim + (h / kvMul) * hs, st = kvDim;
      int32_t j = 0;
      for (; j < hs4; j++) {
        const float pair0 = wt[0] * kv_at(vc, v0 + j, half) + wt[1] * kv_at(vc, v0 + st + j, half);
        const float pair1 = wt[2] * kv_at(vc, v0 + 2 * st + j, half) + wt[3] * kv_at(vc, v0 + 3 * st + j, half);
        oh[j] = oh[j] + (pair0 + pair1);
      }
      for (; j < hs; j++)
        oh[j] = oh[j] + wt[0] * kv_at(vc, v0 + j, half) + wt[1] * kv_at(vc, v0 + st + j, half) +
                wt[2] * kv_at(vc, v0 + 2 * st + j, half) + wt[3] * kv_at(vc, v0 + 3 * st + j, half);
    }
  }
  for (; t < count; t++) {
    for (int32_t h = h0; h < h1; h++) {
      const float weight = att[h * count + t];
      float *oh = out + h * hs;
      const int64_t vt = (int64_t)t * kvDim + (h / kvMul) * hs;
      for (int32_t j = 0; j < hs; j++) oh[j] = oh[j] + weight * kv_at(vc, vt + j, half);
    }
  }
}

/* ------------------------------------------------------------------------------------------------ the checkpoint */

static int layer_norm(const he_config *c) { return c->arch == HE_ARCH_GPT2 || c->arch == HE_ARCH_NEOX; }

/* the tensors of the form (public/llama2_convert.py:32-83) */
static int present(const he_config *c, int32_t id) {
  switch (id) {
    case HE_T_WCLS: return !c->shared_classifier;
    case HE_T_W3: return !layer_norm(c);
    case HE_T_BQ:
    case HE_T_BK:
    case HE_T_BV: return layer_norm(c) || c->qkv_bias;
    case HE_T_Q_NORM:
    case HE_T_K_NORM: return !layer_norm(c) && c->qk_norm;
    case HE_T_POSITIONS: return c->arch == HE_ARCH_GPT2;
    case HE_T_LN_ATT_BIAS:
    case HE_T_LN_FFN_BIAS:
    case HE_T_LN_FINAL_BIAS:
    case HE_T_BO:
    case HE_T_B1:
    case HE_T_B2: return layer_norm(c);
  }
  return 1;
}

/* a tensor's value count and row length (0 for float32 vectors) */
static void tensor_shape(const he_config *c, int32_t id, int64_t *count, int64_t *last) {
  const int64_t L = c->n_layers, dim = c->dim, hidden = c->hidden_dim, vocab = c->vocab_size;
  const int64_t qdim = (int64_t)c->n_heads * c->head_size, kvdim = (int64_t)c->n_kv_heads * c->head_size;
  const int64_t counts[HE_T_COUNT] = {vocab * dim, L * dim, L * qdim * dim, L * kvdim * dim, L * kvdim * dim,
                                      L * dim * qdim, L * dim, L * hidden * dim, L * dim * hidden, L * hidden * dim,
                                      dim, vocab * dim, L * qdim, L * kvdim, L * kvdim,
                                      L * c->head_size, L * c->head_size, (int64_t)c->seq_len * dim, L * dim, L * dim,
                                      dim, L * dim, L * hidden, L * dim};
  const int64_t lasts[HE_T_COUNT] = {dim, 0, dim, dim, dim, qdim, 0, dim, hidden, dim, 0, dim, 0, 0, 0,
                                     0, 0, dim, 0, 0, 0, 0, 0, 0};
  *count = counts[id];
  *last = lasts[id];
}

/* public/llama2_numpy.py:751-775 Places.take over the tensor order of the form: llama_tensors (:1149-1179, Qwen2's
 * biases and Qwen3's head norms last) or gpt2_tensors (:1203-1240), as public/llama2_convert.py:32-83 writes them, of
 * an int8 or int6 checkpoint (no RoPE tables in such a file), from the 28-byte header on. Returns the file size. */
int64_t or_places(const he_config *c, he_tensor *t) {
  int64_t offset = 28;
  memset(t, 0, sizeof(he_tensor) * HE_T_COUNT);
#define TAKE(id)                                                              \
  do {                                                                        \
    int64_t n_, last_;                                                        \
    tensor_shape(c, (id), &n_, &last_);                                       \
    t[id].offset = offset;                                                    \
    if (last_) {                                                              \
      const int64_t grp_ = or_group_size((int32_t)last_);                     \
      const int64_t stored_ = c->six ? n_ * 3 / 4 : n_;                       \
      t[id].scales = offset + stored_;                                        \
      offset += stored_ + 4 * (n_ / grp_);                                    \
    } else {                                                                  \
      offset += 4 * n_;                                                       \
    }                                                                         \
  } while (0)
  if (layer_norm(c)) {
    static const int32_t order[] = {HE_T_EMBEDDING, HE_T_POSITIONS, HE_T_RMS_ATT, HE_T_LN_ATT_BIAS, HE_T_WQ, HE_T_WK,
                                    HE_T_WV, HE_T_BQ, HE_T_BK, HE_T_BV, HE_T_WO, HE_T_BO, HE_T_RMS_FFN,
                                    HE_T_LN_FFN_BIAS, HE_T_W1, HE_T_B1, HE_T_W2, HE_T_B2, HE_T_RMS_FINAL,
                                    HE_T_LN_FINAL_BIAS, HE_T_WCLS};
    for (size_t i = 0; i < sizeof order / sizeof order[0]; i++)
      if (present(c, order[i])) TAKE(order[i]);
  } else {
    static const int32_t order[] = {HE_T_EMBEDDING, HE_T_RMS_ATT, HE_T_WQ, HE_T_WK, HE_T_WV, HE_T_WO, HE_T_RMS_FFN,
                                    HE_T_W1, HE_T_W2, HE_T_W3, HE_T_RMS_FINAL, HE_T_WCLS, HE_T_BQ, HE_T_BK, HE_T_BV,
                                    HE_T_Q_NORM, HE_T_K_NORM};
    for (size_t i = 0; i < sizeof order / sizeof order[0]; i++)
      if (present(c, order[i])) TAKE(order[i]);
  }
  if (c->shared_classifier) t[HE_T_WCLS] = t[HE_T_EMBEDDING];
#undef TAKE
  return offset;
}

static int norm_weight(int32_t id) {
  return id == HE_T_RMS_ATT || id == HE_T_RMS_FFN || id == HE_T_RMS_FINAL || id == HE_T_Q_NORM || id == HE_T_K_NORM;
}

/* quantize.py:22-40 on a synthetic float32 model: matrices N(0, 0.02) by or_synth_value (stream = the tensor's
 * HE_T_* index, index = the value's place in the tensor), quantize() or quantize6()+pack6(); norm weights 1.0;
 * biases N(0, 0.02). The 28-byte header is the llama2.c one (vocab negative where the classifier is its own). */
void or_synth_checkpoint(const he_config *c, const he_tensor *t, uint8_t *out, int64_t size, uint64_t seed) {
  (void)size;
  int32_t header[7] = {c->dim, c->hidden_dim, c->n_layers, c->n_heads, c->n_kv_heads,
                       c->shared_classifier ? c->vocab_size : -c->vocab_size, c->seq_len};
  memcpy(out, header, 28);
  for (int32_t id = 0; id < HE_T_COUNT; id++) {
    if (!present(c, id)) continue;
    int64_t n, last;
    tensor_shape(c, id, &n, &last);
    if (!last && norm_weight(id)) {
      float *v = (float *)(out + t[id].offset);
      for (int64_t i = 0; i < n; i++) v[i] = 1.0f;
      continue;
    }
    /* one piece of rows at a time (a vector: one row) */
    const int64_t K = last ? last : n;
    const int64_t piece_rows = (1 << 22) / K + 1;
    float *vals = (float *)malloc(sizeof(float) * (size_t)(piece_rows * K));
    int8_t *q = (int8_t *)malloc((size_t)(piece_rows * K));
    for (int64_t r0 = 0; r0 < n / K; r0 += piece_rows) {
      const int64_t rows = (n / K - r0) < piece_rows ? (n / K - r0) : piece_rows;
      or_synth_fill(vals, (uint64_t)(rows * K), seed, id, (uint64_t)(r0 * K), 0.02);
      if (!last) {
        memcpy(out + t[id].offset + 4 * r0 * K, vals, sizeof(float) * (size_t)(rows * K));
        continue;
      }
      const int32_t grp = c->six ? 32 : or_group_size((int32_t)K);
      const int64_t g0 = r0 * K / grp, groups = rows * K / grp;
      float *scales = (float *)(out + t[id].scales) + g0;
      if (c->six) {
        or_quantize6(q, scales, vals, groups);
        or_pack6(out + t[id].offset + g0 * 24, q, groups);
      } else {
        or_quantize(q, scales, vals, rows * K, grp);
        memcpy(out + t[id].offset + r0 * K, q, (size_t)(rows * K));
      }
    }
    free(q);
    free(vals);
  }
}

/* public/llama2_numpy.py:484-542 (no scaling): angles = pos * 1 / theta ** (arange(0, hs, 2) / hs) in float64,
 * cos and sin rounded to float32 (:1177-1179) */
void or_rope_tables(float *cos_out, float *sin_out, int32_t seq_len, int32_t hs, double theta) {
  const int32_t half = hs / 2;
  for (int32_t i = 0; i < half; i++) {
    const double freq = 1.0 / pow(theta, (double)(2 * i) / (double)hs);
    for (int32_t p = 0; p < seq_len; p++) {
      const double angle = (double)p * freq;
      cos_out[(int64_t)p * half + i] = (float)cos(angle);
      sin_out[(int64_t)p * half + i] = (float)sin(angle);
    }
  }
}

/* ------------------------------------------------------------------------------------------------ the model */

struct or_model {
  he_config c;
  he_tensor t[HE_T_COUNT];
  const uint8_t *ck;
  float *cosT, *sinT;
  int32_t max_block, qdim, kvdim, bias, xw;
  void *keys, *values; /* [layers][seq_len][kvdim], f32 or f16 */
  /* frames (public/forward.js:250-255, 765-769): per token */
  float *x, *xb, *xb2, *q, *k, *v, *hb, *hb2, *att, *logits;
  int8_t *xq;
  float *xs;
  float *before;          /* the layer's input (parallel residual) */
  float *columns, picked[HE_OUTLIERS_MOST]; /* the outlier channels' float32 classifier columns [n][vocab] */
};

static const int8_t *mat_values(const or_model *m, int32_t id, int32_t l, int64_t rows, int64_t K) {
  const int64_t per = m->c.six ? rows * K * 3 / 4 : rows * K;
  return (const int8_t *)(m->ck + m->t[id].offset + l * per);
}
static const float *mat_scales(const or_model *m, int32_t id, int32_t l, int64_t rows, int64_t K) {
  return (const float *)(m->ck + m->t[id].scales) + l * rows * (K / GS);
}
static const float *vec(const or_model *m, int32_t id, int64_t at) {
  return (const float *)(m->ck + m->t[id].offset) + at;
}

or_model *or_model_open(const he_config *c, const he_tensor *t, const uint8_t *checkpoint, const float *rope_cos,
                        const float *rope_sin, int32_t max_block) {
  or_model *m = (or_model *)calloc(1, sizeof(or_model));
  m->c = *c;
  memcpy(m->t, t, sizeof(he_tensor) * HE_T_COUNT);
  m->ck = checkpoint;
  m->max_block = max_block;
  m->qdim = c->n_heads * c->head_size;
  m->kvdim = c->n_kv_heads * c->head_size;
  m->bias = c->relaxed ? 64 : 0;
  m->xw = c->dim > m->qdim ? c->dim : m->qdim;
  const int64_t table = (int64_t)c->seq_len * (c->head_size / 2);
  m->cosT = (float *)malloc(sizeof(float) * (size_t)table);
  m->sinT = (float *)malloc(sizeof(float) * (size_t)table);
  memcpy(m->cosT, rope_cos, sizeof(float) * (size_t)table);
  memcpy(m->sinT, rope_sin, sizeof(float) * (size_t)table);
  const size_t e = c->half_kv ? 2 : 4;
  const size_t kv = (size_t)c->n_layers * c->seq_len * m->kvdim * e;
  m->keys = calloc(1, kv);
  m->values = calloc(1, kv);
  const int64_t B = max_block, widest = c->hidden_dim > c->dim ? c->hidden_dim : c->dim;
  const int64_t wq = widest > m->qdim ? widest : m->qdim;
  m->x = (float *)calloc((size_t)(B * c->dim), 4);
  m->xb = (float *)calloc((size_t)(B * wq), 4);
  m->xb2 = (float *)calloc((size_t)(B * c->dim), 4);
  m->q = (float *)calloc((size_t)(B * m->qdim), 4);
  m->k = (float *)calloc((size_t)(B * m->kvdim), 4);
  m->v = (float *)calloc((size_t)(B * m->kvdim), 4);
  m->hb = (float *)calloc((size_t)(B * c->hidden_dim), 4);
  m->hb2 = (float *)calloc((size_t)(B * c->hidden_dim), 4);
  m->att = (float *)calloc((size_t)(B * c->n_heads * (int64_t)c->seq_len), 4);
  m->logits = (float *)calloc((size_t)c->vocab_size, 4);
  m->xq = (int8_t *)calloc((size_t)(B * wq), 1);
  m->xs = (float *)calloc((size_t)(B * wq / GS + 1), 4);
  m->before = (float *)calloc((size_t)(B * c->dim), 4);
  /* public/forward.js:801-812: columns[i][v] = f32(weight(v, c_i) * the scale of its group) */
  m->columns = (float *)calloc((size_t)c->n_outliers * (size_t)c->vocab_size + 1, 4);
  if (c->n_outliers) {
    const int32_t dim = c->dim, grp = c->six ? 32 : or_group_size(dim);
    const float *scales = (const float *)(checkpoint + t[HE_T_WCLS].scales);
    int8_t *wide = (int8_t *)malloc((size_t)dim);
    for (int32_t v = 0; v < c->vocab_size; v++) {
      const int64_t row = (int64_t)v * dim;
      if (c->six) or_unpack6(wide, checkpoint + t[HE_T_WCLS].offset + row / GS * 24, dim / GS);
      else memcpy(wide, checkpoint + t[HE_T_WCLS].offset + row, (size_t)dim);
      for (int32_t i = 0; i < c->n_outliers; i++) {
        const int32_t ch = c->outliers[i];
        m->columns[(int64_t)i * c->vocab_size + v] = (float)wide[ch] * scales[(row + ch) / grp];
      }
    }
    free(wide);
  }
  return m;
}

void or_model_close(or_model *m) {
  if (!m) return;
  free(m->cosT); free(m->sinT); free(m->keys); free(m->values);
  free(m->x); free(m->xb); free(m->xb2); free(m->q); free(m->k); free(m->v);
  free(m->hb); free(m->hb2); free(m->att); free(m->logits); free(m->xq); free(m->xs);
  free(m->before); free(m->columns);
  free(m);
}

/* kernels/kernel_relaxed.ts:84-183 matmul_q8r_tile (public/jobs.js:96 runs it on prompt blocks): a row's weights
 * against every token of the block while the row is at hand. Per (row, token) it is the one-token kernel to the bit
 * (the same exact group sums, relaxed_row / plain_row in the same order), so this only changes how often a row is
 * read: once a block instead of once a token. xq [count][K] from quantize_x(bias), xs [count][K/32]. */
static void matmul_tokens(float *out, int64_t out_stride, const int8_t *xq, const float *xs, const void *w,
                          const float *ws, int32_t rows, int32_t K, int32_t count, int32_t bias, int32_t six) {
  const int32_t ng = K / GS;
  int8_t *xc = (int8_t *)malloc((size_t)count * (size_t)K);
  if (bias) centred(xc, xq, count * K);
  else memcpy(xc, xq, (size_t)count * (size_t)K);
#pragma omp parallel
  {
    int8_t *wide = (int8_t *)malloc((size_t)K);
    int32_t *S = (int32_t *)malloc(sizeof(int32_t) * 4 * (size_t)ng);
#pragma omp for schedule(dynamic, 8)
    for (int32_t r = 0; r < rows; r++) {
      const int8_t *row;
      if (six) {
        or_unpack6(wide, (const uint8_t *)w + (int64_t)r * ng * 24, ng);
        row = wide;
      } else {
        row = (const int8_t *)w + (int64_t)r * K;
      }
      for (int32_t t = 0; t < count; t++) {
        const int8_t *x = xc + (int64_t)t * K;
        const float *st = xs + (int64_t)t * ng;
        if (bias) {
          for (int32_t g = 0; g < ng; g++) S[g] = dot32(row + g * GS, x + g * GS);
          out[t * out_stride + r] = relaxed_row(S, ws + (int64_t)r * ng, st, ng);
        } else {
          for (int32_t g = 0; g < ng; g++) lanes32(S + 4 * g, row + g * GS, x + g * GS);
          out[t * out_stride + r] = plain_row(S, ws + (int64_t)r * ng, st, ng);
        }
      }
    }
    free(S);
    free(wide);
  }
  free(xc);
}

/* public/forward.js:954-960 matmuls(): every token's input quantized once, then every matrix of the list */
static void matmuls(or_model *m, const float *input, int64_t in_stride, int32_t count, int32_t K, int32_t id,
                    int32_t l, int32_t rows, float *out, int64_t out_stride) {
  const int8_t *w = mat_values(m, id, l, rows, K);
  const float *ws = mat_scales(m, id, l, rows, K);
  if (count > 1) {
    for (int32_t t = 0; t < count; t++)
      or_quantize_x(m->xq + (int64_t)t * K, m->xs + (int64_t)t * (K / GS), input + t * in_stride, K, m->bias);
    matmul_tokens(out, out_stride, m->xq, m->xs, w, ws, rows, K, count, m->bias, m->c.six);
    return;
  }
  for (int32_t t = 0; t < count; t++) {
    int8_t *xq = m->xq + (int64_t)t * K;
    float *xs = m->xs + (int64_t)t * (K / GS);
    or_quantize_x(xq, xs, input + t * in_stride, K, m->bias);
    float *y = out + t * out_stride;
    if (m->c.six) {
      if (m->bias) or_matmul_q6r(y, xq, xs, (const uint8_t *)w, ws, K, 0, rows);
      else or_matmul_q6(y, xq, xs, (const uint8_t *)w, ws, K, 0, rows);
    } else {
      if (m->bias) or_matmul_q8r(y, xq, xs, w, ws, K, 0, rows);
      else or_matmul_q8(y, xq, xs, w, ws, K, 0, rows);
    }
  }
}

/* valueAt (public/forward.js:672-696) over a row of an int8 / int6 table: f32(value * scale of its group) */
static void widen_row(const or_model *m, int32_t id, int64_t r, float *x) {
  const int32_t dim = m->c.dim, grp = m->c.six ? 32 : or_group_size(dim);
  const float *scales = (const float *)(m->ck + m->t[id].scales);
  const int64_t row = r * dim;
  if (m->c.six) {
    int8_t *wide = (int8_t *)malloc((size_t)dim);
    or_unpack6(wide, m->ck + m->t[id].offset + row / GS * 24, dim / GS);
    for (int32_t i = 0; i < dim; i++) x[i] = (float)wide[i] * scales[(row + i) / grp];
    free(wide);
  } else {
    const int8_t *v = (const int8_t *)(m->ck + m->t[id].offset) + row;
    for (int32_t i = 0; i < dim; i++) x[i] = (float)v[i] * scales[(row + i) / grp];
  }
}

/* public/forward.js:962-973 embed(): the token's row widened; GPT-2's row of positions (widened too, floats()) added */
static void embed(or_model *m, int32_t token, int32_t pos, float *x) {
  widen_row(m, HE_T_EMBEDDING, token, x);
  if (m->c.arch == HE_ARCH_GPT2) {
    float *p = (float *)malloc(sizeof(float) * (size_t)m->c.dim);
    widen_row(m, HE_T_POSITIONS, pos, p);
    or_add(x, p, m->c.dim);
    free(p);
  }
}

static void write_cache(or_model *m, void *cache, int32_t l, int32_t pos, const float *src) {
  const int64_t at = ((int64_t)l * m->c.seq_len + pos) * m->kvdim;
  if (m->c.half_kv) or_to_f16((uint16_t *)cache + at, src, m->kvdim);
  else memcpy((float *)cache + at, src, sizeof(float) * (size_t)m->kvdim);
}

/* public/forward.js:1011-1090 run(): count tokens at pos0.., every token computed as it would be alone; the logits,
 * if asked for, the last token's. The llama form (RMSNorm, RoPE, SwiGLU; Qwen2's q/k/v biases, Qwen3's head norms)
 * and GPT-2 / GPT-NeoX (LayerNorm, learned positions or RoPE over the first `rotary` values, GELU, a bias after every
 * matrix, the parallel residual); the outlier channels multiplied apart at the classifier. */
int32_t or_model_run(or_model *m, const int32_t *tokens, int32_t count, int32_t pos0, int32_t need_logits) {
  const he_config *c = &m->c;
  if (count < 1 || count > m->max_block || pos0 < 0 || pos0 + count > c->seq_len) return -1;
  const int32_t dim = c->dim, hidden = c->hidden_dim, qdim = m->qdim, kvdim = m->kvdim, hs = c->head_size, xw = m->xw;
  const float eps = c->rms_norm_eps;
  const size_t e = c->half_kv ? 2 : 4;
  const int ln = layer_norm(c), biases = ln || c->qkv_bias;
  for (int32_t t = 0; t < count; t++) embed(m, tokens[t], pos0 + t, m->x + (int64_t)t * dim);
  for (int32_t l = 0; l < c->n_layers; l++) {
    for (int32_t t = 0; t < count; t++) {
      float *xbt = m->xb + (int64_t)t * xw, *xt = m->x + (int64_t)t * dim;
      if (ln) or_layernorm(xbt, xt, vec(m, HE_T_RMS_ATT, (int64_t)l * dim), vec(m, HE_T_LN_ATT_BIAS, (int64_t)l * dim),
                           dim);
      else or_rmsnorm(xbt, xt, vec(m, HE_T_RMS_ATT, (int64_t)l * dim), dim, eps);
      if (c->parallel_residual) memcpy(m->before + (int64_t)t * dim, xt, sizeof(float) * (size_t)dim);
    }
    matmuls(m, m->xb, xw, count, dim, HE_T_WQ, l, qdim, m->q, qdim);
    matmuls(m, m->xb, xw, count, dim, HE_T_WK, l, kvdim, m->k, kvdim);
    matmuls(m, m->xb, xw, count, dim, HE_T_WV, l, kvdim, m->v, kvdim);
    for (int32_t t = 0; t < count; t++) {
      float *qt = m->q + (int64_t)t * qdim, *kt = m->k + (int64_t)t * kvdim, *vt = m->v + (int64_t)t * kvdim;
      const int32_t pos = pos0 + t;
      if (biases) {
        or_add(qt, vec(m, HE_T_BQ, (int64_t)l * qdim), qdim);
        or_add(kt, vec(m, HE_T_BK, (int64_t)l * kvdim), kvdim);
        or_add(vt, vec(m, HE_T_BV, (int64_t)l * kvdim), kvdim);
      }
      if (c->qk_norm) {
        for (int32_t h = 0; h < c->n_heads; h++)
          or_rmsnorm(qt + h * hs, qt + h * hs, vec(m, HE_T_Q_NORM, (int64_t)l * hs), hs, eps);
        for (int32_t h = 0; h < c->n_kv_heads; h++)
          or_rmsnorm(kt + h * hs, kt + h * hs, vec(m, HE_T_K_NORM, (int64_t)l * hs), hs, eps);
      }
      if (c->arch != HE_ARCH_GPT2) {
        const float *cs = m->cosT + (int64_t)pos * (hs / 2), *sn = m->sinT + (int64_t)pos * (hs / 2);
        const int32_t rot = c->arch == HE_ARCH_NEOX ? c->rotary : 0;
        or_rope(qt, cs, sn, c->n_heads, hs, rot);
        or_rope(kt, cs, sn, c->n_kv_heads, hs, rot);
      }
      write_cache(m, m->keys, l, pos, kt);
      write_cache(m, m->values, l, pos, vt);
    }
    const uint8_t *kc = (const uint8_t *)m->keys + (size_t)l * c->seq_len * kvdim * e;
    const uint8_t *vc = (const uint8_t *)m->values + (size_t)l * c->seq_len * kvdim * e;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int32_t t = 0; t < count; t++)
      for (int32_t h = 0; h < c->n_heads; h++)
        or_attention(m->xb + (int64_t)t * xw, m->q + (int64_t)t * qdim, kc, vc,
                     m->att + (int64_t)t * c->n_heads * c->seq_len, pos0 + t, c->n_heads, c->n_kv_heads, hs, h, h + 1,
                     c->half_kv);
    matmuls(m, m->xb, xw, count, qdim, HE_T_WO, l, dim, m->xb2, dim);
    for (int32_t t = 0; t < count; t++) or_add(m->x + (int64_t)t * dim, m->xb2 + (int64_t)t * dim, dim);
    if (ln) {
      for (int32_t t = 0; t < count; t++) {
        or_add(m->x + (int64_t)t * dim, vec(m, HE_T_BO, (int64_t)l * dim), dim);
        or_layernorm(m->xb + (int64_t)t * xw, (c->parallel_residual ? m->before : m->x) + (int64_t)t * dim,
                     vec(m, HE_T_RMS_FFN, (int64_t)l * dim), vec(m, HE_T_LN_FFN_BIAS, (int64_t)l * dim), dim);
      }
      matmuls(m, m->xb, xw, count, dim, HE_T_W1, l, hidden, m->hb, hidden);
      for (int32_t t = 0; t < count; t++)
        or_gelu(m->hb + (int64_t)t * hidden, m->hb + (int64_t)t * hidden, vec(m, HE_T_B1, (int64_t)l * hidden), hidden);
      matmuls(m, m->hb, hidden, count, hidden, HE_T_W2, l, dim, m->xb2, dim);
      for (int32_t t = 0; t < count; t++) {
        or_add(m->x + (int64_t)t * dim, m->xb2 + (int64_t)t * dim, dim);
        or_add(m->x + (int64_t)t * dim, vec(m, HE_T_B2, (int64_t)l * dim), dim);
      }
      continue;
    }
    for (int32_t t = 0; t < count; t++)
      or_rmsnorm(m->xb + (int64_t)t * xw, m->x + (int64_t)t * dim, vec(m, HE_T_RMS_FFN, (int64_t)l * dim), dim, eps);
    matmuls(m, m->xb, xw, count, dim, HE_T_W1, l, hidden, m->hb, hidden);
    matmuls(m, m->xb, xw, count, dim, HE_T_W3, l, hidden, m->hb2, hidden);
    for (int32_t t = 0; t < count; t++)
      or_swiglu(m->hb + (int64_t)t * hidden, m->hb + (int64_t)t * hidden, m->hb2 + (int64_t)t * hidden, hidden);
    matmuls(m, m->hb, hidden, count, hidden, HE_T_W2, l, dim, m->xb2, dim);
    for (int32_t t = 0; t < count; t++) or_add(m->x + (int64_t)t * dim, m->xb2 + (int64_t)t * dim, dim);
  }
  if (!need_logits) return 0;
  const float *last = m->x + (int64_t)(count - 1) * dim;
  if (ln) or_layernorm(m->xb, last, vec(m, HE_T_RMS_FINAL, 0), vec(m, HE_T_LN_FINAL_BIAS, 0), dim);
  else or_rmsnorm(m->xb, last, vec(m, HE_T_RMS_FINAL, 0), dim, eps);
  for (int32_t i = 0; i < c->n_outliers; i++) { /* public/forward.js:1084-1087 */
    m->picked[i] = m->xb[c->outliers[i]];
    m->xb[c->outliers[i]] = 0.0f;
  }
  matmuls(m, m->xb, xw, 1, dim, HE_T_WCLS, 0, c->vocab_size, m->logits, 0);
  if (c->n_outliers) or_add_columns(m->logits, m->columns, m->picked, c->n_outliers, c->vocab_size);
  return 0;
}

const float *or_model_logits(const or_model *m) { return m->logits; }

/* public/forward.js:1939-1953 keysAndValues(): float32 [layers][count][kvdim] */
void or_model_kv(const or_model *m, int32_t from, int32_t count, float *keys, float *values) {
  for (int32_t l = 0; l < m->c.n_layers; l++)
    for (int32_t t = 0; t < count; t++) {
      const int64_t at = ((int64_t)l * m->c.seq_len + from + t) * m->kvdim;
      float *ko = keys + ((int64_t)l * count + t) * m->kvdim, *vo = values + ((int64_t)l * count + t) * m->kvdim;
      if (m->c.half_kv) {
        for (int32_t i = 0; i < m->kvdim; i++) {
          ko[i] = half_to_float(((const uint16_t *)m->keys)[at + i]);
          vo[i] = half_to_float(((const uint16_t *)m->values)[at + i]);
        }
      } else {
        memcpy(ko, (const float *)m->keys + at, sizeof(float) * (size_t)m->kvdim);
        memcpy(vo, (const float *)m->values + at, sizeof(float) * (size_t)m->kvdim);
      }
    }
}

/* public/llama2_numpy.py:1565-1651 generate() with temperature 0 and no stop tokens: fed = [BOS] + prompt[:-1]
 * through forwardMany in blocks of `block`, then from the last prompt token one greedy step a position until
 * `steps` positions. Writes the chosen tokens; returns their number. */
int32_t or_generate(or_model *m, const int32_t *prompt, int32_t n_prompt, int32_t steps, int32_t block,
                    int32_t *out_tokens, float *last_logits) {
  int32_t token = 1, pos = 0, n = 0;
  if (n_prompt >= 1) {
    int32_t *fed = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_prompt);
    fed[0] = 1;
    for (int32_t i = 1; i < n_prompt; i++) fed[i] = prompt[i - 1];
    for (int32_t at = 0; at < n_prompt; at += block) {
      const int32_t len = n_prompt - at < block ? n_prompt - at : block;
      if (or_model_run(m, fed + at, len, at, 0)) {
        free(fed);
        return -1;
      }
    }
    free(fed);
    token = prompt[n_prompt - 1];
    pos = n_prompt;
  }
  for (; pos < steps; pos++) {
    if (or_model_run(m, &token, 1, pos, 1)) return -1;
    token = or_argmax(m->logits, m->c.vocab_size);
    out_tokens[n++] = token;
  }
  if (last_logits) memcpy(last_logits, m->logits, sizeof(float) * (size_t)m->c.vocab_size);
  return n;
}

/* the C layout of include/pyodide_llm_hip.h's structs, for the hosts' ctypes mirrors: sizeof(he_config), the offsets
 * of rms_norm_eps, arch and outliers in it, sizeof(he_tensor), HE_T_COUNT */
void or_abi_layout(int64_t *out) {
  out[0] = (int64_t)sizeof(he_config);
  out[1] = (int64_t)offsetof(he_config, rms_norm_eps);
  out[2] = (int64_t)offsetof(he_config, arch);
  out[3] = (int64_t)offsetof(he_config, outliers);
  out[4] = (int64_t)sizeof(he_tensor);
  out[5] = HE_T_COUNT;
}

void or_set_threads(int32_t n) { omp_set_num_threads(n > 0 ? n : 1); }
int32_t or_get_threads(void) { return omp_get_max_threads(); }
