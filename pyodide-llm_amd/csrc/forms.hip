// forms.hip — the kernels of the model forms beside the Llama/Qwen2 one, each in the reference's float32 order:
//   layernorm (kernels/kernel.ts:610-634) then quantize_x: GPT-2 and GPT-NeoX (public/forward.js:1031,1063,1082);
//   gelu with the bias of w1 (kernels/kernel.ts:636-652) then quantize_x;
//   the biases added after wo and w2 (add_inplace, kernels/kernel.ts:691-693; public/forward.js:1061,1070-1071);
//   Qwen3's q/k head norms: rmsnorm (kernels/kernel.ts:330-342) over every head of q and k after the biases
//   (public/forward.js:1038-1047);
//   the outlier channels of the classifier's input (public/forward.js:801-812,1084-1089): their float32 columns of the
//   classifier, the channels taken out of its input, and add_columns (kernels/kernel.ts:671-689) after it.
#pragma clang fp contract(off)

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

namespace {

// layernorm of one token a block: the sum of x in four lanes (j % 4) added in order by four threads, hsum
// ((l0 + l1) + l2) + l3, the tail in order, mean = f32(total / n); the same for (x - mean)^2; s = f32(1 / f32(sqrt(
// f32(ss / n) + 1e-5))); out = f32(f32(w * f32(s * f32(x - mean))) + b); then quantize_x of out. copy (optional)
// receives x itself: the layer's input, which a parallel residual's FFN normalizes again (public/forward.js:1033).
__global__ __launch_bounds__(1024) void layernorm_quant_kernel(int8_t *xq, float *xs, float *out, float *copy,
                                                              const float *x, const float *w, const float *b,
                                                              int32_t n, int32_t x_stride, int32_t xq_stride,
                                                              int32_t xs_stride, int32_t out_stride, int32_t bias) {
  extern __shared__ float sm[];
  const int n4 = n & ~3, q4 = n4 >> 2, qs = chain_rowstride(q4);
  float *xv = sm;      // n
  float *sq = sm + n;  // 4 * qs, transposed: lane k's values side by side
  __shared__ float part[4];
  __shared__ float smean, sval;
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *xt = x + (int64_t)t * x_stride;
  for (int j = tid; j < n; j += 1024) {
    const float v = xt[j];
    xv[j] = v;
    if (j < n4) sq[(j & 3) * qs + (j >> 2)] = v;
    if (copy && blockIdx.y == 0) copy[(int64_t)t * x_stride + j] = v;
  }
  __syncthreads();
  if (tid < 4) part[tid] = lds_chain(sq + tid * qs, q4, 0.0f);
  __syncthreads();
  if (tid == 0) {
    float total = ((part[0] + part[1]) + part[2]) + part[3];
    for (int j = n4; j < n; ++j) total = total + xv[j];
    smean = total / (float)n;
  }
  __syncthreads();
  const float mean = smean;
  for (int j = tid; j < n4; j += 1024) {
    const float d = xv[j] - mean;
    sq[(j & 3) * qs + (j >> 2)] = d * d;
  }
  __syncthreads();
  if (tid < 4) part[tid] = lds_chain(sq + tid * qs, q4, 0.0f);
  __syncthreads();
  if (tid == 0) {
    float ss = ((part[0] + part[1]) + part[2]) + part[3];
    for (int j = n4; j < n; ++j) {
      const float d = xv[j] - mean;
      ss = ss + d * d;
    }
    sval = 1.0f / __builtin_sqrtf(ss / (float)n + 1e-5f);
  }
  __syncthreads();
  const float s = sval;
  int8_t *q = xq + (int64_t)t * xq_stride;
  float *sc = xs + (int64_t)t * xs_stride;
  // this block's share of the groups (gridDim.y blocks a token, as the rmsnorm kernel splits them)
  for (int g = (tid >> 5) * gridDim.y + blockIdx.y; g < n / GS; g += 32 * gridDim.y) {
    const int j = g * GS + (tid & 31);
    const float o = w[j] * (s * (xv[j] - mean)) + b[j];
    if (out) out[(int64_t)t * out_stride + j] = o;
    quantize_group(o, q, sc, j, g, bias);
  }
}

// gelu_new with the bias first: v = h + b; inner = f32(c * f32(v + f32(f32(f32(0.044715 * v) * v) * v)));
// out = f32(v / f32(1 + vexp(-2 * inner))); then quantize_x (rows of whole groups of 32: no scalar tail)
__global__ __launch_bounds__(256) void gelu_quant_kernel(int8_t *xq, float *xs, float *out, const float *h,
                                                         const float *b, int32_t m, int32_t n, int32_t h_stride,
                                                         int32_t xq_stride, int32_t xs_stride, int32_t bias) {
  const int groups = n / GS;
  const int64_t gid = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (gid >= (int64_t)m * groups) return;  // whole half-waves leave together
  const int t = (int)(gid / groups), g = (int)(gid % groups), j = g * GS + (threadIdx.x & 31);
  const float v = h[(int64_t)t * h_stride + j] + b[j];
  const float inner = 0.7978845608028654f * (v + ((0.044715f * v) * v) * v);
  const float o = v / (1.0f + vexp(-2.0f * inner));
  if (out) out[(int64_t)t * h_stride + j] = o;
  quantize_group(o, xq + (int64_t)t * xq_stride, xs + (int64_t)t * xs_stride, j, g, bias);
}

// x[t][j] = f32(x[t][j] + b[j])
__global__ __launch_bounds__(256) void add_rows_kernel(float *x, const float *b, int32_t n, int32_t stride) {
  const int t = blockIdx.y;
  for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
    float *p = x + (int64_t)t * stride + j;
    *p = *p + b[j];
  }
}

// Qwen3: every head of q and k (a wave each): + its bias where given, then rmsnorm over the head's hs values in place
// (four lanes over j % 4 from LDS, hsum ((l0 + l1) + l2) + l3, s = f32(1 / f32(sqrt(f32(ss / hs) + eps))),
// out = f32(w * f32(s * x))). Heads past the last keep to the barriers and do nothing.
__global__ __launch_bounds__(256) void head_norm_kernel(float *q, float *k, const float *bq, const float *bk,
                                                        const float *qw, const float *kw, int32_t nh, int32_t nkv,
                                                        int32_t hs, int32_t q_stride, int32_t kv_stride, float eps) {
  constexpr int RS = 64 + 1;  // a lane's row of squares (hs / 4 <= 64), padded off the next row's banks
  __shared__ float sq[4][4 * RS];
  __shared__ float part[4][4];
  const int t = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = blockIdx.x * 4 + wave;
  const bool live = h < nh + nkv;
  const bool isq = h < nh;
  float *x = nullptr;
  const float *bias = nullptr, *w = nullptr;
  if (live) {
    x = isq ? q + (int64_t)t * q_stride + (int64_t)h * hs : k + (int64_t)t * kv_stride + (int64_t)(h - nh) * hs;
    bias = isq ? (bq ? bq + (int64_t)h * hs : nullptr) : (bk ? bk + (int64_t)(h - nh) * hs : nullptr);
    w = isq ? qw : kw;
  }
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j = lane + 64 * u;
    if (live && j < hs) {
      float a = x[j];
      if (bias) a = a + bias[j];
      v[u] = a;
      sq[wave][(j & 3) * RS + (j >> 2)] = a * a;
    }
  }
  __syncthreads();
  if (live && lane < 4) {
    float acc = 0.0f;
    for (int i = 0; i < hs / 4; ++i) acc = acc + sq[wave][lane * RS + i];
    part[wave][lane] = acc;
  }
  __syncthreads();
  if (!live) return;
  const float ss = ((part[wave][0] + part[wave][1]) + part[wave][2]) + part[wave][3];
  const float s = 1.0f / __builtin_sqrtf(ss / (float)hs + eps);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j = lane + 64 * u;
    if (j < hs) x[j] = w[j] * (s * v[u]);
  }
}

// columns[i][v] = f32(weight(v, c_i) * its group's scale): the classifier's float32 column of each outlier channel
__global__ __launch_bounds__(256) void outlier_columns_kernel(float *columns, const uint8_t *table,
                                                              const float *scales, int32_t vocab, int32_t dim,
                                                              int32_t group, int32_t six, OutlierSet set) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= (int64_t)set.n * vocab) return;
  const int i = (int)(id / vocab), v = (int)(id % vocab);
  const int64_t at = (int64_t)v * dim + set.c[i];
  int32_t w;
  if (six) {
    const uint8_t *gb = table + (at >> 5) * 24;
    const int j = (int)(at & 31);
    const int low = j < 16 ? (gb[j] & 15) : (gb[j - 16] >> 4);
    const int top = (gb[16 + (j & 7)] >> (2 * (j >> 3))) & 3;
    w = (int8_t)(uint8_t)((low | (top << 4)) << 2);
  } else {
    w = (int8_t)table[at];
  }
  columns[id] = (float)w * scales[at / group];
}

// picked[i] = x[c_i]; x[c_i] = 0 (the channels are distinct)
__global__ void pick_kernel(float *x, float *picked, OutlierSet set) {
  if (threadIdx.x != 0) return;
  for (int i = 0; i < set.n; ++i) {
    picked[i] = x[set.c[i]];
    x[set.c[i]] = 0.0f;
  }
}

// y[v] = f32(... f32(y[v] + f32(a_0 * columns[0][v])) ... + f32(a_{n-1} * columns[n-1][v]))
__global__ __launch_bounds__(256) void add_columns_kernel(float *y, const float *columns, const float *a, int32_t n,
                                                          int32_t vocab) {
  const int v = blockIdx.x * 256 + threadIdx.x;
  if (v >= vocab) return;
  float acc = y[v];
  for (int c = 0; c < n; ++c) acc = acc + a[c] * columns[(int64_t)c * vocab + v];
  y[v] = acc;
}

}  // namespace

hipError_t launch_layernorm_quant(int8_t *xq, float *xs, float *out, float *copy, const float *x, const float *w,
                                  const float *b, int32_t m, int32_t n, int32_t x_stride, int32_t xq_stride,
                                  int32_t xs_stride, int32_t out_stride, int32_t bias, hipStream_t s) {
  if (n > 16384) return hipErrorInvalidValue;  // x and the lanes' rows stay within the block's LDS
  const size_t lds = sizeof(float) * (size_t)(n + 4 * chain_rowstride((n & ~3) >> 2) + 16);
  static bool sized = false;  // once a process: let the kernel take LDS past 64 KiB
  if (lds > 65536 && !sized) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&layernorm_quant_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
    if (e != hipSuccess) return e;
    sized = true;
  }
  const int split = m < 64 ? 4 : 1;
  hipLaunchKernelGGL(layernorm_quant_kernel, dim3(m, split), dim3(1024), lds, s, xq, xs, out, copy, x, w, b, n,
                     x_stride, xq_stride, xs_stride, out_stride, bias);
  return hipGetLastError();
}

hipError_t launch_gelu_quant(int8_t *xq, float *xs, float *out, const float *h, const float *b, int32_t m, int32_t n,
                             int32_t h_stride, int32_t xq_stride, int32_t xs_stride, int32_t bias, hipStream_t s) {
  const int64_t groups = (int64_t)m * (n / GS);
  hipLaunchKernelGGL(gelu_quant_kernel, dim3((unsigned)((groups + 7) / 8)), dim3(256), 0, s, xq, xs, out, h, b, m, n,
                     h_stride, xq_stride, xs_stride, bias);
  return hipGetLastError();
}

hipError_t launch_add_rows(float *x, const float *b, int32_t m, int32_t n, int32_t stride, hipStream_t s) {
  const int blocks = std::min(64, (n + 255) / 256);
  hipLaunchKernelGGL(add_rows_kernel, dim3(blocks, m), dim3(256), 0, s, x, b, n, stride);
  return hipGetLastError();
}

hipError_t launch_head_norm(float *q, float *k, const float *bq, const float *bk, const float *qw, const float *kw,
                            int32_t m, int32_t nh, int32_t nkv, int32_t hs, int32_t q_stride, int32_t kv_stride,
                            float eps, hipStream_t s) {
  if (hs > 256 || hs % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(head_norm_kernel, dim3((nh + nkv + 3) / 4, m), dim3(256), 0, s, q, k, bq, bk, qw, kw, nh, nkv, hs,
                     q_stride, kv_stride, eps);
  return hipGetLastError();
}

hipError_t launch_outlier_columns(float *columns, const uint8_t *table, const float *scales, int32_t vocab,
                                  int32_t dim, int32_t group, bool six, const OutlierSet &set, hipStream_t s) {
  const int64_t n = (int64_t)set.n * vocab;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(outlier_columns_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, columns, table,
                     scales, vocab, dim, group, (int32_t)six, set);
  return hipGetLastError();
}

hipError_t launch_pick(float *x, float *picked, const OutlierSet &set, hipStream_t s) {
  hipLaunchKernelGGL(pick_kernel, dim3(1), dim3(64), 0, s, x, picked, set);
  return hipGetLastError();
}

hipError_t launch_add_columns(float *y, const float *columns, const float *a, int32_t n, int32_t vocab, hipStream_t s) {
  hipLaunchKernelGGL(add_columns_kernel, dim3((vocab + 255) / 256), dim3(256), 0, s, y, columns, a, n, vocab);
  return hipGetLastError();
}

}  // namespace ple
