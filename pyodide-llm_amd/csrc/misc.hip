// misc.hip — the per-token elementwise work around the matmuls, each in the reference's float32 order:
//   quantize_x (kernels/kernel.ts:129-156), rmsnorm (:330-342) then quantize_x, swiglu (:654-667) then quantize_x,
//   embed (public/forward.js:962-973 with valueAt :692-696; GPT-2's positions added), the q/k/v bias add (:691-693,
//   public/forward.js:1038-1042), rope (:344-357, over the first `rot` values of each head) and the KV-cache write (to_f16 :570-599 or a copy, public/forward.js:998-1006), argmax (:695-699),
//   and the device twin of the oracle's synthetic checkpoint.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "l2fetch.hpp"

namespace ple {

namespace {

// the row stride of rmsnorm's four sums of squares in LDS: room for WAVE_CHAIN_MOST values where the wave's register
// chain takes them
__host__ __device__ constexpr int norm_rowstride(int q4) {
  return chain_rowstride(q4 <= WAVE_CHAIN_MOST ? WAVE_CHAIN_MOST : q4);
}

__global__ __launch_bounds__(256) void quantize_kernel(int8_t *xq, float *xs, const float *x, int32_t m, int32_t n,
                                                       int32_t x_stride, int32_t xq_stride, int32_t xs_stride,
                                                       int32_t bias) {
  const int groups = n / GS;
  const int64_t gid = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (gid >= (int64_t)m * groups) return;  // whole half-waves leave together
  const int t = (int)(gid / groups), g = (int)(gid % groups), j = g * GS + (threadIdx.x & 31);
  quantize_group(x[(int64_t)t * x_stride + j], xq + (int64_t)t * xq_stride, xs + (int64_t)t * xs_stride, j, g, bias);
}

// rmsnorm of one token a block: the squares in four lanes (j % 4) added in order by four threads, hsum
// ((l0 + l1) + l2) + l3, the tail in order; s = f32(1 / f32(sqrt(f32(ss / n) + eps))); out = w * (s * x); then
// quantize_x of out. x and w are staged in LDS first, so that no global load waits inside the ordered parts.
__global__ __launch_bounds__(1024) void rmsnorm_quant_kernel(int8_t *xq, float *xs, float *out, const float *x,
                                                            const float *w, int32_t n, int32_t x_stride,
                                                            int32_t xq_stride, int32_t xs_stride, int32_t out_stride,
                                                            float eps, int32_t bias, const L2Fetch f) {
  // the last f.blocks rows of blocks (one token) fill the next GEMV's L2 lines instead
  const int split = gridDim.y - f.blocks;
  if ((int)blockIdx.y >= split) {
    l2_fetch(f, blockIdx.y - split, blockIdx.y);
    return;
  }
  extern __shared__ float sm[];
  const int n4 = n & ~3, q4 = n4 >> 2, qs = norm_rowstride(q4);
  float *xv = sm;            // n
  float *wv = sm + n;        // n
  float *sq = sm + 2 * n;    // 4 * qs, transposed: lane k's squares side by side
  __shared__ float part[4];
  __shared__ float sval;
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *xt = x + (int64_t)t * x_stride;
  if ((n & 3) == 0 && n <= 8 * 1024) {
    // every load first (up to 2 float4 of x and of w a thread), then the stores
    float4 xr[2], wr[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j4 = min(tid + u * 1024, n / 4 - 1);  // clamped: the loads are unconditional, so none waits
      xr[u] = reinterpret_cast<const float4 *>(xt)[j4];
      wr[u] = reinterpret_cast<const float4 *>(w)[j4];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j4 = tid + u * 1024;
      if (j4 < n / 4) {
        const float4 v = xr[u];
        reinterpret_cast<float4 *>(xv)[j4] = v;
        reinterpret_cast<float4 *>(wv)[j4] = wr[u];
        sq[0 * qs + j4] = v.x * v.x;
        sq[1 * qs + j4] = v.y * v.y;
        sq[2 * qs + j4] = v.z * v.z;
        sq[3 * qs + j4] = v.w * v.w;
      }
    }
  } else {
    for (int j = tid; j < n; j += 1024) {
      const float v = xt[j];
      xv[j] = v;
      wv[j] = w[j];
      if (j < n4) sq[(j & 3) * qs + (j >> 2)] = v * v;
    }
  }
  if (q4 <= WAVE_CHAIN_MOST) {
    // the four sums from registers (waves 0 and 1): their rows padded with +0.0 to WAVE_CHAIN_MOST
    for (int j = q4 + tid; j < WAVE_CHAIN_MOST; j += 1024) {
#pragma unroll
      for (int k = 0; k < 4; ++k) sq[k * qs + j] = 0.0f;
    }
    __syncthreads();
    if (tid < 128) {
      const float sum = chain4_registers(sq, qs, tid);
      if ((tid & 31) == 31) part[tid >> 5] = sum;
    }
  } else {
    __syncthreads();
    if (tid < 4) part[tid] = lds_chain(sq + tid * qs, q4, 0.0f);
  }
  __syncthreads();
  if (tid == 0) {
    float ss = ((part[0] + part[1]) + part[2]) + part[3];
    for (int j = n4; j < n; ++j) ss = ss + xv[j] * xv[j];
    sval = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
  }
  __syncthreads();
  const float s = sval;
  int8_t *q = xq + (int64_t)t * xq_stride;
  float *sc = xs + (int64_t)t * xs_stride;
  // this block's share of the groups: gridDim.y blocks of a token each run the (short) sums themselves and quantize
  // every gridDim.y-th group, so that no one CU does all the divisions
  for (int g = (tid >> 5) * split + blockIdx.y; g < n / GS; g += 32 * split) {
    const int j = g * GS + (tid & 31);
    const float o = wv[j] * (s * xv[j]);
    if (out) out[(int64_t)t * out_stride + j] = o;
    quantize_group(o, q, sc, j, g, bias);
  }
}

// swiglu: h1 / (1 + vexp(-h1)) * h3 (the scalar tail's fexp gives the same bits), then quantize_x
__global__ __launch_bounds__(256) void swiglu_quant_kernel(int8_t *xq, float *xs, float *out, const float *h1,
                                                           const float *h3, int32_t m, int32_t n, int32_t h_stride,
                                                           int32_t xq_stride, int32_t xs_stride, int32_t bias) {
  const int groups = n / GS;
  const int64_t gid = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (gid >= (int64_t)m * groups) return;
  const int t = (int)(gid / groups), g = (int)(gid % groups), j = g * GS + (threadIdx.x & 31);
  const float v = h1[(int64_t)t * h_stride + j];
  const float o = v / (1.0f + vexp(-v)) * h3[(int64_t)t * h_stride + j];
  if (out) out[(int64_t)t * h_stride + j] = o;
  quantize_group(o, xq + (int64_t)t * xq_stride, xs + (int64_t)t * xs_stride, j, g, bias);
}

// quantize_x of one group of 32 held four values a lane by its 8 lanes (aligned, all present): the largest magnitude
// by the lanes' own maxima and three DPP steps (xor 1, xor 2, the mirror across the two quads), the scale and its
// reciprocal as quantize_group computes them, four bytes stored at xq[j..j+3]
__device__ __forceinline__ void quantize_group4(float4 o, int8_t *xq, float *xs, int j, int g, int32_t bias) {
  float a = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(o.x), __builtin_fabsf(o.y)),
                            __builtin_fmaxf(__builtin_fabsf(o.z), __builtin_fabsf(o.w)));
  a = __builtin_fmaxf(a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0xB1, 0xF, 0xF, true)));
  a = __builtin_fmaxf(a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x4E, 0xF, 0xF, true)));
  a = __builtin_fmaxf(a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x141, 0xF, 0xF, true)));
  const float qmax = bias == 0 ? 127.0f : 63.0f;
  const float scale = a / qmax;
  const float inv = scale > 0 ? 1.0f / scale : 0.0f;
  const uint32_t q = (uint32_t)(uint8_t)quant_value(o.x, inv, bias) | ((uint32_t)(uint8_t)quant_value(o.y, inv, bias) << 8) |
                     ((uint32_t)(uint8_t)quant_value(o.z, inv, bias) << 16) |
                     ((uint32_t)(uint8_t)quant_value(o.w, inv, bias) << 24);
  *reinterpret_cast<uint32_t *>(xq + j) = q;
  if ((threadIdx.x & 7) == 0) xs[g] = scale;
}

// rmsnorm + quantize_x of many tokens (a prompt pass), one token a block of 256 threads: the same steps and order as
// rmsnorm_quant_kernel, with each of the four ordered sums of squares in one wave's registers (lane s holds the sum's
// values 16 s .. 16 s + 15, zeros past the count; round s starts every lane from the running sum and hands lane s's
// result on as a scalar), so that eight tokens share a CU (the 1024-thread blocks of rmsnorm_quant_kernel left
// fourteen of their sixteen waves idle through the sums). Rows of whole groups of 32, at most 4096 values.
constexpr int RT_SEG = 16;              // values a lane of a sum
constexpr int RT_LANE = RT_SEG + 4;     // floats a lane's segment takes in LDS: 16-byte reads of 16 lanes on distinct banks
constexpr int RT_ROW = 64 * RT_LANE;    // floats a sum's row
constexpr int RT_MOST = 4 * 64 * RT_SEG;  // values a token at most
constexpr int RT_TOKENS = 8;            // tokens a launch from which rmsnorm_tokens_kernel takes it
__global__ __launch_bounds__(256) void rmsnorm_tokens_kernel(int8_t *xq, float *xs, float *out, const float *x,
                                                             const float *w, int32_t n, int32_t x_stride,
                                                             int32_t xq_stride, int32_t xs_stride, int32_t out_stride,
                                                             float eps, int32_t bias) {
  __shared__ float sq[4 * RT_ROW];
  __shared__ float part[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q4 = n >> 2, nseg = (q4 + RT_SEG - 1) / RT_SEG;
  const float4 *x4 = reinterpret_cast<const float4 *>(x + (int64_t)t * x_stride);
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  // float4 j4 = tid + 256 u of the token and of the weights, requested at once (clamped: loaded, never used past q4)
  float4 xr[4], wr[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j4 = min(tid + 256 * u, q4 - 1);
    xr[u] = x4[j4];
    wr[u] = w4[j4];
  }
  // the squares into the four sums' rows (sum k: x[4 j4 + k]^2 as its value j4), zeros up to the last whole segment
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j4 = tid + 256 * u, at = (j4 / RT_SEG) * RT_LANE + j4 % RT_SEG;
    if (j4 < q4) {
      sq[at] = xr[u].x * xr[u].x;
      sq[RT_ROW + at] = xr[u].y * xr[u].y;
      sq[2 * RT_ROW + at] = xr[u].z * xr[u].z;
      sq[3 * RT_ROW + at] = xr[u].w * xr[u].w;
    } else if (j4 < nseg * RT_SEG) {
#pragma unroll
      for (int k = 0; k < 4; ++k) sq[k * RT_ROW + at] = 0.0f;
    }
  }
  __syncthreads();
  {
    // wave k: sum k over its lanes' segments (lanes past the last read the first; what they add is never used)
    const float4 *seg = reinterpret_cast<const float4 *>(sq + wave * RT_ROW + (lane < nseg ? lane : 0) * RT_LANE);
    const float4 v0 = seg[0], v1 = seg[1], v2 = seg[2], v3 = seg[3];
    float run = 0.0f;
    for (int r = 0; r < nseg; ++r) {
      float acc = run;
      acc = acc + v0.x; acc = acc + v0.y; acc = acc + v0.z; acc = acc + v0.w;
      acc = acc + v1.x; acc = acc + v1.y; acc = acc + v1.z; acc = acc + v1.w;
      acc = acc + v2.x; acc = acc + v2.y; acc = acc + v2.z; acc = acc + v2.w;
      acc = acc + v3.x; acc = acc + v3.y; acc = acc + v3.z; acc = acc + v3.w;
      run = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), r));
    }
    if (lane == 0) part[wave] = run;
  }
  __syncthreads();
  // ((l0 + l1) + l2) + l3 (no tail: n % 4 == 0), s = f32(1 / f32(sqrt(f32(ss / n) + eps))), by every thread
  const float ss = ((part[0] + part[1]) + part[2]) + part[3];
  const float sv = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
  int8_t *q = xq + (int64_t)t * xq_stride;
  float *sc = xs + (int64_t)t * xs_stride;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j4 = tid + 256 * u;
    if (j4 < q4) {  // whole groups of 32: the 8 lanes of a group take this branch together
      const float4 o = make_float4(wr[u].x * (sv * xr[u].x), wr[u].y * (sv * xr[u].y), wr[u].z * (sv * xr[u].z),
                                   wr[u].w * (sv * xr[u].w));
      if (out) *reinterpret_cast<float4 *>(out + (int64_t)t * out_stride + 4 * j4) = o;
      quantize_group4(o, q, sc, 4 * j4, j4 >> 3, bias);
    }
  }
}

// the same as quantize_kernel four values a lane (rows whose strides keep the vectors aligned)
__global__ __launch_bounds__(256) void quantize4_kernel(int8_t *xq, float *xs, const float *x, int32_t m, int32_t n,
                                                        int32_t x_stride, int32_t xq_stride, int32_t xs_stride,
                                                        int32_t bias) {
  const int groups = n / GS;
  const int64_t gid = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (gid >= (int64_t)m * groups) return;  // whole 8-lane groups leave together
  const int t = (int)(gid / groups), g = (int)(gid % groups), j = g * GS + 4 * (threadIdx.x & 7);
  quantize_group4(*reinterpret_cast<const float4 *>(x + (int64_t)t * x_stride + j), xq + (int64_t)t * xq_stride,
                  xs + (int64_t)t * xs_stride, j, g, bias);
}

// swiglu_quant_kernel four values a lane (float4 loads, quantize_group4): a group's scale and its reciprocal are
// computed by 8 lanes instead of 32. For rows whose strides keep the vectors aligned (launch_swiglu_quant checks).
__global__ __launch_bounds__(256) void swiglu_quant4_kernel(int8_t *xq, float *xs, float *out, const float *h1,
                                                            const float *h3, int32_t m, int32_t n, int32_t h_stride,
                                                            int32_t xq_stride, int32_t xs_stride, int32_t bias) {
  const int groups = n / GS;
  const int64_t gid = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (gid >= (int64_t)m * groups) return;  // (whole 8-lane groups leave together)
  const int t = (int)(gid / groups), g = (int)(gid % groups), j = g * GS + 4 * (threadIdx.x & 7);
  const float4 v = *reinterpret_cast<const float4 *>(h1 + (int64_t)t * h_stride + j);
  const float4 w = *reinterpret_cast<const float4 *>(h3 + (int64_t)t * h_stride + j);
  float4 o;
  o.x = v.x / (1.0f + vexp(-v.x)) * w.x;
  o.y = v.y / (1.0f + vexp(-v.y)) * w.y;
  o.z = v.z / (1.0f + vexp(-v.z)) * w.z;
  o.w = v.w / (1.0f + vexp(-v.w)) * w.w;
  if (out) *reinterpret_cast<float4 *>(out + (int64_t)t * h_stride + j) = o;
  quantize_group4(o, xq + (int64_t)t * xq_stride, xs + (int64_t)t * xs_stride, j, g, bias);
}

// valueAt (public/forward.js:672-696): f32(int8 or unpacked int6 value * the scale of its group)
__device__ __forceinline__ float value_at(const uint8_t *table, const float *scales, int64_t at, int32_t group,
                                          int32_t six) {
  int32_t v;
  if (six) {
    const uint8_t *b = table + (at >> 5) * 24;
    const int j = (int)(at & 31);
    const int low = j < 16 ? (b[j] & 15) : (b[j - 16] >> 4);
    const int top = (b[16 + (j & 7)] >> (2 * (j >> 3))) & 3;
    v = (int8_t)(uint8_t)((low | (top << 4)) << 2);
  } else {
    v = (int8_t)table[at];
  }
  return (float)v * scales[at / group];
}

// embed: x_i = f32(int8 * scale of its group) for the token's row; GPT-2's position row (widened the same way) added
__global__ __launch_bounds__(256) void embed_kernel(float *x, const int32_t *tokens, const uint8_t *table,
                                                    const float *scales, int32_t dim, int32_t x_stride, int32_t group,
                                                    int32_t six, const Positions p) {
  const int t = blockIdx.y;
  const int64_t row = (int64_t)tokens[t] * dim;
  const int64_t prow = p.table ? (int64_t)((p.dpos ? *p.dpos : p.pos0) + t) * dim : 0;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < dim; i += gridDim.x * 256) {
    float v = value_at(table, scales, row + i, group, six);
    if (p.table) v = v + value_at(p.table, p.scales, prow + i, p.group, six);
    x[(int64_t)t * x_stride + i] = v;
  }
}

// per token: bias (q, k, v), rope on q and k at its position, k and v into the cache
__global__ __launch_bounds__(256) void qkv_post_kernel(const QkvPost a) {
  const int t = blockIdx.y;
  const int pos = (a.dpos ? *a.dpos : a.pos0) + t;
  const int qdim = a.nh * a.hs, kvdim = a.nkv * a.hs, half = a.hs / 2;
  float *q = a.q + (int64_t)t * a.q_stride, *k = a.k + (int64_t)t * a.kv_stride, *v = a.v + (int64_t)t * a.kv_stride;
  const float *cs = a.cos_t + (int64_t)pos * half, *sn = a.sin_t + (int64_t)pos * half;
  const int pairs = (qdim + kvdim) / 2;
  for (int p = blockIdx.x * 256 + threadIdx.x; p < pairs + kvdim; p += gridDim.x * 256) {
    if (p < pairs) {
      const bool isq = p < qdim / 2;
      float *base = isq ? q : k;
      const float *bias = isq ? a.bq : a.bk;
      const int i = 2 * (isq ? p : p - qdim / 2);  // the pair's first value
      float v0 = base[i], v1 = base[i + 1];
      if (bias) {
        v0 = v0 + bias[i];
        v1 = v1 + bias[i + 1];
      }
      float o0 = v0, o1 = v1;
      if (i % a.hs < a.rot) {
        const int ci = (i % a.hs) >> 1;
        const float c = cs[ci], s = sn[ci];
        o0 = v0 * c - v1 * s;
        o1 = v0 * s + v1 * c;
      }
      base[i] = o0;
      base[i + 1] = o1;
      if (!isq) {
        const int64_t at = (int64_t)pos * kvdim + i;
        if (a.half) {
          reinterpret_cast<uint16_t *>(a.kcache)[at] = to_f16(o0);
          reinterpret_cast<uint16_t *>(a.kcache)[at + 1] = to_f16(o1);
        } else {
          reinterpret_cast<float *>(a.kcache)[at] = o0;
          reinterpret_cast<float *>(a.kcache)[at + 1] = o1;
        }
      }
    } else {
      const int i = p - pairs;
      float o = v[i];
      if (a.bv) o = o + a.bv[i];
      v[i] = o;
      const int64_t at = (int64_t)i * a.vstride + pos;
      if (a.half) reinterpret_cast<uint16_t *>(a.vcache)[at] = to_f16(o);
      else reinterpret_cast<float *>(a.vcache)[at] = o;
    }
  }
}

// argmax, first of the largest: per block the best (value, index), then one block over the blocks; the host reports a
// winner that is not finite (NOT_FINITE)
// NumPy's argmax order (public/llama2_numpy.py:1521-1527): a NaN is the largest, the first of equals wins; on finite
// logits this is kernels/kernel.ts:695-699's first index of the largest
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  if (v != v) return bv == bv || i < bi;
  if (bv != bv) return false;
  return v > bv || (v == bv && i < bi);
}
__global__ __launch_bounds__(256) void argmax_stage(float *ov, int32_t *oi, const float *x, const int32_t *xi,
                                                    int32_t n) {
  __shared__ float sv[256];
  __shared__ int si[256];
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
    const float v = x[j];
    const int i = xi ? xi[j] : j;
    if (bi == 0x7fffffff || better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      const float v = sv[threadIdx.x + w];
      const int i = si[threadIdx.x + w];
      if (i != 0x7fffffff && (si[threadIdx.x] == 0x7fffffff || better(v, i, sv[threadIdx.x], si[threadIdx.x]))) {
        sv[threadIdx.x] = v;
        si[threadIdx.x] = i;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    ov[blockIdx.x] = sv[0];
    oi[blockIdx.x] = si[0];
  }
}

// ---- the device twin of the oracle's synthetic checkpoint (oracle/oracle.c or_synth_value, or_quantize,
// or_quantize6, or_pack6): a splitmix64 hash of (seed, stream, index), four 16-bit quarters summed, one float multiply
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}
__device__ __forceinline__ float synth_value(uint64_t key, uint64_t index, float factor) {
  const uint64_t r = mix64(key + index * 0x9E3779B97F4A7C15ull);
  const int32_t s = (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) +
                    (int32_t)(r >> 48);
  return (float)(s - 131070) * factor;
}

// one group of 32 a half-wave: the values, then quantize() (int8, scale f32(amax / 127)) or quantize6()+pack6()
__global__ __launch_bounds__(256) void synth_matrix_kernel(uint8_t *values, float *scales, int64_t groups,
                                                           uint64_t key, float factor, int32_t six) {
  const int64_t g = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (g >= groups) return;
  const int j = threadIdx.x & 31;
  const float v = synth_value(key, (uint64_t)(g * GS + j), factor);
  const float amax = wave_max32(__builtin_fabsf(v));
  if (!six) {
    const float scale = amax / 127.0f;
    const float inverse = scale > 0 ? 1.0f / scale : 0.0f;
    values[g * GS + j] = (uint8_t)(int8_t)__builtin_rintf(v * inverse);
    if (j == 0) scales[g] = scale;
    return;
  }
  const float scale = amax / 31.0f;
  const float inverse = scale > 0 ? 1.0f / scale : 0.0f;
  float r = __builtin_rintf(v * inverse);
  r = r < -32.0f ? -32.0f : (r > 31.0f ? 31.0f : r);
  const uint32_t b = (uint32_t)(((int32_t)r * 4) & 0xff) >> 2 & 63;  // the six bits
  // pack6: byte j (< 16) = low nibble of j | low nibble of j + 16 << 4; byte 16 + k = tops of k, k+8, k+16, k+24
  const uint32_t other = __shfl_xor(b, 16, 64);  // lane j < 16 gets value j + 16's bits
  uint8_t *o = values + g * 24;
  if (j < 16) o[j] = (uint8_t)((b & 15) | ((other & 15) << 4));
  const uint32_t t1 = __shfl(b, (threadIdx.x & 32) + (j & 7) + 8, 64);
  const uint32_t t2 = __shfl(b, (threadIdx.x & 32) + (j & 7) + 16, 64);
  const uint32_t t3 = __shfl(b, (threadIdx.x & 32) + (j & 7) + 24, 64);
  const uint32_t t0 = __shfl(b, (threadIdx.x & 32) + (j & 7), 64);
  if (j < 8) o[16 + j] = (uint8_t)((t0 >> 4) | ((t1 >> 4) << 2) | ((t2 >> 4) << 4) | ((t3 >> 4) << 6));
  if (j == 0) scales[g] = scale / 4.0f;
}

__global__ __launch_bounds__(256) void synth_vector_kernel(float *out, int64_t n, uint64_t key, float factor,
                                                           int32_t ones) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    out[i] = ones ? 1.0f : synth_value(key, (uint64_t)i, factor);
}

uint64_t synth_key(uint64_t seed, int32_t stream) {
  uint64_t z = seed * 0x9E3779B97F4A7C15ull ^ ((uint64_t)(uint32_t)stream * 0xD1B54A32D192ED03ull);
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}

int blocks_for(int64_t items, int64_t per_block, int64_t cap = 1 << 20) {
  int64_t b = (items + per_block - 1) / per_block;
  if (b < 1) b = 1;
  return (int)(b > cap ? cap : b);
}

}  // namespace

hipError_t launch_quantize(int8_t *xq, float *xs, const float *x, int32_t m, int32_t n, int32_t x_stride,
                           int32_t xq_stride, int32_t xs_stride, int32_t bias, hipStream_t s) {
  const int64_t groups = (int64_t)m * (n / GS);
  const bool aligned = x_stride % 4 == 0 && xq_stride % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(xq) % 4 == 0;
  if (aligned)
    hipLaunchKernelGGL(quantize4_kernel, dim3(blocks_for(groups, 32)), dim3(256), 0, s, xq, xs, x, m, n, x_stride,
                       xq_stride, xs_stride, bias);
  else
    hipLaunchKernelGGL(quantize_kernel, dim3(blocks_for(groups, 8)), dim3(256), 0, s, xq, xs, x, m, n, x_stride,
                       xq_stride, xs_stride, bias);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_quant(int8_t *xq, float *xs, float *out, const float *x, const float *w, int32_t m,
                                int32_t n, int32_t x_stride, int32_t xq_stride, int32_t xs_stride, int32_t out_stride,
                                float eps, int32_t bias, hipStream_t s, const L2Fetch *fetch) {
  const bool aligned = x_stride % 4 == 0 && xq_stride % 4 == 0 && (!out || out_stride % 4 == 0) &&
                       reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(xq) % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
  if (m >= RT_TOKENS && n % GS == 0 && n <= RT_MOST && aligned) {
    hipLaunchKernelGGL(rmsnorm_tokens_kernel, dim3(m), dim3(256), 0, s, xq, xs, out, x, w, n, x_stride, xq_stride,
                       xs_stride, out_stride, eps, bias);
    return hipGetLastError();
  }
  const size_t lds = sizeof(float) * (size_t)(2 * n + 4 * norm_rowstride((n & ~3) >> 2) + 16);
  // one token: 4 blocks share its groups (more tokens fill the chip by themselves)
  const int split = m < 64 ? 4 : 1;
  const L2Fetch f = fetch && m == 1 ? *fetch : L2Fetch{};
  hipLaunchKernelGGL(rmsnorm_quant_kernel, dim3(m, split + f.blocks), dim3(1024), lds, s, xq, xs, out, x, w, n,
                     x_stride, xq_stride, xs_stride, out_stride, eps, bias, f);
  return hipGetLastError();
}

hipError_t launch_swiglu_quant(int8_t *xq, float *xs, float *out, const float *h1, const float *h3, int32_t m,
                               int32_t n, int32_t h_stride, int32_t xq_stride, int32_t xs_stride, int32_t bias,
                               hipStream_t s) {
  const int64_t groups = (int64_t)m * (n / GS);
  const bool aligned = h_stride % 4 == 0 && xq_stride % 4 == 0 && reinterpret_cast<uintptr_t>(h1) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(h3) % 16 == 0 && reinterpret_cast<uintptr_t>(xq) % 4 == 0 &&
                       (!out || reinterpret_cast<uintptr_t>(out) % 16 == 0);
  if (aligned)
    hipLaunchKernelGGL(swiglu_quant4_kernel, dim3(blocks_for(groups, 32)), dim3(256), 0, s, xq, xs, out, h1, h3, m, n,
                       h_stride, xq_stride, xs_stride, bias);
  else
    hipLaunchKernelGGL(swiglu_quant_kernel, dim3(blocks_for(groups, 8)), dim3(256), 0, s, xq, xs, out, h1, h3, m, n,
                       h_stride, xq_stride, xs_stride, bias);
  return hipGetLastError();
}

hipError_t launch_embed(float *x, const int32_t *tokens, const uint8_t *table, const float *scales, int32_t m,
                        int32_t dim, int32_t x_stride, int32_t group, bool six, const Positions &positions,
                        hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(blocks_for(dim, 256, 64), m), dim3(256), 0, s, x, tokens, table, scales, dim,
                     x_stride, group, (int32_t)six, positions);
  return hipGetLastError();
}

hipError_t launch_qkv_post(const QkvPost &a, hipStream_t s) {
  const int64_t items = (int64_t)(a.nh * a.hs + a.nkv * a.hs) / 2 + a.nkv * a.hs;
  hipLaunchKernelGGL(qkv_post_kernel, dim3(blocks_for(items, 256, 64), a.m), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_argmax(int32_t *out, float *value, const float *x, int32_t n, float *scratch_v, int32_t *scratch_i,
                         hipStream_t s) {
  const int blocks = 256;
  hipLaunchKernelGGL(argmax_stage, dim3(blocks), dim3(256), 0, s, scratch_v, scratch_i, x, (const int32_t *)nullptr,
                     n);
  hipLaunchKernelGGL(argmax_stage, dim3(1), dim3(256), 0, s, value, out, (const float *)scratch_v,
                     (const int32_t *)scratch_i, blocks);
  return hipGetLastError();
}

hipError_t launch_synth_matrix(uint8_t *values, float *scales, int64_t rows, int32_t k, uint64_t seed, int32_t stream,
                               float factor, bool six, hipStream_t s) {
  const int64_t groups = rows * (k / GS);
  hipLaunchKernelGGL(synth_matrix_kernel, dim3(blocks_for(groups, 8, 1ll << 31)), dim3(256), 0, s, values, scales,
                     groups, synth_key(seed, stream), factor, (int32_t)six);
  return hipGetLastError();
}

hipError_t launch_synth_vector(float *out, int64_t n, uint64_t seed, int32_t stream, float factor, bool ones,
                               hipStream_t s) {
  hipLaunchKernelGGL(synth_vector_kernel, dim3(blocks_for(n, 256, 4096)), dim3(256), 0, s, out, n,
                     synth_key(seed, stream), factor, (int32_t)ones);
  return hipGetLastError();
}

}  // namespace ple
