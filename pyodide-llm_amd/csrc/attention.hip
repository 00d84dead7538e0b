// attention.hip — causal grouped-query attention of m tokens (token t at position pos0 + t over the cache rows
// 0..pos0+t), to the bit of kernels/kernel.ts:448-566 attentionOf:
//   score = (l0 + l2) + (l1 + l3) of four lanes over j (q_j * k_j rounded, added in order), the tail added, times
//           isq = f32(1 / f32(sqrt(hs)));
//   softmax: the largest (order-free); e = vexp(s - max) for the positions below count & ~3, fexp past them; the sum
//           in four lanes (t % 4) in order, hsum ((l0 + l1) + l2) + l3, the tail added in order; p = e * f32(1 / sum);
//   out_j: blocks of four positions in order, out = out + ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)), then the positions past
//           the fours one at a time, out = out + p v.
// Four launches, each wide over positions so that every CU streams the cache: (A) scores and per-tile maxima,
// (B) the softmax of each (token, head), (C) the four-position blocks of weighted values, (D) the ordered sums over
// the blocks. Keys and values are staged in LDS once per kv head for the nh / nkv query heads that share them.
#pragma clang fp contract(off)

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

namespace {

constexpr int TILE = 64;  // positions a block of (A) and (C)

__device__ __forceinline__ float cache_at(const void *c, int64_t i, int half) {
  return half ? from_f16(reinterpret_cast<const uint16_t *>(c)[i]) : reinterpret_cast<const float *>(c)[i];
}

// (A) grid (tiles, nkv, m)
__global__ __launch_bounds__(256) void scores_kernel(const AttnArgs a) {
  extern __shared__ float sm[];
  const int tile = blockIdx.x, kh = blockIdx.y, t = blockIdx.z;
  const int count = a.pos0 + t + 1;
  const int p0 = tile * TILE;
  if (p0 >= count) return;
  const int hs = a.hs, kvdim = a.nkv * hs, mul = a.nh / a.nkv, ld = hs + 4;
  float *ks = sm;                   // [TILE][hs + 4]
  float *qs = sm + TILE * ld;       // [mul][hs]
  const int np = min(TILE, count - p0);
  for (int i = threadIdx.x; i < np * hs; i += 256) {
    const int p = i / hs, j = i % hs;
    ks[p * ld + j] = cache_at(a.kcache, (int64_t)(p0 + p) * kvdim + kh * hs + j, a.half);
  }
  const float *q = a.q + (int64_t)t * a.q_stride + (int64_t)kh * mul * hs;
  for (int i = threadIdx.x; i < mul * hs; i += 256) qs[i] = q[i];
  __syncthreads();
  const float isq = 1.0f / __builtin_sqrtf((float)hs);
  const int hs4 = hs & ~3;
  float *scores = a.scores + (int64_t)t * a.nh * a.seq_len;
  for (int idx = threadIdx.x; idx < mul * TILE; idx += 256) {
    const int hl = idx / TILE, p = idx % TILE;
    float sc = -__builtin_inff();
    if (p < np) {
      const float *kr = ks + p * ld, *qr = qs + hl * hs;
      float l0 = 0.0f, l1 = 0.0f, l2 = 0.0f, l3 = 0.0f;
      int j = 0;
      for (; j < hs4; j += 4) {
        const float4 kv = *reinterpret_cast<const float4 *>(kr + j);
        const float4 qv = *reinterpret_cast<const float4 *>(qr + j);
        l0 = l0 + qv.x * kv.x;
        l1 = l1 + qv.y * kv.y;
        l2 = l2 + qv.z * kv.z;
        l3 = l3 + qv.w * kv.w;
      }
      sc = (l0 + l2) + (l1 + l3);
      for (; j < hs; ++j) sc = sc + qr[j] * kr[j];
      sc = sc * isq;
      scores[(int64_t)(kh * mul + hl) * a.seq_len + p0 + p] = sc;
    }
    // the tile's largest of this head: p runs over one wave's lanes when TILE == 64
    float mx = sc;
    for (int o = 32; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (p == 0) a.tilemax[((int64_t)t * a.nh + kh * mul + hl) * (a.seq_len / TILE + 1) + tile] = mx;
  }
}

// (B) one block a (head, token)
__global__ __launch_bounds__(256) void softmax_kernel(const AttnArgs a) {
  extern __shared__ float sm[];  // count4 exponentials, transposed: lane k's side by side
  __shared__ float part[4];
  __shared__ float shared_max, shared_inv;
  const int h = blockIdx.x, t = blockIdx.y;
  const int count = a.pos0 + t + 1, count4 = count & ~3, q4 = count4 >> 2;
  const int tiles = (count + TILE - 1) / TILE;
  float *scores = a.scores + ((int64_t)t * a.nh + h) * a.seq_len;
  const float *tm = a.tilemax + ((int64_t)t * a.nh + h) * (a.seq_len / TILE + 1);
  if (threadIdx.x < 64) {
    float mx = -3.4028234663852886e38f;
    for (int i = threadIdx.x; i < tiles; i += 64) mx = wmax(mx, tm[i]);
    for (int o = 32; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (threadIdx.x == 0) shared_max = mx;
  }
  __syncthreads();
  const float mx = shared_max;
  for (int i = threadIdx.x; i < count; i += 256) {
    const float d = scores[i] - mx;
    if (i < count4) {
      const float e = vexp(d);
      scores[i] = e;
      sm[(i & 3) * q4 + (i >> 2)] = e;
    } else {
      scores[i] = fexp(d);
    }
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    const float *c = sm + threadIdx.x * q4;
    float acc = 0.0f;
    int i = 0;
    if ((q4 & 3) == 0) {
      const float4 *c4 = reinterpret_cast<const float4 *>(c);
      for (; i < q4; i += 4) {
        const float4 v = c4[i >> 2];
        acc = acc + v.x;
        acc = acc + v.y;
        acc = acc + v.z;
        acc = acc + v.w;
      }
    }
    for (; i < q4; ++i) acc = acc + c[i];
    part[threadIdx.x] = acc;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = ((part[0] + part[1]) + part[2]) + part[3];
    for (int i = count4; i < count; ++i) sum = sum + scores[i];
    shared_inv = 1.0f / sum;
  }
  __syncthreads();
  const float inv = shared_inv;
  for (int i = threadIdx.x; i < count; i += 256) scores[i] = scores[i] * inv;
}

// (C) grid (tiles, nkv, m): block b of a head, (p0 v0 + p1 v1) + (p2 v2 + p3 v3), and the single products past the
// fours, into partial[t][h][b][j]
__global__ __launch_bounds__(256) void blocks_kernel(const AttnArgs a) {
  extern __shared__ float sm[];
  const int tile = blockIdx.x, kh = blockIdx.y, t = blockIdx.z;
  const int count = a.pos0 + t + 1, count4 = count & ~3;
  const int p0 = tile * TILE;
  if (p0 >= count) return;
  const int hs = a.hs, kvdim = a.nkv * hs, mul = a.nh / a.nkv;
  const int np = min(TILE, count - p0);
  float *vs = sm;               // [TILE][hs]
  float *ps = sm + TILE * hs;   // [mul][TILE]
  for (int i = threadIdx.x; i < np * hs; i += 256) {
    const int p = i / hs, j = i % hs;
    vs[p * hs + j] = cache_at(a.vcache, (int64_t)(p0 + p) * kvdim + kh * hs + j, a.half);
  }
  const float *scores = a.scores + (int64_t)t * a.nh * a.seq_len;
  for (int i = threadIdx.x; i < mul * TILE; i += 256) {
    const int hl = i / TILE, p = i % TILE;
    ps[i] = p < np ? scores[(int64_t)(kh * mul + hl) * a.seq_len + p0 + p] : 0.0f;
  }
  __syncthreads();
  const int nblocks = TILE / 4;
  const int64_t per_head = (int64_t)(a.seq_len / 4 + 4) * hs;
  for (int idx = threadIdx.x; idx < mul * nblocks * hs; idx += 256) {
    const int j = idx % hs, b = (idx / hs) % nblocks, hl = idx / (hs * nblocks);
    const int pb = p0 + 4 * b;  // the block's first position
    float *out = a.partial + ((int64_t)t * a.nh + kh * mul + hl) * per_head;
    const float *pp = ps + hl * TILE + 4 * b;
    const float *vv = vs + 4 * b * hs + j;
    if (pb + 4 <= count4) {
      const float pair0 = pp[0] * vv[0] + pp[1] * vv[hs];
      const float pair1 = pp[2] * vv[2 * hs] + pp[3] * vv[3 * hs];
      out[(int64_t)(pb >> 2) * hs + j] = pair0 + pair1;
    } else if (pb < count) {
      // positions past the fours: one product each, after the blocks (index count4 / 4 + i)
      for (int i = 0; i < 4; ++i)
        if (pb + i >= count4 && pb + i < count)
          out[(int64_t)((count4 >> 2) + (pb + i - count4)) * hs + j] = pp[i] * vv[i * hs];
    }
  }
}

// (D) one thread a (token, head, j): the blocks added in order, then the single products
__global__ __launch_bounds__(256) void chain_kernel(const AttnArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int hs = a.hs;
  if (idx >= (int64_t)a.m * a.nh * hs) return;
  const int j = (int)(idx % hs), h = (int)((idx / hs) % a.nh), t = (int)(idx / ((int64_t)hs * a.nh));
  const int count = a.pos0 + t + 1, count4 = count & ~3, nb = count4 >> 2;
  const int64_t per_head = (int64_t)(a.seq_len / 4 + 4) * hs;
  const float *pb = a.partial + ((int64_t)t * a.nh + h) * per_head + j;
  float acc = 0.0f;
  int b = 0;
  for (; b + 8 <= nb; b += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = pb[(int64_t)(b + i) * hs];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = acc + v[i];
  }
  for (; b < nb; ++b) acc = acc + pb[(int64_t)b * hs];
  for (int i = 0; i < count - count4; ++i) acc = acc + pb[(int64_t)(nb + i) * hs];
  a.out[(int64_t)t * a.out_stride + h * hs + j] = acc;
}

}  // namespace

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
  if (a.hs % 4 != 0 || a.nh % a.nkv != 0) return hipErrorInvalidValue;
  const int mul = a.nh / a.nkv;
  const int tiles = (a.pos0 + a.m + TILE - 1) / TILE;
  const size_t lds_a = sizeof(float) * (size_t)(TILE * (a.hs + 4) + mul * a.hs);
  hipLaunchKernelGGL(scores_kernel, dim3(tiles, a.nkv, a.m), dim3(256), lds_a, s, a);
  const int most = a.pos0 + a.m;
  const size_t lds_b = sizeof(float) * (size_t)(most & ~3);
  hipLaunchKernelGGL(softmax_kernel, dim3(a.nh, a.m), dim3(256), lds_b, s, a);
  const size_t lds_c = sizeof(float) * (size_t)(TILE * a.hs + mul * TILE);
  hipLaunchKernelGGL(blocks_kernel, dim3(tiles, a.nkv, a.m), dim3(256), lds_c, s, a);
  const int64_t threads = (int64_t)a.m * a.nh * a.hs;
  hipLaunchKernelGGL(chain_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace ple
