// attention.hip — causal grouped-query attention of m tokens (token t at position pos0 + t over the cache rows
// 0..pos0+t), to the bit of kernels/kernel.ts:448-566 attentionOf:
//   score = (l0 + l2) + (l1 + l3) of four lanes over j (q_j * k_j rounded, added in order), the tail added, times
//           isq = f32(1 / f32(sqrt(hs)));
//   softmax: the largest (order-free); e = vexp(s - max) for the positions below count & ~3, fexp past them; the sum
//           in four lanes (t % 4) in order, hsum ((l0 + l1) + l2) + l3, the tail added in order; p = e * f32(1 / sum);
//   out_j: blocks of four positions in order, out = out + ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)), then the positions past
//           the fours one at a time, out = out + p v.
// Three launches: (A) the scores of 64-position tiles, every CU streaming keys once for the nh / nkv query heads
// that share them, with each tile's maxima; (B) one block a (token, head): the exponentials, their ordered sum from
// LDS, the weights p written over the scores; (C) the weighted values: for a few tokens (decode) a ring of LDS slots
// that producer waves fill with the four-position products ahead of the wave that runs the ordered sums; for a prompt
// block, blocks of tokens that share the values they stage, a thread a (token, head, column) sum.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

namespace {

constexpr int TILE = 64;   // positions a block of (A)
constexpr int MAXMUL = 8;  // query heads a kv head at most
constexpr int PVJ = 8;     // columns a block of (C)
constexpr int RING_TOKENS = 8;  // up to this many tokens the weighted values run on the ring kernel (below)

template <bool HALF>
__device__ __forceinline__ float4 cache4(const void *c, int64_t i) {  // four values from element i (i % 4 == 0)
  if constexpr (HALF) {
    const uint2 h = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(c) + i);
    return make_float4(from_f16((uint16_t)(h.x & 0xffff)), from_f16((uint16_t)(h.x >> 16)),
                       from_f16((uint16_t)(h.y & 0xffff)), from_f16((uint16_t)(h.y >> 16)));
  } else {
    return *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(c) + i);
  }
}
template <bool HALF>
__device__ __forceinline__ float cache1(const void *c, int64_t i) {
  if constexpr (HALF) return from_f16(reinterpret_cast<const uint16_t *>(c)[i]);
  else return reinterpret_cast<const float *>(c)[i];
}

// (A) grid (tiles, nkv, m)
template <int HS, bool HALF>
__global__ __launch_bounds__(256) void scores_kernel(const AttnArgs a) {
  constexpr int LD = HS + 4, C4 = HS / 4;
  __shared__ float ks[TILE * LD];
  __shared__ float qs[MAXMUL * HS];
  const int tile = blockIdx.x, kh = blockIdx.y, t = blockIdx.z;
  const int count = a.pos0 + t + 1;
  const int p0 = tile * TILE;
  if (p0 >= count) return;
  const int kvdim = a.nkv * HS, mul = a.nh / a.nkv;
  const int np = min(TILE, count - p0);
  constexpr int NL = (TILE * C4 + 255) / 256;  // float4 of keys a thread, requested together
  float4 kr4[NL];
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int i = threadIdx.x + u * 256, p = min(i / C4, np - 1), c = i % C4;  // clamped, unconditional
    kr4[u] = cache4<HALF>(a.kcache, (int64_t)(p0 + p) * kvdim + kh * HS + 4 * c);
  }
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int i = threadIdx.x + u * 256, p = i / C4, c = i % C4;
    if (p < np) *reinterpret_cast<float4 *>(ks + p * LD + 4 * c) = kr4[u];
  }
  const float *q = a.q + (int64_t)t * a.q_stride + (int64_t)kh * mul * HS;
  for (int i = threadIdx.x; i < mul * C4; i += 256)
    *reinterpret_cast<float4 *>(qs + 4 * i) = *reinterpret_cast<const float4 *>(q + 4 * i);
  __syncthreads();
  const float isq = 1.0f / __builtin_sqrtf((float)HS);
  float *scores = a.scores + (int64_t)t * a.nh * a.seq_len;
  for (int idx = threadIdx.x; idx < mul * TILE; idx += 256) {
    const int hl = idx / TILE, p = idx % TILE;
    float sc = -__builtin_inff();
    if (p < np) {
      const float *kr = ks + p * LD, *qr = qs + hl * HS;
      float l0 = 0.0f, l1 = 0.0f, l2 = 0.0f, l3 = 0.0f;
#pragma unroll 8
      for (int j = 0; j < HS; j += 4) {
        const float4 kv = *reinterpret_cast<const float4 *>(kr + j);
        const float4 qv = *reinterpret_cast<const float4 *>(qr + j);
        l0 = l0 + qv.x * kv.x;
        l1 = l1 + qv.y * kv.y;
        l2 = l2 + qv.z * kv.z;
        l3 = l3 + qv.w * kv.w;
      }
      sc = ((l0 + l2) + (l1 + l3)) * isq;
      scores[(int64_t)(kh * mul + hl) * a.seq_len + p0 + p] = sc;
    }
    float mx = sc;  // the tile's largest of this head (a wave is one head's 64 positions)
    for (int o = 32; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (p == 0) a.tilemax[((int64_t)t * a.nh + kh * mul + hl) * (a.seq_len / TILE + 1) + tile] = mx;
  }
}

// (A) for many tokens (a prompt block): one block a (64-position tile, kv head, 32 / mul tokens): the tile's keys
// staged once in LDS for every (token, head) row of the block, 32 rows; wave w takes rows w, w + 4, ..., a lane one
// position, and runs the 8 rows' four lane sums side by side over the head (the keys read once for the 8). The
// rows' tile maxima by wave reductions.
constexpr int SROWS = 32;  // (token, head) rows a block

template <int HS, bool HALF>
__global__ __launch_bounds__(256) void scores_tokens_kernel(const AttnArgs a) {
  constexpr int LD = HS + 4, C4 = HS / 4;
  __shared__ float ks[TILE * LD];
  __shared__ float qs[SROWS * HS];
  const int tile = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mul = a.nh / a.nkv, tt_n = max(1, SROWS / mul);
  const int t0 = blockIdx.z * tt_n, last = min(t0 + tt_n, a.m) - 1;
  const int p0 = tile * TILE;
  if (p0 >= a.pos0 + last + 1) return;  // past every token of the block (uniform: before any barrier)
  const int kvdim = a.nkv * HS;
  const int np = min(TILE, a.pos0 + last + 1 - p0);  // positions any token of the block reaches
  // keys: TILE * C4 float4, and the rows' queries: SROWS * C4 float4, requested together (clamped, unconditional)
  constexpr int NK = TILE * C4 / 256, NQ = (SROWS * C4 + 255) / 256;
  float4 kr[NK], qr[NQ];
#pragma unroll
  for (int u = 0; u < NK; ++u) {
    const int i = tid + u * 256, p = min(i / C4, np - 1), c = i % C4;
    kr[u] = cache4<HALF>(a.kcache, (int64_t)(p0 + p) * kvdim + kh * HS + 4 * c);
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = min(tid + u * 256, SROWS * C4 - 1), r = i / C4, c = i % C4;
    const int t = min(t0 + r / mul, last), h = kh * mul + r % mul;
    qr[u] = *reinterpret_cast<const float4 *>(a.q + (int64_t)t * a.q_stride + (int64_t)h * HS + 4 * c);
  }
#pragma unroll
  for (int u = 0; u < NK; ++u) {
    const int i = tid + u * 256, p = i / C4, c = i % C4;
    *reinterpret_cast<float4 *>(ks + p * LD + 4 * c) = kr[u];
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = tid + u * 256;
    if (i < SROWS * C4) *reinterpret_cast<float4 *>(qs + 4 * i) = qr[u];
  }
  __syncthreads();
  const float isq = 1.0f / __builtin_sqrtf((float)HS);
  float l[8][4];
#pragma unroll
  for (int u = 0; u < 8; ++u) l[u][0] = l[u][1] = l[u][2] = l[u][3] = 0.0f;
  const float *kp = ks + lane * LD;
#pragma unroll 4
  for (int j = 0; j < HS; j += 4) {
    const float4 kv = *reinterpret_cast<const float4 *>(kp + j);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float4 qv = *reinterpret_cast<const float4 *>(qs + (wave + 4 * u) * HS + j);
      l[u][0] = l[u][0] + qv.x * kv.x;
      l[u][1] = l[u][1] + qv.y * kv.y;
      l[u][2] = l[u][2] + qv.z * kv.z;
      l[u][3] = l[u][3] + qv.w * kv.w;
    }
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int r = wave + 4 * u, tt = r / mul, hl = r % mul, t = t0 + tt;
    const bool row = tt < tt_n && t < a.m;  // uniform over the wave
    const int count = a.pos0 + min(t, a.m - 1) + 1;
    float sc = -__builtin_inff();
    if (row && p0 + lane < count) {
      sc = ((l[u][0] + l[u][2]) + (l[u][1] + l[u][3])) * isq;
      a.scores[((int64_t)t * a.nh + kh * mul + hl) * a.seq_len + p0 + lane] = sc;
    }
    float mx = sc;  // the tile's largest of this (token, head)
    for (int o = 32; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (row && lane == 0 && p0 < count) a.tilemax[((int64_t)t * a.nh + kh * mul + hl) * (a.seq_len / TILE + 1) + tile] = mx;
  }
}

// (B) one block a (head, token): grid (nh, m), block 256. The scores requested at once, the exponentials by every
// thread into LDS (lane k's positions t % 4 == k side by side), the four ordered sums by four threads, the weights.
__global__ __launch_bounds__(256) void softmax_kernel(const AttnArgs a) {
  extern __shared__ float e4[];  // 4 rows of q4s exponentials, then the tail
  __shared__ float part[4];
  __shared__ float shared_mx, shared_inv;
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const int count = a.pos0 + t + 1, count4 = count & ~3, q4 = count4 >> 2, q4s = (q4 + 3) & ~3;
  const int tiles = (count + TILE - 1) / TILE;
  float *scores = a.scores + ((int64_t)t * a.nh + h) * a.seq_len;
  const float *tm = a.tilemax + ((int64_t)t * a.nh + h) * (a.seq_len / TILE + 1);
  float sv[16];  // up to 16 scores a thread, requested with the tile maxima
#pragma unroll
  for (int u = 0; u < 16; ++u) sv[u] = scores[min(tid + 256 * u, count - 1)];  // clamped, unconditional
  if (tid < 64) {
    float mx = -3.4028234663852886e38f;
    for (int i = tid; i < tiles; i += 64) mx = wmax(mx, tm[i]);
    for (int o = 32; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (tid == 0) shared_mx = mx;
  }
  __syncthreads();
  const float mx = shared_mx;
  float *tail = e4 + 4 * q4s;
  for (int base = 0; base < count; base += 256 * 16) {
    if (base > 0) {
#pragma unroll
      for (int u = 0; u < 16; ++u) sv[u] = scores[min(base + tid + 256 * u, count - 1)];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int i = base + tid + 256 * u;
      if (i < count) {
        const float d = sv[u] - mx;
        if (i < count4) e4[(i & 3) * q4s + (i >> 2)] = vexp(d);
        else tail[i - count4] = fexp(d);
      }
    }
  }
  __syncthreads();
  if (tid < 4) part[tid] = lds_chain(e4 + tid * q4s, q4, 0.0f);
  __syncthreads();
  if (tid == 0) {
    float sum = ((part[0] + part[1]) + part[2]) + part[3];
    for (int i = 0; i < count - count4; ++i) sum = sum + tail[i];
    shared_inv = 1.0f / sum;
  }
  __syncthreads();
  const float inv = shared_inv;
  for (int i = tid; i < count; i += 256) {
    const float e = i < count4 ? e4[(i & 3) * q4s + (i >> 2)] : tail[i - count4];
    scores[i] = e * inv;
  }
}

// (C) for many tokens (a prompt block): one block of 256 threads a (kv head, 32 of its columns (16 where hs is not a
// multiple of 32), 256 / (columns * mul) tokens), a thread a (token, head, column) whose ordered sum over the
// four-position blocks it runs itself: out = out + ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)) from LDS, where 128-position
// chunks of the values (transposed: a column's positions side by side) and of the weights are staged, the next
// chunk's loads in flight meanwhile. The block's tokens share every value they read; each stops at its own last four.
constexpr int TPC = 128;  // positions a chunk

template <int HS, bool HALF>
__global__ __launch_bounds__(256) void pv_tokens_kernel(const AttnArgs a) {
  constexpr int COLS = HS % 32 == 0 ? 32 : 16;   // columns a block
  constexpr int ROWS = 256 / COLS;               // (token, head) weight rows a block at most
  constexpr int TVS = TPC + 4;                   // LDS row of a column's values (16 lanes' float4 on distinct banks)
  constexpr int VPT = TPC * (COLS / 4) / 256;    // float4 of values a thread a chunk
  constexpr int WPT = ROWS * (TPC / 4) / 256;    // float4 of weights a thread a chunk
  __shared__ float vs[2][COLS * TVS];  // [column][position]
  __shared__ float ps[2][ROWS * TPC];  // [token * mul + head][position]
  const int tid = threadIdx.x, kh = blockIdx.y;
  const int mul = a.nh / a.nkv, tt_n = max(1, ROWS / mul);
  const int j0 = blockIdx.x * COLS, t0 = blockIdx.z * tt_n;
  const int kvdim = a.nkv * HS;
  const int j = tid % COLS, hl = (tid / COLS) % mul, tt = tid / (COLS * mul);
  const bool chain = tt < tt_n && t0 + tt < a.m;
  const int t = min(t0 + tt, a.m - 1);
  const int count = a.pos0 + t + 1, count4 = count & ~3;
  const int last = min(t0 + tt_n, a.m) - 1;  // the block's last token reads the most positions
  const int most4 = (a.pos0 + last + 1) & ~3;
  const int chunks = (most4 + TPC - 1) / TPC;
  const int rows = (last - t0 + 1) * mul;  // weight rows of the block
  float4 v[VPT], w[WPT];
  // a chunk's loads, from clamped addresses (unconditional; what lies past a token's count4 is never added), and their
  // stores into LDS: written out as macros, so that v and w stay in registers
#define PVT_FETCH(c_)                                                                                             \
  do {                                                                                                            \
    _Pragma("unroll") for (int u = 0; u < VPT; ++u) {                                                             \
      const int i = tid + 256 * u, pos = min((c_) * TPC + i / (COLS / 4), most4 - 1), q = i % (COLS / 4);        \
      v[u] = cache4<HALF>(a.vcache, (int64_t)pos * kvdim + kh * HS + j0 + 4 * q);                                 \
    }                                                                                                             \
    _Pragma("unroll") for (int u = 0; u < WPT; ++u) {                                                             \
      const int i = tid + 256 * u;                                                                                \
      const int r = min(i / (TPC / 4), rows - 1), pos = min((c_) * TPC + 4 * (i % (TPC / 4)), most4 - 4);       \
      w[u] = *reinterpret_cast<const float4 *>(a.scores + ((int64_t)(t0 + r / mul) * a.nh + kh * mul + r % mul) * \
                                                              a.seq_len + pos);                                   \
    }                                                                                                             \
  } while (0)
#define PVT_STAGE(buf_)                                                                                           \
  do {                                                                                                            \
    _Pragma("unroll") for (int u = 0; u < VPT; ++u) {                                                             \
      const int i = tid + 256 * u, pl = i / (COLS / 4), q = i % (COLS / 4);                                       \
      float *col = vs[(buf_)] + (4 * q) * TVS + pl;                                                               \
      col[0] = v[u].x;                                                                                            \
      col[TVS] = v[u].y;                                                                                          \
      col[2 * TVS] = v[u].z;                                                                                      \
      col[3 * TVS] = v[u].w;                                                                                      \
    }                                                                                                             \
    _Pragma("unroll") for (int u = 0; u < WPT; ++u) {                                                             \
      reinterpret_cast<float4 *>(ps[(buf_)])[tid + 256 * u] = w[u]; /* every row, the block's or clamped copies */ \
    }                                                                                                             \
  } while (0)
  if (chunks > 0) {
    PVT_FETCH(0);
    PVT_STAGE(0);
  }
  __syncthreads();
  float acc = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    PVT_FETCH(c + 1);  // the next chunk's loads fly while this one is added (after the last: clamped, unused)
    const float *vc = vs[c & 1] + j * TVS;
    const float *prow = ps[c & 1] + (tt * mul + hl) * TPC;
    const int nb = chain ? max(0, min(TPC, count4 - c * TPC)) >> 2 : 0;
    for (int b = 0; b < nb; ++b) {
      const float4 pw = *reinterpret_cast<const float4 *>(prow + 4 * b);
      const float4 vv = *reinterpret_cast<const float4 *>(vc + 4 * b);
      acc = acc + ((pw.x * vv.x + pw.y * vv.y) + (pw.z * vv.z + pw.w * vv.w));
    }
    PVT_STAGE((c + 1) & 1);  // the other buffer: its last readers passed the previous barrier
    __syncthreads();
  }
#undef PVT_FETCH
#undef PVT_STAGE
  if (chain) {
    const float *pt = a.scores + ((int64_t)t * a.nh + kh * mul + hl) * a.seq_len;
    for (int p = count4; p < count; ++p) acc = acc + pt[p] * cache1<HALF>(a.vcache, (int64_t)p * kvdim + kh * HS + j0 + j);
    a.out[(int64_t)t * a.out_stride + (kh * mul + hl) * HS + j0 + j] = acc;
  }
}

// (C) for a few tokens (decode): one block of 256 threads a (token, kv head, 8 of the head's columns), after (B) has
// turned the scores into the weights p. Wave 0 runs the ordered sums of every (head, column); waves 1-3 each produce
// every 3rd chunk of 256 positions of what those sums add, the four-position products
// ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)), into a ring of LDS slots, as far ahead as the ring allows, with the loads of
// their next chunk in flight meanwhile. An LDS flag a slot says it is filled and a counter says how many chunks wave 0
// has added: no block-wide barrier a chunk. Every wait is on another wave of the same block, for a chunk of a lower
// index, so every wait ends.
constexpr int RP = 256, RB = RP / 4, RR = RB + 4;  // positions, four-position blocks, LDS row (floats) of a chunk
constexpr int NSLOT = 3;                           // ring slots
constexpr int SLOT = MAXMUL * PVJ * RR;            // floats a slot
constexpr int NPROD = 3;                           // producer waves

__device__ __forceinline__ int lds_load(const int *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void lds_store(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void wait_at_least(const int *p, int v) {
  while (lds_load(p) < v) __builtin_amdgcn_s_sleep(1);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <int HS, bool HALF>
__global__ __launch_bounds__(256) void pv_ring_kernel(const AttnArgs a) {
  __shared__ float ring[NSLOT * SLOT];
  __shared__ int filled[NSLOT], used;
  const int j0 = blockIdx.x * PVJ, kh = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int count = a.pos0 + t + 1, count4 = count & ~3;
  const int kvdim = a.nkv * HS, mul = a.nh / a.nkv;
  const float *weights = a.scores + (int64_t)t * a.nh * a.seq_len + (int64_t)kh * mul * a.seq_len;
  const int64_t vbase = (int64_t)kh * HS + j0;
  const int chunks = (count4 + RP - 1) / RP;

  if (tid < NSLOT) filled[tid] = 0;
  if (tid == NSLOT) used = 0;
  // wave 0, lane hl * 8 + j: the weights and values of the positions past the fours (at most 3), requested now and
  // used at the end
  float tp[3], tv[3];
  if (wave == 0) {
    const int hl = min(lane / PVJ, mul - 1), j = lane % PVJ;
#pragma unroll
    for (int r = 0; r < 3; ++r) {
      const int p = min(count4 + r, count - 1);
      tp[r] = weights[(int64_t)hl * a.seq_len + p];
      tv[r] = cache1<HALF>(a.vcache, (int64_t)p * kvdim + vbase + j);
    }
  }

  float acc = 0.0f;  // wave 0, lane hl * 8 + j
  // lane = the four-position block b of the chunk: its 4 value rows (8 columns) and every head's 4 weights; a
  // producer's first chunk is requested before the block's barrier
  float4 va[8], vn[8], pa[MAXMUL], pn[MAXMUL];
  auto fetch = [&](int c, float4 *v, float4 *pw) {
    const int p = min(c * RP + 4 * lane, count4 - 4);  // clamped: never added past count4
    const int64_t at = (int64_t)p * kvdim + vbase;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[2 * r] = cache4<HALF>(a.vcache, at + r * kvdim);
      v[2 * r + 1] = cache4<HALF>(a.vcache, at + r * kvdim + 4);
    }
#pragma unroll
    for (int hl = 0; hl < MAXMUL; ++hl)
      pw[hl] = *reinterpret_cast<const float4 *>(weights + (int64_t)min(hl, mul - 1) * a.seq_len + p);
  };
  if (wave > 0 && wave - 1 < chunks) fetch(wave - 1, va, pa);
  __syncthreads();
  if (wave > 0) {
    for (int c = wave - 1; c < chunks; c += NPROD) {
      if (c + NPROD < chunks) fetch(c + NPROD, vn, pn);  // the wave's next chunk flies meanwhile
      wait_at_least(&used, c - NSLOT + 1);                // the slot's last chunk has been added
      float *slot = ring + (c % NSLOT) * SLOT;
#pragma unroll
      for (int hl = 0; hl < MAXMUL; ++hl) {
        if (hl < mul) {
          const float p0 = pa[hl].x, p1 = pa[hl].y, p2 = pa[hl].z, p3 = pa[hl].w;
          float *row = slot + hl * PVJ * RR + lane;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float4 x0 = va[h], x1 = va[2 + h], x2 = va[4 + h], x3 = va[6 + h];
            row[(4 * h + 0) * RR] = (p0 * x0.x + p1 * x1.x) + (p2 * x2.x + p3 * x3.x);
            row[(4 * h + 1) * RR] = (p0 * x0.y + p1 * x1.y) + (p2 * x2.y + p3 * x3.y);
            row[(4 * h + 2) * RR] = (p0 * x0.z + p1 * x1.z) + (p2 * x2.z + p3 * x3.z);
            row[(4 * h + 3) * RR] = (p0 * x0.w + p1 * x1.w) + (p2 * x2.w + p3 * x3.w);
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) lds_store(&filled[c % NSLOT], c + 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) va[i] = vn[i];
#pragma unroll
      for (int hl = 0; hl < MAXMUL; ++hl) pa[hl] = pn[hl];
    }
  } else {
    for (int c = 0; c < chunks; ++c) {
      wait_at_least(&filled[c % NSLOT], c + 1);
      if (lane < mul * PVJ) {
        const int nb = min(RP, count4 - c * RP) >> 2;
        acc = lds_chain(ring + (c % NSLOT) * SLOT + lane * RR, nb, acc);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) lds_store(&used, c + 1);
    }
    if (lane < mul * PVJ) {
      const int hl = lane / PVJ, j = lane % PVJ;
#pragma unroll
      for (int r = 0; r < 3; ++r)
        if (r < count - count4) acc = acc + tp[r] * tv[r];
      a.out[(int64_t)t * a.out_stride + (kh * mul + hl) * HS + j0 + j] = acc;
    }
  }
}

template <int HS, bool HALF>
hipError_t launch_hs(const AttnArgs &a, hipStream_t s) {
  const int tiles = (a.pos0 + a.m + TILE - 1) / TILE;
  if (a.m <= RING_TOKENS) {
    hipLaunchKernelGGL((scores_kernel<HS, HALF>), dim3(tiles, a.nkv, a.m), dim3(256), 0, s, a);
  } else {
    const int tt = std::max(1, SROWS / (a.nh / a.nkv));
    hipLaunchKernelGGL((scores_tokens_kernel<HS, HALF>), dim3(tiles, a.nkv, (a.m + tt - 1) / tt), dim3(256), 0, s, a);
  }
  const int most4 = (a.pos0 + a.m) & ~3;
  const size_t lds_b = sizeof(float) * (size_t)(4 * ((most4 / 4 + 3) & ~3) + 4);
  hipLaunchKernelGGL(softmax_kernel, dim3(a.nh, a.m), dim3(256), lds_b, s, a);
  if (a.m <= RING_TOKENS) {
    hipLaunchKernelGGL((pv_ring_kernel<HS, HALF>), dim3(HS / PVJ, a.nkv, a.m), dim3(256), 0, s, a);
  } else {
    constexpr int COLS = HS % 32 == 0 ? 32 : 16;
    const int tt = std::max(1, 256 / COLS / (a.nh / a.nkv));
    hipLaunchKernelGGL((pv_tokens_kernel<HS, HALF>), dim3(HS / COLS, a.nkv, (a.m + tt - 1) / tt), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

template <bool HALF>
hipError_t launch_half(const AttnArgs &a, hipStream_t s) {
  switch (a.hs) {
    case 16: return launch_hs<16, HALF>(a, s);
    case 32: return launch_hs<32, HALF>(a, s);
    case 48: return launch_hs<48, HALF>(a, s);
    case 64: return launch_hs<64, HALF>(a, s);
    case 96: return launch_hs<96, HALF>(a, s);
    case 128: return launch_hs<128, HALF>(a, s);
    case 256: return launch_hs<256, HALF>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool attention_supported(int32_t hs, int32_t nh, int32_t nkv) {
  const bool sizes = hs == 16 || hs == 32 || hs == 48 || hs == 64 || hs == 96 || hs == 128 || hs == 256;
  return sizes && nkv > 0 && nh % nkv == 0 && nh / nkv <= MAXMUL;
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
  if (!attention_supported(a.hs, a.nh, a.nkv)) return hipErrorInvalidValue;
  return a.half ? launch_half<true>(a, s) : launch_half<false>(a, s);
}

}  // namespace ple
