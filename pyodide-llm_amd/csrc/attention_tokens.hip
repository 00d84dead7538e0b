// attention_tokens.hip — the attention of a prompt block (many tokens a launch), to the bit of kernels/kernel.ts:448-566
// attentionOf in the order attention.hip states: (A) the scores of 64-position tiles for blocks of (token, head) rows
// that share each staged key tile, with each tile's maxima; (B) one block a (token, head) writing the weights p over
// the scores; (C) blocks of tokens that share the values they stage, a thread two (token, head, column) sums. (B) and
// (C) also take the decode launches whose context is past the decode kernels' LDS. In a file of their own, so that
// the decode kernels' code object does not change with them.
#pragma clang fp contract(off)

#include <algorithm>

#include "attention.hpp"

namespace ple {

namespace {

// (A) for many tokens (a prompt block): one block a (64-position tile, kv head, SR / mul tokens): the tile's keys
// staged once in LDS for every (token, head) row of the block, SR rows (64; 32 for head size 256). A lane takes two
// positions (2 pl, 2 pl + 1 of the tile) and the rows of its half-wave: wave w's half h takes rows
// w + 4 (u + RW h), u < RW = SR / 8, and runs their four lane sums for both positions side by side over the head
// (a query read serves two positions, a key read RW rows). The rows' tile maxima by half-wave reductions.
template <int HS> constexpr int scores_rows() { return HS <= 128 ? 32 : 16; }

template <int HS, bool HALF>
__global__ __launch_bounds__(256) void scores_tokens_kernel(const AttnArgs a) {
  constexpr int LD = HS + 4, C4 = HS / 4, SR = scores_rows<HS>(), RW = SR / 8;
  __shared__ float ks[TILE * LD];
  __shared__ float qs[SR * HS];
  const int tile = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, pl = lane & 31;
  const int mul = a.nh / a.nkv, tt_n = max(1, SR / mul);
  const int t0 = blockIdx.z * tt_n, last = min(t0 + tt_n, a.m) - 1;
  const int p0 = tile * TILE, pos0 = first_position(a);
  if (p0 >= pos0 + last + 1) return;  // past every token of the block (uniform: before any barrier)
  const int kvdim = a.nkv * HS;
  const int np = min(TILE, pos0 + last + 1 - p0);  // positions any token of the block reaches
  // keys: TILE * C4 float4, and the rows' queries: SR * C4 float4, requested together (clamped, unconditional)
  constexpr int NK = TILE * C4 / 256, NQ = (SR * C4 + 255) / 256;
  float4 kr[NK], qr[NQ];
#pragma unroll
  for (int u = 0; u < NK; ++u) {
    const int i = tid + u * 256, p = min(i / C4, np - 1), c = i % C4;
    kr[u] = cache4<HALF>(a.kcache, (int64_t)(p0 + p) * kvdim + kh * HS + 4 * c);
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = min(tid + u * 256, SR * C4 - 1), r = i / C4, c = i % C4;
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
    if (i < SR * C4) *reinterpret_cast<float4 *>(qs + 4 * i) = qr[u];
  }
  __syncthreads();
  const float isq = 1.0f / __builtin_sqrtf((float)HS);
  float l[2][RW][4];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int u = 0; u < RW; ++u) l[e][u][0] = l[e][u][1] = l[e][u][2] = l[e][u][3] = 0.0f;
  const float *kp0 = ks + (2 * pl) * LD, *kp1 = kp0 + LD;
  const float *qb = qs + (wave + 4 * RW * half) * HS;  // row u of the half-wave at qb + 4 u HS
#pragma unroll 4
  for (int j = 0; j < HS; j += 4) {
    const float4 k0 = *reinterpret_cast<const float4 *>(kp0 + j);
    const float4 k1 = *reinterpret_cast<const float4 *>(kp1 + j);
#pragma unroll
    for (int u = 0; u < RW; ++u) {
      const float4 qv = *reinterpret_cast<const float4 *>(qb + 4 * u * HS + j);
      l[0][u][0] = l[0][u][0] + qv.x * k0.x;
      l[0][u][1] = l[0][u][1] + qv.y * k0.y;
      l[0][u][2] = l[0][u][2] + qv.z * k0.z;
      l[0][u][3] = l[0][u][3] + qv.w * k0.w;
      l[1][u][0] = l[1][u][0] + qv.x * k1.x;
      l[1][u][1] = l[1][u][1] + qv.y * k1.y;
      l[1][u][2] = l[1][u][2] + qv.z * k1.z;
      l[1][u][3] = l[1][u][3] + qv.w * k1.w;
    }
  }
#pragma unroll
  for (int u = 0; u < RW; ++u) {
    const int r = wave + 4 * (u + RW * half), tt = r / mul, hl = r % mul, t = t0 + tt;
    const bool row = tt < tt_n && t < a.m;  // uniform over the half-wave
    const int count = first_position(a) + min(t, a.m - 1) + 1;
    float *srow = a.scores + ((int64_t)t * a.nh + kh * mul + hl) * a.seq_len;
    float mx = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int p = p0 + 2 * pl + e;
      if (row && p < count) {
        const float sc = ((l[e][u][0] + l[e][u][2]) + (l[e][u][1] + l[e][u][3])) * isq;
        srow[p] = sc;
        mx = wmax(mx, sc);
      }
    }
    // the tile's largest of this (token, head): the 32 lanes of the half-wave (xor offsets below 32 stay in it)
    for (int o = 16; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (row && pl == 0 && p0 < count) a.tilemax[((int64_t)t * a.nh + kh * mul + hl) * (a.seq_len / TILE + 1) + tile] = mx;
  }
}

// (B) one block a (head, token): grid (nh, m), block 256. The scores requested at once, the exponentials by every
// thread into LDS (lane k's positions t % 4 == k side by side), the four ordered sums by four threads, the weights.
__global__ __launch_bounds__(256) void softmax_kernel(const AttnArgs a) {
  extern __shared__ float e4[];  // 4 rows of q4s exponentials, then the tail
  __shared__ float part[4];
  __shared__ float shared_mx, shared_inv;
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const int count = first_position(a) + t + 1, count4 = count & ~3, q4 = count4 >> 2, q4s = chain_rowstride(q4);
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
      if (base + 256 * u < count) {  // the block's test first (a scalar branch): no exponentials past the count
        const int i = base + tid + 256 * u;
        if (i < count) {
          const float d = sv[u] - mx;
          if (i < count4) e4[(i & 3) * q4s + (i >> 2)] = vexp(d);
          else tail[i - count4] = fexp(d);
        }
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
// multiple of 32), 2 * 256 / (columns * mul) tokens), a thread two (token, head, column) ordered sums over the
// four-position blocks, run side by side (tokens tt and tt + 256 / (columns * mul) of the block, one value read for
// both): out = out + ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)) from LDS, where 128-position chunks of the values (a column's
// positions side by side, as the cache holds them) and of the weights are staged, the next chunk's loads in flight
// meanwhile. The block's tokens share every value they read; each stops at its own last four.
constexpr int TPC = 128;  // positions a chunk

template <int HS, bool HALF>
__global__ __launch_bounds__(256) void pv_tokens_kernel(const AttnArgs a) {
  constexpr int COLS = HS % 32 == 0 ? 32 : 16;   // columns a block
  constexpr int TROWS = 256 / COLS;              // (token, head) rows of one pass over the block's threads
  constexpr int ROWS = 2 * TROWS;                // weight rows a block at most: a thread runs two rows' sums
  constexpr int TVS = TPC + 4;                   // LDS row of a column's values (16 lanes' float4 on distinct banks)
  constexpr int VPT = TPC * (COLS / 4) / 256;    // float4 of values a thread a chunk
  constexpr int WPT = ROWS * (TPC / 4) / 256;    // float4 of weights a thread a chunk
  __shared__ float vs[2][COLS * TVS];  // [column][position]
  __shared__ float ps[2][ROWS * TPC];  // [token * mul + head][position]
  const int tid = threadIdx.x, kh = blockIdx.y;
  const int mul = a.nh / a.nkv, tt_n = max(1, TROWS / mul);  // tokens of one pass; the block takes two passes' worth
  const int j0 = blockIdx.x * COLS, t0 = blockIdx.z * 2 * tt_n;
  const int j = tid % COLS, hl = (tid / COLS) % mul, tt = tid / (COLS * mul);
  // the thread's two sums, tokens t0 + tt and t0 + tt + tt_n of the same head and column: two independent chains,
  // every value read serves both
  const bool in = tt < tt_n;
  const bool chain0 = in && t0 + tt < a.m, chain1 = in && t0 + tt + tt_n < a.m;
  const int ta = min(t0 + tt, a.m - 1), tb = min(t0 + tt + tt_n, a.m - 1);
  const int pos0 = first_position(a);
  const int count_a = pos0 + ta + 1, count4_a = count_a & ~3, count_b = pos0 + tb + 1, count4_b = count_b & ~3;
  const int last = min(t0 + 2 * tt_n, a.m) - 1;  // the block's last token reads the most positions
  const int most4 = (pos0 + last + 1) & ~3;
  const int chunks = (most4 + TPC - 1) / TPC;
  const int rows = (last - t0 + 1) * mul;  // weight rows of the block
  float4 v[VPT], w[WPT];
  // a chunk's loads, from clamped addresses (unconditional; what lies past a token's count4 is never added), and their
  // stores into LDS: written out as macros, so that v and w stay in registers
#define PVT_FETCH(c_)                                                                                             \
  do {                                                                                                            \
    _Pragma("unroll") for (int u = 0; u < VPT; ++u) {                                                             \
      const int i = tid + 256 * u, cc = i / (TPC / 4), pos = min((c_) * TPC + 4 * (i % (TPC / 4)), most4 - 4);   \
      v[u] = cache4<HALF>(a.vcache, (int64_t)(kh * HS + j0 + cc) * a.vstride + pos);                              \
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
      const int i = tid + 256 * u;                                                                                \
      *reinterpret_cast<float4 *>(vs[(buf_)] + (i / (TPC / 4)) * TVS + 4 * (i % (TPC / 4))) = v[u];               \
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
  float acc0 = 0.0f, acc1 = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    PVT_FETCH(c + 1);  // the next chunk's loads fly while this one is added (after the last: clamped, unused)
    const float *vc = vs[c & 1] + j * TVS;
    const float *pa = ps[c & 1] + (tt * mul + hl) * TPC;
    const float *pb = ps[c & 1] + ((tt + tt_n) * mul + hl) * TPC;
    const int na = chain0 ? max(0, min(TPC, count4_a - c * TPC)) >> 2 : 0;
    const int nb = chain1 ? max(0, min(TPC, count4_b - c * TPC)) >> 2 : 0;
    const int both = min(na, nb);
    int b = 0;
    for (; b < both; ++b) {
      const float4 vv = *reinterpret_cast<const float4 *>(vc + 4 * b);
      const float4 wa = *reinterpret_cast<const float4 *>(pa + 4 * b);
      const float4 wb = *reinterpret_cast<const float4 *>(pb + 4 * b);
      acc0 = acc0 + ((wa.x * vv.x + wa.y * vv.y) + (wa.z * vv.z + wa.w * vv.w));
      acc1 = acc1 + ((wb.x * vv.x + wb.y * vv.y) + (wb.z * vv.z + wb.w * vv.w));
    }
    for (int e = b; e < na; ++e) {  // the earlier token's own positions (only where the later one has no sum)
      const float4 vv = *reinterpret_cast<const float4 *>(vc + 4 * e);
      const float4 wa = *reinterpret_cast<const float4 *>(pa + 4 * e);
      acc0 = acc0 + ((wa.x * vv.x + wa.y * vv.y) + (wa.z * vv.z + wa.w * vv.w));
    }
    for (int e = b; e < nb; ++e) {  // the later token's positions past the earlier one's
      const float4 vv = *reinterpret_cast<const float4 *>(vc + 4 * e);
      const float4 wb = *reinterpret_cast<const float4 *>(pb + 4 * e);
      acc1 = acc1 + ((wb.x * vv.x + wb.y * vv.y) + (wb.z * vv.z + wb.w * vv.w));
    }
    PVT_STAGE((c + 1) & 1);  // the other buffer: its last readers passed the previous barrier
    __syncthreads();
  }
#undef PVT_FETCH
#undef PVT_STAGE
  const int64_t vcol = (int64_t)(kh * HS + j0 + j) * a.vstride;
  if (chain0) {
    const float *pt = a.scores + ((int64_t)ta * a.nh + kh * mul + hl) * a.seq_len;
    for (int p = count4_a; p < count_a; ++p) acc0 = acc0 + pt[p] * cache1<HALF>(a.vcache, vcol + p);
    a.out[(int64_t)ta * a.out_stride + (kh * mul + hl) * HS + j0 + j] = acc0;
  }
  if (chain1) {
    const float *pt = a.scores + ((int64_t)tb * a.nh + kh * mul + hl) * a.seq_len;
    for (int p = count4_b; p < count_b; ++p) acc1 = acc1 + pt[p] * cache1<HALF>(a.vcache, vcol + p);
    a.out[(int64_t)tb * a.out_stride + (kh * mul + hl) * HS + j0 + j] = acc1;
  }
}


template <int HS, bool HALF>
hipError_t scores_tokens_hs(const AttnArgs &a, hipStream_t s) {
  const int tiles = (a.pos0 + a.m + TILE - 1) / TILE;
  const int tt = std::max(1, scores_rows<HS>() / (a.nh / a.nkv));
  hipLaunchKernelGGL((scores_tokens_kernel<HS, HALF>), dim3(tiles, a.nkv, (a.m + tt - 1) / tt), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int HS, bool HALF>
hipError_t softmax_pv_hs(const AttnArgs &a, hipStream_t s) {
  const size_t lds_b = softmax_lds(a.pos0 + a.m);
  if (lds_b > (size_t)ALDS) return hipErrorInvalidValue;
  if (lds_b > 64 * 1024) {
    static bool sized = false;  // once a process: let the kernel take LDS past 64 KiB
    if (!sized) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&softmax_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, ALDS);
      if (e != hipSuccess) return e;
      sized = true;
    }
  }
  hipLaunchKernelGGL(softmax_kernel, dim3(a.nh, a.m), dim3(256), lds_b, s, a);
  constexpr int COLS = HS % 32 == 0 ? 32 : 16;
  const int tt = 2 * std::max(1, 256 / COLS / (a.nh / a.nkv));  // tokens a block: two sums a thread
  hipLaunchKernelGGL((pv_tokens_kernel<HS, HALF>), dim3(HS / COLS, a.nkv, (a.m + tt - 1) / tt), dim3(256), 0, s, a);
  return hipGetLastError();
}

// the head sizes the kernels take (attention_supported)
template <bool HALF>
hipError_t scores_tokens_by_hs(const AttnArgs &a, hipStream_t s) {
  switch (a.hs) {
    case 16: return scores_tokens_hs<16, HALF>(a, s);
    case 32: return scores_tokens_hs<32, HALF>(a, s);
    case 48: return scores_tokens_hs<48, HALF>(a, s);
    case 64: return scores_tokens_hs<64, HALF>(a, s);
    case 96: return scores_tokens_hs<96, HALF>(a, s);
    case 128: return scores_tokens_hs<128, HALF>(a, s);
    case 256: return scores_tokens_hs<256, HALF>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <bool HALF>
hipError_t softmax_pv_by_hs(const AttnArgs &a, hipStream_t s) {
  switch (a.hs) {
    case 16: return softmax_pv_hs<16, HALF>(a, s);
    case 32: return softmax_pv_hs<32, HALF>(a, s);
    case 48: return softmax_pv_hs<48, HALF>(a, s);
    case 64: return softmax_pv_hs<64, HALF>(a, s);
    case 96: return softmax_pv_hs<96, HALF>(a, s);
    case 128: return softmax_pv_hs<128, HALF>(a, s);
    case 256: return softmax_pv_hs<256, HALF>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

size_t softmax_lds(int count) { return sizeof(float) * (size_t)(4 * chain_rowstride((count & ~3) / 4) + 4); }

hipError_t launch_scores_tokens(const AttnArgs &a, hipStream_t s) {
  return a.half ? scores_tokens_by_hs<true>(a, s) : scores_tokens_by_hs<false>(a, s);
}

hipError_t launch_softmax_pv(const AttnArgs &a, hipStream_t s) {
  return a.half ? softmax_pv_by_hs<true>(a, s) : softmax_pv_by_hs<false>(a, s);
}

}  // namespace ple
