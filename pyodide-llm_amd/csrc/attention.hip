// attention.hip — causal grouped-query attention of m tokens (token t at position pos0 + t over the cache rows
// 0..pos0+t), to the bit of kernels/kernel.ts:448-566 attentionOf:
//   score = (l0 + l2) + (l1 + l3) of four lanes over j (q_j * k_j rounded, added in order), the tail added, times
//           isq = f32(1 / f32(sqrt(hs)));
//   softmax: the largest (order-free); e = vexp(s - max) for the positions below count & ~3, fexp past them; the sum
//           in four lanes (t % 4) in order, hsum ((l0 + l1) + l2) + l3, the tail added in order; p = e * f32(1 / sum);
//   out_j: blocks of four positions in order, out = out + ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)), then the positions past
//           the fours one at a time, out = out + p v.
// The keys lie as the positions' rows ([seq_len][kv_dim]), the values as the columns' runs of positions
// ([kv_dim][vstride]). Launches: (A) the scores of 64-position tiles, every CU streaming keys once for the nh / nkv
// query heads that share them, with each tile's maxima; then for a few tokens (decode) one launch (B + C) a
// (token, head, 16 or 32 columns): the exponentials, their ordered sum, and the weighted values. A prompt block's
// scores, and the separate softmax and weighted values of prompt blocks and of contexts past these kernels' LDS, are
// attention_tokens.hip's.
#pragma clang fp contract(off)

#include <algorithm>

#include "attention.hpp"

namespace ple {

namespace {

// (A) grid (tiles, nkv, m)
template <int HS, bool HALF>
__global__ __launch_bounds__(256) void scores_kernel(const AttnArgs a) {
  constexpr int LD = HS + 4, C4 = HS / 4;
  __shared__ float ks[TILE * LD];
  __shared__ float qs[MAXMUL * HS];
  const int tile = blockIdx.x, kh = blockIdx.y, t = blockIdx.z;
  const int count = first_position(a) + t + 1;
  const int p0 = tile * TILE;
  if (p0 >= count) return;
  const int kvdim = a.nkv * HS, mul = a.nh / a.nkv;
  const int np = min(TILE, count - p0);
  constexpr int NL = (TILE * C4 + 255) / 256;  // float4 of keys a thread, requested together
  constexpr int NQ = (MAXMUL * C4 + 255) / 256;  // float4 of the queries a thread, requested with them
  const float *q = a.q + (int64_t)t * a.q_stride + (int64_t)kh * mul * HS;
  float4 qr[NQ];
#pragma unroll
  for (int u = 0; u < NQ; ++u) qr[u] = *reinterpret_cast<const float4 *>(q + 4 * min((int)threadIdx.x + u * 256, mul * C4 - 1));
  float4 kr4[NL];
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int i = threadIdx.x + u * 256, p = min(i / C4, np - 1), c = i % C4;  // clamped, unconditional
    kr4[u] = cache4<HALF>(a.kcache, (int64_t)(p0 + p) * kvdim + kh * HS + 4 * c);
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = threadIdx.x + u * 256;
    if (i < mul * C4) *reinterpret_cast<float4 *>(qs + 4 * i) = qr[u];
  }
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int i = threadIdx.x + u * 256, p = i / C4, c = i % C4;
    if (p < np) *reinterpret_cast<float4 *>(ks + p * LD + 4 * c) = kr4[u];
  }
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

// (B + C) for a few tokens (decode), in one launch: one block a (token, query head, 32 of the head's columns: one
// quantization group, 16 where the head size is not a multiple of 32). The block requests everything it reads at
// once: the head's tile maxima (wave 0), its scores (every thread), the producer waves' first value chunks and the
// tail values (wave 0). Then the exponentials go into LDS (lane k's positions t % 4 == k side by side), four lanes of
// wave 0 run the ordered sums and the block has f32(1 / sum); then the producer waves each turn every NP-th item (a
// chunk of 256 positions and 16 columns, the next two requested ahead) into the four-position products ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)),
// p = e * f32(1 / sum), in a ring of LDS slots, and wave 0's first lanes add them in order, a lane a column. An LDS flag
// a (slot, half) says it is filled and a counter says how many chunks wave 0 has added; every wait is on another wave
// of the block for a chunk of a lower index, so every wait ends. With a whole group, wave 0 also runs quantize_x on
// its 32 sums (the output projection's activations, no launch of their own).
// The blocks of the nh / nkv heads that share a kv head's columns are dealt to one XCD (the hardware deals blocks to
// the 8 XCDs in turn), so that the values they all read come from that XCD's L2 after the first.
constexpr int RP = 256, RB = RP / 4, RR = RB + 4;  // positions, four-position blocks, LDS row (floats) of a chunk
constexpr int ASLOTS = 8;                   // ring slots at most

template <int HS> struct Attend {
  static constexpr int AC = HS % 32 == 0 ? 32 : 16;  // columns a block
  static constexpr int H = AC / 16;                   // 16-column items a chunk
  static constexpr int NT = 512;                      // threads a block
  static constexpr int NP = NT / 64 - 1;              // producer waves
  static constexpr int SV = 16;                       // scores a thread a pass (8192 positions)
};

__device__ __forceinline__ int lds_load(const int *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void lds_store(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void wait_at_least(const int *p, int v) {
  while (lds_load(p) < v) __builtin_amdgcn_s_sleep(1);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// an item's values: lane = four-position block, one float4 of positions a column of the item's 16 (clamped: never
// added past count4)
#define ATT_FETCH(item, v)                                                                                    \
  {                                                                                                           \
    const int64_t at_ = vcol + (int64_t)((item) % H * 16) * a.vstride + min((item) / H * RP + 4 * lane, count4 - 4); \
    _Pragma("unroll") for (int j_ = 0; j_ < 16; ++j_) v[j_] = cache4<HALF>(a.vcache, at_ + (int64_t)j_ * a.vstride); \
  }

template <int HS, bool HALF>
__global__ __launch_bounds__(Attend<HS>::NT) void attend_kernel(const AttnArgs a, const int nslot) {
  using P = Attend<HS>;
  constexpr int AC = P::AC, H = P::H, NT = P::NT, NP = P::NP, ASV = P::SV;
  extern __shared__ float4 lds4[];
  float *const lds = reinterpret_cast<float *>(lds4);
  __shared__ float shared_mx, shared_inv;
  __shared__ int filled[ASLOTS][H], used;
  constexpr int S = HS / AC;  // column slices a kv head
  const int mul = a.nh / a.nkv, groups = a.nkv * S;
  const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3, hl = idx % mul, g = (idx / mul) * 8 + xcd;
  if (g >= groups) return;  // the grid's rounding up: whole blocks leave
  const int kh = g / S, j0 = (g % S) * AC, h = kh * mul + hl;
  const int t = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, pw = wave - 1;
  const int count = first_position(a) + t + 1, count4 = count & ~3, q4 = count4 >> 2, rs = chain_rowstride(q4);
  float *const e4 = lds;              // [4][rs]
  float *const tail = lds + 4 * rs;   // [4]
  float *const ring = tail + 4;       // [nslot][AC][RR]
  const float *sc = a.scores + ((int64_t)t * a.nh + h) * a.seq_len;
  const int64_t vcol = (int64_t)(kh * HS + j0) * a.vstride;  // the block's first value column
  const int chunks = (count4 + RP - 1) / RP, items = chunks * H;

  if (tid < ASLOTS * H) filled[tid / H][tid % H] = 0;
  if (tid == ASLOTS * H) used = 0;
  // every load of the block, requested before anything waits: tile maxima, scores, values
  const int tiles = (count + TILE - 1) / TILE;
  const float *tm = a.tilemax + ((int64_t)t * a.nh + h) * (a.seq_len / TILE + 1);
  float tmr[2];
  if (wave == 0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) tmr[u] = tm[min(lane + 64 * u, tiles - 1)];  // clamped: a repeat changes no max
  }
  float sv[ASV];
#pragma unroll
  for (int u = 0; u < ASV; ++u) sv[u] = sc[min(tid + NT * u, count - 1)];
  float4 va[16], vn[16];  // a producer's next two items
  if (wave > 0 && pw < items) ATT_FETCH(pw, va);
  if (wave > 0 && pw + NP < items) ATT_FETCH(pw + NP, vn);
  float tv[3];  // wave 0, lane j < AC: column j's values past the fours (at most 3)
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 3; ++r)
      tv[r] = cache1<HALF>(a.vcache, vcol + (int64_t)(lane % AC) * a.vstride + min(count4 + r, count - 1));
  }
  if (wave == 0) {
    float mx = wmax(tmr[0], tmr[1]);
    for (int i = lane + 128; i < tiles; i += 64) mx = wmax(mx, tm[i]);  // past 8192 positions
    for (int o = 32; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) shared_mx = mx;
  }
  __syncthreads();
  const float mx = shared_mx;
  for (int base = 0; base < count; base += NT * ASV) {
    if (base > 0) {
#pragma unroll
      for (int u = 0; u < ASV; ++u) sv[u] = sc[min(base + tid + NT * u, count - 1)];
    }
#pragma unroll
    for (int u = 0; u < ASV; ++u) {
      // the block's test first (the same for every thread: a scalar branch), so that no wave runs the exponentials
      // of positions past the count with its lanes switched off
      if (base + NT * u < count) {
        const int i = base + tid + NT * u;
        if (i < count) {
          const float d = sv[u] - mx;
          if (i < count4) e4[(i & 3) * rs + (i >> 2)] = vexp(d);
          else tail[i - count4] = fexp(d);
        }
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
    // lanes 0-3: lane k's sum; ((l0 + l1) + l2) + l3, the tail in order, 1 / sum
    const float part = lane < 4 ? lds_chain(e4 + lane * rs, q4, 0.0f) : 0.0f;
    const float c1 = __shfl(part, 1, 64), c2 = __shfl(part, 2, 64), c3 = __shfl(part, 3, 64);
    if (lane == 0) {
      float sum = ((part + c1) + c2) + c3;
      for (int r = 0; r < count - count4; ++r) sum = sum + tail[r];
      shared_inv = 1.0f / sum;
    }
  }
  __syncthreads();
  const float inv = shared_inv;
  if (wave > 0) {
    for (int it = pw; it < items; it += NP) {
      const int c = it / H, half = it % H;
      wait_at_least(&used, c - nslot + 1);  // the slot's last chunk has been added
      float *slot = ring + (c % nslot) * (AC * RR) + half * 16 * RR + lane;
      const int b = min(c * RB + lane, q4 - 1);  // the lane's four-position block (clamped: never added past q4)
      const float p0 = e4[b] * inv, p1 = e4[rs + b] * inv, p2 = e4[2 * rs + b] * inv, p3 = e4[3 * rs + b] * inv;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float4 x = va[j];
        slot[j * RR] = (p0 * x.x + p1 * x.y) + (p2 * x.z + p3 * x.w);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) lds_store(&filled[c % nslot][half], c + 1);
#pragma unroll
      for (int j = 0; j < 16; ++j) va[j] = vn[j];
      if (it + 2 * NP < items) ATT_FETCH(it + 2 * NP, vn);  // in flight while the wave waits
    }
  } else {
    // lane j < AC: column j0 + j (lanes past AC repeat column AC - 1 and store nothing). Chunks in pairs, two
    // register sets: chunk c + 1 is requested (after its flags) before chunk c's adds, which hide its latency. The
    // slot of c + 1 is free once c - 1 is released, so waiting for c + 1 before releasing c needs nslot >= 2.
    float acc = 0.0f;
    const int lr = min(lane, AC - 1);
    float4 xa[RB / 4], xb[RB / 4];
    auto ready = [&](int c) {  // every half of chunk c filled: the flags requested together, then one wait
      const int *f = filled[c % nslot];
      for (;;) {
        int least = lds_load(f);
#pragma unroll
        for (int hh = 1; hh < H; ++hh) least = min(least, lds_load(f + hh));
        if (least >= c + 1) break;
        __builtin_amdgcn_s_sleep(1);
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    };
    auto fetch = [&](int c, float4 (&x)[RB / 4]) {
      const float4 *row = reinterpret_cast<const float4 *>(ring + (c % nslot) * (AC * RR) + lr * RR);
#pragma unroll
      for (int u = 0; u < RB / 4; ++u) x[u] = row[u];
    };
    auto consume = [&](int c, const float4 (&x)[RB / 4]) {
      const int nb = min(RP, count4 - c * RP) >> 2;
      if (nb == RB) {
        acc = add32(acc, x);
        acc = add32(acc, x + 8);
      } else {  // the last chunk, part full: from LDS
        acc = lds_chain(ring + (c % nslot) * (AC * RR) + lr * RR, nb, acc);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) lds_store(&used, c + 1);
    };
    if (chunks > 0) {
      ready(0);
      fetch(0, xa);
    }
    for (int c = 0; c < chunks; c += 2) {
      if (c + 1 < chunks) {
        ready(c + 1);
        fetch(c + 1, xb);
      }
      consume(c, xa);
      if (c + 1 < chunks) {
        if (c + 2 < chunks) {
          ready(c + 2);
          fetch(c + 2, xa);
        }
        consume(c + 1, xb);
      }
    }
#pragma unroll
    for (int r = 0; r < 3; ++r)
      if (r < count - count4) acc = acc + (tail[r] * inv) * tv[r];
    const int col = h * HS + j0 + lane;
    if (lane < AC) a.out[(int64_t)t * a.out_stride + col] = acc;
    if (AC == 32 && a.xq) {
      // quantize_x of the group (lanes 0-31): the largest magnitude, scale = amax / qmax, the values
      const float amax = wave_max32(__builtin_fabsf(acc));
      const float scale = amax / (a.bias == 0 ? 127.0f : 63.0f);
      const float qinv = scale > 0 ? 1.0f / scale : 0.0f;
      if (lane < 32) a.xq[(int64_t)t * a.xq_stride + col] = quant_value(acc, qinv, a.bias);
      if (lane == 0) a.xs[(int64_t)t * a.xs_stride + col / GS] = scale;
    }
  }
}
#undef ATT_FETCH

// (B + C) for a few tokens (decode) whose output the caller quantizes itself: one block of 1024 threads a (token,
// query head, 16 columns), thread b owning the four-position block b (positions 4b .. 4b+3) of the weighted values.
// The head's tile maxima and scores are requested at once, the exponentials go into LDS by lane (four rows: positions
// t % 4 == k); then every thread requests its block's 16 columns x 4 values while four lanes of wave 0 run the
// ordered sums, turns them into the columns' four-position products ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)), p = e *
// f32(1 / sum), into LDS rows (one a column), and 16 lanes of wave 0 add their column's products in order, then the
// tail. (The values are requested once the exponentials are in LDS: requested at the start, their arrival slowed the
// scores' loads and the exponentials.) Blocks of the query heads that share a kv head's columns go to one XCD, as in
// attend_kernel.
constexpr int A2_NT = 1024;  // threads a block
constexpr int A2_AC = 16;    // columns a block
constexpr int A2_SV = 4;     // scores a thread a pass (4096 positions)
constexpr int A2_MOST = 2 * 4 * A2_NT;  // positions: two four-position blocks a thread at most

// LDS bytes of attend2_kernel for the largest count of a launch: the exponentials' four rows, the tail, the columns'
// rows of products
size_t attend2_lds(int count) {
  const int rs = chain_rowstride((count & ~3) >> 2);
  return sizeof(float) * (size_t)((4 + A2_AC) * rs + 4);
}

template <int HS, bool HALF>
__global__ __launch_bounds__(A2_NT) void attend2_kernel(const AttnArgs a) {
  constexpr int NT = A2_NT, AC = A2_AC, S = HS / AC;
  extern __shared__ float4 lds4[];
  float *const lds = reinterpret_cast<float *>(lds4);
  __shared__ float shared_mx, shared_inv;
  const int mul = a.nh / a.nkv, groups = a.nkv * S;
  const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3, hl = idx % mul, g = (idx / mul) * 8 + xcd;
  if (g >= groups) return;  // the grid's rounding up: whole blocks leave
  const int kh = g / S, j0 = (g % S) * AC, h = kh * mul + hl;
  const int t = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int count = first_position(a) + t + 1, count4 = count & ~3, q4 = count4 >> 2, rs = chain_rowstride(q4);
  float *const e4 = lds;             // [4][rs]
  float *const tail = lds + 4 * rs;  // [4]
  float *const blk = tail + 4;       // [AC][rs] (16-byte aligned: rs is a multiple of 16)
  const float *sc = a.scores + ((int64_t)t * a.nh + h) * a.seq_len;
  const int64_t vcol = (int64_t)(kh * HS + j0) * a.vstride;  // the block's first value column
  const int tiles = (count + TILE - 1) / TILE;
  const float *tm = a.tilemax + ((int64_t)t * a.nh + h) * (a.seq_len / TILE + 1);
  float tmr[2];
  if (wave == 0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) tmr[u] = tm[min(lane + 64 * u, tiles - 1)];  // clamped: a repeat changes no max
  }
  float sv[A2_SV];
#pragma unroll
  for (int u = 0; u < A2_SV; ++u) sv[u] = sc[min(tid + NT * u, count - 1)];  // clamped, unconditional
  float tv[3];  // wave 0, lane j < AC: column j's values past the fours (at most 3)
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 3; ++r)
      tv[r] = cache1<HALF>(a.vcache, vcol + (int64_t)(lane % AC) * a.vstride + min(count4 + r, count - 1));
  }
  if (wave == 0) {
    float mx = wmax(tmr[0], tmr[1]);
    for (int i = lane + 128; i < tiles; i += 64) mx = wmax(mx, tm[i]);  // past 8192 positions
    for (int o = 32; o >= 1; o >>= 1) mx = wmax(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) shared_mx = mx;
  }
  __syncthreads();
  const float mx = shared_mx;
  for (int base = 0; base < count; base += NT * A2_SV) {
    if (base > 0) {
#pragma unroll
      for (int u = 0; u < A2_SV; ++u) sv[u] = sc[min(base + tid + NT * u, count - 1)];
    }
#pragma unroll
    for (int u = 0; u < A2_SV; ++u) {
      if (base + NT * u < count) {  // the block's test first (a scalar branch): no exponentials past the count
        const int i = base + tid + NT * u;
        if (i < count) {
          const float d = sv[u] - mx;
          if (i < count4) e4[(i & 3) * rs + (i >> 2)] = vexp(d);
          else tail[i - count4] = fexp(d);
        }
      }
    }
  }
  __syncthreads();
  // the first pass's values requested now (clamped into the column: never used past q4): they fly while wave 0 runs
  // the exponentials' ordered sum (its reads 32 values at a time, so that both fit the registers)
  float4 v0[AC];
  {
    const int bc = max(min(tid, q4 - 1), 0);
#pragma unroll
    for (int j = 0; j < AC; ++j) v0[j] = cache4<HALF>(a.vcache, vcol + (int64_t)j * a.vstride + 4 * bc);
  }
  if (wave == 0) {
    // lanes 0-3: lane k's sum; ((l0 + l1) + l2) + l3, the tail in order, 1 / sum
    const float part = lane < 4 ? lds_chain_h<4>(e4 + lane * rs, q4, 0.0f) : 0.0f;
    const float c1 = __shfl(part, 1, 64), c2 = __shfl(part, 2, 64), c3 = __shfl(part, 3, 64);
    if (lane == 0) {
      float sum = ((part + c1) + c2) + c3;
      for (int r = 0; r < count - count4; ++r) sum = sum + tail[r];
      shared_inv = 1.0f / sum;
    }
  }
  __syncthreads();
  const float inv = shared_inv;
  // block b's products: (p0 v0 + p1 v1) + (p2 v2 + p3 v3) for the 16 columns, into the columns' rows
  auto products = [&](int b, const float4 (&v)[AC]) {
    if (b < q4) {
      const float p0 = e4[b] * inv, p1 = e4[rs + b] * inv, p2 = e4[2 * rs + b] * inv, p3 = e4[3 * rs + b] * inv;
#pragma unroll
      for (int j = 0; j < AC; ++j) {
        const float4 x = v[j];
        blk[j * rs + b] = (p0 * x.x + p1 * x.y) + (p2 * x.z + p3 * x.w);
      }
    }
  };
  products(tid, v0);
  for (int b0 = NT; b0 < q4; b0 += NT) {  // (a scalar loop: every thread takes the same passes)
    const int b = b0 + tid, bc = min(b, q4 - 1);  // clamped: never stored past q4
    float4 v[AC];
#pragma unroll
    for (int j = 0; j < AC; ++j) v[j] = cache4<HALF>(a.vcache, vcol + (int64_t)j * a.vstride + 4 * bc);
    products(b, v);
  }
  __syncthreads();
  if (wave == 0 && lane < AC) {
    float acc = lds_chain(blk + lane * rs, q4, 0.0f);
#pragma unroll
    for (int r = 0; r < 3; ++r)
      if (r < count - count4) acc = acc + (tail[r] * inv) * tv[r];
    a.out[(int64_t)t * a.out_stride + h * HS + j0 + lane] = acc;
  }
}

// LDS bytes of attend_kernel for the largest count of a launch (ring slots into *nslot), 0 where it does not fit
template <int HS>
int attend_lds(const AttnArgs &a, int *nslot) {
  const int count = a.pos0 + a.m;
  const int head = (int)sizeof(float) * (4 * chain_rowstride((count & ~3) >> 2) + 4);
  const int slot = (int)sizeof(float) * Attend<HS>::AC * RR;
  const int n = std::min(ASLOTS, (ALDS - head) / slot);
  if (n < 2) return 0;
  *nslot = n;
  return head + n * slot;
}

// whether attend2_kernel takes a decode launch: head sizes of whole 16-column slices, a context that fits its LDS
// and its two four-position blocks a thread
bool attend2_takes(const AttnArgs &a) {
  const int count = a.pos0 + a.m;
  return a.hs % A2_AC == 0 && count <= A2_MOST && attend2_lds(count) <= (size_t)ALDS;
}

template <int HS, bool HALF>
hipError_t launch_hs(const AttnArgs &a, hipStream_t s) {
  const int tiles = (a.pos0 + a.m + TILE - 1) / TILE;
  if (a.m <= DECODE_TOKENS) {
    hipLaunchKernelGGL((scores_kernel<HS, HALF>), dim3(tiles, a.nkv, a.m), dim3(256), 0, s, a);
  } else {
    const hipError_t e = launch_scores_tokens(a, s);
    if (e != hipSuccess) return e;
  }
  if (a.m <= DECODE_TOKENS && !a.split && !a.xq && attend2_takes(a)) {
    // the caller quantizes the output itself: blocks of 16 columns
    const size_t lds = attend2_lds(a.pos0 + a.m);
    if (lds > 64 * 1024) {
      static bool sized = false;  // once a process: let the kernel take LDS past 64 KiB
      if (!sized) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&attend2_kernel<HS, HALF>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, ALDS);
        if (e != hipSuccess) return e;
        sized = true;
      }
    }
    const int groups = a.nkv * (HS / A2_AC), g8 = (groups + 7) & ~7;
    hipLaunchKernelGGL((attend2_kernel<HS, HALF>), dim3(g8 * (a.nh / a.nkv), 1, a.m), dim3(A2_NT), lds, s, a);
    return hipGetLastError();
  }
  int nslot = 0;
  const int fused = a.m <= DECODE_TOKENS && !a.split ? attend_lds<HS>(a, &nslot) : 0;
  if (fused) {
    static bool sized = false;  // once a process: let the kernel take LDS past 64 KiB
    if (!sized) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&attend_kernel<HS, HALF>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, ALDS);
      if (e != hipSuccess) return e;
      sized = true;
    }
    const int groups = a.nkv * (HS / Attend<HS>::AC), g8 = (groups + 7) & ~7;
    hipLaunchKernelGGL((attend_kernel<HS, HALF>), dim3(g8 * (a.nh / a.nkv), 1, a.m), dim3(Attend<HS>::NT), fused, s,
                       a, nslot);
    return hipGetLastError();
  }
  return launch_softmax_pv(a, s);
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

int32_t attention_most_positions() {
  int32_t n = (ALDS / 4) & ~3;
  while (n > 0 && softmax_lds(n) > (size_t)ALDS) n -= 4;
  return n;
}

bool attention_quantizes(const AttnArgs &a) {
  if (!attention_supported(a.hs, a.nh, a.nkv) || a.m > DECODE_TOKENS || a.hs % 32 || a.split) return false;
  int nslot = 0;
  switch (a.hs) {
    case 32: return attend_lds<32>(a, &nslot) > 0;
    case 64: return attend_lds<64>(a, &nslot) > 0;
    case 96: return attend_lds<96>(a, &nslot) > 0;
    case 128: return attend_lds<128>(a, &nslot) > 0;
    case 256: return attend_lds<256>(a, &nslot) > 0;
    default: return false;
  }
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
  if (!attention_supported(a.hs, a.nh, a.nkv)) return hipErrorInvalidValue;
  // pieces of equal size (each past DECODE_TOKENS when m is past ATTN_ROWS), one after another on the stream
  const int pieces = a.dpos ? 1 : (a.m + ATTN_ROWS - 1) / ATTN_ROWS, size = (a.m + pieces - 1) / pieces;
  for (int at = 0; at < a.m; at += size) {
    AttnArgs p = a;
    p.q = a.q + (int64_t)at * a.q_stride;
    p.out = a.out + (int64_t)at * a.out_stride;
    p.pos0 = a.pos0 + at;
    p.m = std::min(size, a.m - at);
    if (p.xq) {
      p.xq = a.xq + (int64_t)at * a.xq_stride;
      p.xs = a.xs + (int64_t)at * a.xs_stride;
    }
    const hipError_t e = a.half ? launch_half<true>(p, s) : launch_half<false>(p, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ple
