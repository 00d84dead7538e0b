// attention_tokens.hip — the attention of a prompt block (many tokens a launch), to the bit of kernels/kernel.ts:448-566
// attentionOf in the order attention.hip states: (A) the scores of 64-position tiles for blocks of 64 (token, head)
// rows that share each staged key tile, their products on the matrix core; (B) one block a (token, head) taking the
// row's largest score and writing the weights p over the scores; (C) blocks of tokens that share the values they
// stage, a thread two (token, head, column) sums. (B) and (C) also take the decode launches whose context is past the
// decode kernels' LDS. In a file of their own, so that the decode kernels' code object does not change with them.
#pragma clang fp contract(off)

#include <algorithm>

#include "attention.hpp"

namespace ple {

namespace {

// (A) for many tokens (a prompt block), products on the matrix core: one block a (64-position tile, kv head,
// 64 / mul tokens): 64 (token, head) rows x 64 positions, a wave 32 rows x 32 positions. v_mfma_f32_32x32x1_2b_f32
// with a zero accumulator makes 2 x 32 x 32 single products q[row][d] * k[pos][d], each the correctly rounded float32
// product (as the VALU's multiply, subnormals kept: a zero accumulator adds nothing), two dims at once (block 0 from
// lanes 0-31, block 1 from lanes 32-63): dims 4j and 4j + 2 in one, 4j + 1 and 4j + 3 in the next. The VALU then adds
// each product to its (row, position)'s lane chain d % 4 in order of d, the sums kernels/kernel.ts:448-566 fixes: one
// add a product instead of a multiply and an add. The head is staged in chunks of DC dims (the rows' queries and the
// tile's keys, double buffered in LDS: the next chunk's loads in flight while this one is summed). No tile maxima:
// the softmax takes each row's largest score from the scores themselves.
template <int HS> constexpr int score_chunk() { return HS % 32 == 0 ? 32 : 16; }
constexpr int SCORE_ROWS = 64;  // (token, head) rows a block

typedef float v32f __attribute__((ext_vector_type(32)));

// the 16 values live in registers here: an empty asm that takes and gives them keeps the compiler from moving the
// adds that make them below this point
__device__ __forceinline__ void pin16(float (&x)[16]) {
  asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7]),
               "+v"(x[8]), "+v"(x[9]), "+v"(x[10]), "+v"(x[11]), "+v"(x[12]), "+v"(x[13]), "+v"(x[14]), "+v"(x[15]));
}

template <int HS, bool HALF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void scores_tokens_kernel(const AttnArgs a) {
  constexpr int DC = score_chunk<HS>(), NC = HS / DC;
  constexpr int LDC = DC + 2;  // floats a staged row: the b64 reads of 32 rows fall on distinct banks
  constexpr int NF = TILE * DC / 4 / 256;  // float4 of keys (and of queries) a thread stages a chunk
  __shared__ float ks[2][TILE * LDC];
  __shared__ float qs[2][SCORE_ROWS * LDC];
  const int kh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave & 1, wp = wave >> 1;  // the wave's 32 rows and 32 positions
  const int h = lane >> 5, l32 = lane & 31;
  const int mul = a.nh / a.nkv, tt_n = max(1, SCORE_ROWS / mul);
  const int t0 = blockIdx.z * tt_n, last = min(t0 + tt_n, a.m) - 1;
  const int tile = blockIdx.x, p0 = tile * TILE, pos0 = first_position(a), reach = pos0 + last + 1;
  if (p0 >= reach) return;  // past every token of the block (uniform: before any barrier)
  const int kvdim = a.nkv * HS;
  // a chunk's loads: keys of positions (clamped to the reach: loaded, never used) and queries of rows (token
  // t0 + r / mul, clamped to the block's last, head kh * mul + r % mul), row/position i / (DC / 4), float4
  // i % (DC / 4); as 32-bit element offsets from the two bases (the launch checks that the cache and the queries fit)
  uint32_t ko[NF], qo[NF];
#pragma unroll
  for (int u = 0; u < NF; ++u) {
    const int i = tid + 256 * u, r = i / (DC / 4), c4 = i % (DC / 4);
    ko[u] = (uint32_t)min(p0 + r, reach - 1) * (uint32_t)kvdim + (uint32_t)(kh * HS + 4 * c4);
    const int t = min(t0 + r / mul, last), hh = kh * mul + r % mul;
    qo[u] = (uint32_t)t * (uint32_t)a.q_stride + (uint32_t)(hh * HS + 4 * c4);
  }
  float4 kf[NF], qf[NF];
  auto fetch = [&](int c) {
#pragma unroll
    for (int u = 0; u < NF; ++u) {
      kf[u] = cache4<HALF>(a.kcache, ko[u] + (uint32_t)(c * DC));
      qf[u] = *reinterpret_cast<const float4 *>(a.q + (qo[u] + (uint32_t)(c * DC)));
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < NF; ++u) {
      const int i = tid + 256 * u, r = i / (DC / 4), c4 = i % (DC / 4);
      float2 *kd = reinterpret_cast<float2 *>(ks[buf] + r * LDC + 4 * c4);
      float2 *qd = reinterpret_cast<float2 *>(qs[buf] + r * LDC + 4 * c4);
      kd[0] = make_float2(kf[u].x, kf[u].y);
      kd[1] = make_float2(kf[u].z, kf[u].w);
      qd[0] = make_float2(qf[u].x, qf[u].y);
      qd[1] = make_float2(qf[u].z, qf[u].w);
    }
  };
  fetch(0);
  stage(0);
  __syncthreads();
  float acc[4][16];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;
  const v32f zero = {};
  for (int c = 0; c < NC; ++c) {
    const bool more = c + 1 < NC;  // uniform
    if (more) fetch(c + 1);
    // this lane's operands: row wr * 32 + lane % 32 of the queries and position wp * 32 + lane % 32 of the keys, the
    // dims 4j + 2 h and 4j + 2 h + 1 of the chunk
    const float *qb = qs[c & 1] + (wr * 32 + l32) * LDC + 2 * h;
    const float *kb = ks[c & 1] + (wp * 32 + l32) * LDC + 2 * h;
#pragma unroll
    for (int j = 0; j < DC / 4; ++j) {
      const float2 qv = *reinterpret_cast<const float2 *>(qb + 4 * j);
      const float2 kv = *reinterpret_cast<const float2 *>(kb + 4 * j);
      // one product block in registers at a time: the sums are pinned where they are made (the compiler would
      // otherwise sink the adds below later MFMAs and keep every product block); the other waves of the SIMD hide
      // each MFMA's latency
      v32f d = __builtin_amdgcn_mfma_f32_32x32x1f32(qv.x, kv.x, zero, 0, 0, 0);  // dims 4j, 4j + 2
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        acc[0][v] = acc[0][v] + d[v];
        acc[2][v] = acc[2][v] + d[16 + v];
      }
      pin16(acc[0]);
      pin16(acc[2]);
      d = __builtin_amdgcn_mfma_f32_32x32x1f32(qv.y, kv.y, zero, 0, 0, 0);  // dims 4j + 1, 4j + 3
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        acc[1][v] = acc[1][v] + d[v];
        acc[3][v] = acc[3][v] + d[16 + v];
      }
      pin16(acc[1]);
      pin16(acc[3]);
    }
    if (more) {
      stage((c + 1) & 1);  // the other buffer: its last readers passed the previous barrier
      __syncthreads();
    }
  }
  // the lane's 16 outputs: rows wr * 32 + (v / 4) * 8 + h * 4 + v % 4 (uniform over the half-wave), position
  // p0 + wp * 32 + lane % 32
  const float isq = 1.0f / __builtin_sqrtf((float)HS);
  const int p = p0 + wp * 32 + l32;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int r = wr * 32 + (v >> 2) * 8 + h * 4 + (v & 3), tt = r / mul, t = t0 + tt;
    const int count = pos0 + min(t, a.m - 1) + 1;
    if (tt < tt_n && t < a.m && p < count)
      a.scores[((int64_t)t * a.nh + kh * mul + r % mul) * a.seq_len + p] =
          ((acc[0][v] + acc[2][v]) + (acc[1][v] + acc[3][v])) * isq;
  }
}

// (B) one block a (head, token): grid (nh, m), block 256. The scores requested at once, their largest by a block
// reduction, the exponentials by every thread into LDS (lane k's positions t % 4 == k side by side), the four ordered
// sums by four threads, the weights.
__global__ __launch_bounds__(256) void softmax_kernel(const AttnArgs a) {
  extern __shared__ float e4[];  // 4 rows of q4s exponentials, then the tail
  __shared__ float part[4];
  __shared__ float shared_mx, shared_inv, wave_mx[4];
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const int count = first_position(a) + t + 1, count4 = count & ~3, q4 = count4 >> 2, q4s = chain_rowstride(q4);
  float *scores = a.scores + ((int64_t)t * a.nh + h) * a.seq_len;
  float sv[16];  // up to 16 scores a thread
#pragma unroll
  for (int u = 0; u < 16; ++u) sv[u] = scores[min(tid + 256 * u, count - 1)];  // clamped, unconditional
  // the largest score, from the lowest finite float32 (order-free: every score once, clamped copies of the last
  // changing nothing)
  float lm = -3.4028234663852886e38f;
#pragma unroll
  for (int u = 0; u < 16; ++u) lm = wmax(lm, sv[u]);
  for (int base = 256 * 16; base < count; base += 256 * 16)  // past 4096 positions: the rest, read once more below
    for (int u = 0; u < 16; ++u) lm = wmax(lm, scores[min(base + tid + 256 * u, count - 1)]);
  for (int o = 32; o >= 1; o >>= 1) lm = wmax(lm, __shfl_xor(lm, o, 64));
  if ((tid & 63) == 0) wave_mx[tid >> 6] = lm;
  __syncthreads();
  if (tid == 0) shared_mx = wmax(wmax(wave_mx[0], wave_mx[1]), wmax(wave_mx[2], wave_mx[3]));
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

// (B') one wave a (token, head) row, four rows (heads h4 * 4 ..) a block: grid (ceil(nh / 4), m), block 256. The same
// steps as (B) inside one wave (its largest, the exponentials into the wave's own LDS rows, the four ordered sums by
// four of its lanes, the weights), with no block barrier: a row takes a wave, not a block, so more rows share a CU
// while their sums run. For contexts whose four rows of exponentials fit the LDS (softmax4_lds).
constexpr int SM4_HELD = 32;  // scores a lane holds (rows of up to 2048 positions read once)
__global__ __launch_bounds__(256) void softmax4_kernel(const AttnArgs a) {
  extern __shared__ float e4all[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x * 4 + wave, t = blockIdx.y;
  if (h >= a.nh) return;  // (uniform over the wave; no block barrier follows)
  const int count = first_position(a) + t + 1, count4 = count & ~3, q4 = count4 >> 2, q4s = chain_rowstride(q4);
  float *e4 = e4all + wave * (4 * q4s + 4), *tail = e4 + 4 * q4s;
  float *scores = a.scores + ((int64_t)t * a.nh + h) * a.seq_len;
  // the largest score, from the lowest finite float32 (order-free): lane maxima, rotations inside 16-lane rows
  // (DPP), the four rows' values by readlane
  // the row's first 64 * SM4_HELD scores held in registers from the maximum's pass to the exponentials' (a uniform
  // test a load, so that a short row requests only what it has)
  float held[SM4_HELD];
#pragma unroll
  for (int u = 0; u < SM4_HELD; ++u) held[u] = 64 * u < count ? scores[min(lane + 64 * u, count - 1)] : 0.0f;
  float lm = -3.4028234663852886e38f;
#pragma unroll
  for (int u = 0; u < SM4_HELD; ++u)
    if (64 * u < count) lm = wmax(lm, held[u]);  // a clamped copy of the last score changes no maximum
  for (int i = lane + 64 * SM4_HELD; i < count; i += 64) lm = wmax(lm, scores[i]);
  {
    int src = __float_as_int(lm);
    lm = wmax(lm, __int_as_float(__builtin_amdgcn_update_dpp(src, src, 0x128, 0xF, 0xF, false)));  // row_ror:8
    src = __float_as_int(lm);
    lm = wmax(lm, __int_as_float(__builtin_amdgcn_update_dpp(src, src, 0x124, 0xF, 0xF, false)));  // row_ror:4
    src = __float_as_int(lm);
    lm = wmax(lm, __int_as_float(__builtin_amdgcn_update_dpp(src, src, 0x122, 0xF, 0xF, false)));  // row_ror:2
    src = __float_as_int(lm);
    lm = wmax(lm, __int_as_float(__builtin_amdgcn_update_dpp(src, src, 0x121, 0xF, 0xF, false)));  // row_ror:1
    src = __float_as_int(lm);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(src, 0)), r1 = __int_as_float(__builtin_amdgcn_readlane(src, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(src, 32)), r3 = __int_as_float(__builtin_amdgcn_readlane(src, 48));
    lm = wmax(wmax(r0, r1), wmax(r2, r3));
  }
  const float mx = lm;
#pragma unroll
  for (int u = 0; u < SM4_HELD; ++u) {
    const int i = lane + 64 * u;
    if (i < count) {
      const float d = held[u] - mx;
      if (i < count4) e4[(i & 3) * q4s + (i >> 2)] = vexp(d);
      else tail[i - count4] = fexp(d);
    }
  }
  for (int i = lane + 64 * SM4_HELD; i < count; i += 64) {
    const float d = scores[i] - mx;
    if (i < count4) e4[(i & 3) * q4s + (i >> 2)] = vexp(d);
    else tail[i - count4] = fexp(d);
  }
  wave_sync_lds();
  float part = 0.0f;
  if (lane < 4) part = lds_chain(e4 + lane * q4s, q4, 0.0f);
  // ((l0 + l1) + l2) + l3, then the tail in order (every lane computes it from the four lanes' sums)
  const float p0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 0));
  const float p1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 1));
  const float p2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 2));
  const float p3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 3));
  float sum = ((p0 + p1) + p2) + p3;
  for (int i = 0; i < count - count4; ++i) sum = sum + tail[i];
  const float inv = 1.0f / sum;
  for (int i = lane; i < count; i += 64) {
    const float e = i < count4 ? e4[(i & 3) * q4s + (i >> 2)] : tail[i - count4];
    scores[i] = e * inv;
  }
}

// (C) for many tokens (a prompt block), products on the matrix core: v_mfma_f32_16x16x1_4b_f32 with a zero
// accumulator makes 4 x 16 x 16 single products, block b of the four being position 4k + b: p[row][4k + b] *
// v[4k + b][col], each the correctly rounded float32 product. A lane then holds, for each of its 4 (row, column)
// outputs, the four products of one four-position block, and adds them as kernels/kernel.ts:448-566 does:
// out = out + ((p0 v0 + p1 v1) + (p2 v2 + p3 v3)), one add a product. A block of 256 threads takes R (token, head) rows
// (R = 1024 / C) and C columns of one kv head, 4 tiles of 16 x 16, one a wave (the positions are the long dimension
// and their order is fixed, so the outputs are split as finely as the matrix core allows, for as many waves as can
// share a CU); the weights and the values of a 32-position chunk are staged in LDS (double buffered: the next chunk's
// loads in flight). The block's tokens end at different positions: a four-position block past a row's last whole four
// is not added to it, and the positions past its fours are added one at a time at the end, out = out + p v.
template <int HS> constexpr int pv_cols() { return HS % 32 == 0 ? 32 : 16; }
constexpr int TPC = 32;        // positions a chunk
constexpr int LDP = TPC + 4;   // floats a staged row: 16 rows x 4 positions of a read on distinct banks

typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ void pin4(float (&x)[4]) {
  asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
}

// (at most 128 VGPRs a lane: the MFMA then writes VGPRs, with no copies out of AGPRs)
template <int HS, bool HALF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void pv_tokens_kernel(const AttnArgs a) {
  constexpr int C = pv_cols<HS>(), R = 1024 / C, CT = C / 16;  // columns, rows, column tiles of a block
  constexpr int NP = R * TPC / 4 / 256;                       // float4 of weights a thread stages (1 or 2)
  static_assert(NP >= 1 && NP <= 2 && C * TPC / 4 <= 256, "pv staging shape");
  __shared__ float ps[2][R * LDP];  // weights [row][position]
  __shared__ float vs[2][C * LDP];  // values [column][position]
  const int kh = blockIdx.y, j0 = blockIdx.x * C, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;  // the lane's position in a four (its operands) and row/column in a tile
  const int trow = (wave / CT) * 16, tcol = (wave % CT) * 16;  // the wave's tile
  const int mul = a.nh / a.nkv, tt_n = max(1, R / mul);
  const int t0 = blockIdx.z * tt_n, last = min(t0 + tt_n, a.m) - 1;
  const int pos0 = first_position(a);
  const int most4 = (pos0 + last + 1) & ~3;   // the block's last token's whole fours: every four any row adds
  const int least4 = (pos0 + t0 + 1) & ~3;    // the first token's: every row adds the fours below it
  const int chunks = (most4 + TPC - 1) / TPC;
  // staging loads: weights of rows tid / 8 (+ 32) (token t0 + r / mul clamped to the block's last, head
  // kh * mul + r % mul), values of column tid / 8, float4 tid % 8 of the chunk; positions clamped below most4 (loaded,
  // never added). Written out as macros with named registers, so that the staged values stay in registers.
  const float *prow0, *prow1 = nullptr;
  {
    auto row_of = [&](int r) {
      const int t = min(t0 + r / mul, last), hh = kh * mul + r % mul;
      return a.scores + ((int64_t)t * a.nh + hh) * a.seq_len + 4 * (tid % 8);
    };
    prow0 = row_of(tid / 8);
    if constexpr (NP > 1) prow1 = row_of(tid / 8 + 32);
  }
  const int64_t vrow = (int64_t)(kh * HS + j0 + min(tid, C * TPC / 4 - 1) / 8) * a.vstride + 4 * (tid % 8);
  float4 pf0, pf1, vf0;
#define PV_FETCH(c_)                                                                                               \
  do {                                                                                                             \
    const int po = min((c_) * TPC, most4 - 4 - 4 * (tid % 8));                                                    \
    pf0 = *reinterpret_cast<const float4 *>(prow0 + po);                                                           \
    if constexpr (NP > 1) pf1 = *reinterpret_cast<const float4 *>(prow1 + po);                                      \
    vf0 = cache4<HALF>(a.vcache, vrow + po);                                                                       \
  } while (0)
#define PV_STAGE(buf_)                                                                                             \
  do {                                                                                                             \
    float *pd = ps[(buf_)] + (tid / 8) * LDP + 4 * (tid % 8);                                                      \
    *reinterpret_cast<float4 *>(pd) = pf0;                                                                         \
    if constexpr (NP > 1) *reinterpret_cast<float4 *>(pd + 32 * LDP) = pf1;                                        \
    if (tid < C * TPC / 4) *reinterpret_cast<float4 *>(vs[(buf_)] + (tid / 8) * LDP + 4 * (tid % 8)) = vf0;         \
  } while (0)
  // the lane's outputs: rows trow + g * 4 + q, q < 4, column tcol + lane % 16; a row's whole fours
  int nb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = trow + g * 4 + q, t = min(t0 + r / mul, last);
    nb[q] = ((pos0 + t + 1) & ~3) >> 2;
  }
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const v16f zero = {};
  if (chunks > 0) {
    PV_FETCH(0);
    PV_STAGE(0);
  }
  __syncthreads();
  for (int c = 0; c < chunks; ++c) {
    const bool more = c + 1 < chunks;  // uniform
    if (more) PV_FETCH(c + 1);
    const float *pb = ps[c & 1] + (trow + l16) * LDP + g, *vb = vs[c & 1] + (tcol + l16) * LDP + g;
    const int b0 = c * (TPC / 4);  // the chunk's first four, from position 0
    if ((c + 1) * TPC <= least4) {  // every row of the block adds every four of the chunk (uniform)
#pragma unroll
      for (int k = 0; k < TPC / 4; ++k) {
        const v16f d = __builtin_amdgcn_mfma_f32_16x16x1f32(pb[4 * k], vb[4 * k], zero, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = acc[q] + ((d[q] + d[4 + q]) + (d[8 + q] + d[12 + q]));
        pin4(acc);
      }
    } else {  // each row adds the fours below its own last whole four (the fours past most4: staged, never added)
#pragma unroll
      for (int k = 0; k < TPC / 4; ++k) {
        const v16f d = __builtin_amdgcn_mfma_f32_16x16x1f32(pb[4 * k], vb[4 * k], zero, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float sum = acc[q] + ((d[q] + d[4 + q]) + (d[8 + q] + d[12 + q]));
          acc[q] = b0 + k < nb[q] ? sum : acc[q];
        }
        pin4(acc);
      }
    }
    if (more) {
      PV_STAGE((c + 1) & 1);  // the other buffer: its last readers passed the previous barrier
      __syncthreads();
    }
  }
#undef PV_FETCH
#undef PV_STAGE
  // each row's positions past its fours, one at a time, then the outputs
  const int col = j0 + tcol + l16;
  const int64_t vcol = (int64_t)(kh * HS + col) * a.vstride;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = trow + g * 4 + q, tt = r / mul, t = t0 + tt;
    if (tt >= tt_n || t >= a.m) continue;
    const int count = pos0 + t + 1, hh = kh * mul + r % mul;
    const float *pt = a.scores + ((int64_t)t * a.nh + hh) * a.seq_len;
    float o = acc[q];
    for (int p = count & ~3; p < count; ++p) o = o + pt[p] * cache1<HALF>(a.vcache, vcol + p);
    a.out[(int64_t)t * a.out_stride + hh * HS + col] = o;
  }
}

template <int HS, bool HALF>
hipError_t scores_tokens_hs(const AttnArgs &a, hipStream_t s) {
  // the kernel's element offsets are 32-bit
  if ((int64_t)a.seq_len * a.nkv * HS >= (1ll << 32) || (int64_t)a.m * a.q_stride >= (1ll << 32)) return hipErrorInvalidValue;
  const int tiles = (a.pos0 + a.m + TILE - 1) / TILE;
  const int tt = std::max(1, SCORE_ROWS / (a.nh / a.nkv));
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
  const size_t lds4 = softmax4_lds(a.pos0 + a.m);
  if (lds4 <= (size_t)ALDS) {
    if (lds4 > 64 * 1024) {
      static bool sized4 = false;  // once a process: let the kernel take LDS past 64 KiB
      if (!sized4) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&softmax4_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, ALDS);
        if (e != hipSuccess) return e;
        sized4 = true;
      }
    }
    hipLaunchKernelGGL(softmax4_kernel, dim3((a.nh + 3) / 4, a.m), dim3(256), lds4, s, a);
  } else {
    hipLaunchKernelGGL(softmax_kernel, dim3(a.nh, a.m), dim3(256), lds_b, s, a);
  }
  constexpr int C = pv_cols<HS>();
  const int tt = std::max(1, (1024 / C) / (a.nh / a.nkv));  // tokens a block
  hipLaunchKernelGGL((pv_tokens_kernel<HS, HALF>), dim3(HS / C, a.nkv, (a.m + tt - 1) / tt), dim3(256), 0, s, a);
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
// four rows of softmax_lds (softmax4_kernel)
size_t softmax4_lds(int count) { return 4 * softmax_lds(count); }

hipError_t launch_scores_tokens(const AttnArgs &a, hipStream_t s) {
  return a.half ? scores_tokens_by_hs<true>(a, s) : scores_tokens_by_hs<false>(a, s);
}

hipError_t launch_softmax_pv(const AttnArgs &a, hipStream_t s) {
  return a.half ? softmax_pv_by_hs<true>(a, s) : softmax_pv_by_hs<false>(a, s);
}

}  // namespace ple
