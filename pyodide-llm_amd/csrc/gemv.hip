// gemv.hip — the decode matmul (m <= 8 tokens) of int8/int6 rows against quantized activations, to the bit of the
// reference's CPU kernels:
//   bias 64: kernels/kernel_relaxed.ts:34-67 matmul_q8r (and :195-218 matmul_q6r): per group the exact integer
//            S_g = dot(w, q - 64); lane g % 4 of four float32 accumulators adds f32(S_g) * f32(ws * xs) for the groups
//            in fours, in order; the lanes are added ((l0 + l1) + l2) + l3; the groups past the fours one at a time.
//   bias 0:  kernels/kernel.ts:231-258 matmul_q8 (and :261-278 matmul_q6): four int32 lane sums a group (lane k:
//            products 2k, 2k+1, 2k+8, 2k+9 of each half), each scaled into its own accumulator over every group in
//            order, the four added in order.
// Layout: one wave a row. An int8 row is read 16 bytes a lane (a group is a lane pair, 1 KiB a wave step), an int6
// row 24 bytes a lane (a group a lane, 1.5 KiB a step); a wave requests up to 8 steps of its row (8 or 12 KiB) before
// it uses the first, so that HBM sees whole rows in flight. The int32 sums come from v_dot4_i32_i8; the products of
// the whole row go to LDS, laid out so that the lane holding accumulator k of token t reads its groups in order.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace ple {
#if GEMV_PAD
extern "C" __global__ void ple_pad_kernel(int *out) {
  if (out) asm volatile(".fill %0, 4, 0xbf800000" ::"i"(GEMV_PAD / 4));
}
#endif

namespace {

constexpr int WAVES = 4;
// wave steps requested at once: 8 (8 KiB of an int8 row a wave) for one or two tokens, fewer where every token's
// activations ride along in registers
template <int M>
constexpr int chunk_of() { return M <= 2 ? 8 : (M <= 4 ? 4 : 2); }

struct RowLayout {  // a token's products in LDS: 4 accumulator rows of q floats, then the (up to 3) tail groups
  int q, stride;
};
__host__ __device__ inline RowLayout row_layout(int k, bool relaxed) {
  const int g = k / GS;
  const int q = relaxed ? (((g & ~3) / 4 + 3) & ~3) : ((g + 3) & ~3);
  return {q, 4 * q + 4};
}

// the segment (matrix) of a launch's row r, with constant indices into the arguments only, so that they stay in
// scalar registers (a dynamic index makes the compiler read them from memory and wait on every load before it)
struct RowAt {
  const uint8_t *w;
  const float *ws;
  float *y;
  int32_t r, y_stride, accumulate;
};
__device__ __forceinline__ RowAt row_at(const MatArgs &a, int row) {
  const int n0 = a.seg[0].rows, n1 = a.seg[1].rows;
  if (a.nseg > 2 && row >= n0 + n1)
    return {a.seg[2].w, a.seg[2].ws, a.seg[2].y, row - n0 - n1, a.seg[2].y_stride, a.seg[2].accumulate};
  if (a.nseg > 1 && row >= n0) return {a.seg[1].w, a.seg[1].ws, a.seg[1].y, row - n0, a.seg[1].y_stride, a.seg[1].accumulate};
  return {a.seg[0].w, a.seg[0].ws, a.seg[0].y, row, a.seg[0].y_stride, a.seg[0].accumulate};
}

// the decode paths' store of row `row`'s result: y = sum (or y + sum). With a.qkv on (every lane of the wave calls
// it, rows in pairs on lanes 2i, 2i + 1): + bias, RoPE on q and k rows (kernels/kernel.ts:344-357: pair (v0, v1) ->
// (v0 c - v1 s, v0 s + v1 c)), and k and v rows into the cache too (float16 by to_f16 where the cache is half).
__device__ __forceinline__ void store_row(const MatArgs &a, int row, float sum, bool valid) {
  const RowAt at = row_at(a, min(row, a.total_rows - 1));
  float *y = at.y + at.r;
  if (!a.qkv.on) {
    if (valid) *y = at.accumulate ? *y + sum : sum;
    return;
  }
  // (every field read by value: a reference into the kernel's argument struct makes the compiler copy it to scratch)
  const float *bq = a.qkv.bq, *bk = a.qkv.bk, *bv = a.qkv.bv, *cos_t = a.qkv.cos_t, *sin_t = a.qkv.sin_t;
  void *kcache = a.qkv.kcache, *vcache = a.qkv.vcache;
  const int32_t *dpos = a.qkv.dpos;
  const int pos = dpos ? *dpos : a.qkv.pos, hs = a.qkv.hs, kvdim = a.qkv.kvdim, half = a.qkv.half;
  const int vstride = a.qkv.vstride;
  const int n0 = a.seg[0].rows, n1 = a.seg[1].rows;
  const int seg = row < n0 ? 0 : (row < n0 + n1 ? 1 : 2), r = at.r;
  const float *bias = seg == 0 ? bq : (seg == 1 ? bk : bv);
  const float v = bias ? sum + bias[r] : sum;
  const float partner = dpp_xor1(v);  // the pair's other row (lanes 2i, 2i + 1)
  float o = v;
  if (seg < 2) {
    const int ci = (r % hs) >> 1;
    const float c = cos_t[(int64_t)pos * (hs / 2) + ci], s = sin_t[(int64_t)pos * (hs / 2) + ci];
    const bool even = (r & 1) == 0;
    const float v0 = even ? v : partner, v1 = even ? partner : v;
    o = even ? v0 * c - v1 * s : v0 * s + v1 * c;
  }
  if (!valid) return;
  *y = o;
  if (seg > 0) {
    void *cache = seg == 1 ? kcache : vcache;
    const int64_t i = seg == 1 ? (int64_t)pos * kvdim + r : (int64_t)r * vstride + pos;
    if (half) reinterpret_cast<uint16_t *>(cache)[i] = to_f16(o);
    else reinterpret_cast<float *>(cache)[i] = o;
  }
}

template <int M, bool SIX, bool RELAXED, bool SUMS>
__global__ __launch_bounds__(256) void gemv_kernel(const MatArgs a) {
  constexpr int GPI = SIX ? 64 : 32;  // groups a wave step
  constexpr int NW = SIX ? 8 : 4;     // words of weights a lane a step
  constexpr int NX = SIX ? 8 : 4;     // words of a token's activations a lane a step
  constexpr int CHUNK = chunk_of<M>();
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * WAVES + wave;
  if (row >= a.total_rows) return;  // a whole wave leaves: nothing below waits on the block
  const int K = a.k, G = K / GS, G4 = G & ~3;
  const RowLayout lay = row_layout(K, RELAXED);
  float *P = smem + wave * M * lay.stride;
  const int steps = (G + GPI - 1) / GPI;
  const bool holder = SIX ? true : ((lane & 1) == 0);
  const int mylocal = SIX ? lane : (lane >> 1);

  const RowAt sg = row_at(a, row);
  const int r = sg.r;
  const uint8_t *wrow = sg.w + (int64_t)r * (SIX ? (int64_t)G * 24 : (int64_t)K);
  const float *srow = SUMS ? nullptr : sg.ws + (int64_t)r * G;

  for (int c0 = 0; c0 < steps; c0 += CHUNK) {
    uint32_t wv[CHUNK][NW];
    uint32_t xv[CHUNK][M][NX];
    float wsv[CHUNK], xsv[CHUNK][M];
    // every load of the chunk first: the row's weights and scales, the tokens' activations and scales
#pragma unroll
    for (int u = 0; u < CHUNK; ++u) {
      const int g = min((c0 + u) * GPI + mylocal, G - 1);  // clamped: every load unconditional
      {
        if constexpr (SIX) {
          const uint2 *p = reinterpret_cast<const uint2 *>(wrow + (int64_t)g * 24);
          const uint2 l0 = p[0], l1 = p[1], tops = p[2];
          wv[u][0] = l0.x; wv[u][1] = l0.y; wv[u][2] = l1.x; wv[u][3] = l1.y; wv[u][4] = tops.x; wv[u][5] = tops.y;
        } else {
          const uint4 v = *reinterpret_cast<const uint4 *>(wrow + (int64_t)g * 32 + (lane & 1) * 16);
          wv[u][0] = v.x; wv[u][1] = v.y; wv[u][2] = v.z; wv[u][3] = v.w;
        }
        if constexpr (!SUMS) {
          wsv[u] = srow[g];
#pragma unroll
          for (int t = 0; t < M; ++t) xsv[u][t] = a.xs[(int64_t)t * a.xs_stride + g];
        }
#pragma unroll
        for (int t = 0; t < M; ++t) {
          const int8_t *xt = a.xq + (int64_t)t * a.xq_stride + g * 32;
          if constexpr (SIX) {
            const uint4 x0 = reinterpret_cast<const uint4 *>(xt)[0], x1 = reinterpret_cast<const uint4 *>(xt)[1];
            xv[u][t][0] = x0.x; xv[u][t][1] = x0.y; xv[u][t][2] = x0.z; xv[u][t][3] = x0.w;
            xv[u][t][4] = x1.x; xv[u][t][5] = x1.y; xv[u][t][6] = x1.z; xv[u][t][7] = x1.w;
          } else {
            const uint4 x0 = *reinterpret_cast<const uint4 *>(xt + (lane & 1) * 16);
            xv[u][t][0] = x0.x; xv[u][t][1] = x0.y; xv[u][t][2] = x0.z; xv[u][t][3] = x0.w;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < CHUNK; ++u) {
      if (c0 + u >= steps) break;
      const int g = (c0 + u) * GPI + mylocal;
      const bool active = g < G;
      uint32_t w[8];
      if constexpr (SIX) {
        const uint32_t L[4] = {wv[u][0], wv[u][1], wv[u][2], wv[u][3]};
        six_widen(L, wv[u][4], wv[u][5], w);
      } else {
        w[0] = wv[u][0]; w[1] = wv[u][1]; w[2] = wv[u][2]; w[3] = wv[u][3];
      }
      int32_t S[M][RELAXED ? 1 : 4];
#pragma unroll
      for (int t = 0; t < M; ++t) {
#pragma unroll
        for (int k = 0; k < (RELAXED ? 1 : 4); ++k) S[t][k] = 0;
        if (active) {
          const uint32_t *x = xv[u][t];
          if constexpr (RELAXED) {
            int32_t acc = 0;
#pragma unroll
            for (int i = 0; i < NX; ++i) acc = dot4(w[i], centre4(x[i]), acc);
            S[t][0] = acc;
          } else {
            // lane k of kernels/kernel.ts:222-229: bytes {2k, 2k+1} of words 0/2 (k < 2) or 1/3 (k >= 2) of each half
#pragma unroll
            for (int h = 0; h < NX; h += 4) {
              const int32_t even = dot4(w[h], x[h], dot4(w[h + 2], x[h + 2], 0));
              const int32_t odd = dot4(w[h + 1], x[h + 1], dot4(w[h + 3], x[h + 3], 0));
              const int32_t l0 = dot4(w[h] & 0xFFFFu, x[h], dot4(w[h + 2] & 0xFFFFu, x[h + 2], 0));
              const int32_t l2 = dot4(w[h + 1] & 0xFFFFu, x[h + 1], dot4(w[h + 3] & 0xFFFFu, x[h + 3], 0));
              S[t][0] += l0;
              S[t][1] += even - l0;
              S[t][2] += l2;
              S[t][3] += odd - l2;
            }
          }
        }
        if constexpr (!SIX) {
#pragma unroll
          for (int k = 0; k < (RELAXED ? 1 : 4); ++k) S[t][k] += dpp_xor1(S[t][k]);
        }
      }
      if (!(holder && active)) continue;
      if constexpr (SUMS) {
#pragma unroll
        for (int t = 0; t < M; ++t) {
          int32_t *o = a.sums + (((int64_t)t * a.total_rows + row) * G + g) * (RELAXED ? 1 : 4);
#pragma unroll
          for (int k = 0; k < (RELAXED ? 1 : 4); ++k) o[k] = S[t][k];
        }
      } else {
#pragma unroll
        for (int t = 0; t < M; ++t) {
          const float scale = wsv[u] * xsv[u][t];
          float *pt = P + t * lay.stride;
          if constexpr (RELAXED) {
            const float p = (float)S[t][0] * scale;
            if (g < G4) pt[(g & 3) * lay.q + (g >> 2)] = p;
            else pt[4 * lay.q + (g - G4)] = p;
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) pt[k * lay.q + g] = (float)S[t][k] * scale;
          }
        }
      }
    }
  }
  if constexpr (SUMS) return;
  wave_sync_lds();
  float chain = 0.0f;  // lane 4t + k (t < M): accumulator k of token t
  if (lane < 4 * M) {
    const int t = lane >> 2, k = lane & 3;
    chain = lds_chain(P + t * lay.stride + k * lay.q, RELAXED ? G4 / 4 : G, 0.0f);
  }
  const int src = (lane < M ? lane : 0) * 4;
  const float c0 = __shfl(chain, src, 64), c1 = __shfl(chain, src + 1, 64);
  const float c2 = __shfl(chain, src + 2, 64), c3 = __shfl(chain, src + 3, 64);
  if (lane < M) {
    float sum = ((c0 + c1) + c2) + c3;
    if constexpr (RELAXED) {
      const float *tl = P + lane * lay.stride + 4 * lay.q;
      for (int g = G4; g < G; ++g) sum = sum + tl[g - G4];
    }
    float *y = sg.y + (int64_t)lane * sg.y_stride + r;
    *y = sg.accumulate ? *y + sum : sum;
  }
}

// The activations of a decode launch from the float32 token instead of quantize_x's output, in the block itself (no
// launch of their own): with a.xnorm, rmsnorm first (kernels/kernel.ts:330-342: the squares in four lanes j % 4 added
// in order by four threads, hsum ((l0 + l1) + l2) + l3, the tail; s = f32(1 / f32(sqrt(f32(ss / n) + eps)));
// out = w * (s * x)), then quantize_x with bias 64 (kernels/kernel.ts:129-156), stored centred (q - 64) into xl with the
// group scales into xsl. Every block computes the same bits. Thread tid of the block's NT takes the MAXU consecutive
// positions from tid * MAXU (MAXU a divisor of 32 and a multiple of 4; MAXU * NT >= K), requested by load_f32 before
// the rows as float4; a group of 32 is then 32 / MAXU neighbouring lanes, whose largest magnitude is their own
// maxima's (DPP within the group's lanes), so that a lane computes one group's scale and its reciprocal, not MAXU of
// them. sq: 4 * chain_rowstride(K / 4) floats of LDS.
// NORM (rmsnorm with a.xnorm) is a template argument: a load under a run-time test of the pointer is waited for
// before the next is requested, which made the token's loads one round trip each.
template <int MAXU, bool NORM, int NT = 256>
__device__ __forceinline__ void load_f32(const MatArgs &a, float (&xv)[MAXU], float (&wv)[MAXU]) {
  static_assert(MAXU % 4 == 0 && 32 % MAXU == 0, "a lane's positions: whole float4, within one group");
#pragma unroll
  for (int u = 0; u < MAXU / 4; ++u) {
    const int j = min((int)threadIdx.x * MAXU + 4 * u, a.k - 4);  // clamped: every load unconditional
    const float4 x4 = *reinterpret_cast<const float4 *>(a.xf + j);
    xv[4 * u] = x4.x; xv[4 * u + 1] = x4.y; xv[4 * u + 2] = x4.z; xv[4 * u + 3] = x4.w;
    if constexpr (NORM) {
      const float4 w4 = *reinterpret_cast<const float4 *>(a.xnorm + j);
      wv[4 * u] = w4.x; wv[4 * u + 1] = w4.y; wv[4 * u + 2] = w4.z; wv[4 * u + 3] = w4.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) wv[4 * u + e] = 1.0f;
    }
  }
}
template <int MAXU, bool NORM, int NT = 256>
__device__ __forceinline__ void stage_from_f32(const MatArgs &a, const float (&xv)[MAXU], const float (&wv)[MAXU],
                                               uint8_t *xl, float *xsl, float *sq) {
  __shared__ float part[4], sval;
  constexpr int LG = 32 / MAXU;  // lanes a group
  const int tid = threadIdx.x, K = a.k, q4 = K >> 2, qs = chain_rowstride(q4), j0 = tid * MAXU;
  float sc = 1.0f;
  if constexpr (NORM) {
    if (j0 < K) {
#pragma unroll
      for (int i = 0; i < MAXU; ++i) sq[(i & 3) * qs + ((j0 + i) >> 2)] = xv[i] * xv[i];
    }
    lds_barrier();
    if (tid < 4) part[tid] = lds_chain(sq + tid * qs, q4, 0.0f);
    lds_barrier();
    if (tid == 0) sval = 1.0f / __builtin_sqrtf((((part[0] + part[1]) + part[2]) + part[3]) / (float)K + a.eps);
    lds_barrier();
    sc = sval;
  }
  float o[MAXU];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXU; ++i) {
    o[i] = NORM ? wv[i] * (sc * xv[i]) : xv[i];
    m = __builtin_fmaxf(m, __builtin_fabsf(o[i]));
  }
  // the group's largest magnitude (order-free): xor 1 and xor 2 within quads, then the mirror within 8 lanes
  if constexpr (LG >= 2) m = __builtin_fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0xB1, 0xF, 0xF, true)));
  if constexpr (LG >= 4) m = __builtin_fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x4E, 0xF, 0xF, true)));
  if constexpr (LG >= 8) m = __builtin_fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x141, 0xF, 0xF, true)));
  const float scale = m / 63.0f;
  const float inv = scale > 0 ? 1.0f / scale : 0.0f;
  uint32_t words[MAXU / 4];
#pragma unroll
  for (int u = 0; u < MAXU / 4; ++u) {
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) w |= (uint32_t)(uint8_t)(quant_value(o[4 * u + e], inv, 64) - 64) << (8 * e);
    words[u] = w;
  }
  if (j0 < K) {  // whole groups (K is a multiple of 32)
#pragma unroll
    for (int u = 0; u < MAXU / 4; ++u) reinterpret_cast<uint32_t *>(xl + j0)[u] = words[u];
    if (tid % LG == 0) xsl[j0 >> 5] = scale;
  }
}

// The decode path proper (one token, int8, bias 64): a wave takes R consecutive rows (about 16 KiB of weights) and
// requests all of them with their scales before anything else (a scheduling barrier keeps the compiler from sinking
// the loads next to their uses); meanwhile the block stages the token's activations, centred, and their scales in
// LDS once. The R rows' products go to LDS and 4R lanes add them in the reference's order at once.
// NS: wave steps (1 KiB of a row), NS * 1024 >= K.
// SRC: 0 the activations from xq / xs; 1 the float32 token (a.xf); 2 a.xf after rmsnorm with a.xnorm
template <int R, int NS, int SRC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void gemv1_kernel(const MatArgs a) {
  constexpr bool F32 = SRC != 0;
  constexpr int SV = (NS * 32 + 255) / 256;  // float4 of a row's scales a lane
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.k, G = K / GS, G4 = G & ~3, G16 = (G + 3) & ~3;
  const int steps = (G + 31) / 32;
  const RowLayout lay = row_layout(K, true);
  uint32_t *xl = reinterpret_cast<uint32_t *>(smem);   // K bytes of centred activations
  float *xsl = smem + K / 4;                           // G scales of the activations
  float *wsl = xsl + G16 + wave * R * G16;             // this wave's rows' weight scales
  float *P = xsl + G16 + WAVES * R * G16 + wave * R * lay.stride;  // this wave's products
  const bool holder = (lane & 1) == 0;
  const int half = (lane & 1) * 16;
  const int row0 = min((blockIdx.x * WAVES + wave) * R, a.total_rows - 1);
  // every load of the block, in the order their uses come: the token's activations (small, staged first), the rows'
  // scales, the rows (about 16 KiB a wave); unconditional loads from clamped (always valid) addresses, since a load
  // under a branch is waited for before the next
  constexpr int XL = (NS * 1024 / 16 + 255) / 256;
  constexpr int XSV = (NS * 32 + 255) / 256;
  constexpr int FU = F32 ? NS * 4 : 1;
  uint4 xv[XL];
  float sv[XSV];
  float fx[FU], fw[FU];
  if constexpr (F32) {
    static_assert(NS <= 4, "the float32 token is held a thread at a time");
    load_f32<FU, SRC == 2>(a, fx, fw);
  } else {
#pragma unroll
    for (int u = 0; u < XL; ++u) xv[u] = reinterpret_cast<const uint4 *>(a.xq)[min((int)threadIdx.x + 256 * u, K / 16 - 1)];
#pragma unroll
    for (int u = 0; u < XSV; ++u) sv[u] = a.xs[min((int)threadIdx.x + 256 * u, G - 1)];
  }
  uint32_t wr[R][NS][4];
  float4 sr[R][SV];
  const uint8_t *wrow[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const RowAt at = row_at(a, min(row0 + i, a.total_rows - 1));  // rows past the end: the last again, unused
    wrow[i] = at.w + (int64_t)at.r * K;
    const float *ws = at.ws + (int64_t)at.r * G;
    // the row's scales as float4 (a row's scales start 4-byte aligned only: read them one float at a time where
    // the row does not start on 16 bytes)
#pragma unroll
    for (int u = 0; u < SV; ++u) {
      const int f = min(4 * (lane + 64 * u), G16 - 4);
      if ((reinterpret_cast<uintptr_t>(ws) & 15) == 0 && f + 4 <= G) {
        sr[i][u] = *reinterpret_cast<const float4 *>(ws + f);
      } else {
        sr[i][u] = make_float4(ws[min(f, G - 1)], ws[min(f + 1, G - 1)], ws[min(f + 2, G - 1)], ws[min(f + 3, G - 1)]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int g = min(u * 32 + (lane >> 1), G - 1);
      const uint4 v = *reinterpret_cast<const uint4 *>(wrow[i] + (int64_t)g * 32 + half);
      wr[i][u][0] = v.x; wr[i][u][1] = v.y; wr[i][u][2] = v.z; wr[i][u][3] = v.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // the block's activations into LDS: K / 16 uint4, centred (or made here from the float32 token)
  if constexpr (F32) {
    stage_from_f32<FU, SRC == 2>(a, fx, fw, reinterpret_cast<uint8_t *>(xl), xsl, P - wave * R * lay.stride);
  } else {
#pragma unroll
    for (int u = 0; u < XL; ++u) {
      const int i = threadIdx.x + 256 * u;
      if (i < K / 16)
        reinterpret_cast<uint4 *>(xl)[i] = make_uint4(centre4(xv[u].x), centre4(xv[u].y), centre4(xv[u].z),
                                                      centre4(xv[u].w));
    }
#pragma unroll
    for (int u = 0; u < XSV; ++u) {
      const int i = threadIdx.x + 256 * u;
      if (i < G) xsl[i] = sv[u];
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int u = 0; u < SV; ++u) {
      const int f = 4 * (lane + 64 * u);
      if (f < G16) *reinterpret_cast<float4 *>(wsl + i * G16 + f) = sr[i][u];
    }
  lds_barrier();
  if ((blockIdx.x * WAVES + wave) * R >= a.total_rows) return;  // (after the block's barrier)
  // fully unrolled (no early exit), so that wr stays in registers
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (u < steps) {
    const int g = u * 32 + (lane >> 1);
    const int gc = min(g, G - 1);
    const uint4 x4 = reinterpret_cast<const uint4 *>(xl)[(gc * 32 + half) / 16];
    const uint32_t xc[4] = {x4.x, x4.y, x4.z, x4.w};
    const float xs_g = xsl[gc];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      int32_t S = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) S = dot4(wr[i][u][j], xc[j], S);
      S += dpp_xor1(S);
      if (holder && g < G) {
        const float p = (float)S * (wsl[i * G16 + g] * xs_g);
        float *pi = P + i * lay.stride;
        if (g < G4) pi[(g & 3) * lay.q + (g >> 2)] = p;
        else pi[4 * lay.q + (g - G4)] = p;
      }
    }
    }
  }
  wave_sync_lds();
  float chain = 0.0f;  // lane 4i + k: accumulator k of row row0 + i
  if (lane < 4 * R) chain = lds_chain(P + (lane >> 2) * lay.stride + (lane & 3) * lay.q, G4 / 4, 0.0f);
  const int src = (lane < R ? lane : 0) * 4;
  const float c0 = __shfl(chain, src, 64), c1 = __shfl(chain, src + 1, 64);
  const float c2 = __shfl(chain, src + 2, 64), c3 = __shfl(chain, src + 3, 64);
  float sum = ((c0 + c1) + c2) + c3;
  if (lane < R) {
    const float *tl = P + lane * lay.stride + 4 * lay.q;
    for (int g = G4; g < G; ++g) sum = sum + tl[g - G4];
  }
  store_row(a, row0 + lane, sum, lane < R && row0 + lane < a.total_rows);
}

// The persistent decode path (one token, int8, bias 64; a launch that asks for it: MatArgs.persistent): one block of
// PW waves a CU, and wave w
// of block b takes the row groups gw, gw + NWV, gw + 2 NWV, ... (gw = b PW + w, NWV = every wave of the grid) of R
// consecutive rows, requesting a group's rows and scales, then adding them up, then the next group. The CU hides each
// wave's load latency behind its other waves' groups. The block stages the token's activations in LDS once, while
// every wave's first group is in flight: from xq / xs (centred), or (F32) from the float32 token, after rmsnorm where
// a.xnorm is given, in the block itself (stage_from_f32), so that the norm's ordered sum runs once a CU while HBM
// delivers the first rows, instead of in a launch of its own. Per row the arithmetic is gemv1_kernel's: exact group
// sums by v_dot4, their float32 products into LDS, 4R lanes adding the reference's four chains in order, and
// store_row (the residual add, or the q / k / v epilogue).
template <int R, int NS>
struct RowSet {
  uint32_t w[R][NS][4];
  float s[R][(NS * 32 + 255) / 256][4];
};

// the launch's segments as named scalars, read once: a segment picked among them by a wave-uniform row is a scalar
// select (picked among the argument struct's array members, the compiler can turn it into an indexed copy in scratch)
struct SegPick {
  const uint8_t *w0, *w1, *w2;
  const float *s0, *s1, *s2;
  int32_t n0, n1, nseg;
};
__device__ __forceinline__ SegPick seg_pick(const MatArgs &a) {
  return {a.seg[0].w, a.seg[1].w, a.seg[2].w, a.seg[0].ws, a.seg[1].ws, a.seg[2].ws, a.seg[0].rows, a.seg[1].rows,
          a.nseg};
}
// the values and scales of row `row` (wave-uniform)
__device__ __forceinline__ void pick_row(const SegPick &p, int row, int k, int g, const uint8_t **w, const float **ws) {
  if (p.nseg > 2 && row >= p.n0 + p.n1) {
    *w = p.w2 + (int64_t)(row - p.n0 - p.n1) * k;
    *ws = p.s2 + (int64_t)(row - p.n0 - p.n1) * g;
  } else if (p.nseg > 1 && row >= p.n0) {
    *w = p.w1 + (int64_t)(row - p.n0) * k;
    *ws = p.s1 + (int64_t)(row - p.n0) * g;
  } else {
    *w = p.w0 + (int64_t)row * k;
    *ws = p.s0 + (int64_t)row * g;
  }
}

// a group's rows and scales (every load unconditional, from clamped addresses); ALIGNED: every row's scales start on
// 16 bytes, read as float4
template <int R, int NS, bool ALIGNED>
__device__ __forceinline__ void request_rows(RowSet<R, NS> &b, const SegPick &sp, int K, int total_rows, int group,
                                             int ngroups, int lane) {
  constexpr int SV = (NS * 32 + 255) / 256;
  const int G = K / GS, G16 = (G + 3) & ~3, half = (lane & 1) * 16;
  const int row0 = __builtin_amdgcn_readfirstlane(min(group, ngroups - 1) * R);
  const uint8_t *wrows[R];
  const float *srows[R];
#pragma unroll
  for (int i = 0; i < R; ++i) pick_row(sp, min(row0 + i, total_rows - 1), K, G, &wrows[i], &srows[i]);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const float *ws = srows[i];
#pragma unroll
    for (int u = 0; u < SV; ++u) {
      const int f = min(4 * (lane + 64 * u), G16 - 4);
      if constexpr (ALIGNED) {
        const float4 v = *reinterpret_cast<const float4 *>(ws + f);
        b.s[i][u][0] = v.x; b.s[i][u][1] = v.y; b.s[i][u][2] = v.z; b.s[i][u][3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) b.s[i][u][e] = ws[min(f + e, G - 1)];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint8_t *wrow = wrows[i];
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int g = min(u * 32 + (lane >> 1), G - 1);
      const uint4 v = *reinterpret_cast<const uint4 *>(wrow + (int64_t)g * 32 + half);
      b.w[i][u][0] = v.x; b.w[i][u][1] = v.y; b.w[i][u][2] = v.z; b.w[i][u][3] = v.w;
    }
  }
}

// one group's rows against the staged activations: the products into P, the four chains of each row, the store
template <int R, int NS>
__device__ __forceinline__ void finish_rows(const RowSet<R, NS> &b, const MatArgs &a, int group, const uint32_t *xl,
                                            const float *xsl, float *wsl, float *P, int lane) {
  constexpr int SV = (NS * 32 + 255) / 256;
  const int K = a.k, G = K / GS, G4 = G & ~3, G16 = (G + 3) & ~3;
  const int steps = (G + 31) / 32, half = (lane & 1) * 16;
  const bool holder = (lane & 1) == 0;
  const RowLayout lay = row_layout(K, true);
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int u = 0; u < SV; ++u) {
      const int f = 4 * (lane + 64 * u);
      if (f < G16)
        *reinterpret_cast<float4 *>(wsl + i * G16 + f) = make_float4(b.s[i][u][0], b.s[i][u][1], b.s[i][u][2], b.s[i][u][3]);
    }
  wave_sync_lds();
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (u < steps) {
      const int g = u * 32 + (lane >> 1);
      const int gc = min(g, G - 1);
      const uint4 x4 = reinterpret_cast<const uint4 *>(xl)[(gc * 32 + half) / 16];
      const uint32_t xc[4] = {x4.x, x4.y, x4.z, x4.w};
      const float xs_g = xsl[gc];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        int32_t S = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) S = dot4(b.w[i][u][j], xc[j], S);
        S += dpp_xor1(S);
        if (holder && g < G) {
          const float p = (float)S * (wsl[i * G16 + g] * xs_g);
          float *pi = P + i * lay.stride;
          if (g < G4) pi[(g & 3) * lay.q + (g >> 2)] = p;
          else pi[4 * lay.q + (g - G4)] = p;
        }
      }
    }
  }
  wave_sync_lds();
  float chain = 0.0f;  // lane 4i + k: accumulator k of row row0 + i
  if (lane < 4 * R) chain = lds_chain(P + (lane >> 2) * lay.stride + (lane & 3) * lay.q, G4 / 4, 0.0f);
  const int src = (lane < R ? lane : 0) * 4;
  const float c0 = __shfl(chain, src, 64), c1 = __shfl(chain, src + 1, 64);
  const float c2 = __shfl(chain, src + 2, 64), c3 = __shfl(chain, src + 3, 64);
  float sum = ((c0 + c1) + c2) + c3;
  if (lane < R) {
    const float *tl = P + lane * lay.stride + 4 * lay.q;
    for (int g = G4; g < G; ++g) sum = sum + tl[g - G4];
  }
  const int row0 = __builtin_amdgcn_readfirstlane(group * R);
  store_row(a, row0 + lane, sum, lane < R && row0 + lane < a.total_rows);
  wave_sync_lds();  // the next group writes wsl and P again
}

// SRC: 0 the activations from xq / xs; 1 the float32 token (a.xf); 2 a.xf after rmsnorm with a.xnorm
template <int PW, int R, int NS, int SRC, bool ALIGNED>
__global__ __launch_bounds__(64 * PW) void gemvp_kernel(const MatArgs a) {
  constexpr int PNT = 64 * PW;
  constexpr bool F32 = SRC != 0;
  extern __shared__ float smem[];
  // the wave's index in a scalar register: every row index below is the wave's own, so segment picks stay scalar
  // (an index the compiler takes for a lane's makes it copy the argument struct to scratch and index it there)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = a.k, G = K / GS, G16 = (G + 3) & ~3;
  const RowLayout lay = row_layout(K, true);
  uint32_t *xl = reinterpret_cast<uint32_t *>(smem);               // K bytes of centred activations
  float *xsl = smem + K / 4;                                       // G scales of the activations
  float *wsl = xsl + G16 + wave * R * G16;                         // this wave's rows' weight scales
  float *P = xsl + G16 + PW * R * G16 + wave * R * lay.stride;     // this wave's products
  float *sq = xsl + G16 + PW * R * G16 + PW * R * lay.stride;      // F32 with a norm: the squares' four rows
  const int ngroups = (a.total_rows + R - 1) / R, nwv = gridDim.x * PW;
  int group = blockIdx.x * PW + wave;
  const SegPick sp = seg_pick(a);
  RowSet<R, NS> rows;
  // the token first (small; staged while the rows fly), then the first group's rows
  constexpr int XL = (NS * 1024 / 16 + PNT - 1) / PNT;
  constexpr int XSV = (NS * 32 + PNT - 1) / PNT;
  constexpr int FU = F32 ? (NS * 1024 + PNT - 1) / PNT : 1;
  uint4 xv[XL];
  float sv[XSV];
  float fx[FU], fw[FU];
  if constexpr (F32) {
    load_f32<FU, SRC == 2, PNT>(a, fx, fw);
  } else {
#pragma unroll
    for (int u = 0; u < XL; ++u) xv[u] = reinterpret_cast<const uint4 *>(a.xq)[min((int)threadIdx.x + PNT * u, K / 16 - 1)];
#pragma unroll
    for (int u = 0; u < XSV; ++u) sv[u] = a.xs[min((int)threadIdx.x + PNT * u, G - 1)];
  }
  request_rows<R, NS, ALIGNED>(rows, sp, K, a.total_rows, group, ngroups, lane);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (F32) {
    stage_from_f32<FU, SRC == 2, PNT>(a, fx, fw, reinterpret_cast<uint8_t *>(xl), xsl, sq);
  } else {
#pragma unroll
    for (int u = 0; u < XL; ++u) {
      const int i = threadIdx.x + PNT * u;
      if (i < K / 16)
        reinterpret_cast<uint4 *>(xl)[i] = make_uint4(centre4(xv[u].x), centre4(xv[u].y), centre4(xv[u].z),
                                                      centre4(xv[u].w));
    }
#pragma unroll
    for (int u = 0; u < XSV; ++u) {
      const int i = threadIdx.x + PNT * u;
      if (i < G) xsl[i] = sv[u];
    }
  }
  lds_barrier();
  if (group >= ngroups) return;  // (after the block's barrier; no barrier follows)
  finish_rows<R, NS>(rows, a, group, xl, xsl, wsl, P, lane);
  for (group += nwv; group < ngroups; group += nwv) {
    request_rows<R, NS, ALIGNED>(rows, sp, K, a.total_rows, group, ngroups, lane);
    finish_rows<R, NS>(rows, a, group, xl, xsl, wsl, P, lane);
  }
}

// The int6 decode path (one token, six.ts groups, bias 64: kernels/kernel_relaxed.ts:189-218 matmul_q6r): as
// gemv1_kernel, with a lane taking two consecutive groups of 24 bytes (48 bytes, three 16-byte loads) of each of its
// wave's R rows, 128 groups a wave step, widened to int8 in registers (kernels/six.ts) next to their use.
// NS: wave steps, NS * 128 groups >= K / 32.
// SRC: 0 the activations from xq / xs; 1 the float32 token (a.xf); 2 a.xf after rmsnorm with a.xnorm
// W: waves a block (the float32 token's blocks take 16, so that quantize_x of the token is 4 values a thread)
template <int R, int NS, int SRC, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(1, 4))) void gemv6_kernel(const MatArgs a) {
  constexpr bool F32 = SRC != 0;
  constexpr int NT = 64 * W;
  constexpr int SV = (NS * 128 + 255) / 256;  // float4 of a row's scales a lane
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.k, G = K / GS, G4 = G & ~3, G16 = (G + 3) & ~3;
  const int steps = (G + 127) / 128;
  const RowLayout lay = row_layout(K, true);
  uint32_t *xl = reinterpret_cast<uint32_t *>(smem);   // K bytes of centred activations
  float *xsl = smem + K / 4;                           // G scales of the activations
  float *wsl = xsl + G16 + wave * R * G16;             // this wave's rows' weight scales
  float *P = xsl + G16 + W * R * G16 + wave * R * lay.stride;  // this wave's products
  const int row0 = min((blockIdx.x * W + wave) * R, a.total_rows - 1);
  // every load of the block, in the order their uses come: the token's activations and their scales (staged first),
  // the rows' scales, the rows; unconditional loads from clamped (always valid) addresses (the staging waits only for
  // the first, and each wave step only for its own rows)
  constexpr int XL = (NS * 4096 / 16 + NT - 1) / NT;
  constexpr int XSV = (NS * 128 + NT - 1) / NT;
  constexpr int FU = F32 ? (NS * 4096 + NT - 1) / NT : 1;
  uint4 xv[XL];
  float sv[XSV];
  float fx[FU], fw[FU];
  if constexpr (F32) {
    static_assert(NS == 1, "the float32 token is held a thread at a time");
    load_f32<FU, SRC == 2, NT>(a, fx, fw);
  } else {
#pragma unroll
    for (int u = 0; u < XL; ++u) xv[u] = reinterpret_cast<const uint4 *>(a.xq)[min((int)threadIdx.x + NT * u, K / 16 - 1)];
#pragma unroll
    for (int u = 0; u < XSV; ++u) sv[u] = a.xs[min((int)threadIdx.x + NT * u, G - 1)];
  }
  uint4 wr[R][NS][3];
  float4 sr[R][SV];
  const uint8_t *wrow[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const RowAt at = row_at(a, min(row0 + i, a.total_rows - 1));  // rows past the end: the last again, unused
    wrow[i] = at.w + (int64_t)at.r * G * 24;
    const float *ws = at.ws + (int64_t)at.r * G;
#pragma unroll
    for (int u = 0; u < SV; ++u) {
      const int f = min(4 * (lane + 64 * u), G16 - 4);
      if ((reinterpret_cast<uintptr_t>(ws) & 15) == 0 && f + 4 <= G) {
        sr[i][u] = *reinterpret_cast<const float4 *>(ws + f);
      } else {
        sr[i][u] = make_float4(ws[min(f, G - 1)], ws[min(f + 1, G - 1)], ws[min(f + 2, G - 1)], ws[min(f + 3, G - 1)]);
      }
    }
  }
  // groups 2 * pair and 2 * pair + 1 of each wave step
#pragma unroll
  for (int u = 0; u < NS; ++u)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int pair = min(u * 64 + lane, (G - 2) >> 1);  // G is even where it matters; an odd G's last pair clamps
      const uint4 *p = reinterpret_cast<const uint4 *>(wrow[i] + (int64_t)pair * 48);
      wr[i][u][0] = p[0];
      wr[i][u][1] = p[1];
      wr[i][u][2] = p[2];
    }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (F32) {
    stage_from_f32<FU, SRC == 2, NT>(a, fx, fw, reinterpret_cast<uint8_t *>(xl), xsl, P - wave * R * lay.stride);
  } else {
#pragma unroll
    for (int u = 0; u < XL; ++u) {
      const int i = threadIdx.x + NT * u;
      if (i < K / 16)
        reinterpret_cast<uint4 *>(xl)[i] = make_uint4(centre4(xv[u].x), centre4(xv[u].y), centre4(xv[u].z),
                                                      centre4(xv[u].w));
    }
#pragma unroll
    for (int u = 0; u < XSV; ++u) {
      const int i = threadIdx.x + NT * u;
      if (i < G) xsl[i] = sv[u];
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int u = 0; u < SV; ++u) {
      const int f = 4 * (lane + 64 * u);
      if (f < G16) *reinterpret_cast<float4 *>(wsl + i * G16 + f) = sr[i][u];
    }
  lds_barrier();
  if ((blockIdx.x * W + wave) * R >= a.total_rows) return;  // (after the block's barrier)
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (u < steps) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int g = u * 128 + 2 * lane + h;
        const int gc = min(g, G - 1);
        const uint4 x0 = reinterpret_cast<const uint4 *>(xl)[gc * 2], x1 = reinterpret_cast<const uint4 *>(xl)[gc * 2 + 1];
        const uint32_t xc[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const float xs_g = xsl[gc];
#pragma unroll
        for (int i = 0; i < R; ++i) {
          // group h of the lane's 48 bytes: its 16 low-nibble bytes and 8 bytes of top bits
          const uint4 q0 = wr[i][u][0], q1 = wr[i][u][1], q2 = wr[i][u][2];
          uint32_t L[4], T0, T1;
          if (h == 0) {
            L[0] = q0.x; L[1] = q0.y; L[2] = q0.z; L[3] = q0.w; T0 = q1.x; T1 = q1.y;
          } else {
            L[0] = q1.z; L[1] = q1.w; L[2] = q2.x; L[3] = q2.y; T0 = q2.z; T1 = q2.w;
          }
          uint32_t wv[8];
          six_widen(L, T0, T1, wv);
          int32_t S = 0;
#pragma unroll
          for (int j = 0; j < 8; ++j) S = dot4(wv[j], xc[j], S);
          if (g < G) {
            const float p = (float)S * (wsl[i * G16 + g] * xs_g);
            float *pi = P + i * lay.stride;
            if (g < G4) pi[(g & 3) * lay.q + (g >> 2)] = p;
            else pi[4 * lay.q + (g - G4)] = p;
          }
        }
      }
    }
  }
  wave_sync_lds();
  float chain = 0.0f;  // lane 4i + k: accumulator k of row row0 + i
  if (lane < 4 * R) chain = lds_chain(P + (lane >> 2) * lay.stride + (lane & 3) * lay.q, G4 / 4, 0.0f);
  const int src = (lane < R ? lane : 0) * 4;
  const float c0 = __shfl(chain, src, 64), c1 = __shfl(chain, src + 1, 64);
  const float c2 = __shfl(chain, src + 2, 64), c3 = __shfl(chain, src + 3, 64);
  float sum = ((c0 + c1) + c2) + c3;
  if (lane < R) {
    const float *tl = P + lane * lay.stride + 4 * lay.q;
    for (int g = G4; g < G; ++g) sum = sum + tl[g - G4];
  }
  store_row(a, row0 + lane, sum, lane < R && row0 + lane < a.total_rows);
}

template <int R, int NS, int W = WAVES>
hipError_t launch_gemv6(const MatArgs &a, hipStream_t s) {
  if (a.xf && (NS > 1 || a.k % 32)) return hipErrorInvalidValue;
  const int waves = (a.total_rows + R - 1) / R;
  const int blocks = (waves + W - 1) / W;
  const size_t g16 = ((a.k / GS) + 3) & ~3;
  const size_t head = (size_t)a.k + sizeof(float) * g16 * (1 + W * R);
  size_t products = sizeof(float) * W * R * (size_t)row_layout(a.k, true).stride;
  if (a.xf) products = std::max(products, sizeof(float) * 4 * (size_t)chain_rowstride(a.k / 4));  // the squares
  const size_t lds = head + products;
  if constexpr (NS == 1) {
    if (a.xf) {
      if (a.xnorm) hipLaunchKernelGGL((gemv6_kernel<R, NS, 2, W>), dim3(blocks), dim3(64 * W), lds, s, a);
      else hipLaunchKernelGGL((gemv6_kernel<R, NS, 1, W>), dim3(blocks), dim3(64 * W), lds, s, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv6_kernel<R, NS, 0, W>), dim3(blocks), dim3(64 * W), lds, s, a);
  return hipGetLastError();
}

constexpr int32_t SMALL_ROWS6 = 8192;

hipError_t launch_decode6(const MatArgs &a, hipStream_t s) {
  const int steps = (a.k / GS + 127) / 128;  // 3 KiB steps of a row
  // the float32 token: 16 rows a block as the 4 waves of 4 rows, but 16 waves of one row (8 of two where the q/k/v
  // epilogue takes rows in pairs), so that quantize_x of the token is 4 values a thread
  if (steps <= 1) {
    // from xq: two rows a wave for the small matrices (q/k/v, wo: measured on cold copies at K = 3584, 4 rows a wave
    // leave too few waves for their few MB: q/k/v 7.0 -> 6.1 µs, wo 5.7 -> 5.4), four for the large
    if (!a.xf) return a.total_rows <= SMALL_ROWS6 ? launch_gemv6<2, 1>(a, s) : launch_gemv6<4, 1>(a, s);
    return a.qkv.on ? launch_gemv6<2, 1, 8>(a, s) : launch_gemv6<1, 1, 16>(a, s);
  }
  if (a.xf) return hipErrorInvalidValue;
  if (steps <= 2) return launch_gemv6<2, 2>(a, s);
  if (steps <= 4) return launch_gemv6<1, 4>(a, s);
  if (steps <= 5) return launch_gemv6<1, 5>(a, s);
  if (steps <= 6) return launch_gemv6<1, 6>(a, s);
  return hipErrorInvalidValue;
}

template <int R, int NS>
hipError_t launch_gemv1(const MatArgs &a, hipStream_t s) {
  if (a.xf && (NS > 4 || a.k % 32)) return hipErrorInvalidValue;
  const int waves = (a.total_rows + R - 1) / R;
  const int blocks = (waves + WAVES - 1) / WAVES;
  const size_t g16 = ((a.k / GS) + 3) & ~3;
  const size_t head = (size_t)a.k + sizeof(float) * g16 * (1 + WAVES * R);
  size_t products = sizeof(float) * WAVES * R * (size_t)row_layout(a.k, true).stride;
  if (a.xf) products = std::max(products, sizeof(float) * 4 * (size_t)chain_rowstride(a.k / 4));  // the squares
  const size_t lds = head + products;
  if constexpr (NS <= 4) {
    if (a.xf) {
      if (a.xnorm) hipLaunchKernelGGL((gemv1_kernel<R, NS, 2>), dim3(blocks), dim3(64 * WAVES), lds, s, a);
      else hipLaunchKernelGGL((gemv1_kernel<R, NS, 1>), dim3(blocks), dim3(64 * WAVES), lds, s, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv1_kernel<R, NS, 0>), dim3(blocks), dim3(64 * WAVES), lds, s, a);
  return hipGetLastError();
}

// the persistent grid: one block a CU (the device's count, asked once)
int persistent_blocks() {
  static int cus = 0;
  if (!cus) {
    int device = 0, n = 0;
    if (hipGetDevice(&device) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

constexpr size_t PLDS = 160 * 1024 - 1024;  // LDS a persistent block may take (gfx950: 160 KiB a workgroup)

// the LDS of a persistent block: the activations and their scales, every wave's rows' scales and products, the squares
size_t gemvp_lds(int pw, int r, int k, bool norm) {
  const size_t g16 = ((k / GS) + 3) & ~3;
  size_t lds = (size_t)k + sizeof(float) * g16 * (1 + (size_t)pw * r) +
               sizeof(float) * (size_t)pw * r * (size_t)row_layout(k, true).stride;
  if (norm) lds += sizeof(float) * 4 * (size_t)chain_rowstride(k / 4);
  return lds;
}

template <int PW, int R, int NS, int SRC, bool ALIGNED>
hipError_t launch_gemvp_one(const MatArgs &a, int blocks, size_t lds, hipStream_t s) {
  if (lds > 64 * 1024) {
    static bool sized = false;  // once a process: let the kernel take LDS past 64 KiB
    if (!sized) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemvp_kernel<PW, R, NS, SRC, ALIGNED>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)PLDS);
      if (e != hipSuccess) return e;
      sized = true;
    }
  }
  hipLaunchKernelGGL((gemvp_kernel<PW, R, NS, SRC, ALIGNED>), dim3(blocks), dim3(64 * PW), lds, s, a);
  return hipGetLastError();
}

// a persistent launch of PW waves a block and R rows a group over the device's CUs (one block a CU)
template <int PW, int R, int NS>
hipError_t launch_gemvp(const MatArgs &a, hipStream_t s, int blocks_a_cu = 1) {
  const bool f32 = a.xf != nullptr;
  if (f32 && (NS > 4 || a.k % 32)) return hipErrorInvalidValue;
  const int G = a.k / GS, ngroups = (a.total_rows + R - 1) / R;
  const int blocks = std::min((ngroups + PW - 1) / PW, blocks_a_cu * persistent_blocks());
  const size_t lds = gemvp_lds(PW, R, a.k, f32 && a.xnorm);
  if (lds > PLDS) return hipErrorInvalidValue;
  // the rows' scales as float4 where every segment's start and row length keep them on 16 bytes
  bool aligned = G % 4 == 0;
  for (int i = 0; i < a.nseg; ++i) aligned = aligned && reinterpret_cast<uintptr_t>(a.seg[i].ws) % 16 == 0;
  if constexpr (NS <= 4) {
    if (f32 && a.xnorm)
      return aligned ? launch_gemvp_one<PW, R, NS, 2, true>(a, blocks, lds, s)
                     : launch_gemvp_one<PW, R, NS, 2, false>(a, blocks, lds, s);
    if (f32)
      return aligned ? launch_gemvp_one<PW, R, NS, 1, true>(a, blocks, lds, s)
                     : launch_gemvp_one<PW, R, NS, 1, false>(a, blocks, lds, s);
  }
  return aligned ? launch_gemvp_one<PW, R, NS, 0, true>(a, blocks, lds, s)
                 : launch_gemvp_one<PW, R, NS, 0, false>(a, blocks, lds, s);
}

// the persistent path (measured on the 8B shapes: 8 waves a block and 2 rows a group for rows of 2-4 KiB, the output
// projection from the attention's float32 output 7.35 against 9.44 us for gemv1_kernel<4, 4>)
hipError_t launch_persistent(const MatArgs &a, hipStream_t s) {
  const int steps = (a.k / GS + 31) / 32;  // 1 KiB steps of a row
  if (steps <= 2) return launch_gemvp<8, 2, 2>(a, s);
  if (steps <= 4) return launch_gemvp<8, 2, 4>(a, s);
  return hipErrorInvalidValue;
}

hipError_t launch_decode(const MatArgs &a, hipStream_t s) {
  const int steps = (a.k / GS + 31) / 32;  // 1 KiB steps of a row
  if (steps <= 1) return launch_gemv1<4, 1>(a, s);
  if (steps <= 2) return launch_gemv1<4, 2>(a, s);
  // 4 KiB rows (measured over the Llama-3-8B shapes): 2 rows a wave for the larger matrices, 1 for 4096 rows or fewer
  // (a block that quantizes its own token: 4 rows a wave, so that fewer blocks repeat it)
  if (steps <= 4) {
    if (a.xf) return launch_gemv1<4, 4>(a, s);
    return a.total_rows > 4096 || a.qkv.on ? launch_gemv1<2, 4>(a, s) : launch_gemv1<1, 4>(a, s);
  }
  if (steps <= 8) return launch_gemv1<2, 8>(a, s);
  // 14 KiB rows (the 8B's w2) in exactly 14 steps: 16 steps a wave idle on 2 of them and run 4% slower
  if (steps <= 14) return launch_gemv1<1, 14>(a, s);
  if (steps <= 16) return launch_gemv1<1, 16>(a, s);
  if (steps <= 20) return launch_gemv1<1, 20>(a, s);
  return hipErrorInvalidValue;
}

template <int M, bool SIX, bool RELAXED, bool SUMS>
hipError_t launch_m(const MatArgs &a, hipStream_t s) {
  const int blocks = (a.total_rows + WAVES - 1) / WAVES;
  const size_t lds = SUMS ? 0 : sizeof(float) * WAVES * M * (size_t)row_layout(a.k, RELAXED).stride;
  hipLaunchKernelGGL((gemv_kernel<M, SIX, RELAXED, SUMS>), dim3(blocks), dim3(64 * WAVES), lds, s, a);
  return hipGetLastError();
}

template <bool SIX, bool RELAXED, bool SUMS>
hipError_t launch_sel(const MatArgs &a, hipStream_t s) {
  switch (a.m) {
    case 1: return launch_m<1, SIX, RELAXED, SUMS>(a, s);
    case 2: return launch_m<2, SIX, RELAXED, SUMS>(a, s);
    case 3: return launch_m<3, SIX, RELAXED, SUMS>(a, s);
    case 4: return launch_m<4, SIX, RELAXED, SUMS>(a, s);
    case 5: return launch_m<5, SIX, RELAXED, SUMS>(a, s);
    case 6: return launch_m<6, SIX, RELAXED, SUMS>(a, s);
    case 7: return launch_m<7, SIX, RELAXED, SUMS>(a, s);
    case 8: return launch_m<8, SIX, RELAXED, SUMS>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int32_t gemv_tokens(int32_t k, bool relaxed) {
  // the most tokens one launch takes: 8, fewer where a block's products would pass 64 KiB of LDS
  const size_t per_token = sizeof(float) * WAVES * (size_t)row_layout(k, relaxed).stride;
  int32_t m = (int32_t)((64 * 1024) / per_token);
  return m < 1 ? 0 : (m > 8 ? 8 : m);
}

bool decode_takes_f32(int32_t k, bool six, bool relaxed) {
  // int8 rows up to 4 KiB; int6 rows of one wave step (an even count of groups, up to 128)
  if (six) return relaxed && k <= 4 * 1024 && k % 64 == 0;
  return relaxed && k <= 4 * 1024 && k % 32 == 0;
}

bool decode_persistent(int32_t k, bool six, bool relaxed) { return !six && relaxed && k > 1024 && k <= 4 * 1024; }

// the decode paths whose waves take rows in pairs: int8 rows up to 8 KiB, int6 rows up to 256 groups (even)
bool decode_fuses_qkv(int32_t k, bool six, bool relaxed) {
  if (!relaxed) return false;
  return six ? (k / GS) % 2 == 0 && k <= 256 * GS : k <= 8 * 1024;
}

int32_t decode_block_rows(int32_t k, int32_t total_rows, bool six, bool relaxed, bool xf, bool qkv_on) {
  // launch_decode's and launch_decode6's choices of rows a wave (launch_gemv's one-token paths)
  if (!relaxed) return 0;
  if (!six) {
    if (k > 20 * 1024) return 0;
    const int steps = (k / GS + 31) / 32;
    if (steps <= 2) return 4 * WAVES;
    if (steps <= 4) return (xf ? 4 : (total_rows > 4096 || qkv_on ? 2 : 1)) * WAVES;
    if (steps <= 8) return 2 * WAVES;
    return WAVES;
  }
  if (k > 24 * 1024 || (k / GS) % 2) return 0;
  const int steps = (k / GS + 127) / 128;
  if (steps <= 1) return (!xf && total_rows <= SMALL_ROWS6 ? 2 : 4) * WAVES;
  if (steps <= 2) return 2 * WAVES;
  if (steps <= 6) return WAVES;
  return 0;
}

hipError_t launch_gemv(const MatArgs &a, bool six, bool relaxed, hipStream_t s) {
  const bool sums = a.sums != nullptr;
  if (a.xf && (sums || a.m != 1 || !decode_takes_f32(a.k, six, relaxed))) return hipErrorInvalidValue;
  if (a.qkv.on && (sums || a.m != 1 || !decode_fuses_qkv(a.k, six, relaxed))) return hipErrorInvalidValue;
  if (a.persistent && (sums || a.m != 1 || !decode_persistent(a.k, six, relaxed))) return hipErrorInvalidValue;
  if (a.persistent) return launch_persistent(a, s);
  if (!sums && !six && relaxed && a.m == 1 && a.k <= 20 * 1024) return launch_decode(a, s);
  if (!sums && six && relaxed && a.m == 1 && a.k <= 24 * 1024 && (a.k / GS) % 2 == 0) return launch_decode6(a, s);
  if (!sums && a.m > gemv_tokens(a.k, relaxed)) return hipErrorInvalidValue;
  if (six) {
    if (relaxed) return sums ? launch_sel<true, true, true>(a, s) : launch_sel<true, true, false>(a, s);
    return sums ? launch_sel<true, false, true>(a, s) : launch_sel<true, false, false>(a, s);
  }
  if (relaxed) return sums ? launch_sel<false, true, true>(a, s) : launch_sel<false, true, false>(a, s);
  return sums ? launch_sel<false, false, true>(a, s) : launch_sel<false, false, false>(a, s);
}

}  // namespace ple
