// gemv.hip — the decode matmul (m <= 8 tokens) of int8/int6 rows against quantized activations, to the bit of the
// reference's CPU kernels:
//   bias 64: kernels/kernel_relaxed.ts:34-67 matmul_q8r (and :195-218 matmul_q6r): per group the exact integer
//            S_g = dot(w, q - 64); lane g % 4 of four float32 accumulators adds f32(S_g) * f32(ws * xs) for the groups
//            in fours, in order; the lanes are added ((l0 + l1) + l2) + l3; the groups past the fours one at a time.
//   bias 0:  kernels/kernel.ts:231-258 matmul_q8 (and :261-278 matmul_q6): four int32 lane sums a group (lane k:
//            products 2k, 2k+1, 2k+8, 2k+9 of each half), each scaled into its own accumulator over every group in
//            order, the four added in order.
// Layout: one wave streams one row (grid-stride over rows). An int8 row is read 16 bytes a lane (a group is a lane
// pair, 1 KiB a wave step); an int6 row 24 bytes a lane (a group a lane, 1.5 KiB a step). The int32 sums come from
// v_dot4_i32_i8; the products go through LDS to the lanes that hold the float32 accumulators (4 per token), which add
// them in the reference's order while the next step's loads are in flight.
#pragma clang fp contract(off)

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

namespace {

constexpr int WAVES = 4;

template <int M, bool SIX, bool RELAXED>
struct GemvShape {
  static constexpr int GPI = SIX ? 64 : 32;                   // groups a wave step
  static constexpr int PER = RELAXED ? GPI : GPI * 4;          // products a token a step
};

template <int M, bool SIX, bool RELAXED, bool SUMS>
__global__ __launch_bounds__(256) void gemv_kernel(const MatArgs a) {
  using Sh = GemvShape<M, SIX, RELAXED>;
  constexpr int GPI = Sh::GPI;
  __shared__ float prod[WAVES][M * Sh::PER];
  __shared__ float tail[WAVES][M * 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float *P = prod[wave];
  const int K = a.k, G = K / GS, G4 = G & ~3;
  const int iters = (G + GPI - 1) / GPI;
  const bool holder = SIX ? true : ((lane & 1) == 0);
  const int mylocal = SIX ? lane : (lane >> 1);  // this lane's group within a step

  for (int row = blockIdx.x * WAVES + wave; row < a.total_rows; row += gridDim.x * WAVES) {
    int s = 0, r = row;
    while (s + 1 < a.nseg && r >= a.seg[s].rows) {
      r -= a.seg[s].rows;
      ++s;
    }
    const MatSeg sg = a.seg[s];
    const uint8_t *wrow = sg.w + (int64_t)r * (SIX ? (int64_t)G * 24 : (int64_t)K);
    const float *srow = sg.ws + (int64_t)r * G;
    float chain = 0.0f;  // lane 4t + k (t < M): accumulator k of token t

    for (int it = 0; it < iters; ++it) {
      const int g = it * GPI + mylocal;
      const bool active = g < G;
      int32_t S[M][RELAXED ? 1 : 4];
#pragma unroll
      for (int t = 0; t < M; ++t)
#pragma unroll
        for (int k = 0; k < (RELAXED ? 1 : 4); ++k) S[t][k] = 0;
      if (active) {
        uint32_t w[SIX ? 8 : 4];
        if constexpr (SIX) {
          const uint2 *p = reinterpret_cast<const uint2 *>(wrow + (int64_t)g * 24);
          const uint2 l0 = p[0], l1 = p[1], tops = p[2];
          const uint32_t L[4] = {l0.x, l0.y, l1.x, l1.y};
          six_widen(L, tops.x, tops.y, w);
        } else {
          const uint4 v = *reinterpret_cast<const uint4 *>(wrow + (int64_t)g * 32 + (lane & 1) * 16);
          w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        }
#pragma unroll
        for (int t = 0; t < M; ++t) {
          const int8_t *xt = a.xq + (int64_t)t * a.xq_stride + g * 32;
          uint32_t x[SIX ? 8 : 4];
          if constexpr (SIX) {
            const uint4 x0 = reinterpret_cast<const uint4 *>(xt)[0], x1 = reinterpret_cast<const uint4 *>(xt)[1];
            x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w; x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
          } else {
            const uint4 x0 = *reinterpret_cast<const uint4 *>(xt + (lane & 1) * 16);
            x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
          }
          constexpr int NW = SIX ? 8 : 4;
          if constexpr (RELAXED) {
            int32_t acc = 0;
#pragma unroll
            for (int i = 0; i < NW; ++i) acc = dot4(w[i], centre4(x[i]), acc);
            S[t][0] = acc;
          } else {
            // lane k of kernels/kernel.ts:222-229: bytes {2k, 2k+1} of words 0/2 (k < 2) or 1/3 (k >= 2) of each half
#pragma unroll
            for (int h = 0; h < NW; h += 4) {
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
      }
      if constexpr (!SIX) {
#pragma unroll
        for (int t = 0; t < M; ++t)
#pragma unroll
          for (int k = 0; k < (RELAXED ? 1 : 4); ++k) S[t][k] += __shfl_xor(S[t][k], 1, 64);
      }
      if constexpr (SUMS) {
        if (holder && active) {
#pragma unroll
          for (int t = 0; t < M; ++t) {
            int32_t *o = a.sums + (((int64_t)t * a.total_rows + row) * G + g) * (RELAXED ? 1 : 4);
#pragma unroll
            for (int k = 0; k < (RELAXED ? 1 : 4); ++k) o[k] = S[t][k];
          }
        }
        continue;
      }
      if (holder && active) {
        const float wsg = srow[g];
#pragma unroll
        for (int t = 0; t < M; ++t) {
          const float scale = wsg * a.xs[(int64_t)t * a.xs_stride + g];
          if constexpr (RELAXED) {
            const float p = (float)S[t][0] * scale;
            if (g < G4) P[t * GPI + (mylocal & 3) * (GPI / 4) + (mylocal >> 2)] = p;
            else tail[wave][t * 4 + (g - G4)] = p;
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) P[t * GPI * 4 + k * GPI + mylocal] = (float)S[t][k] * scale;
          }
        }
      }
      wave_sync_lds();
      if (lane < 4 * M) {
        const int t = lane >> 2, k = lane & 3;
        if constexpr (RELAXED) {
          const int n = min(GPI, G4 - it * GPI);  // groups of this step below G4 (a multiple of 4, or <= 0)
          const float *c = P + t * GPI + k * (GPI / 4);
          for (int j = 0; j < n / 4; ++j) chain = chain + c[j];
        } else {
          const int n = min(GPI, G - it * GPI);
          const float *c = P + t * GPI * 4 + k * GPI;
          for (int j = 0; j < n; ++j) chain = chain + c[j];
        }
      }
      wave_sync_lds();
    }
    if constexpr (SUMS) continue;
    const int src = (lane < M ? lane : 0) * 4;
    const float c0 = __shfl(chain, src, 64), c1 = __shfl(chain, src + 1, 64);
    const float c2 = __shfl(chain, src + 2, 64), c3 = __shfl(chain, src + 3, 64);
    if (lane < M) {
      float sum = ((c0 + c1) + c2) + c3;
      if constexpr (RELAXED) {
        for (int g = G4; g < G; ++g) sum = sum + tail[wave][lane * 4 + (g - G4)];
      }
      float *y = sg.y + (int64_t)lane * sg.y_stride + r;
      *y = sg.accumulate ? *y + sum : sum;
    }
    wave_sync_lds();
  }
}

template <int M, bool SIX, bool RELAXED, bool SUMS>
hipError_t launch_m(const MatArgs &a, hipStream_t s) {
  const int64_t waves = a.total_rows;
  int blocks = (int)((waves + WAVES - 1) / WAVES);
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL((gemv_kernel<M, SIX, RELAXED, SUMS>), dim3(blocks), dim3(64 * WAVES), 0, s, a);
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

hipError_t launch_gemv(const MatArgs &a, bool six, bool relaxed, hipStream_t s) {
  const bool sums = a.sums != nullptr;
  if (six) {
    if (relaxed) return sums ? launch_sel<true, true, true>(a, s) : launch_sel<true, true, false>(a, s);
    return sums ? launch_sel<true, false, true>(a, s) : launch_sel<true, false, false>(a, s);
  }
  if (relaxed) return sums ? launch_sel<false, true, true>(a, s) : launch_sel<false, true, false>(a, s);
  return sums ? launch_sel<false, false, true>(a, s) : launch_sel<false, false, false>(a, s);
}

}  // namespace ple
