// sampling.hip — the repetition penalty and the draw of one token from temperature-scaled logits (restricted to the
// nucleus where 0 < topp < 1), to the token of kernels/kernel.ts:705-868 (penalize, sample, with largest at
// :423-445 and the nucleus of sortNucleus/intoNucleus at :729-787):
//   best = the largest logit (a NaN anywhere gives NaN): no token (-1) unless it is finite;
//   floor = nucleus ? best - temperature * 16.118095 : -FLT_MAX; kept, in index order: v - best for v >= floor;
//   p = vexp((v - best) * f32(1 / temperature)) for the first 4 * floor(count / 4), fexp((v - best) / temperature)
//   past them; total = their float64 sum in that order, top = the largest p;
//   nucleus: cutoff = min((1 - topp) / max(count - 1, 1) * total, top) in float64, the kept p >= cutoff sorted from
//   the most probable (equal ones in index order: the reference's quicksort leaves their order open), their float64
//   running sum up to the first >= topp * total;
//   the first token whose running float64 sum passes random * mass, else the last one taken.
// One block of 1024 threads: the order-free parts (the largest, the filters, the exponentials, the sort) in parallel,
// the float64 running sums by one thread from LDS in the reference's order.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

namespace {

constexpr int ST = 1024;         // threads of the sampling block
constexpr int SORT_MOST = 8192;  // nucleus tokens one block sorts (more: the step is declined, SAMPLE_DECLINED)
constexpr int STAGE = 16384;     // probabilities staged in LDS at a time for the running sums

// kernels/kernel.ts:705-719: each distinct token of tokens[0..count) once, value > 0 ? value / penalty : value * penalty
__global__ __launch_bounds__(64) void penalize_kernel(float *logits, const int32_t *tokens, int32_t count,
                                                     float penalty) {
  const int i = threadIdx.x;
  if (i >= count) return;
  const int32_t t = tokens[i];
  for (int j = 0; j < i; ++j)
    if (tokens[j] == t) return;  // a repeat: its first occurrence takes it
  const float v = logits[t];
  logits[t] = v > 0 ? v / penalty : v * penalty;
}

// the exclusive prefix sum of every thread's c over the block (threads in order), and the total
__device__ __forceinline__ int block_scan(int c, int *wave_sums, int *total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_sums[wave] = x;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < ST / 64; ++w) {
      const int s = wave_sums[w];
      wave_sums[w] = run;
      run += s;
    }
    *total = run;
  }
  __syncthreads();
  return wave_sums[wave] + x - c;
}

// (p, token) pairs: a before b where p is larger, or equal and the token smaller
__device__ __forceinline__ bool before(float pa, int ia, float pb, int ib) { return pa > pb || (pa == pb && ia < ib); }

__global__ __launch_bounds__(ST) void sample_kernel(const float *logits, int32_t n, float temperature, float topp,
                                                    double random, float *probs, int32_t *index, int32_t *out_token,
                                                    float *out_best) {
  __shared__ float4 area[SORT_MOST / 2];  // the sort's probabilities then tokens; the running sums' staging
  float *const sp = reinterpret_cast<float *>(area);
  int *const si = reinterpret_cast<int *>(area) + SORT_MOST;
  __shared__ float wf[ST / 64];
  __shared__ int wi[ST / 64];
  __shared__ float shared_best, shared_top;
  __shared__ int shared_count, shared_likely, shared_token;
  __shared__ double shared_total, shared_cutoff;
  static_assert(STAGE <= 2 * SORT_MOST, "the staging area is the sort's");
  float *const stage = reinterpret_cast<float *>(area);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // the largest logit (order-free: wmax keeps a NaN and puts +0 above -0)
  float b = logits[0];
  for (int i = tid; i < n; i += ST) b = wmax(b, logits[i]);
  for (int o = 32; o >= 1; o >>= 1) b = wmax(b, __shfl_xor(b, o, 64));
  if (lane == 0) wf[wave] = b;
  __syncthreads();
  if (tid == 0) {
    float x = wf[0];
    for (int w = 1; w < ST / 64; ++w) x = wmax(x, wf[w]);
    shared_best = x;
  }
  __syncthreads();
  const float best = shared_best;
  if (!__builtin_isfinite(best)) {
    if (tid == 0) {
      *out_token = SAMPLE_NOT_FINITE;
      *out_best = best;
    }
    return;  // the whole block
  }
  const bool nucleus = topp > 0 && topp < 1;
  const float floor_ = nucleus ? best - temperature * 16.118095f : -3.4028234663852886e38f;

  // kept: v - best for v >= floor in index order (each thread a contiguous run of the vocabulary), then p
  const int seg = (n + ST - 1) / ST, lo = min(n, tid * seg), hi = min(n, lo + seg);
  int c = 0;
  for (int i = lo; i < hi; ++i) c += logits[i] >= floor_;
  int k = block_scan(c, wi, &shared_count);
  const int count = shared_count, simd = count & ~3;
  const float inverse = 1.0f / temperature;
  for (int i = lo; i < hi; ++i) {
    const float v = logits[i];
    if (v >= floor_) {
      const float d = v - best;
      probs[k] = k < simd ? vexp(d * inverse) : fexp(d / temperature);
      index[k] = i;
      ++k;
    }
  }
  __syncthreads();

  // top (order-free) and total (float64, in order: one thread from LDS)
  float t = 0.0f;
  for (int j = tid; j < count; j += ST) t = __builtin_fmaxf(t, probs[j]);
  for (int o = 32; o >= 1; o >>= 1) t = __builtin_fmaxf(t, __shfl_xor(t, o, 64));
  if (lane == 0) wf[wave] = t;
  double total = 0.0;
  for (int base = 0; base < count; base += STAGE) {
    const int len = min(STAGE, count - base);
    __syncthreads();
    for (int j = tid; j < len; j += ST) stage[j] = probs[base + j];
    __syncthreads();
    if (tid == 0)
      for (int j = 0; j < len; ++j) total += (double)stage[j];
  }
  if (tid == 0) {
    float x = wf[0];
    for (int w = 1; w < ST / 64; ++w) x = __builtin_fmaxf(x, wf[w]);
    shared_top = x;
    shared_total = total;
  }
  __syncthreads();
  total = shared_total;

  if (!nucleus) {
    // the running sum in index order up to the first that passes random * total
    const double target = random * total;
    double cumulative = 0.0;
    int token = -1;
    for (int base = 0; base < count && token < 0; base += STAGE) {
      const int len = min(STAGE, count - base);
      __syncthreads();
      for (int j = tid; j < len; j += ST) stage[j] = probs[base + j];
      __syncthreads();
      if (tid == 0) {
        for (int j = 0; j < len; ++j) {
          cumulative += (double)stage[j];
          if (cumulative > target) {
            shared_token = base + j;
            break;
          }
        }
        if (!(cumulative > target)) shared_token = -1;
      }
      __syncthreads();
      token = shared_token;
    }
    if (tid == 0) {
      *out_token = index[token >= 0 ? token : count - 1];
      *out_best = best;
    }
    return;
  }

  // the nucleus: the kept p >= cutoff, sorted from the most probable
  if (tid == 0) {
    const double ceiling = (1.0 - (double)topp) / (double)(count > 1 ? count - 1 : 1) * total;
    const double top = (double)shared_top;
    shared_cutoff = ceiling < top ? ceiling : top;
  }
  __syncthreads();
  const double cutoff = shared_cutoff;
  const int kseg = (count + ST - 1) / ST, klo = min(count, tid * kseg), khi = min(count, klo + kseg);
  int lc = 0;
  for (int j = klo; j < khi; ++j) lc += (double)probs[j] >= cutoff;
  int at = block_scan(lc, wi, &shared_likely);
  const int likely = shared_likely;
  if (likely > SORT_MOST) {
    if (tid == 0) {
      *out_token = SAMPLE_DECLINED;
      *out_best = best;
    }
    return;
  }
  for (int j = klo; j < khi; ++j) {
    const float p = probs[j];
    if ((double)p >= cutoff) {
      sp[at] = p;
      si[at] = index[j];
      ++at;
    }
  }
  int size = 1;
  while (size < likely) size <<= 1;
  for (int j = likely + tid; j < size; j += ST) {
    sp[j] = -1.0f;  // below every probability: sorted last
    si[j] = 0x7fffffff;
  }
  __syncthreads();
  // bitonic sort of size pairs into the order of before()
  for (int width = 2; width <= size; width <<= 1) {
    for (int stride = width >> 1; stride > 0; stride >>= 1) {
      for (int j = tid; j < size; j += ST) {
        const int partner = j ^ stride;
        if (partner > j) {
          const bool forward = (j & width) == 0;
          const float pa = sp[j], pb = sp[partner];
          const int ia = si[j], ib = si[partner];
          if (before(pb, ib, pa, ia) == forward) {
            sp[j] = pb;
            si[j] = ib;
            sp[partner] = pa;
            si[partner] = ia;
          }
        }
      }
      __syncthreads();
    }
  }
  if (tid == 0) {
    const double limit = (double)topp * total;
    double mass = 0.0;
    int last = likely - 1;
    for (int j = 0; j < likely; ++j) {
      mass += (double)sp[j];
      if (mass >= limit) {
        last = j;
        break;
      }
    }
    const double target = random * mass;
    double cumulative = 0.0;
    int token = si[last];
    for (int j = 0; j <= last; ++j) {
      cumulative += (double)sp[j];
      if (cumulative > target) {
        token = si[j];
        break;
      }
    }
    *out_token = token;
    *out_best = best;
  }
}

}  // namespace

hipError_t launch_penalize(float *logits, const int32_t *tokens, int32_t count, float penalty, hipStream_t s) {
  if (count < 1) return hipSuccess;
  if (count > 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL(penalize_kernel, dim3(1), dim3(64), 0, s, logits, tokens, count, penalty);
  return hipGetLastError();
}

hipError_t launch_sample(const float *logits, int32_t n, float temperature, float topp, double random, float *probs,
                         int32_t *index, int32_t *out_token, float *out_best, hipStream_t s) {
  if (n < 1 || !(temperature > 0)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(ST), 0, s, logits, n, temperature, topp, random, probs, index,
                     out_token, out_best);
  return hipGetLastError();
}

}  // namespace ple
