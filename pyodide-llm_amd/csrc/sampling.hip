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
// One block of 1024 threads: the order-free parts (the largest, the filters, the exponentials, the sort) in parallel;
// the float64 total in the reference's order by one wave from registers (sum_wave), the draw's running sums by one
// thread from the total's checkpoints.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

namespace {

constexpr int ST = 1024;         // threads of the sampling block
constexpr int SORT_MOST = 8192;  // nucleus tokens one block sorts (more: the step is declined, SAMPLE_DECLINED)
constexpr int VU = 8;            // loads of the vocabulary a thread has in flight in the block's passes over it
constexpr int STAGE = 16384;     // floats of the LDS area the sort and the running sums' staging share

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

// The float64 running sums of the draw are sequential (the reference's order: one add after another in index order).
// The total runs from registers: a dependent float64 add takes about 6 cycles from registers and about twice that
// when its values come from LDS reads, whose issue then sets the pace.
constexpr int CP_BLOCK = 256;                     // values between two checkpoints of the running sum
constexpr int CP_MOST = SAMPLE_MOST / CP_BLOCK;   // checkpoints of the largest vocabulary
constexpr int SEG = 32;                           // values a lane adds in its turn
constexpr int CHUNK = 64 * SEG;                   // values a wave holds at a time
static_assert(CHUNK == SAMPLE_CHUNK, "the probabilities' buffers hold whole chunks");
static_assert(CP_BLOCK % SEG == 0, "a checkpoint falls on a lane's first value");

// the 64-bit value of lane - 1 (lane 0: any), by DPP: a row shift by one, or (EDGE, for a row's first lane) lane 15
// of the row before
template <bool EDGE>
__device__ __forceinline__ double from_lane_below(double x) {
  constexpr int ctrl = EDGE ? 0x142 : 0x111;  // row_bcast:15, row_shr:1
  const int lo = __double2loint(x), hi = __double2hiint(x);
  return __hiloint2double(__builtin_amdgcn_update_dpp(hi, hi, ctrl, 0xF, 0xF, false),
                          __builtin_amdgcn_update_dpp(lo, lo, ctrl, 0xF, 0xF, false));
}

// p[0] + p[1] + ... + p[count-1] in float64 (each p widened exactly), in order, by one wave: lane L holds
// p[b + 32 L .. b + 32 L + 31] of a chunk of 2048 in registers (+0.0 past count, which changes no sum), and in turn s
// lane s adds its 32 to the running sum lane s - 1 handed it, so that an add waits on the add before it only; the
// next chunk's reads fly meanwhile. With cp, cp[i / CP_BLOCK] = the sum before value i for every multiple i of
// CP_BLOCK below count. Every lane returns the total. (p: 16-byte aligned, count >= 1, room for whole chunks:
// sample_probs_floats(count) floats.)
__device__ double sum_wave(const float *p, int count, double *cp) {
  const int lane = threadIdx.x & 63;
  float4 nx[SEG / 4];
  auto fetch = [&](int b) {  // (past count: what the buffer holds there, masked to +0.0 below)
    const int i0 = b + lane * SEG;
#pragma unroll
    for (int u = 0; u < SEG / 4; ++u) nx[u] = reinterpret_cast<const float4 *>(p + i0)[u];
  };
  double run = 0.0;  // the sum before the chunk
  fetch(0);
  for (int b = 0; b < count; b += CHUNK) {
    double v[SEG];
    const int left = count - b - lane * SEG;  // this lane's values below count
#pragma unroll
    for (int u = 0; u < SEG / 4; ++u) {
      v[4 * u] = 4 * u < left ? (double)nx[u].x : 0.0;
      v[4 * u + 1] = 4 * u + 1 < left ? (double)nx[u].y : 0.0;
      v[4 * u + 2] = 4 * u + 2 < left ? (double)nx[u].z : 0.0;
      v[4 * u + 3] = 4 * u + 3 < left ? (double)nx[u].w : 0.0;
    }
    if (b + CHUNK < count) fetch(b + CHUNK);
    // acc: lane 0's start now, each other lane's from its turn on (the sum before its values); the turns unrolled
    // by rows of 16, so that each hand-on's DPP form is fixed
    double acc = run;
    double sum = run;
    for (int s0 = 0; s0 < 64; s0 += 16) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        sum = acc;
#pragma unroll
        for (int u = 0; u < SEG; ++u) sum = sum + v[u];
        const double moved = k == 15 ? from_lane_below<true>(sum) : from_lane_below<false>(sum);
        acc = lane == s0 + k + 1 ? moved : acc;
      }
    }
    if (cp && lane % (CP_BLOCK / SEG) == 0 && b + SEG * lane < count) cp[(b + SEG * lane) / CP_BLOCK] = acc;
    run = __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(sum), 63),
                           __builtin_amdgcn_readlane(__double2loint(sum), 63));
  }
  return run;
}

// the first j < len whose running sum acc + v[0] + ... + v[j] (float64, in order) passes target (REACH: reaches it), or
// -1; *acc_out the sum reached (v 16-byte aligned)
template <bool REACH = false>
__device__ __forceinline__ int first_past(const float *v, int len, double acc, double target, double *acc_out) {
  auto past = [&](double a) { return REACH ? a >= target : a > target; };
  const float4 *v4 = reinterpret_cast<const float4 *>(v);
  int i = 0;
  for (; i + 32 <= len; i += 32) {
    float4 a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] = v4[i / 4 + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float x[4] = {a[u].x, a[u].y, a[u].z, a[u].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc += (double)x[k];
        if (past(acc)) {
          *acc_out = acc;
          return i + 4 * u + k;
        }
      }
    }
  }
  for (; i < len; ++i) {
    acc += (double)v[i];
    if (past(acc)) {
      *acc_out = acc;
      return i;
    }
  }
  *acc_out = acc;
  return -1;
}

// (p, token) pairs: a before b where p is larger, or equal and the token smaller
__device__ __forceinline__ bool before(float pa, int ia, float pb, int ib) { return pa > pb || (pa == pb && ia < ib); }

__device__ __forceinline__ void sample_block(const float *logits, int32_t n, float temperature, float topp,
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
  __shared__ double checkpoints[CP_MOST];  // the running sum of the kept p before every CP_BLOCK of them
  static_assert(STAGE <= 2 * SORT_MOST, "the staging area is the sort's");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // the largest logit (order-free: wmax keeps a NaN and puts +0 above -0)
  float b = logits[0];
  for (int i0 = tid; i0 < n; i0 += ST * VU) {  // VU loads in flight a thread (clamped: a repeat changes no max)
    float v[VU];
#pragma unroll
    for (int u = 0; u < VU; ++u) v[u] = logits[min(i0 + ST * u, n - 1)];
#pragma unroll
    for (int u = 0; u < VU; ++u) b = wmax(b, v[u]);
  }
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

  // kept: v - best for v >= floor in index order, then p. Each wave takes a contiguous run of the vocabulary, 64
  // values a step side by side: the count of its run, a block scan over the waves, then the kept values' places in
  // order (the lanes below in the step, the steps before)
  const int wrun = ((n + ST / 64 - 1) / (ST / 64) + 63) & ~63, wlo = min(n, wave * wrun), whi = min(n, wlo + wrun);
  const uint64_t below = (1ull << lane) - 1;
  int c = 0;
  for (int i0 = wlo + lane; i0 < whi; i0 += 64 * VU) {
    float v[VU];
#pragma unroll
    for (int u = 0; u < VU; ++u) v[u] = logits[min(i0 + 64 * u, n - 1)];
#pragma unroll
    for (int u = 0; u < VU; ++u) c += i0 + 64 * u < whi && v[u] >= floor_;
  }
  for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
  int k = block_scan(lane == 0 ? c : 0, wi, &shared_count);
  k = __shfl(k, 0, 64);
  const int count = shared_count, simd = count & ~3;
  const float inverse = 1.0f / temperature;
  for (int j0 = wlo; j0 < whi; j0 += 64 * VU) {
    float vs[VU];  // every load of the pass requested before its stores (clamped, unconditional)
#pragma unroll
    for (int u = 0; u < VU; ++u) vs[u] = logits[min(j0 + 64 * u + lane, n - 1)];
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int i = j0 + 64 * u + lane;
      const float v = vs[u];
      const bool keep = i < whi && v >= floor_;
      const uint64_t mask = __ballot(keep);
      if (keep) {
        const int at = k + __popcll(mask & below);
        const float d = v - best;
        probs[at] = at < simd ? vexp(d * inverse) : fexp(d / temperature);
        index[at] = i;
      }
      k += __popcll(mask);
    }
  }
  __syncthreads();

  // top (order-free) and total (float64, in order: one thread from LDS)
  float t = 0.0f;
  for (int j = tid; j < count; j += ST) t = __builtin_fmaxf(t, probs[j]);
  for (int o = 32; o >= 1; o >>= 1) t = __builtin_fmaxf(t, __shfl_xor(t, o, 64));
  if (lane == 0) wf[wave] = t;
  // total: float64, in order, by wave 0 from registers
  double total = 0.0;
  if (wave == 0) total = sum_wave(probs, count, checkpoints);
  __syncthreads();  // (the waves' maxima in wf too)
  if (tid == 0) {
    float x = wf[0];
    for (int w = 1; w < ST / 64; ++w) x = __builtin_fmaxf(x, wf[w]);
    shared_top = x;
    shared_total = total;
  }
  __syncthreads();
  total = shared_total;

  if (!nucleus) {
    // the running sum in index order up to the first that passes random * total: the block of CP_BLOCK where it
    // passes, from the checkpoints (the sum never decreases: every p >= 0), then that block's adds again from its
    // checkpoint (the same adds, the same bits)
    if (tid == 0) {
      const double target = random * total;
      const int blocks = (count + CP_BLOCK - 1) / CP_BLOCK;
      // the first block b whose end (the sum before block b + 1, or the total) passes target, blocks if none: the ends
      // never decrease, so by halving
      int b = 0, hi = blocks;
      while (b < hi) {
        const int mid = (b + hi) / 2;
        if ((mid + 1 < blocks ? checkpoints[mid + 1] : total) <= target) b = mid + 1;
        else hi = mid;
      }
      int token = -1;
      if (b < blocks) {
        double reached = 0.0;
        const int j = first_past(probs + b * CP_BLOCK, min(CP_BLOCK, count - b * CP_BLOCK), checkpoints[b], target,
                                 &reached);
        if (j >= 0) token = b * CP_BLOCK + j;
      }
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
  // the kept p >= cutoff, in order: a wave a contiguous run, as above
  const int krun = ((count + ST / 64 - 1) / (ST / 64) + 63) & ~63, klo = min(count, wave * krun),
            khi = min(count, klo + krun);
  int lc = 0;
  for (int j = klo + lane; j < khi; j += 64) lc += (double)probs[j] >= cutoff;
  for (int o = 32; o >= 1; o >>= 1) lc += __shfl_xor(lc, o, 64);
  int at = block_scan(lane == 0 ? lc : 0, wi, &shared_likely);
  at = __shfl(at, 0, 64);
  const int likely = shared_likely;
  if (likely > SORT_MOST) {
    if (tid == 0) {
      *out_token = SAMPLE_DECLINED;
      *out_best = best;
    }
    return;
  }
  for (int j0 = klo; j0 < khi; j0 += 64) {
    const int j = j0 + lane;
    const float p = j < khi ? probs[j] : 0.0f;
    const bool keep = j < khi && (double)p >= cutoff;
    const uint64_t mask = __ballot(keep);
    if (keep) {
      const int to = at + __popcll(mask & below);
      sp[to] = p;
      si[to] = index[j];
    }
    at += __popcll(mask);
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
    // the nucleus: the running sum from the most probable up to the first that reaches topp * total; then the draw
    // within it
    const double limit = (double)topp * total;
    double mass = 0.0;
    int last = first_past<true>(sp, likely, 0.0, limit, &mass);
    if (last < 0) last = likely - 1;
    const double target = random * mass;
    double reached = 0.0;
    const int j = first_past(sp, last + 1, 0.0, target, &reached);
    *out_token = si[j >= 0 ? j : last];
    *out_best = best;
  }
}

__global__ __launch_bounds__(ST) void sample_kernel(const float *logits, int32_t n, float temperature, float topp,
                                                    double random, float *probs, int32_t *index, int32_t *out_token,
                                                    float *out_best) {
  sample_block(logits, n, temperature, topp, random, probs, index, out_token, out_best);
}

// ---- the sampled steps of a replayed graph: settings, random numbers and the penalty's window in device memory ----

// a step's draw: the temperature and top-p of the call, the round's random number of this step (state[STATE_STEP])
__global__ __launch_bounds__(ST) void sample_steps_kernel(const float *logits, int32_t n, const RunParams *params,
                                                          const int32_t *state, float *probs, int32_t *index,
                                                          int32_t *out_token, float *out_best) {
  sample_block(logits, n, params->temperature, params->topp, params->randoms[state[STATE_STEP]], probs, index,
               out_token, out_best);
}

// the penalty of the call over the window's state[STATE_WINDOW] tokens (in any order: each distinct one once)
__global__ __launch_bounds__(64) void penalize_steps_kernel(float *logits, const int32_t *window, const int32_t *state,
                                                           const RunParams *params) {
  const int i = threadIdx.x, count = state[STATE_WINDOW];
  if (i >= count) return;
  const int32_t t = window[i];
  for (int j = 0; j < i; ++j)
    if (window[j] == t) return;  // a repeat: its first occurrence takes it
  const float penalty = params->penalty, v = logits[t];
  logits[t] = v > 0 ? v / penalty : v * penalty;
}

// whether the step that chose `token` with largest logit `value` ends the call: a token that is not one (the draw's
// SAMPLE_NOT_FINITE or SAMPLE_DECLINED), a largest logit that is not finite, or a stop token
__device__ __forceinline__ bool halts(int32_t token, float value, const RunParams *params) {
  if (token < 0 || !__builtin_isfinite(value)) return true;
  const int ns = params->n_stops;
  for (int j = 0; j < RUN_STOPS_MOST; ++j)
    if (j < ns && params->stops[j] == token) return true;
  return false;
}

// the logits of the step that ends the call, kept (the replays after it in the round overwrite the step's own)
__global__ __launch_bounds__(256) void keep_halting_kernel(const float *logits, int32_t n, float *kept,
                                                           const int32_t *token, const float *value,
                                                           const int32_t *state, const RunParams *params) {
  if (state[STATE_HALTED] != 0 || !halts(*token, *value, params)) return;  // (the same for every block)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    kept[i] = logits[i];
}

// the end of a replayed step: its token and largest logit into ids / values at the step, the halting step noted
// (state[STATE_HALTED] = step + 1, the first one only), the token appended to the penalty's window (a ring of
// REPETITION_WINDOW once full), the token made the next step's input (a valid one after a step that chose none), the
// position and the step advanced
__global__ void advance_steps_kernel(int32_t *tokens, int32_t *state, const int32_t *token, const float *value,
                                     int32_t *ids, float *values, int32_t *window, const RunParams *params) {
  const int32_t step = state[STATE_STEP], b = *token;
  const float v = *value;
  ids[step] = b;
  values[step] = v;
  if (state[STATE_HALTED] == 0 && halts(b, v, params)) state[STATE_HALTED] = step + 1;
  if (b >= 0) {
    const int32_t count = state[STATE_WINDOW];
    if (count < RUN_WINDOW) {
      window[count] = b;
      state[STATE_WINDOW] = count + 1;
    } else {
      const int32_t head = state[STATE_HEAD];
      window[head] = b;
      state[STATE_HEAD] = head + 1 == RUN_WINDOW ? 0 : head + 1;
    }
  }
  tokens[0] = b >= 0 ? b : 0;
  state[STATE_POS] = state[STATE_POS] + 1;
  state[STATE_STEP] = step + 1;
}

}  // namespace

hipError_t launch_sample_steps(const float *logits, int32_t n, const RunParams *params, const int32_t *state,
                               float *probs, int32_t *index, int32_t *out_token, float *out_best, hipStream_t s) {
  if (n < 1 || n > SAMPLE_MOST) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_steps_kernel, dim3(1), dim3(ST), 0, s, logits, n, params, state, probs, index, out_token,
                     out_best);
  return hipGetLastError();
}

hipError_t launch_penalize_steps(float *logits, const int32_t *window, const int32_t *state, const RunParams *params,
                                 hipStream_t s) {
  hipLaunchKernelGGL(penalize_steps_kernel, dim3(1), dim3(RUN_WINDOW), 0, s, logits, window, state, params);
  return hipGetLastError();
}

hipError_t launch_step_end(const float *logits, int32_t n, float *kept, int32_t *tokens, int32_t *state,
                           const int32_t *token, const float *value, int32_t *ids, float *values, int32_t *window,
                           const RunParams *params, hipStream_t s) {
  const int blocks = (int)std::min<int64_t>(128, ((int64_t)n + 1023) / 1024);
  hipLaunchKernelGGL(keep_halting_kernel, dim3(blocks), dim3(256), 0, s, logits, n, kept, token, value, state, params);
  hipLaunchKernelGGL(advance_steps_kernel, dim3(1), dim3(1), 0, s, tokens, state, token, value, ids, values, window,
                     params);
  return hipGetLastError();
}

hipError_t launch_penalize(float *logits, const int32_t *tokens, int32_t count, float penalty, hipStream_t s) {
  if (count < 1) return hipSuccess;
  if (count > 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL(penalize_kernel, dim3(1), dim3(64), 0, s, logits, tokens, count, penalty);
  return hipGetLastError();
}

hipError_t launch_sample(const float *logits, int32_t n, float temperature, float topp, double random, float *probs,
                         int32_t *index, int32_t *out_token, float *out_best, hipStream_t s) {
  if (n < 1 || n > SAMPLE_MOST || !(temperature > 0)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(ST), 0, s, logits, n, temperature, topp, random, probs, index,
                     out_token, out_best);
  return hipGetLastError();
}

}  // namespace ple
