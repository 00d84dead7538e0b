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
// the float64 total with the bits of the reference's order, taken in parallel (sum_block), the draw's running sums by
// one thread from the total's checkpoints.
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
template <int NT = ST>
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
    for (int w = 0; w < NT / 64; ++w) {
      const int s = wave_sums[w];
      wave_sums[w] = run;
      run += s;
    }
    *total = run;
  }
  __syncthreads();
  return wave_sums[wave] + x - c;
}

// The float64 running sums of the draw are sequential in the reference's order (one add after another in index order):
// the total takes their bits in parallel (sum_block), the draw's search runs them from a checkpoint.
constexpr int CP_BLOCK = SAMPLE_CHECKPOINT;       // values between two checkpoints of the running sum
constexpr int CP_MOST = SAMPLE_MOST / CP_BLOCK;   // checkpoints of the largest vocabulary
constexpr int SEG = 32;                           // values a lane holds of a chunk
constexpr int CHUNK = 64 * SEG;                   // values a wave holds at a time
static_assert(CHUNK == SAMPLE_CHUNK, "the probabilities' buffers hold whole chunks");
static_assert(CP_BLOCK % SEG == 0, "a checkpoint falls on a lane's first value");

// A chunk's float64 sum in parallel, with the bits of the sequential adds, while the running sum stays in one binade.
// With run in [2^e, 2^(e+1)) every sum that stays below 2^(e+1) is a multiple of u = 2^(e-52), and fl(s + x) = s + r u
// where r is x / u rounded to the nearest integer: that does not depend on s, except on an exact tie (x / u = q + 1/2),
// which rounds to the even multiple, so that r = q + ((s / u + q) odd) and the sum after it is even. So each lane
// takes its 32 r as a function of the parity of s / u before them (none of them a tie: a fixed sum and a flip of the
// parity; else a sum plus 0 or 1 by the incoming parity at the first tie, and a fixed parity after), the lanes'
// incoming parities follow from lane masks (the last lane with a tie and the flips since), and the r are exact
// integers in float64 below 2^53. Lanes below from take no part (their values are done). Returns the first lane
// (from..63) whose values take the sum to 2^(e+1) or past it, 64 if none; *start is the sum before this lane's values
// (right for the lanes from..the returned one), *end the chunk's end where 64 is returned.
// a lane's 32 values as r at grid 2^(e-52) (see above): the sum of r with the first tie's 1 left out, whether a tie was
// seen, the parity flips after the last tie (or of all of them where none was), and the first tie's c
struct LaneR {
  double s0;
  int seen, x, cfirst;
};

__device__ __forceinline__ LaneR lane_r(const float (&v)[SEG], int e) {
  // per value (all exact): y = x / u, q = floor(y); g = 2 (y - q) in [0, 2), ge = floor(g) (y - q >= 1/2), whole =
  // g has no fraction; tie = ge and whole, up = ge and not whole; odd = q's last bit. The flags are made 0 / 1 by
  // arithmetic and kept as integers, and the q summed on their own, so that nothing waits on the ties' order.
  // The lane's state in one integer: bit 0 the flips since the last tie, bit 1 a tie seen, bit 2 the first tie's c,
  // from bit 3 up the 1s added.
  int st = 0;
  double sq = 0.0;  // the lane's sum of q
#pragma unroll
  for (int u = 0; u < SEG; ++u) {
    float vu = v[u];
    asm volatile("" : "+v"(vu));  // (each value's work starts here: none of it is hoisted above the last's)
    const double y = __builtin_ldexp((double)vu, 52 - e);  // x / u, exact
    const double q = __builtin_floor(y);
    const double g = (y - q) * 2.0, gi = __builtin_floor(g);
    const double h = q * 0.5;
    const int odd = (int)((h - __builtin_floor(h)) * 2.0);
    const int ge = (int)gi, frac = (int)__builtin_ceil(g - gi);
    const int tie = ge & (frac ^ 1), up = ge & frac;
    sq = sq + q;
    const int x = st & 1, seen = (st >> 1) & 1;
    const int a = x ^ odd;  // a tie's extra 1 given the parity since the last tie
    const int add = (tie & seen & a) | ((tie ^ 1) & up);
    const int nx = (tie ^ 1) & (x ^ odd ^ up);
    st = ((st & ~3) | nx | ((seen | tie) << 1) | ((tie & (seen ^ 1) & a) << 2)) + (add << 3);
    // the lane's state made here, value by value (an empty asm that takes and gives it): left to itself the compiler
    // holds every value's q and flags to the end and spills
    asm volatile("" : "+v"(sq), "+v"(st));
  }
  return {sq + (double)(st >> 3), (st >> 1) & 1, st & 1, (st >> 2) & 1};
}

__device__ __forceinline__ LanePack pack(const LaneR &r) { return {r.s0, r.x | (r.seen << 1) | (r.cfirst << 2), 0}; }
__device__ __forceinline__ LaneR unpack(const LanePack &p) {
  return {p.s0, (p.flags >> 1) & 1, p.flags & 1, (p.flags >> 2) & 1};
}

// the parity (of the sum / u) that this lane receives, where lane `from` (the lowest with mine) receives pin0 and
// each lane with mine hands on either a fixed parity (seen: x) or the one it received flipped by x: from lane masks,
// the last lane below with a fixed parity and the flips since
__device__ __forceinline__ int parity_in(bool mine, int seen, int x, int pin0) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = (1ull << lane) - 1;
  const uint64_t mt = __ballot(mine && seen), mk = __ballot(mine && seen && x), mx = __ballot(mine && !seen && x);
  if (mt & below) {
    const int last = 63 - __builtin_clzll(mt & below);
    const uint64_t since = below & ~((2ull << last) - 1);
    return (int)((mk >> last) & 1) ^ (__builtin_popcountll(mx & since) & 1);
  }
  return pin0 ^ (__builtin_popcountll(mx & below) & 1);
}

// the lane's sum of r where lane from's incoming parity is pin0 (lanes below from: 0)
__device__ __forceinline__ double lane_t(const LaneR &r, int from, int pin0) {
  const bool mine = (int)(threadIdx.x & 63) >= from;
  const int pin = parity_in(mine, r.seen, r.x, pin0);
  return mine ? r.s0 + (r.seen ? (double)(pin ^ r.cfirst) : 0.0) : 0.0;
}

// a double moved across the lanes by a DPP control (lanes with no source, or in rows the mask leaves out, get 0)
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ double dpp_move(double x) {
  return __hiloint2double(__builtin_amdgcn_update_dpp(0, __double2hiint(x), CTRL, ROWS, 0xf, true),
                          __builtin_amdgcn_update_dpp(0, __double2loint(x), CTRL, ROWS, 0xf, true));
}

// the sum of t over the lanes up to this one: row shifts by 1, 2, 4 and 8, then lane 15 of each row into the next and
// lane 31 into the upper half. Exact on integers whose sum up to this lane is below 2^53, whatever the order of the
// adds (every partial sum is below it too); past the first lane whose sum leaves the binade nothing is used.
__device__ __forceinline__ double lanes_upto(double t) {
  t = t + dpp_move<0x111>(t);
  t = t + dpp_move<0x112>(t);
  t = t + dpp_move<0x114>(t);
  t = t + dpp_move<0x118>(t);
  t = t + dpp_move<0x142, 0xa>(t);
  t = t + dpp_move<0x143, 0xc>(t);
  return t;
}
// the value of the lane below (lane 0: 0)
__device__ __forceinline__ double lane_below(double x) { return dpp_move<0x138>(x); }

// a double that is the same in every lane, or lane l's, as a uniform value
__device__ __forceinline__ double uniform(double x) {
  return __hiloint2double(__builtin_amdgcn_readfirstlane(__double2hiint(x)),
                          __builtin_amdgcn_readfirstlane(__double2loint(x)));
}
__device__ __forceinline__ double from_lane(double x, int l) {
  return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(x), l),
                          __builtin_amdgcn_readlane(__double2loint(x), l));
}

__device__ __forceinline__ int binade(double s) { return ((__double2hiint(s) >> 20) & 0x7ff) - 1023; }  // s > 0, normal

// Lanes from..63 of a chunk in parallel at run's binade e (lanes below from take no part: their values are done).
// Returns the first lane whose values take the sum to 2^(e+1) or past it, 64 if none; *start is the sum before this
// lane's values (right for the lanes from..the returned one), *end the chunk's end where 64 is returned.
// (r: the lanes' values taken at run's binade, lane_r)
__device__ __forceinline__ int chunk_lanes_r(const LaneR &r, double run, int from, double *start, double *end) {
  const int lane = threadIdx.x & 63;
  const int e = binade(run);
  const double t = lane_t(r, from, __double2loint(run) & 1);  // lane from: the parity of run / u
  const double inc = lanes_upto(t);
  const double base = __builtin_ldexp(run, 52 - e);  // run / u
  const uint64_t over = __ballot(!(base + inc < 9007199254740992.0));  // lanes whose sum reaches 2^(e+1)
  const double excl = lane_below(inc);  // the lanes below (inc - t would not be exact in a lane past 2^53)
  *start = run + __builtin_ldexp(excl, e - 52);
  if (over) return __builtin_ctzll(over);
  *end = run + __builtin_ldexp(from_lane(inc, 63), e - 52);
  return 64;
}
__device__ __forceinline__ int chunk_lanes(const float (&v)[SEG], double run, int from, double *start, double *end) {
  return chunk_lanes_r(lane_r(v, binade(run)), run, from, start, end);
}

// One chunk (values b.., lane L's 32 at b + 32 L) exactly from run, by one wave: the lanes in parallel while the sum
// stays in one binade; a lane that takes it out of its binade, and the first lane while the sum is 0, adds its values
// one after another; then the lanes after it in parallel again. After two such lanes (a sum that still crosses
// binades often: a parallel pass costs about as much as twenty lanes' adds in turn) the rest of the chunk goes lane
// by lane, each adding its values to the sum the lane below hands it. Returns the chunk's end (every lane); with cp,
// the checkpoints of the chunk's values.
__device__ __forceinline__ double chunk_exact(const float (&v)[SEG], double run, int b, int count, double *cp) {
  const int lane = threadIdx.x & 63;
  double pre = 0.0;  // this lane's sum before its values
  int from = 0;
  for (int crossed = 0; from < 64 && crossed < 2; ++crossed) {
    int cross = from;
    double start = run, end = 0.0;
    if (run > 0.0) cross = chunk_lanes(v, run, from, &start, &end);
    if (lane >= from && lane <= cross) pre = start;
    if (cross == 64) {
      run = uniform(end);
      from = 64;
      break;
    }
    // lane cross's values in order from its start (every lane adds its own; lane cross's sum is kept)
    double acc = from_lane(start, cross);
#pragma unroll
    for (int u = 0; u < SEG; ++u) {
      float t = v[u];
      asm volatile("" : "+v"(t));  // (widened here, one at a time: all 32 held widened would not fit)
      acc = acc + (double)t;
    }
    run = from_lane(acc, cross);
    from = cross + 1;
  }
  // lane by lane: in turn s lane s adds its values to the sum in acc (every lane adds its own; lane s + 1 takes lane
  // s's sum, by a readlane: the turns are few enough here that the hand-on's latency does not matter)
  for (int s = from; s < 64; ++s) {
    if (lane == s) pre = run;
    double acc = run;
#pragma unroll
    for (int u = 0; u < SEG; ++u) {
      float t = v[u];
      asm volatile("" : "+v"(t));
      acc = acc + (double)t;
    }
    run = from_lane(acc, s);
  }
  if (cp && lane % (CP_BLOCK / SEG) == 0 && b + SEG * lane < count) cp[(b + SEG * lane) / CP_BLOCK] = pre;
  return run;
}

// lane from's values added in order to run (every lane adds its own; lane from's sum is kept): the sum after them, and
// lane from's pre (its sum before them) set to run
__device__ __forceinline__ double lane_in_order(const float (&v)[SEG], double run, int from, double &pre) {
  if ((int)(threadIdx.x & 63) == from) pre = run;
  double acc = run;
#pragma unroll
  for (int u = 0; u < SEG; ++u) {
    float t = v[u];
    asm volatile("" : "+v"(t));
    acc = acc + (double)t;
  }
  return from_lane(acc, from);
}

// One chunk (values b.., lane L's 32 at b + 32 L) exactly from run > 0 at lane from (the lanes below it done, their
// sums before them in pre), from its lanes already taken at binades E .. E + W - 1 (at(k): binade E + k): each run of
// lanes that keeps the sum in one binade in parallel, as chunk_exact, and each lane that takes it out of its binade by
// its adds in order, however many there are; while the sum is below 2^E, a lane at a time in order. Returns false,
// having written nothing, where the sum reaches a binade above those; else true, *end the chunk's end and, with cp,
// the checkpoints of the chunk's values.
template <int W, typename At>
__device__ __forceinline__ bool chunk_walk(const float (&v)[SEG], double run, int from, double pre, int E, At at, int b,
                                           int count, double *cp, double *end) {
  const int lane = threadIdx.x & 63;
  while (from < 64) {
    const int k = binade(run) - E;
    if (k >= W) return false;  // (uniform)
    if (k < 0) {
      run = lane_in_order(v, run, from, pre);
      ++from;
      continue;
    }
    double start = run, stop = 0.0;
    const int cross = chunk_lanes_r(at(k), run, from, &start, &stop);
    if (lane >= from && lane <= cross) pre = start;
    if (cross == 64) {
      run = uniform(stop);
      break;
    }
    // lane cross's values in order from its start (every lane adds its own; lane cross's sum is kept)
    double acc = from_lane(start, cross);
#pragma unroll
    for (int u = 0; u < SEG; ++u) {
      float t = v[u];
      asm volatile("" : "+v"(t));
      acc = acc + (double)t;
    }
    run = from_lane(acc, cross);
    from = cross + 1;
  }
  if (cp && lane % (CP_BLOCK / SEG) == 0 && b + SEG * lane < count) cp[(b + SEG * lane) / CP_BLOCK] = pre;
  *end = run;
  return true;
}

// one chunk taken at binade e, for either parity of the sum before it: its sum of r and its lanes' sums of r before
// them (every lane of the wave calls; lanes 0, 8, .., 56 and 63 write)
__device__ __forceinline__ void chunk_guess_s(double inc0, double inc1, ChunkGuess &g) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int P = 0; P < 2; ++P) {
    const double inc = P ? inc1 : inc0;
    const double excl = lane_below(inc);
    if (lane % (CP_BLOCK / SEG) == 0) g.pre[P][lane / (CP_BLOCK / SEG)] = excl;
    if (lane == 63) g.t[P] = inc;
  }
}
// the lanes' sums of r in order from lane 0, for parity P there
__device__ __forceinline__ double scan_from0(const LaneR &r, int P) { return lanes_upto(lane_t(r, 0, P)); }
__device__ __forceinline__ void chunk_guess(const float (&v)[SEG], int e, ChunkGuess &g) {
  const LaneR r = lane_r(v, e);
  chunk_guess_s(scan_from0(r, 0), scan_from0(r, 1), g);
}

// what the block's waves leave for the in-order pass: each chunk's guessed binade (NO_GUESS: none) and, at it, the
// chunk's sum of r and its lanes' (0, 8, .., 56) sums of r before them, for either parity of the sum before the chunk
constexpr int MOST_CHUNKS = SAMPLE_MOST / CHUNK;
constexpr int NO_GUESS = -100000;
static_assert(sizeof(ChunkGuess) == sizeof(double) * 2 * (1 + CHUNK / CP_BLOCK), "a chunk's guess");
struct SumShared {
  double approx[MOST_CHUNKS];  // each chunk's sum in any order
  int guess[MOST_CHUNKS];
  ChunkGuess g[MOST_CHUNKS];
};
// p[0] + p[1] + ... + p[count-1] in float64 (each p widened exactly), with the bits of the adds in index order, by the
// block (all of it calls): chunks of 2048, lane L of a wave holding p[b + 32 L .. b + 32 L + 31] (+0.0 past count,
// which changes no sum). (1) Every chunk's sum in any order, and from them the binade the running sum probably has
// at each chunk's start. (2) Each wave takes every waves-th chunk at its guessed binade (lane_r, then lane_t and the
// lanes' sums for both parities of the sum before it). (3) Wave 0 goes through the chunks in order: a run of chunks
// whose sums before them have the guessed binade and whose sums of r keep it below the next power of two is taken at
// once, a lane a chunk (their ends and checkpoints follow from (2) exactly); the chunk that ends such a run is walked
// from its lanes at two binades where given has them (chunk_walk), else taken by chunk_exact. With cp,
// cp[i / CP_BLOCK] = the sum before value i for every multiple i of CP_BLOCK below count. With given, steps (1) and
// (2) are its guesses and the first chunk its exact end and checkpoints (vocab_guess_kernel's; copied: the guesses
// already in sh). Wave 0 returns the total. (p: 16-byte aligned, count >= 1, whole chunks: +0.0 from count up to
// sample_probs_floats(count).)
__device__ __forceinline__ double sum_block(const float *p, int count, double *cp, SumShared &sh,
                                            const DrawParts *given = nullptr, bool copied = false) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const int chunks = (count + CHUNK - 1) / CHUNK;
  auto load = [&](int c, float(&v)[SEG]) {
#pragma unroll
    for (int u = 0; u < SEG / 4; ++u) {
      const float4 r = reinterpret_cast<const float4 *>(p + c * CHUNK + lane * SEG)[u];
      v[4 * u] = r.x;
      v[4 * u + 1] = r.y;
      v[4 * u + 2] = r.z;
      v[4 * u + 3] = r.w;
    }
  };
  if (given) {  // steps (1) and (2) done by other blocks (copied: their guesses already in sh)
    if (!copied)
      for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
        sh.guess[c] = given->guess[c];
        sh.g[c] = given->g[c];
      }
  } else {
    for (int c = wave; c < chunks; c += 2 * waves) {  // two chunks at a time, so that their loads fly together
      const int d = min(c + waves, chunks - 1);  // (past the last chunk: the last again, its sum written twice)
      float v[SEG], w[SEG];
      load(c, v);
      load(d, w);
      float a = 0.0f, z = 0.0f;  // (float32: these sums only guess the binades)
#pragma unroll
      for (int u = 0; u < SEG; ++u) {
        a += v[u];
        z += w[u];
      }
      double s = a, t = z;
      for (int o = 32; o >= 1; o >>= 1) {
        s += __shfl_xor(s, o, 64);
        t += __shfl_xor(t, o, 64);
      }
      if (lane == 0) {
        sh.approx[c] = s;
        sh.approx[d] = t;
      }
    }
    __syncthreads();
    if (wave == 0) {
      // the approximate sums before chunks 2L and 2L + 1
      const int c0 = 2 * lane, c1 = c0 + 1;
      const double a0 = c0 < chunks ? sh.approx[c0] : 0.0, a1 = c1 < chunks ? sh.approx[c1] : 0.0;
      const double before = lanes_upto(a0 + a1) - (a0 + a1), mid = before + a0;
      if (c0 < chunks) sh.guess[c0] = before > 0.0 ? binade(before) : NO_GUESS;
      if (c1 < chunks) sh.guess[c1] = mid > 0.0 ? binade(mid) : NO_GUESS;
    }
    __syncthreads();
    for (int c = wave; c < chunks; c += waves) {
      const int e = sh.guess[c];
      if (e == NO_GUESS) continue;  // (uniform)
      float v[SEG];
      load(c, v);
      chunk_guess(v, e, sh.g[c]);
    }
  }
  __syncthreads();
  // in order (wave 0), the chunks' guesses in lanes (lane L: chunks L and L + 64), read by readlane; the checkpoints
  // of the chunks taken from their guesses are written afterwards, all at once
  double run = 0.0;
  if (wave == 0) {
    static_assert(MOST_CHUNKS <= 128, "two chunks a lane");
    // (two of each, named, not arrays: an index that is not a constant would put an array in scratch memory)
    const int c0 = lane, c1 = lane + 64;
    const int eg0 = c0 < chunks ? sh.guess[c0] : NO_GUESS, eg1 = c1 < chunks ? sh.guess[c1] : NO_GUESS;
    const double t00 = c0 < chunks ? sh.g[c0].t[0] : 0.0, t01 = c0 < chunks ? sh.g[c0].t[1] : 0.0;
    const double t10 = c1 < chunks ? sh.g[c1].t[0] : 0.0, t11 = c1 < chunks ? sh.g[c1].t[1] : 0.0;
    double before0 = -1.0, before1 = -1.0;  // the sum before a chunk taken from its guess (-1: not so taken)
    int c = 0;
    if (given) {  // the first chunk, from 0, done by vocab_guess_kernel
      run = given->first_end;
      if (cp && lane < CHUNK / CP_BLOCK && lane * CP_BLOCK < count) cp[lane] = given->first_cp[lane];
      c = 1;
    }
    while (c < chunks) {
      if (run > 0.0) {
        // the chunks from c to the end of its group of 64 (a lane each) that keep the sum in run's binade E, at once:
        // a chunk's parity out (of the sum / u) is (P + T[P]) mod 2 of its parity in P, so either fixed or P flipped
        // or not; the parities in follow from lane masks (parity_in), then the chunks' T by a scan. The run stops at
        // the first chunk whose guess is not E or whose T takes the sum to 2^(E+1).
        const int h = c >> 6, l = c & 63;
        const int E = binade(run);
        const double Ta = h ? t10 : t00, Tb = h ? t11 : t01;
        const bool fit = lane >= l && 64 * h + lane < chunks && (h ? eg1 : eg0) == E;
        const double ha = Ta * 0.5, hb = Tb * 0.5;
        const int f0 = ha != __builtin_floor(ha), f1 = hb == __builtin_floor(hb);  // the parity out for 0 and for 1
        const int pin = parity_in(fit, f0 == f1, f0, __double2loint(run) & 1);
        const double inc = lanes_upto(fit ? (pin ? Tb : Ta) : 0.0);
        const uint64_t stop_at =
            __ballot(lane >= l && !(fit && __builtin_ldexp(run, 52 - E) + inc < 9007199254740992.0));
        const int stop = stop_at ? __builtin_ctzll(stop_at) : 64;
        if (lane >= l && lane < stop) {
          const double bf = run + __builtin_ldexp(lane_below(inc), E - 52);
          if (h) before1 = bf;
          else before0 = bf;
        }
        if (stop > l) run = run + __builtin_ldexp(from_lane(inc, stop - 1), E - 52);
        c = 64 * h + stop;
        if (stop == 64 || c >= chunks) continue;
      }
      // chunk c alone (its sum leaves the binade, its guess is another binade, or the sum before it is 0)
      const int h = c >> 6, l = c & 63;
      const int e = __builtin_amdgcn_readlane(h ? eg1 : eg0, l);
      {
        float v[SEG];
        load(c, v);
        bool walked = false;
        if (given && e != NO_GUESS && run > 0.0) {  // from the chunk's lanes at binades e and e + 1
          const LaneR r0 = unpack(given->lanes[c][0][lane]), r1 = unpack(given->lanes[c][1][lane]);
          double end = 0.0;
          walked = chunk_walk<2>(v, run, 0, 0.0, e, [&](int k) { return k ? r1 : r0; }, c * CHUNK, count, cp, &end);
          if (walked) run = end;
        }
        if (!walked) run = chunk_exact(v, run, c * CHUNK, count, cp);
      }
      ++c;
    }
    if (cp) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = h ? c1 : c0, e = h ? eg1 : eg0;
        const double bf = h ? before1 : before0;
        if (bf >= 0.0) {
          const int P = __double2loint(bf) & 1;
#pragma unroll
          for (int k = 0; k < CHUNK / CP_BLOCK; ++k)
            if (c * CHUNK + k * CP_BLOCK < count)
              cp[c * (CHUNK / CP_BLOCK) + k] = bf + __builtin_ldexp(sh.g[c].pre[P][k], e - 52);
        }
      }
    }
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

// ---- the draw over the vocabulary in blocks of CHUNK values (many CUs), then one block for the ordered sums ----
// A draw's settings: the call's arguments, or in a replayed step the call's settings and the round's random number of
// the step from device memory.
struct Settings {
  float temperature, topp;
  double random;
};
__device__ __forceinline__ Settings settings(float temperature, float topp, double random, const RunParams *params,
                                             const int32_t *state) {
  if (params) return {params->temperature, params->topp, params->randoms[state[STATE_STEP]]};
  return {temperature, topp, random};
}

constexpr int VB = 256;            // threads of a vocabulary block: CHUNK / VB consecutive logits a thread
constexpr int VPT = CHUNK / VB;
constexpr int VBLOCKS_MOST = SAMPLE_MOST / CHUNK;

// the largest logit (order-free: wmax keeps a NaN and puts +0 above -0) from the blocks' largest ones (all of them
// read by every caller: at most VBLOCKS_MOST)
__device__ __forceinline__ float best_of(const DrawParts *parts, int blocks, float *wf) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float b = parts->bmax[0];
  for (int i = tid; i < blocks; i += blockDim.x) b = wmax(b, parts->bmax[i]);
  for (int o = 32; o >= 1; o >>= 1) b = wmax(b, __shfl_xor(b, o, 64));
  if (lane == 0) wf[wave] = b;
  __syncthreads();
  float x = wf[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) x = wmax(x, wf[w]);
  __syncthreads();
  return x;
}

// the floor of the kept logits (kernels/kernel.ts:815-817): with a nucleus, best - temperature * 16.118095
__device__ __forceinline__ float floor_of(float best, const Settings &st) {
  const bool nucleus = st.topp > 0 && st.topp < 1;
  return nucleus ? best - st.temperature * 16.118095f : -3.4028234663852886e38f;
}

// (1) each block's largest logit. With window (a replayed step's draw), the call's penalty first, over the window's
// state[STATE_WINDOW] tokens that fall in the block, each distinct one once (penalize_steps_kernel's), the penalized
// logits written back (the draw's later launches and the step's end read them). With counts (a draw that is known to
// have no nucleus, whose floor keeps every logit above -FLT_MAX whatever the largest), each block's count of kept
// logits too, in place of vocab_count_kernel's launch.
__global__ __launch_bounds__(VB) void vocab_max_kernel(const float *logits, int32_t n, DrawParts *parts,
                                                       float *write_back, const int32_t *window, const int32_t *state,
                                                       const RunParams *params, int32_t counts) {
  __shared__ float wf[VB / 64];
  __shared__ uint32_t hit[CHUNK / 32];
  __shared__ int32_t win[RUN_WINDOW];
  __shared__ int wi[VB / 64];
  __shared__ int total;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i0 = blockIdx.x * CHUNK + tid * VPT;
  float v[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) v[u] = logits[min(i0 + u, n - 1)];  // (clamped: a repeat changes no max)
  if (window) {
    static_assert(VPT <= 32 && 32 % VPT == 0, "a thread's logits in one word of the block's marks");
    const int count = state[STATE_WINDOW], b0 = blockIdx.x * CHUNK;
    if (tid < CHUNK / 32) hit[tid] = 0;
    if (tid < count) win[tid] = window[tid];
    __syncthreads();
    if (tid < count) {
      const int32_t t = win[tid];
      bool first = true;
      for (int j = 0; j < tid; ++j) first = first && win[j] != t;
      if (first && t >= b0 && t < b0 + CHUNK) atomicOr(&hit[(t - b0) >> 5], 1u << ((t - b0) & 31));
    }
    __syncthreads();
    const uint32_t marks = hit[(tid * VPT) >> 5] >> ((tid * VPT) & 31);
    if (marks & ((1u << VPT) - 1)) {
      const float penalty = params->penalty;
#pragma unroll
      for (int u = 0; u < VPT; ++u)
        if ((marks >> u) & 1) {  // (a window token: below n)
          v[u] = v[u] > 0 ? v[u] / penalty : v[u] * penalty;
          write_back[i0 + u] = v[u];
        }
    }
  }
  if (counts) {
    const float floor_ = floor_of(0.0f, Settings{1.0f, 1.0f, 0.0});  // (no nucleus: the same for any largest logit)
    int c = 0;
#pragma unroll
    for (int u = 0; u < VPT; ++u) c += i0 + u < n && v[u] >= floor_;
    block_scan<VB>(c, wi, &total);
    if (tid == 0) parts->bcount[blockIdx.x] = total;
  }
  float b = v[0];
#pragma unroll
  for (int u = 1; u < VPT; ++u) b = wmax(b, v[u]);
  for (int o = 32; o >= 1; o >>= 1) b = wmax(b, __shfl_xor(b, o, 64));
  if (lane == 0) wf[wave] = b;
  __syncthreads();
  if (tid == 0) {
    float x = wf[0];
    for (int w = 1; w < VB / 64; ++w) x = wmax(x, wf[w]);
    parts->bmax[blockIdx.x] = x;
  }
}

// (2) each block's count of kept logits (v >= floor)
__global__ __launch_bounds__(VB) void vocab_count_kernel(const float *logits, int32_t n, DrawParts *parts,
                                                         float temperature, float topp, double random,
                                                         const RunParams *params, const int32_t *state) {
  __shared__ float wf[VB / 64];
  __shared__ int wi[VB / 64];
  __shared__ int total;
  const Settings st = settings(temperature, topp, random, params, state);
  const float best = best_of(parts, gridDim.x, wf);
  if (!__builtin_isfinite(best)) return;  // (the whole block: the draw gives SAMPLE_NOT_FINITE)
  const float floor_ = floor_of(best, st);
  const int tid = threadIdx.x, i0 = blockIdx.x * CHUNK + tid * VPT;
  int c = 0;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const float v = logits[min(i0 + u, n - 1)];
    c += i0 + u < n && v >= floor_;
  }
  block_scan<VB>(c, wi, &total);
  if (tid == 0) parts->bcount[blockIdx.x] = total;
}

// (3) each block's kept values in index order at their places (the counts of the blocks before), their p, the
// block's largest p and its sum of p (where nothing is left out: the block's values are the total's chunk, the sum
// the one its binade is guessed from)
__global__ __launch_bounds__(VB) void vocab_kept_kernel(const float *logits, int32_t n, DrawParts *parts, float *probs,
                                                        int32_t *index, float temperature, float topp, double random,
                                                        const RunParams *params, const int32_t *state) {
  __shared__ float wf[VB / 64], ws[VB / 64];
  __shared__ int wi[VB / 64];
  __shared__ int before_, count_, local_;
  const Settings st = settings(temperature, topp, random, params, state);
  const int blocks = gridDim.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float best = best_of(parts, blocks, wf);
  if (!__builtin_isfinite(best)) return;
  const float floor_ = floor_of(best, st);
  if (tid < 64) {  // the kept values of the blocks before this one, and of all
    int a = 0, t = 0;
    for (int i = tid; i < blocks; i += 64) {
      const int c = parts->bcount[i];
      a += i < (int)blockIdx.x ? c : 0;
      t += c;
    }
    for (int o = 32; o >= 1; o >>= 1) {
      a += __shfl_xor(a, o, 64);
      t += __shfl_xor(t, o, 64);
    }
    if (tid == 0) {
      before_ = a;
      count_ = t;
    }
  }
  const int i0 = blockIdx.x * CHUNK + tid * VPT;
  float v[VPT];
  int c = 0;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    v[u] = logits[min(i0 + u, n - 1)];
    c += i0 + u < n && v[u] >= floor_;
  }
  int at = block_scan<VB>(c, wi, &local_);  // (its barriers also publish before_ and count_)
  at += before_;
  const int count = count_, simd = count & ~3;
  if (blockIdx.x == 0)  // +0.0 from count to the end of its chunk: the total reads whole chunks
    for (int j = count + tid; j < (int)sample_probs_floats(count); j += VB) probs[j] = 0.0f;
  const float inverse = 1.0f / st.temperature;
  float top = 0.0f, sum = 0.0f;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    if (i0 + u < n && v[u] >= floor_) {
      const float d = v[u] - best;
      const float pv = at < simd ? vexp(d * inverse) : fexp(d / st.temperature);
      probs[at] = pv;
      index[at] = i0 + u;
      top = __builtin_fmaxf(top, pv);
      sum += pv;
      ++at;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    top = __builtin_fmaxf(top, __shfl_xor(top, o, 64));
    sum += __shfl_xor(sum, o, 64);
  }
  if (lane == 0) {
    wf[wave] = top;
    ws[wave] = sum;
  }
  __syncthreads();
  if (tid == 0) {
    float x = wf[0], y = ws[0];
    for (int w = 1; w < VB / 64; ++w) {
      x = __builtin_fmaxf(x, wf[w]);
      y += ws[w];
    }
    parts->btop[blockIdx.x] = x;
    parts->csum[blockIdx.x] = y;
  }
}

// (4) without a nucleus, each chunk of the total at its guessed binade, a block a chunk: every value is kept, so block
// b's values are the total's chunk b (unless some logits are -inf: then the guesses are only worse), the binade of the
// sum before it is guessed from the blocks' sums of p, and chunk_guess takes the chunk at that binade (wave 0); the
// chunk's lanes are kept at that binade (wave 0) and the next (wave 1), for a chunk whose sum crosses into it. Block 0
// takes the first chunk exactly, since the sum before it is 0 (below). With a nucleus the draw takes the chunks
// itself.
constexpr int GW = 8;  // waves of a guess block
constexpr int NB = 5;  // binades block 0 takes the first chunk's lanes at (waves 1..NB)
static_assert(NB < GW, "a wave for each binade and one that adds in order");
__global__ __launch_bounds__(64 * GW) void vocab_guess_kernel(int32_t n, DrawParts *parts, const float *probs,
                                                              float temperature, float topp, double random,
                                                              const RunParams *params, const int32_t *state) {
  __shared__ float wf[GW];
  __shared__ LanePack first[NB][64];
  const Settings st = settings(temperature, topp, random, params, state);
  if (st.topp > 0 && st.topp < 1) return;
  if (!__builtin_isfinite(best_of(parts, gridDim.x, wf))) return;  // (the draw gives SAMPLE_NOT_FINITE)
  const int b = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (b > 0 && wave >= 2) return;
  float v[SEG];
#pragma unroll
  for (int u = 0; u < SEG / 4; ++u) {
    const float4 r = reinterpret_cast<const float4 *>(probs + b * CHUNK + lane * SEG)[u];
    v[4 * u] = r.x;
    v[4 * u + 1] = r.y;
    v[4 * u + 2] = r.z;
    v[4 * u + 3] = r.w;
  }
  if (b == 0) {
    // the first chunk, from 0: its sum in any order (t) puts its end at about binade Ef. Waves 1..NB take its lanes at
    // binades Ef - NB + 2 .. Ef + 1 while wave 0 adds lanes in order, from the first that holds a value other than 0
    // (the lanes below it sum to 0), up to the first whose sum before it reaches the lowest of those binades (where
    // the binades change every lane or two, in order is the faster); then wave 0 walks the rest through them.
    float tf = 0.0f;
#pragma unroll
    for (int u = 0; u < SEG; ++u) tf += v[u];
    double t = tf;
    for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o, 64);
    const int E = t > 0.0 ? binade(t) - (NB - 2) : 0;
    if (t > 0.0 && wave >= 1 && wave <= NB) first[wave - 1][lane] = pack(lane_r(v, E + wave - 1));
    double run = 0.0, pre = 0.0;
    int from = 64;
    if (wave == 0) {
      bool some = false;
#pragma unroll
      for (int u = 0; u < SEG; ++u) some |= v[u] != 0.0f;
      const uint64_t m = __ballot(some);
      from = m ? __builtin_ctzll(m) : 64;
      while (from < 64 && (run == 0.0 || binade(run) < E)) {
        run = lane_in_order(v, run, from, pre);
        ++from;
      }
    }
    __syncthreads();
    if (wave != 0) return;
    if (lane == 0) parts->guess[0] = NO_GUESS;
    double end = 0.0;
    if (!chunk_walk<NB>(v, run, from, pre, E, [&](int k) { return unpack(first[k][lane]); }, 0, CHUNK,
                        parts->first_cp, &end))
      end = chunk_exact(v, 0.0, 0, CHUNK, parts->first_cp);
    if (lane == 0) parts->first_end = end;
    return;
  }
  double a = 0.0;  // the sum of p before the chunk, in any order
  for (int i = lane; i < b; i += 64) a += parts->csum[i];
  for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o, 64);
  const int e = a > 0.0 ? binade(a) : NO_GUESS;
  if (wave == 0 && lane == 0) parts->guess[b] = e;
  if (e == NO_GUESS) return;
  const LaneR r = lane_r(v, e + wave);
  parts->lanes[b][wave][lane] = pack(r);
  if (wave == 0) chunk_guess_s(scan_from0(r, 0), scan_from0(r, 1), parts->g[b]);
}

// (5) the draw, one block: the largest logit, the count and the largest p from the blocks' parts; the total's chunks
// padded with +0.0; the total, the nucleus and the draw
__device__ __forceinline__ void draw_block(int32_t n, const Settings &st, const DrawParts *parts, float *probs,
                                          int32_t *index, int32_t *out_token, float *out_best) {
  __shared__ float4 area[SORT_MOST / 2];  // the sort's probabilities then tokens; the total's guesses
  float *const sp = reinterpret_cast<float *>(area);
  int *const si = reinterpret_cast<int *>(area) + SORT_MOST;
  __shared__ int wi[ST / 64];
  __shared__ int shared_likely;
  __shared__ double shared_total, shared_cutoff;
  __shared__ double checkpoints[CP_MOST];  // the running sum of the kept p before every CP_BLOCK of them
  static_assert(STAGE <= 2 * SORT_MOST, "the staging area is the sort's");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float temperature = st.temperature, topp = st.topp;
  const double random = st.random;
  const int blocks = (n + CHUNK - 1) / CHUNK;
  const bool nucleus = topp > 0 && topp < 1;
  SumShared &sh = *reinterpret_cast<SumShared *>(area);
  static_assert(sizeof(SumShared) <= sizeof(float4) * (SORT_MOST / 2), "the total's LDS fits the sort's area");
  // every read of the vocabulary launches' parts at once: each wave all of the blocks' largest logits, kept counts
  // and largest p (so that every wave has their reductions, with no barrier), and without a nucleus the block the
  // chunks' guesses into LDS (for sum_block, whose barrier they meet)
  float best = parts->bmax[0], top = 0.0f;
  int c = 0;
  for (int i = lane; i < blocks; i += 64) {
    best = wmax(best, parts->bmax[i]);
    c += parts->bcount[i];
    top = __builtin_fmaxf(top, parts->btop[i]);
  }
  if (!nucleus)
    for (int i = tid; i < blocks; i += ST) {
      sh.guess[i] = parts->guess[i];
      sh.g[i] = parts->g[i];
    }
  for (int o = 32; o >= 1; o >>= 1) {
    best = wmax(best, __shfl_xor(best, o, 64));
    c += __shfl_xor(c, o, 64);
    top = __builtin_fmaxf(top, __shfl_xor(top, o, 64));
  }
  if (!__builtin_isfinite(best)) {
    if (tid == 0) {
      *out_token = SAMPLE_NOT_FINITE;
      *out_best = best;
    }
    return;  // the whole block
  }
  const uint64_t below = (1ull << lane) - 1;
  const int count = __builtin_amdgcn_readfirstlane(c);  // (probs is +0.0 from count to its chunk's end)

  // total: float64, in order, by wave 0 from registers (without a nucleus from vocab_guess_kernel's guesses)
  double total = sum_block(probs, count, checkpoints, sh, nucleus ? nullptr : parts, true);
  if (tid == 0) shared_total = total;
  __syncthreads();
  total = shared_total;

  if (!nucleus) {
    // the running sum in index order up to the first that passes random * total: the block of CP_BLOCK where it
    // passes, from the checkpoints (the sum never decreases: every p >= 0), then that block's adds again from its
    // checkpoint (the same adds, the same bits), by wave 0: the block's values and token indices read at once (a
    // float4 and an int4 a lane) into LDS (the guesses' area, done with), then lane 0's adds, 32 at a time from
    // registers, the first index past target kept by a select
    static_assert(CP_BLOCK == 64 * 4, "a checkpoint block is a float4 a lane");
    if (wave == 0) {
      const double target = random * total;
      const int blocks = (count + CP_BLOCK - 1) / CP_BLOCK;
      // the first block b whose end (the sum before block b + 1, or the total) passes target, blocks if none: the ends
      // never decrease, so the lanes look at every 16th end, then at the 16 of the first group that passes
      static_assert(CP_MOST <= 64 * 16, "two looks over the checkpoints");
      auto passes = [&](int m) { return (m + 1 < blocks ? checkpoints[m + 1] : total) > target; };
      const uint64_t g16 = __ballot(16 * lane < blocks && passes(min(16 * lane + 15, blocks - 1)));
      int b = blocks;
      if (g16) {
        const int g = __builtin_ctzll(g16);
        const uint64_t one = __ballot(lane < 16 && 16 * g + lane < blocks && passes(16 * g + lane));
        b = 16 * g + __builtin_ctzll(one);  // (the group's last passes: one is not 0)
      }
      int token = -1;
      if (b < blocks) {
        const int len = min(CP_BLOCK, count - b * CP_BLOCK);
        float4 *const vals = area;  // (probs holds whole chunks: the block's 256 are there)
        int4 *const ids = reinterpret_cast<int4 *>(area + 64);
        vals[lane] = reinterpret_cast<const float4 *>(probs + b * CP_BLOCK)[lane];
        const int i0 = b * CP_BLOCK + 4 * lane;  // (index holds n: clamped past the count, those never taken)
        ids[lane] = make_int4(index[min(i0, count - 1)], index[min(i0 + 1, count - 1)], index[min(i0 + 2, count - 1)],
                              index[min(i0 + 3, count - 1)]);
        wave_sync_lds();
        if (lane == 0) {
          // 32 adds at a time with one look at the end; the 32 in which the sum passes target again, one at a time
          const float *const x = reinterpret_cast<const float *>(vals);
          double acc = checkpoints[b];
          int j = -1;
          for (int q = 0; q * 32 < len; ++q) {
            float4 a[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) a[u] = vals[q * 8 + u];
            double t = acc;
#pragma unroll
            for (int u = 0; u < 8; ++u) t = (((t + (double)a[u].x) + (double)a[u].y) + (double)a[u].z) + (double)a[u].w;
            if (t > target) {  // (every p >= 0: the sum passes within these 32)
              for (int i = q * 32; i < min(q * 32 + 32, len); ++i) {
                acc += (double)x[i];
                if (acc > target) {
                  j = i;
                  break;
                }
              }
              break;
            }
            acc = t;
          }
          if (j >= 0) token = reinterpret_cast<const int *>(ids)[j];
        }
      }
      if (lane == 0) {
        *out_token = token >= 0 ? token : index[count - 1];
        *out_best = best;
      }
    }
    return;
  }

  // the nucleus: the kept p >= cutoff, sorted from the most probable
  if (tid == 0) {
    const double ceiling = (1.0 - (double)topp) / (double)(count > 1 ? count - 1 : 1) * total;
    shared_cutoff = ceiling < (double)top ? ceiling : (double)top;
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

// the draw's float64 total alone (the same block's work, with given the chunks' guesses of vocab_guess_kernel): *total,
// and checkpoints[i / CP_BLOCK] = the sum before value i
__global__ __launch_bounds__(ST) void ordered_sum_kernel(const float *p, int32_t n, double *total, double *checkpoints,
                                                         const DrawParts *given) {
  __shared__ SumShared sh;
  const double t = sum_block(p, n, checkpoints, sh, given);
  if (threadIdx.x == 0) *total = t;
}

// for the total alone taken as the draw without a nucleus takes it: each chunk's sum of p in any order (the guesses'
// prefix), and a finite largest logit for vocab_guess_kernel
__global__ __launch_bounds__(64) void chunk_sums_kernel(const float *p, DrawParts *parts) {
  const int b = blockIdx.x, lane = threadIdx.x;
  float a = 0.0f;
#pragma unroll
  for (int u = 0; u < SEG / 4; ++u) {
    const float4 r = reinterpret_cast<const float4 *>(p + b * CHUNK + lane * SEG)[u];
    a += (r.x + r.y) + (r.z + r.w);
  }
  for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o, 64);
  if (lane == 0) {
    parts->csum[b] = a;
    parts->bmax[b] = 0.0f;
  }
}

__global__ __launch_bounds__(ST) void draw_kernel(int32_t n, const DrawParts *parts, float *probs, int32_t *index,
                                                  int32_t *out_token, float *out_best, float temperature, float topp,
                                                  double random, const RunParams *params, const int32_t *state) {
  draw_block(n, settings(temperature, topp, random, params, state), parts, probs, index, out_token, out_best);
}

// the five launches of a draw (the settings as values, or with params the call's and the step's from device memory;
// with window, the call's penalty over it applied to the logits first, in the first launch)
hipError_t launch_draw(const float *logits, int32_t n, float temperature, float topp, double random,
                       const RunParams *params, const int32_t *state, float *probs, int32_t *index, DrawParts *parts,
                       int32_t *out_token, float *out_best, hipStream_t s, float *write_back = nullptr,
                       const int32_t *window = nullptr, bool whole = false) {
  const int blocks = (n + CHUNK - 1) / CHUNK;
  hipLaunchKernelGGL(vocab_max_kernel, dim3(blocks), dim3(VB), 0, s, logits, n, parts, write_back, window, state,
                     params, (int32_t)whole);
  if (!whole)
    hipLaunchKernelGGL(vocab_count_kernel, dim3(blocks), dim3(VB), 0, s, logits, n, parts, temperature, topp, random,
                       params, state);
  hipLaunchKernelGGL(vocab_kept_kernel, dim3(blocks), dim3(VB), 0, s, logits, n, parts, probs, index, temperature, topp,
                     random, params, state);
  hipLaunchKernelGGL(vocab_guess_kernel, dim3(blocks), dim3(64 * GW), 0, s, n, parts, probs, temperature, topp, random,
                     params, state);
  hipLaunchKernelGGL(draw_kernel, dim3(1), dim3(ST), 0, s, n, parts, probs, index, out_token, out_best, temperature,
                     topp, random, params, state);
  return hipGetLastError();
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

hipError_t launch_sample_steps(float *logits, int32_t n, const RunParams *params, const int32_t *state,
                               const int32_t *window, bool whole, float *probs, int32_t *index, DrawParts *parts,
                               int32_t *out_token, float *out_best, hipStream_t s) {
  if (n < 1 || n > SAMPLE_MOST) return hipErrorInvalidValue;
  return launch_draw(logits, n, 0.0f, 0.0f, 0.0, params, state, probs, index, parts, out_token, out_best, s,
                     window ? logits : nullptr, window, whole);
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

hipError_t launch_ordered_sum(const float *p, int32_t n, double *total, double *checkpoints, DrawParts *parts,
                              hipStream_t s) {
  if (n < 1 || n > SAMPLE_MOST) return hipErrorInvalidValue;
  if (parts) {
    const int blocks = (n + CHUNK - 1) / CHUNK;
    hipLaunchKernelGGL(chunk_sums_kernel, dim3(blocks), dim3(64), 0, s, p, parts);
    hipLaunchKernelGGL(vocab_guess_kernel, dim3(blocks), dim3(64 * GW), 0, s, n, parts, p, 1.0f, 1.0f, 0.0, nullptr,
                       nullptr);
  }
  hipLaunchKernelGGL(ordered_sum_kernel, dim3(1), dim3(ST), 0, s, p, n, total, checkpoints, parts);
  return hipGetLastError();
}

hipError_t launch_sample(const float *logits, int32_t n, float temperature, float topp, double random, float *probs,
                         int32_t *index, DrawParts *parts, int32_t *out_token, float *out_best, hipStream_t s) {
  if (n < 1 || n > SAMPLE_MOST || !(temperature > 0)) return hipErrorInvalidValue;
  return launch_draw(logits, n, temperature, topp, random, nullptr, nullptr, probs, index, parts, out_token, out_best,
                     s);
}

}  // namespace ple
