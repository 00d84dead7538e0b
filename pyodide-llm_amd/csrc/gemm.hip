// gemm.hip — the prefill matmul on CDNA4 i8 MFMA: many tokens against an int8 (or int6) matrix with per-group
// float32 scales, in the reference's exact float32 order (kernels/kernel_relaxed.ts:34-67 matmul_q8r and :164-183
// matmul_q8r_tile, which is the same per (row, token); matmul_q6r :189-218 on the six.ts-widened values).
//
// For a (row r, token t): S_g = dot(w_g, q_g - 64) is an exact int32 per group g of 32. One
// v_mfma_i32_32x32x32_i8 makes S_g for a 32-row x 32-token tile: K = 32 is exactly one group, so every MFMA output is
// one group sum, never a sum across groups. The float32 part is the reference's: p_g = f32(S_g) * f32(ws_g * xs_g)
// added to lane chain g mod 4 for the groups below 4*floor(G/4), the chains combined ((l0 + l1) + l2) + l3, then the
// tail groups added in order; y = result (or y + result, the fused residual add). Those four float32 steps a group
// (product of scales, conversion, multiply, add; the conversion done as a subtraction, see MAGIC) run on the VALU for
// every (row, token, group), so the kernel is bound by the VALU, not by the MFMA pipe: one MFMA a group a tile against
// 64 VALU instructions.
//
// Tiling: a block of 256 threads (4 waves, one a SIMD) makes 64 rows x 128 tokens; each K step stages 4 groups (128
// bytes of K: one group for each lane chain) of the block's weights, activations (centred: q - 64) and scales in LDS,
// double buffered: the next step's global loads are in flight while the current one is computed. A wave makes two
// 32 x 32 MFMA tiles side by side (32 rows x 64 tokens: the weight operand and the 16 row scales a lane read once for
// both): 2 x 4 chains x 16 accumulators a lane, two waves a SIMD (two blocks a CU). Two tiles a wave at two waves a
// SIMD issue this pattern's float32 work faster than one tile a wave at three (measured: 14.3k against 10.1k group
// tiles a µs), the two tiles' independent instructions filling what one wave's dependent ones leave idle.
#include "common.hpp"
#include "kernels.hpp"

namespace ple {
namespace {

constexpr int BR = 64;             // weight rows a block
constexpr int BT = 128;            // tokens a block
constexpr int NT = 256;            // threads a block: 2 x 2 waves of 32 rows x 64 tokens
constexpr int KS = 4;              // groups a K step: one for each lane chain
constexpr int ROWB = KS * 32 + 16; // LDS bytes of one row of a stage (128 and 16 of padding against bank conflicts)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct Stage {
  uint8_t a[BR * ROWB];  // weights (int6 widened), [row][4 groups x 32]
  uint8_t b[BT * ROWB];  // activations minus 64, [token][4 groups x 32]
  float ws[KS * BR];     // weight scales [group][row]
  float xs[KS * BT];     // activation scales [group][token]
};

struct SegRow {
  const uint8_t *w;
  const float *ws;
  int32_t r;
};
__device__ __forceinline__ SegRow seg_row(const MatArgs &a, int row) {
  const int n0 = a.seg[0].rows, n1 = a.seg[1].rows;
  if (a.nseg > 2 && row >= n0 + n1) return {a.seg[2].w, a.seg[2].ws, row - n0 - n1};
  if (a.nseg > 1 && row >= n0) return {a.seg[1].w, a.seg[1].ws, row - n0};
  return {a.seg[0].w, a.seg[0].ws, row};
}

// what one thread loads of a K step: one (row, group) of the weights (int8: 32 bytes; int6: the 24-byte group) with its
// scale, two (token, group)s of the activations (tokens rt and rt + 64) with their scales. Registers between the
// global load and the LDS store.
template <bool SIX>
struct Fetch {
  uint32_t w[SIX ? 6 : 8];
  float wsv;
  uint4 x[4];
  float xsv[2];
};

// (GLU: r0 is the block's first hidden unit; its rows 0-31 are w1's units r0.., rows 32-63 w3's)
template <bool SIX, bool SUMS, bool GLU>
__device__ __forceinline__ void fetch(Fetch<SIX> &f, const MatArgs &a, int r0, int t0, int g0, int G, int tid) {
  // rows, groups and tokens past the end clamped: the loads stay unconditional and valid; what they bring is never
  // added
  const int g = min(g0 + (tid & 3), G - 1);
  SegRow s;
  if constexpr (GLU) {
    const int r = tid >> 2, unit = min(r0 + (r & 31), a.seg[0].rows - 1);
    s = r < 32 ? SegRow{a.seg[0].w, a.seg[0].ws, unit} : SegRow{a.seg[1].w, a.seg[1].ws, unit};
  } else {
    s = seg_row(a, min(r0 + (tid >> 2), a.total_rows - 1));
  }
  if constexpr (SIX) {
    const uint2 *p = reinterpret_cast<const uint2 *>(s.w + ((int64_t)s.r * G + g) * 24);
    const uint2 l0 = p[0], l1 = p[1], tops = p[2];
    f.w[0] = l0.x; f.w[1] = l0.y; f.w[2] = l1.x; f.w[3] = l1.y; f.w[4] = tops.x; f.w[5] = tops.y;
  } else {
    const uint4 *p = reinterpret_cast<const uint4 *>(s.w + ((int64_t)s.r * G + g) * 32);
    const uint4 v0 = p[0], v1 = p[1];
    f.w[0] = v0.x; f.w[1] = v0.y; f.w[2] = v0.z; f.w[3] = v0.w;
    f.w[4] = v1.x; f.w[5] = v1.y; f.w[6] = v1.z; f.w[7] = v1.w;
  }
  f.wsv = SUMS ? 0.0f : s.ws[(int64_t)s.r * G + g];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = min(t0 + h * 64 + (tid >> 2), a.m - 1);
    const uint4 *p = reinterpret_cast<const uint4 *>(a.xq + (int64_t)t * a.xq_stride + (int64_t)g * 32);
    f.x[2 * h] = p[0];
    f.x[2 * h + 1] = p[1];
    f.xsv[h] = SUMS ? 0.0f : a.xs[(int64_t)t * a.xs_stride + g];
  }
}

__device__ __forceinline__ uint4 centre16(uint4 v) { return {centre4(v.x), centre4(v.y), centre4(v.z), centre4(v.w)}; }

template <bool SIX>
__device__ __forceinline__ void store(Stage &st, const Fetch<SIX> &f, int tid) {
  const int rt = tid >> 2, gi = tid & 3;  // the row (and the token) and the group of this thread
  uint4 *d = reinterpret_cast<uint4 *>(st.a + rt * ROWB + gi * 32);
  if constexpr (SIX) {
    uint32_t w[8];
    const uint32_t L[4] = {f.w[0], f.w[1], f.w[2], f.w[3]};
    six_widen(L, f.w[4], f.w[5], w);
    d[0] = {w[0], w[1], w[2], w[3]};
    d[1] = {w[4], w[5], w[6], w[7]};
  } else {
    d[0] = {f.w[0], f.w[1], f.w[2], f.w[3]};
    d[1] = {f.w[4], f.w[5], f.w[6], f.w[7]};
  }
  st.ws[gi * BR + rt] = f.wsv;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint4 *e = reinterpret_cast<uint4 *>(st.b + (h * 64 + rt) * ROWB + gi * 32);
    e[0] = centre16(f.x[2 * h]);
    e[1] = centre16(f.x[2 * h + 1]);
    st.xs[gi * BT + h * 64 + rt] = f.xsv[h];
  }
}

// The MFMA's accumulator starts at MAGIC (the bits of 1.5 * 2^23), so that it ends at MAGIC + S_g: for |S_g| < 2^22
// (here |S_g| <= 32 * 128 * 64 = 2^18) those are the bits of the float32 1.5 * 2^23 + S_g, and subtracting
// 1.5 * 2^23 gives f32(S_g) exactly (both terms and the difference are integers float32 holds). One float32
// subtraction in place of the int-to-float conversion, which issues at half the rate of a multiply or an add.
constexpr int MAGIC = 0x4B400000;
constexpr float MAGIC_F = 12582912.0f;

// acc += f32(S) * f32(ws * xs) for the 16 outputs of a lane in each of its two MFMA tiles (R = MAGIC + S): rows
// (v / 4) * 8 + (lane / 32) * 4 + v % 4 of the tiles, the tokens lane % 32 (x0) and 32 + lane % 32 (x1)
__device__ __forceinline__ void products2(const v16i &R0, const v16i &R1, const float *ws_rows, float x0, float x1,
                                          float (&acc0)[16], float (&acc1)[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 w4 = *reinterpret_cast<const float4 *>(ws_rows + q * 8);
    const float w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = q * 4 + i;
      acc0[v] = acc0[v] + (__int_as_float(R0[v]) - MAGIC_F) * (w[i] * x0);
      acc1[v] = acc1[v] + (__int_as_float(R1[v]) - MAGIC_F) * (w[i] * x1);
    }
  }
}

// the 16 values live in registers here: an empty asm that takes and gives them keeps the compiler from moving their
// computation below this point (asm volatile statements keep their order; the last one's memory clobber keeps the
// stores that follow below it)
__device__ __forceinline__ void pin16(float (&x)[16]) {
  asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7]),
               "+v"(x[8]), "+v"(x[9]), "+v"(x[10]), "+v"(x[11]), "+v"(x[12]), "+v"(x[13]), "+v"(x[14]), "+v"(x[15]));
}

// the 16 group sums of a lane's tile outputs (rows row0 + (v / 4) * 8 + (lane / 32) * 4 + v % 4, token tok0 + lane % 32)
__device__ __forceinline__ void write_sums(const MatArgs &a, const v16i &S, int row0, int tok0, int g, int G, int lane) {
  const int t = tok0 + (lane & 31);
  if (t >= a.m || g >= G) return;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = row0 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
    if (row < a.total_rows) a.sums[((int64_t)t * a.total_rows + row) * G + g] = S[v];
  }
}

// The SwiGLU epilogue (GLU): the block's rows are 32 hidden units of w1 (the waves wr = 0) and the same units of w3
// (wr = 1), so a lane of wave (0, wt) and the same lane of wave (1, wt) hold h1 and h3 of the same (unit, token) in the
// same registers. Each wave hands its partner the tile it does not finish through LDS: wave (0, wt) finishes tile 0
// (tokens 0-31 of its 64), wave (1, wt) tile 1. o = h1 / (1 + vexp(-h1)) * h3 as swiglu_quant4_kernel computes it,
// then quantize_x of the token's group of 32 units (the block's 32): the largest magnitude over the lane's 16 values
// and its partner lane's (lane ^ 32, the group's other 16; order-free), the scale and its reciprocal as
// quantize_group4 makes them, four bytes a run of four units.
__device__ __forceinline__ void glu_epilogue(const MatArgs &a, float (&out)[2][16], float *xch, int u0, int t0,
                                             int wave, int lane) {
  const int wr = wave & 1, wt = wave >> 1;
  __syncthreads();  // every wave is done reading the stages
#pragma unroll
  for (int v = 0; v < 16; ++v) xch[(wave * 16 + v) * 64 + lane] = wr ? out[0][v] : out[1][v];
  __syncthreads();
  float o[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const float other = xch[((wave ^ 1) * 16 + v) * 64 + lane];
    const float h1 = wr ? other : out[0][v], h3 = wr ? out[1][v] : other;
    o[v] = h1 / (1.0f + vexp(-h1)) * h3;
  }
  float amax = __builtin_fabsf(o[0]);
#pragma unroll
  for (int v = 1; v < 16; ++v) amax = __builtin_fmaxf(amax, __builtin_fabsf(o[v]));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32, 64));
  const int t = t0 + wt * 64 + wr * 32 + (lane & 31);
  if (t >= a.m) return;
  const GluOut &g = a.glu;
  const float qmax = g.bias == 0 ? 127.0f : 63.0f;
  const float scale = amax / qmax;
  const float inv = scale > 0 ? 1.0f / scale : 0.0f;
  int8_t *q = g.q + (int64_t)t * g.q_stride + u0 + (lane >> 5) * 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t w = (uint32_t)(uint8_t)quant_value(o[4 * r], inv, g.bias) |
                       ((uint32_t)(uint8_t)quant_value(o[4 * r + 1], inv, g.bias) << 8) |
                       ((uint32_t)(uint8_t)quant_value(o[4 * r + 2], inv, g.bias) << 16) |
                       ((uint32_t)(uint8_t)quant_value(o[4 * r + 3], inv, g.bias) << 24);
    *reinterpret_cast<uint32_t *>(q + r * 8) = w;  // units u0 + 8 r + (lane / 32) * 4 ..
  }
  if (lane < 32) g.s[(int64_t)t * g.s_stride + u0 / 32] = scale;
}

// with SUMS the kernel writes the exact int32 group sums S_g to a.sums [m][rows][G] instead (one segment); with GLU
// the SwiGLU's quantized output (glu_epilogue)
// (two waves a SIMD: the register budget that keeps the MFMA results in VGPRs, no AGPR copies)
template <bool SIX, bool SUMS, bool GLU>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kernel(const MatArgs a) {
  __shared__ Stage stage[2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave & 1, wt = wave >> 1;  // the wave's 32 rows and 64 tokens of the block
  // block b runs on XCD b % 8; the (row block, token block) pairs, row-block major, are dealt to the XCDs in 8
  // contiguous ranges, so that the token blocks of one row block run one after another on one XCD and its weights
  // come from that XCD's L2 after the first (dealt round-robin, every XCD would read every row block's weights)
  const int tbn = (a.m + BT - 1) / BT, nblk = gridDim.x;
  const int xcd = blockIdx.x % 8, j = blockIdx.x / 8;
  const int idx = xcd * (nblk / 8) + min(xcd, nblk % 8) + j;
  const int r0 = (idx / tbn) * (GLU ? BR / 2 : BR), t0 = (idx % tbn) * BT;
  const int G = a.k / 32, G4 = G & ~3, steps = G4 / KS, tail = G - G4;

  float acc[2][KS][16];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int c = 0; c < KS; ++c)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[h][c][v] = 0.0f;
  // the accumulators' start: 0 for the group sums themselves, MAGIC for the float32 path (products)
  const int c0 = SUMS ? 0 : MAGIC;
  const v16i start = {c0, c0, c0, c0, c0, c0, c0, c0, c0, c0, c0, c0, c0, c0, c0, c0};

  // the operands of this lane in a stage: weights row wr*32 + lane%32, activations tokens wt*64 + lane%32 and 32 later,
  // 16 bytes of each group at (lane / 32) * 16 (A and B take the same k bytes, so the sum is the group's)
  const int a_off = (wr * 32 + (lane & 31)) * ROWB + (lane >> 5) * 16;
  const int b_off = (wt * 64 + (lane & 31)) * ROWB + (lane >> 5) * 16;
  const int ws_off = wr * 32 + (lane >> 5) * 4;
  const int xs_off = wt * 64 + (lane & 31);

  Fetch<SIX> f;
  const int total = steps + (tail ? 1 : 0);
  if (total > 0) {
    fetch<SIX, SUMS, GLU>(f, a, r0, t0, 0, G, tid);
    store<SIX>(stage[0], f, tid);
  }
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const Stage &st = stage[s & 1];
    // the next stage fetched and stored unconditionally (no branch that would let the compiler move the products
    // below the stores): its groups are clamped into the row, and past the last stage what it stores goes to the
    // buffer no later read takes (the tail's stage is a real one: total > steps)
    fetch<SIX, SUMS, GLU>(f, a, r0, t0, (s + 1) * KS, G, tid);
    // a group's two MFMAs issued together, then their float32 work
#pragma unroll
    for (int gi = 0; gi < KS; ++gi) {
      const v4i av = *reinterpret_cast<const v4i *>(st.a + a_off + gi * 32);
      const v4i b0 = *reinterpret_cast<const v4i *>(st.b + b_off + gi * 32);
      const v4i b1 = *reinterpret_cast<const v4i *>(st.b + b_off + 32 * ROWB + gi * 32);
      const v16i S0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b0, start, 0, 0, 0);
      const v16i S1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b1, start, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (SUMS) {
        write_sums(a, S0, r0 + wr * 32, t0 + wt * 64, s * KS + gi, G, lane);
        write_sums(a, S1, r0 + wr * 32, t0 + wt * 64 + 32, s * KS + gi, G, lane);
      } else {
        products2(S0, S1, st.ws + gi * BR + ws_off, st.xs[gi * BT + xs_off], st.xs[gi * BT + xs_off + 32], acc[0][gi],
                  acc[1][gi]);
      }
    }
    // the next stage's stores wait for its global loads: kept after the products (the compiler would move them,
    // and their waits, above the float32 work that hides the loads' latency)
    if constexpr (!SUMS) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int c = 0; c < KS; ++c) pin16(acc[h][c]);
      asm volatile("" ::: "memory");
    }
    __builtin_amdgcn_sched_barrier(0);
    store<SIX>(stage[(s + 1) & 1], f, tid);
    __syncthreads();
  }

  // ((l0 + l1) + l2) + l3, then the tail groups in order
  float out[2][16];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int v = 0; v < 16; ++v) out[h][v] = ((acc[h][0][v] + acc[h][1][v]) + acc[h][2][v]) + acc[h][3][v];
  if (tail) {
    const Stage &st = stage[steps & 1];
#pragma unroll
    for (int gi = 0; gi < KS - 1; ++gi) {
      if (gi < tail) {
        const v4i av = *reinterpret_cast<const v4i *>(st.a + a_off + gi * 32);
        const v4i b0 = *reinterpret_cast<const v4i *>(st.b + b_off + gi * 32);
        const v4i b1 = *reinterpret_cast<const v4i *>(st.b + b_off + 32 * ROWB + gi * 32);
        const v16i S0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b0, start, 0, 0, 0);
        const v16i S1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b1, start, 0, 0, 0);
        if constexpr (SUMS) {
          write_sums(a, S0, r0 + wr * 32, t0 + wt * 64, G4 + gi, G, lane);
          write_sums(a, S1, r0 + wr * 32, t0 + wt * 64 + 32, G4 + gi, G, lane);
        } else {
          products2(S0, S1, st.ws + gi * BR + ws_off, st.xs[gi * BT + xs_off], st.xs[gi * BT + xs_off + 32], out[0],
                    out[1]);
        }
      }
    }
  }

  if constexpr (SUMS) return;
  if constexpr (GLU) {
    glu_epilogue(a, out, reinterpret_cast<float *>(&stage[0]), r0, t0, wave, lane);
    return;
  }
  // y[t][r] = out (or y + out): the lane's two tokens, its 16 rows in 4 runs of 4
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = t0 + wt * 64 + h * 32 + (lane & 31);
    if (t >= a.m) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int row = r0 + wr * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      if (row >= a.total_rows) continue;
      const int n0 = a.seg[0].rows, n1 = a.seg[1].rows;
      int si = 0, r = row;
      if (a.nseg > 2 && row >= n0 + n1) {
        si = 2;
        r = row - n0 - n1;
      } else if (a.nseg > 1 && row >= n0) {
        si = 1;
        r = row - n0;
      }
      float *y = (si == 2 ? a.seg[2].y : si == 1 ? a.seg[1].y : a.seg[0].y);
      const int stride = (si == 2 ? a.seg[2].y_stride : si == 1 ? a.seg[1].y_stride : a.seg[0].y_stride);
      const int accumulate = (si == 2 ? a.seg[2].accumulate : si == 1 ? a.seg[1].accumulate : a.seg[0].accumulate);
      float *dst = y + (int64_t)t * stride + r;
      *dst = accumulate ? *dst + out[h][v] : out[h][v];
    }
  }
}

}  // namespace

bool gemm_supported(int32_t k, bool relaxed) { return relaxed && k >= 32 && k % 32 == 0; }

hipError_t launch_gemm(const MatArgs &a, bool six, bool relaxed, hipStream_t s) {
  if (a.m < 1 || a.total_rows < 1 || !gemm_supported(a.k, relaxed)) return hipErrorInvalidValue;
  if (a.sums && a.nseg != 1) return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)((a.total_rows + BR - 1) / BR) * ((a.m + BT - 1) / BT);
  if (blocks > (1ll << 30)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks);
  if (a.sums) {
    if (six)
      gemm_kernel<true, true, false><<<grid, NT, 0, s>>>(a);
    else
      gemm_kernel<false, true, false><<<grid, NT, 0, s>>>(a);
  } else {
    if (six)
      gemm_kernel<true, false, false><<<grid, NT, 0, s>>>(a);
    else
      gemm_kernel<false, false, false><<<grid, NT, 0, s>>>(a);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_glu(const MatArgs &a, bool six, hipStream_t s) {
  const GluOut &g = a.glu;
  if (a.m < 1 || a.nseg != 2 || a.sums || !gemm_supported(a.k, true)) return hipErrorInvalidValue;
  const int hidden = a.seg[0].rows;
  if (hidden < 32 || hidden % 32 || a.seg[1].rows != hidden || a.total_rows != 2 * hidden) return hipErrorInvalidValue;
  // the output's 4-byte runs and its scales: every store aligned and inside [m][q_stride] / [m][s_stride]
  if (!g.q || !g.s || (g.bias != 0 && g.bias != 64) || g.q_stride < hidden || g.q_stride % 4 ||
      g.s_stride < hidden / 32 || reinterpret_cast<uintptr_t>(g.q) % 4)
    return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)(hidden / 32) * ((a.m + BT - 1) / BT);
  if (blocks > (1ll << 30)) return hipErrorInvalidValue;
  if (six)
    gemm_kernel<true, false, true><<<dim3((unsigned)blocks), NT, 0, s>>>(a);
  else
    gemm_kernel<false, false, true><<<dim3((unsigned)blocks), NT, 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace ple
