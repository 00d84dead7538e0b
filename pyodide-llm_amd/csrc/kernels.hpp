// kernels.hpp — the launch interfaces of the gfx950 kernels (host side). Every launch takes device pointers and a
// stream; shapes are checked by the callers in engine.cpp / the hk_* entry points before a launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ple {

// one matrix of a GEMV/GEMM launch: rows [rows][K] int8 (or int6 groups of 24 bytes), scales [rows][K/32]; the
// output y[t * y_stride + r] for token t, row r (accumulate: y = y + result, the residual add of kernels/kernel.ts:
// 691-693 fused)
struct MatSeg {
  const uint8_t *w;
  const float *ws;
  float *y;
  int32_t rows;
  int32_t y_stride;
  int32_t accumulate;
};

// the value cache holds a column's positions side by side, each column seq_len rounded up to 64 positions (256 bytes
// of float32): the weighted sums read a column's values as contiguous runs
inline int32_t value_stride(int32_t seq_len) { return (seq_len + 63) & ~63; }

// one token's q / k / v matmul (three segments) finishing the token's attention inputs in its epilogue, as
// launch_qkv_post does (the bias add, RoPE on q and k, k and v into the cache): the decode path only, rows in pairs
struct QkvFuse {
  int32_t on;
  const float *bq, *bk, *bv;   // Qwen2 biases or null
  const float *cos_t, *sin_t;  // [seq_len][hs/2]
  void *kcache, *vcache;       // this layer's keys [seq_len][kv_dim] and values [kv_dim][vstride]
  int32_t pos, hs, kvdim, half, vstride;
  const int32_t *dpos;  // the position in device memory (a replayed decode step), or null: pos
};

// An L2 fill ahead of a one-token GEMV, run by extra blocks of the rmsnorm launch before it, which leaves most CUs and
// the HBM idle. A launch's block b runs on XCD b % 8 (the 8 XCDs take blocks in
// turn, every launch from XCD 0), and each XCD has its own 4 MiB L2 that keeps its lines across launches: so the
// extra block whose launch-wide index is L touches every 64-byte line of the rows (values and scales) of the GEMV's
// blocks b = L (mod 8), and the GEMV's block b finds them in its own XCD's L2. Only reads; the results never change.
struct L2Fetch {
  const uint8_t *w[3];   // each segment's values [rows][row_bytes]
  const uint8_t *ws[3];  // and scales [rows][scale_bytes]
  int32_t rows[3];       // each a multiple of block_rows
  int32_t nseg;
  int32_t row_bytes, scale_bytes;
  int32_t block_rows;   // rows a GEMV block takes
  int32_t gemv_blocks;  // the GEMV blocks fetched: the first ones (those of its first round on the CUs)
  int32_t blocks;       // the extra blocks (a multiple of 8; 0: none)
  uint32_t *sink;       // 64 words, written only where the touched words' xor hits a constant (keeps the loads)
};
// The prompt's w1 / w3 GEMM finishing the SwiGLU in its epilogue (launch_gemm_glu): seg[0] is w1 and seg[1] w3, the
// same number of rows (hidden units, a multiple of 32); q / s take quantize_x(bias) of h1 / (1 + vexp(-h1)) * h3, the
// bytes and scales launch_swiglu_quant makes of the two outputs.
struct GluOut {
  int8_t *q;  // [m][q_stride]
  float *s;   // [m][s_stride]
  int32_t q_stride, s_stride, bias;
};
struct MatArgs {
  MatSeg seg[3];
  int32_t nseg;
  int32_t total_rows;
  const int8_t *xq;  // activations of quantize_x(bias), [m][xq_stride]
  const float *xs;   // their scales, [m][xs_stride]
  int32_t xq_stride;
  int32_t xs_stride;
  int32_t k;
  int32_t m;
  int32_t *sums;  // group-sum output (hk_group_sums) or null
  // one token (the decode path, decode_takes_f32): the float32 token instead of xq / xs, quantized in the launch,
  // after rmsnorm with weights xnorm (and eps) where xnorm is not null
  const float *xf;
  const float *xnorm;
  float eps;
  QkvFuse qkv;  // decode_fuses_qkv()
  // one token, rows of 1-4 KiB (decode_persistent): the persistent GEMV, about one block a CU that loops over its
  // rows (no L2Fetch fits it: its blocks take rows in another order)
  int32_t persistent;
  GluOut glu;  // launch_gemm_glu only
};

// rows a block of the one-token decode GEMV takes (launch_gemv with m = 1, bias 64, no sums) for rows of k, 0 where
// the launch goes another way
int32_t decode_block_rows(int32_t k, int32_t total_rows, bool six, bool relaxed, bool xf, bool qkv_on);

// the most tokens the engine gives one GEMV pass: more go to the MFMA GEMM where it takes them
constexpr int32_t GEMV_MOST = 8;

// decode GEMV, m <= 8 tokens: exact int32 group sums, the reference's float32 order
hipError_t launch_gemv(const MatArgs &a, bool six, bool relaxed, hipStream_t s);
// whether a one-token launch_gemv of rows of k takes its activations as float32 (MatArgs.xf)
bool decode_takes_f32(int32_t k, bool six, bool relaxed);
// whether a one-token launch_gemv of rows of k may ask for the persistent path (MatArgs.persistent)
bool decode_persistent(int32_t k, bool six, bool relaxed);
// whether a one-token launch_gemv of rows of k finishes q / k / v itself (MatArgs.qkv)
bool decode_fuses_qkv(int32_t k, bool six, bool relaxed);
// the most tokens one launch_gemv takes for rows of k (its products of a row fit the block's LDS)
int32_t gemv_tokens(int32_t k, bool relaxed);
// prefill GEMM on i8 MFMA, any m (bias 64, int8 or int6): the same bits as launch_gemv per (token, row); with
// a.sums (one segment) the exact int32 group sums [m][rows][K/32] instead
hipError_t launch_gemm(const MatArgs &a, bool six, bool relaxed, hipStream_t s);
// the w1 / w3 GEMM with the SwiGLU and its quantize_x in the epilogue (a.glu; bias 64 weights only)
hipError_t launch_gemm_glu(const MatArgs &a, bool six, hipStream_t s);
bool gemm_supported(int32_t k, bool relaxed);

// quantize_x over m rows of n (x_stride apart) into xq (xq_stride) / xs (xs_stride)
hipError_t launch_quantize(int8_t *xq, float *xs, const float *x, int32_t m, int32_t n, int32_t x_stride,
                           int32_t xq_stride, int32_t xs_stride, int32_t bias, hipStream_t s);
// rmsnorm then quantize_x, m tokens; out (optional) receives the normalized float32 row
hipError_t launch_rmsnorm_quant(int8_t *xq, float *xs, float *out, const float *x, const float *w, int32_t m,
                                int32_t n, int32_t x_stride, int32_t xq_stride, int32_t xs_stride, int32_t out_stride,
                                float eps, int32_t bias, hipStream_t s, const L2Fetch *fetch = nullptr);
// swiglu(h1, h3) then quantize_x, m tokens
hipError_t launch_swiglu_quant(int8_t *xq, float *xs, float *out, const float *h1, const float *h3, int32_t m,
                               int32_t n, int32_t h_stride, int32_t xq_stride, int32_t xs_stride, int32_t bias,
                               hipStream_t s);
// embedding rows of m tokens (int8 or int6 table) into x (x_stride apart); with a positions table (GPT-2's, the same
// kind, its group pgroup), the row of position (dpos ? *dpos : pos0) + t widened and added to each
struct Positions {
  const uint8_t *table;  // null: none
  const float *scales;
  int32_t group, pos0;
  const int32_t *dpos;
};
hipError_t launch_embed(float *x, const int32_t *tokens, const uint8_t *table, const float *scales, int32_t m,
                        int32_t dim, int32_t x_stride, int32_t group, bool six, const Positions &positions,
                        hipStream_t s);
// per token: + bias (optional), RoPE on q and k at pos0 + t, k and v into the cache (f32 or f16)
struct QkvPost {
  float *q;
  float *k;
  float *v;
  int32_t q_stride, kv_stride;
  const float *bq, *bk, *bv;
  const float *cos_t, *sin_t;  // [seq_len][hs/2]
  void *kcache, *vcache;       // this layer's keys [seq_len][kv_dim] and values [kv_dim][vstride]
  int32_t nh, nkv, hs, pos0, m, half, vstride;
  const int32_t *dpos;  // the first position in device memory (a replayed decode step), or null: pos0
  int32_t rot;          // the values of each head RoPE turns (kernels/kernel.ts:344-357): hs all, 0 none (GPT-2)
};
hipError_t launch_qkv_post(const QkvPost &a, hipStream_t s);

// attention of m tokens at positions pos0.. over the cache rows 0..pos0+t; out [m][out_stride]
struct AttnArgs {
  const float *q;
  int32_t q_stride;
  const void *kcache, *vcache;  // keys [seq_len][kv_dim] (a position's row), values [kv_dim][vstride] (a column's)
  float *out;
  int32_t out_stride;
  float *scores;  // [min(m, ATTN_ROWS)][nh][seq_len]
  float *tilemax; // [min(m, ATTN_ROWS)][nh][seq_len / 64 + 1]
  int32_t nh, nkv, hs, pos0, m, seq_len, half, vstride;
  // the first position in device memory (a replayed decode step), or null: pos0; with it, pos0 is only the largest
  // first position the launch may see (grid and LDS sizes)
  const int32_t *dpos;
  // where attention_quantizes(): quantize_x(bias) of out as well, [m][xq_stride] and [m][xs_stride] (null: not)
  int8_t *xq;
  float *xs;
  int32_t xq_stride, xs_stride, bias;
  // decode launches take the prompt's separate softmax and weighted-value kernels, as past the fused kernel's LDS
  int32_t split;
};
// a launch of more tokens runs them in pieces of at most ATTN_ROWS that reuse the score rows: a piece's score matrix
// (ATTN_ROWS x nh x its context, 134 MB at 32 heads and 2048 positions) written and read back through the 256 MB
// MALL, where a whole 1024- or 2048-token pass's would spill to HBM
constexpr int32_t ATTN_ROWS = 512;
hipError_t launch_attention(const AttnArgs &a, hipStream_t s);
// the head sizes and grouping the attention kernels take (hs in {16, 32, 48, 64, 96, 128, 256}, nh / nkv <= 8)
bool attention_supported(int32_t hs, int32_t nh, int32_t nkv);
// the longest context (a multiple of 4) the attention kernels take: a (token, head)'s exponentials are held in one
// block's LDS (160 KiB on gfx950) for their ordered sum
int32_t attention_most_positions();
// whether launch_attention writes quantize_x of its output too (a.xq): decode launches whose head size is a multiple
// of 32 (a block holds a whole group) and whose context fits the decode kernel's LDS
bool attention_quantizes(const AttnArgs &a);

// a streaming read of bytes (a multiple of 16) at p in launch shape `shape` (0 .. read_ceiling_shapes() - 1: loads a
// lane per tile, blocks): block b's sums of its 32-bit words lane by lane (j = word index % 4) into partial[4 b + j],
// for read_ceiling_blocks(bytes, shape) blocks
int32_t read_ceiling_shapes();
int32_t read_ceiling_blocks(int64_t bytes, int32_t shape);
int32_t read_ceiling_loads(int32_t shape);
hipError_t launch_read_ceiling(const void *p, int64_t bytes, int32_t shape, uint32_t *partial, hipStream_t s);
// ceilings.ts fma() in every lane of valu_ceiling_waves() waves, passes times (8 multiplies and 8 adds a pass, each
// rounded): lane 0 of wave i writes its sum of the eight accumulators to out[i]
int32_t valu_ceiling_waves();
hipError_t launch_valu_ceiling(int32_t passes, float w, float x0, float step, float spread, float *out, hipStream_t s);
// four v_mfma_i32_32x32x32_i8 a pass in each of mfma_ceiling_waves() waves: out[i] is wave i's sum (mod 2^32) of its
// accumulators' elements
int32_t mfma_ceiling_waves();
hipError_t launch_mfma_ceiling(int32_t passes, int32_t first, int32_t times, int32_t flip, uint32_t *out,
                               hipStream_t s);
// greedy: the first index of the largest logit into *out (and the value into *value)
hipError_t launch_argmax(int32_t *out, float *value, const float *x, int32_t n, float *scratch_v, int32_t *scratch_i,
                         hipStream_t s);
// the repetition penalty (kernels/kernel.ts:705-719) on the distinct tokens of tokens[0..count), count <= 64
hipError_t launch_penalize(float *logits, const int32_t *tokens, int32_t count, float penalty, hipStream_t s);
// one token drawn from softmax(logits / temperature) (kernels/kernel.ts:803-868) for random in [0, 1), restricted to
// the nucleus where 0 < topp < 1; *out_token is the token, SAMPLE_NOT_FINITE where the largest logit is not finite,
// or SAMPLE_DECLINED where the nucleus holds more tokens than one block sorts. probs: scratch of sample_probs_floats(n)
// (the float64 total reads whole chunks of SAMPLE_CHUNK, using none past n); index: scratch of n.
constexpr int32_t SAMPLE_NOT_FINITE = -1, SAMPLE_DECLINED = -2;
constexpr int32_t SAMPLE_MOST = 262144;  // logits a draw takes at most
constexpr int32_t SAMPLE_CHUNK = 2048;
constexpr size_t sample_probs_floats(int32_t n) { return ((size_t)n + SAMPLE_CHUNK - 1) / SAMPLE_CHUNK * SAMPLE_CHUNK; }
static_assert(SAMPLE_MOST % SAMPLE_CHUNK == 0, "the largest vocabulary is whole chunks");
constexpr int32_t SAMPLE_CHECKPOINT = 256;  // values between two checkpoints of the draw's running sum
// a chunk of the draw's float64 total taken at a guessed binade of the sum before it (sampling.hip, sum_block): the
// chunk's sum of r and its lanes' (0, 8, .., 56) sums of r before them, for either parity of the sum before the chunk
struct ChunkGuess {
  double t[2];
  double pre[2][SAMPLE_CHUNK / 32 / 8];
};
// a lane's 32 values of a chunk taken at one binade, whatever the sum before them (sampling.hip, lane_r): the lane's
// sum of r with its first tie's 1 left out, and its flags (bit 0 the parity flips after the last tie, bit 1 a tie
// seen, bit 2 the first tie's c)
struct LanePack {
  double s0;
  int32_t flags, unused;
};
// what the draw's blocks over the vocabulary (SAMPLE_CHUNK logits each) leave for the draw: each block's largest
// logit, its count of kept logits, its largest p and its sum of p; and without a nucleus, each chunk of the total at
// its guessed binade (guess: the binade, or none), its lanes at that binade and the next, and the first chunk's end and
// checkpoints
struct DrawParts {
  float bmax[SAMPLE_MOST / SAMPLE_CHUNK];
  int32_t bcount[SAMPLE_MOST / SAMPLE_CHUNK];
  float btop[SAMPLE_MOST / SAMPLE_CHUNK];
  float csum[SAMPLE_MOST / SAMPLE_CHUNK];
  int32_t guess[SAMPLE_MOST / SAMPLE_CHUNK];
  ChunkGuess g[SAMPLE_MOST / SAMPLE_CHUNK];
  LanePack lanes[SAMPLE_MOST / SAMPLE_CHUNK][2][64];
  double first_end;
  double first_cp[SAMPLE_CHUNK / SAMPLE_CHECKPOINT];
};
hipError_t launch_sample(const float *logits, int32_t n, float temperature, float topp, double random, float *probs,
                         int32_t *index, DrawParts *parts, int32_t *out_token, float *out_best, hipStream_t s);
// the draw's float64 total of p[0..n) in index order (kernels/kernel.ts:845-850), and the running sum before every
// SAMPLE_CHECKPOINT values (checkpoints: ceil(n / SAMPLE_CHECKPOINT) doubles); p: sample_probs_floats(n) floats. With
// parts, as the draw without a nucleus takes it (the chunks guessed over the CUs first); else as with one
hipError_t launch_ordered_sum(const float *p, int32_t n, double *total, double *checkpoints, DrawParts *parts,
                              hipStream_t s);
// ---- replayed decode steps (a captured graph of one step, replayed a round at a time) ----
// the step's state in device memory: the position, the step of the round, the halting step + 1 (0: none yet), the
// penalty window's count and its oldest entry once full
enum { STATE_POS = 0, STATE_STEP, STATE_HALTED, STATE_WINDOW, STATE_HEAD, STATE_WORDS = 8 };
constexpr int32_t RUN_STOPS_MOST = 8;   // stop tokens a replayed call takes (public/forward.js STOPS_MOST)
constexpr int32_t RUN_WINDOW = 64;      // the penalty's latest tokens (public/llama2_numpy.py:545)
constexpr int32_t RUN_RANDOMS = 64;     // random numbers of a round (its steps at most)
// the settings of a call's replayed steps, in device memory: one captured graph takes every call's
struct RunParams {
  double randoms[RUN_RANDOMS];  // the round's random numbers, step i's at i
  float temperature, topp, penalty;
  int32_t n_stops;
  int32_t stops[RUN_STOPS_MOST];
};
// a step's draw (as launch_sample) with the call's temperature and top-p and the round's random number of the step;
// with window, the call's penalty over the window's state[STATE_WINDOW] tokens first (launch_penalize_steps's, in the
// draw's first launch: the logits penalized in place); whole: the call's top-p is known to take no nucleus (one launch
// fewer)
hipError_t launch_sample_steps(float *logits, int32_t n, const RunParams *params, const int32_t *state,
                               const int32_t *window, bool whole, float *probs, int32_t *index, DrawParts *parts,
                               int32_t *out_token, float *out_best, hipStream_t s);
// the call's penalty over the window's state[STATE_WINDOW] tokens
hipError_t launch_penalize_steps(float *logits, const int32_t *window, const int32_t *state, const RunParams *params,
                                 hipStream_t s);
// the end of a replayed step that chose *token (largest logit *value): where this step ends the call (a stop token,
// no token, a largest logit that is not finite) and none before it did, its logits into kept and state[STATE_HALTED]
// = step + 1; its token and value into ids / values at the step, the token into the window and as the next step's
// input (tokens[0]), the position and the step advanced
hipError_t launch_step_end(const float *logits, int32_t n, float *kept, int32_t *tokens, int32_t *state,
                           const int32_t *token, const float *value, int32_t *ids, float *values, int32_t *window,
                           const RunParams *params, hipStream_t s);

// ---- the other forms (forms.hip) ----
// layernorm (eps 1e-5) then quantize_x, m tokens; out (optional) the float32 rows; copy (optional, x_stride) x itself
hipError_t launch_layernorm_quant(int8_t *xq, float *xs, float *out, float *copy, const float *x, const float *w,
                                  const float *b, int32_t m, int32_t n, int32_t x_stride, int32_t xq_stride,
                                  int32_t xs_stride, int32_t out_stride, int32_t bias, hipStream_t s);
// gelu(h + b) then quantize_x, m tokens (n a multiple of 32)
hipError_t launch_gelu_quant(int8_t *xq, float *xs, float *out, const float *h, const float *b, int32_t m, int32_t n,
                             int32_t h_stride, int32_t xq_stride, int32_t xs_stride, int32_t bias, hipStream_t s);
// x[t][j] += b[j] for m rows of n, stride apart
hipError_t launch_add_rows(float *x, const float *b, int32_t m, int32_t n, int32_t stride, hipStream_t s);
// Qwen3: q and k heads + bias (optional), then RMS-normalized in place by qw / kw (hs values each)
hipError_t launch_head_norm(float *q, float *k, const float *bq, const float *bk, const float *qw, const float *kw,
                            int32_t m, int32_t nh, int32_t nkv, int32_t hs, int32_t q_stride, int32_t kv_stride,
                            float eps, hipStream_t s);
// the outlier channels of the classifier's input
struct OutlierSet {
  int32_t n;
  int32_t c[8];
};
hipError_t launch_outlier_columns(float *columns, const uint8_t *table, const float *scales, int32_t vocab,
                                  int32_t dim, int32_t group, bool six, const OutlierSet &set, hipStream_t s);
hipError_t launch_pick(float *x, float *picked, const OutlierSet &set, hipStream_t s);
hipError_t launch_add_columns(float *y, const float *columns, const float *a, int32_t n, int32_t vocab, hipStream_t s);

// device synthesis of a checkpoint (the oracle's or_synth_checkpoint bits)
hipError_t launch_synth_matrix(uint8_t *values, float *scales, int64_t rows, int32_t k, uint64_t seed, int32_t stream,
                               float factor, bool six, hipStream_t s);
hipError_t launch_synth_vector(float *out, int64_t n, uint64_t seed, int32_t stream, float factor, bool ones,
                               hipStream_t s);

}  // namespace ple
