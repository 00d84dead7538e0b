/*
 * pyodide_llm_hip.h — the C ABI of the MI355X forward engine for pyodide-llm's quantized matmul path.
 *
 * The engine replaces the object public/forward.js:createForward returns (public/forward.js:1676-1955) for int8 / int6
 * checkpoints of the Llama form (with Qwen2's q/k/v biases and Qwen3's q/k head norms) and of the GPT-2 and GPT-NeoX
 * forms (LayerNorm, GELU, a bias after every projection; learned positions or partial RoPE; parallel residual). Every entry point takes plain pointers and sizes; device pointers are `void *`
 * and streams are `void *` (a hipStream_t, NULL = the engine's own stream). Every function returns 0 on success or a
 * negative HE_E* code; he_last_error() then names what failed (a thread-local string).
 *
 * Weights are the checkpoint's own bytes as quantize.py writes them (quantize.py:22-40, the tensor order of
 * public/llama2_convert.py:32-83): an int8 matrix is its int8 values [rows][K] followed by one float32 scale per group
 * of 32 [rows][K/32]; an int6 matrix packs every group into 24 bytes (public/llama2_numpy.py:678-692). The engine
 * uploads those bytes unchanged and addresses every tensor by the offsets the caller's plan gives
 * (public/llama2_numpy.py:751-795, Tensor.plan()).
 *
 * Arithmetic is the reference's CPU path to the bit: activations quantized per group of 32 (kernels/kernel.ts:129-156),
 * exact int32 group sums, and the float32 order of kernels/kernel_relaxed.ts:34-67 (bias 64) or kernels/kernel.ts:
 * 231-258 (bias 0), rmsnorm/layernorm/rope/attention/swiglu/gelu/add_columns in the order of kernels/kernel.ts.
 */
#ifndef PYODIDE_LLM_HIP_H
#define PYODIDE_LLM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes ---- */
#define HE_OK 0
#define HE_E_ARG -1      /* an argument is outside what the engine or the kernel takes */
#define HE_E_HIP -2      /* a HIP call failed (no device, out of memory, a launch failure) */
#define HE_E_STATE -3    /* the call does not fit the engine's state (a position past the context, ...) */
#define HE_E_NOTFINITE -4 /* greedy decoding met logits whose largest value is not finite (llama2_numpy.NOT_FINITE) */

/* plan.arch (public/forward.js:636) */
#define HE_ARCH_LLAMA 0 /* "llama": RMSNorm, RoPE, SwiGLU (Qwen2 and Qwen3 are this form with biases / head norms) */
#define HE_ARCH_GPT2 1  /* "gpt2": LayerNorm, learned positions added to the embedding, GELU, a bias after every matrix */
#define HE_ARCH_NEOX 2  /* "neox": GPT-2's layer with RoPE over the first `rotary` values of every head */
#define HE_OUTLIERS_MOST 8 /* OUTLIER_CHANNELS (public/llama2_numpy.py:561) */

/* The model: the fields of `plan` (public/llama2_numpy.py:1261-1270) the forward reads. */
typedef struct he_config {
  int32_t dim;               /* plan.dim */
  int32_t hidden_dim;        /* plan.hidden_dim */
  int32_t n_layers;          /* plan.n_layers */
  int32_t n_heads;           /* plan.n_heads */
  int32_t n_kv_heads;        /* plan.n_kv_heads */
  int32_t head_size;         /* plan.head_size */
  int32_t vocab_size;        /* plan.vocab_size (positive) */
  int32_t seq_len;           /* plan.seq_len: the context, and the rows of the RoPE tables */
  int32_t shared_classifier; /* plan.shared_classifier: wcls is token_embedding_table */
  int32_t six;               /* the matrices are int6 (Tensor kind "int6"), else int8 */
  int32_t qkv_bias;          /* Qwen2: bq, bk, bv are added after the q, k, v matmuls (public/forward.js:1038-1042) */
  int32_t relaxed;           /* 1: activations with bias 64, matmul_q8r order; 0: bias 0, matmul_q8 lane order */
  int32_t half_kv;           /* keys and values kept in float16 (public/forward.js:762, kernels/kernel.ts:570-608) */
  float rms_norm_eps;        /* plan.rms_norm_eps (RMSNorm; LayerNorm's is 1e-5, kernels/kernel.ts:627) */
  int32_t arch;              /* plan.arch: HE_ARCH_* */
  int32_t rotary;            /* plan.rotary: the values of each head RoPE turns (neox); 0 or head_size: all */
  int32_t parallel_residual; /* plan.parallel_residual: the FFN's LayerNorm reads the layer's input (GPT-NeoX) */
  int32_t qk_norm;           /* Qwen3: every head of q and k RMS-normalized by q_norm / k_norm before RoPE
                                (public/forward.js:1043-1047) */
  int32_t n_outliers;        /* plan.outliers: channels of the classifier's input multiplied apart in float32
                                (public/forward.js:801-812,1084-1089), at most HE_OUTLIERS_MOST */
  int32_t outliers[HE_OUTLIERS_MOST];
} he_config;

/* Where a tensor is: byte offsets from the start of the checkpoint (Tensor.offset, Tensor.scales). */
typedef struct he_tensor {
  int64_t offset;
  int64_t scales; /* matrices only; 0 for float32 vectors */
} he_tensor;

/* The order of he_tensor arrays: the names of public/llama2_numpy.py TENSOR_NAMES the forward reads. */
enum {
  HE_T_EMBEDDING = 0, /* token_embedding_table [vocab][dim], int8 or int6 */
  HE_T_RMS_ATT,       /* rms_att_weight [layers][dim] f32 (LayerNorm's weight in gpt2 and neox) */
  HE_T_WQ,            /* wq [layers][n_heads*head_size][dim] */
  HE_T_WK,            /* wk [layers][kv_dim][dim] */
  HE_T_WV,            /* wv [layers][kv_dim][dim] */
  HE_T_WO,            /* wo [layers][dim][n_heads*head_size] */
  HE_T_RMS_FFN,       /* rms_ffn_weight [layers][dim] f32 (the same) */
  HE_T_W1,            /* w1 [layers][hidden][dim] */
  HE_T_W2,            /* w2 [layers][dim][hidden] */
  HE_T_W3,            /* w3 [layers][hidden][dim] (llama only) */
  HE_T_RMS_FINAL,     /* rms_final_weight [dim] f32 (the same) */
  HE_T_WCLS,          /* wcls [vocab][dim] (the embedding's offsets when shared) */
  HE_T_BQ,            /* bq [layers][q_dim] f32 (qkv_bias; always for gpt2 and neox) */
  HE_T_BK,            /* bk [layers][kv_dim] f32 */
  HE_T_BV,            /* bv [layers][kv_dim] f32 */
  HE_T_Q_NORM,        /* q_norm [layers][head_size] f32 (qk_norm) */
  HE_T_K_NORM,        /* k_norm [layers][head_size] f32 (qk_norm) */
  HE_T_POSITIONS,     /* positions [seq_len][dim], int8 or int6 (gpt2: a learned row added to the embedding) */
  HE_T_LN_ATT_BIAS,   /* ln_att_bias [layers][dim] f32 (gpt2, neox: LayerNorm's bias; its weight is rms_att_weight) */
  HE_T_LN_FFN_BIAS,   /* ln_ffn_bias [layers][dim] f32 */
  HE_T_LN_FINAL_BIAS, /* ln_final_bias [dim] f32 */
  HE_T_BO,            /* bo [layers][dim] f32 (gpt2, neox: the biases after wo, w1, w2) */
  HE_T_B1,            /* b1 [layers][hidden] f32 */
  HE_T_B2,            /* b2 [layers][dim] f32 */
  HE_T_COUNT
};

typedef struct he_engine he_engine;

/* the message of the last failed call on this thread ("" if none) */
const char *he_last_error(void);

/* ---- the engine: public/forward.js external().start(plan) and the object it returns ---- */

/* start(plan) (public/forward.js:571-590, createForward :626): uploads `size` bytes of checkpoint (host memory) to the
 * device, the RoPE tables plan.derived.freq_cis_real/imag ([seq_len][head_size/2] float32, host), and makes the
 * KV cache for the whole context. max_block: the most tokens one he_forward_many call takes (promptBlock).
 * seq_len may be at most 40,704 positions (HE_E_ARG past it): a (token, head)'s exponentials are held in one
 * workgroup's 160 KiB of LDS for their ordered sum (kernels/kernel.ts:499-520). */
int32_t he_open(const he_config *cfg, const he_tensor *tensors, const void *checkpoint, uint64_t size,
                const float *rope_cos, const float *rope_sin, int32_t max_block, he_engine **out);

/* The same, with the checkpoint made on the device from a seed rather than uploaded: every matrix N(0, 0.02) by a
 * counter-based generator (a splitmix64 hash of (seed, tensor, index) whose four 16-bit quarters are summed: a
 * scaled Irwin-Hall(4) variate, so that host and device make the same float32 bits), quantized by the reference's
 * quantize()/quantize6() rules, norm weights 1.0, biases N(0, 0.02). For measurements of models too large to make on
 * the host quickly. `tensors` must place every tensor as Places.take() does (public/llama2_numpy.py:751-775). */
int32_t he_open_synthetic(const he_config *cfg, const he_tensor *tensors, uint64_t size, uint64_t seed,
                          const float *rope_cos, const float *rope_sin, int32_t max_block, he_engine **out);

/* engine.forward(token, pos, needLogits) (public/forward.js:1891-1912): one token at position pos through every
 * layer, its key and value into the cache; with need_logits the logits are computed and, if logits is not NULL,
 * copied into it (vocab_size floats, host). Blocks until done. */
int32_t he_forward(he_engine *e, int32_t token, int32_t pos, int32_t need_logits, float *logits);

/* engine.forwardMany(tokens, pos) (public/forward.js:1755-1769): count tokens at pos, pos+1, ... without logits;
 * every token's numbers are those he_forward gives it alone. count <= he_prompt_block(e). */
int32_t he_forward_many(he_engine *e, const int32_t *tokens, int32_t count, int32_t pos);

/* engine.generateMany(token, pos, history, length, count, temperature, topp, penalty, randoms, stops)
 * (public/forward.js:1831-1890): up to `count` steps from token at pos, each the forward pass with logits, then the
 * repetition penalty where penalty != 1 (kernels/kernel.ts:705-719, over the distinct tokens of the latest 64 of
 * history[0..n_history) followed by the tokens this call has chosen; history ends with `token`, as the caller's
 * history does; `length` is the caller's full history length, kept for the interface), then the next token: with
 * temperature 0 the first index of the largest logit (public/llama2_numpy.py:1521-1527), else a draw from the
 * temperature-scaled logits restricted to the nucleus where 0 < topp < 1 (kernels/kernel.ts:803-868) with randoms[i]
 * for step i (n_randoms >= count; the caller's generator's numbers in [0, 1)).
 * ids receives the tokens chosen, a stop token last where one came; *n_ids their number. The logits of the last step
 * (penalized where the penalty applied) stay readable with he_logits. Returns HE_E_NOTFINITE where a step's largest
 * logit is not finite (nothing of that step is in ids). *n_ids may be less than count without a stop token where a
 * step's nucleus holds more tokens than the device sorts (more than 8192): the caller takes that step itself, and
 * *n_ids = 0 is the reference's "the GPU did not take them" (undefined).
 * With at most 8 stop tokens (public/forward.js STOPS_MOST) the steps after the first are replayed from a captured
 * graph of one step, every choice (greedy, penalty, draw, stop) made on the device and the tokens read back once a
 * round (16 steps with stop tokens, 64 without): where a step ends the call, the round's later replays still run,
 * and their cache rows, past the positions of the ids returned, hold what the next step at those positions
 * overwrites. */
int32_t he_generate_many(he_engine *e, int32_t token, int32_t pos, const int32_t *history, int32_t n_history,
                         int32_t length, int32_t count, float temperature, float topp, float penalty,
                         const double *randoms, int32_t n_randoms, const int32_t *stops, int32_t n_stops, int32_t *ids,
                         int32_t *n_ids);

/* engine.logits() (public/forward.js:1936): the logits of the last step with logits, vocab_size floats (host). */
int32_t he_logits(he_engine *e, float *out);

/* engine.keysAndValues(from, count) (public/forward.js:1939-1953): the cache at positions from..from+count-1 as
 * float32 [layers][count][kv_dim], keys then values (host). */
int32_t he_kv_read(he_engine *e, int32_t from, int32_t count, float *keys, float *values);

/* external().read(offset, length) (public/forward.js:574): bytes of the checkpoint as the device holds them. */
int32_t he_checkpoint_read(he_engine *e, uint64_t offset, uint64_t length, void *out);

/* engine.promptBlock (public/forward.js:1773-1778): how many tokens he_forward_many takes at once. */
int32_t he_prompt_block(he_engine *e);

/* engine.memoryBytes() (public/forward.js:1954): the device bytes the engine holds. */
uint64_t he_device_bytes(he_engine *e);

/* engine.release() (public/forward.js:1918-1935): frees everything the engine holds. */
int32_t he_close(he_engine *e);

/* The kinds of kernel he_profile_forward reports on */
enum {
  HE_K_GEMV = 0,   /* the decode matmuls (m <= 8 tokens) */
  HE_K_GEMM,       /* the prefill matmuls on MFMA */
  HE_K_ATTENTION,  /* scores, softmax, weighted values */
  HE_K_NORM,       /* rmsnorm with quantize_x, quantize_x alone */
  HE_K_ELEMENTWISE,/* embed, bias + RoPE + cache write, swiglu with quantize_x */
  HE_K_ARGMAX,     /* greedy selection */
  HE_K_COUNT
};

/* One forward step timed by kind of kernel: the counterpart of the profiling wrap of public/forward.js:646-647 that
 * tests/profile.mjs uses. Runs he_forward(token, pos, need_logits) with a HIP event pair around every launch on the
 * engine's stream, and fills ms[HE_K_COUNT] (device time), bytes[HE_K_COUNT] (the algorithmic bytes the launches
 * read and write: weights, scales, activations, cache rows) and launches[HE_K_COUNT]. */
int32_t he_profile_forward(he_engine *e, int32_t token, int32_t pos, int32_t need_logits, double *ms, double *bytes,
                           int32_t *launches);

/* he_profile_forward for a prompt chunk: he_forward_many(tokens, count, pos) (count <= the engine's promptBlock)
 * with every launch timed and summed by kind the same way. */
int32_t he_profile_forward_many(he_engine *e, const int32_t *tokens, int32_t count, int32_t pos, double *ms,
                                double *bytes, int32_t *launches);

/* The decode matmuls (one token, m = 1) of the engine's own weights timed on their own, the counterpart of the
 * reference's matmul timing over its weights (tests/q8r-bench.mjs:115-135): `which` -1 runs every matmul of a decode
 * step in the step's order (q/k/v, wo, w1/w3, w2 of each layer, then the classifier), 0..4 only q/k/v, wo, w1/w3, w2
 * or the classifier of every layer. The sequence runs `rounds` times back to back on the engine's stream between one
 * HIP event pair, on the engine's current activations, its outputs into scratch rows (the cache, activations and
 * logits are not touched). *ms: the mean duration of one pass; *bytes: the algorithmic bytes of one pass (weights,
 * scales, activations, outputs); *launches: the launches of one pass. */
int32_t he_profile_matmul(he_engine *e, int32_t which, int32_t rounds, double *ms, double *bytes, int32_t *launches);

/* ---- kernel level: device pointers, for the standalone matmul and the parity tests ---- */

/* quantize_x (kernels/kernel.ts:129-156) of m rows of n float32 (row stride n): int8 rows (stride n) and float32
 * scales (stride n/32), bias 64 (q in 1..127) or 0 (q in -127..127). n % 32 == 0. */
int32_t hk_quantize_x(void *xq, void *xs, const void *x, int32_t m, int32_t n, int32_t bias, void *stream);

/* y[t][r] for m tokens and rows r < rows of an int8 (six = 0) or int6 (six = 1) matrix of K columns, its float32
 * group scales ws [rows][K/32], against activations xq [m][K] / xs [m][K/32] from hk_quantize_x with the same bias:
 * matmul_q8r (kernels/kernel_relaxed.ts:34-67) for bias 64, matmul_q8 (kernels/kernel.ts:231-258) for bias 0,
 * matmul_q6r / matmul_q6 for int6; matmul_q8r_tile (kernels/kernel_relaxed.ts:164-183) is the same per token.
 * y is [m][rows] float32. m <= 8 runs the decode GEMV, larger m the MFMA GEMM; both give the same bits. */
int32_t hk_matmul(void *y, const void *xq, const void *xs, const void *w, const void *ws, int32_t m, int32_t rows,
                  int32_t k, int32_t bias, int32_t six, void *stream);

/* The exact int32 sums the matmuls scale, through the same loaders: for bias 64 one per (token, row, group),
 * dot(w, q - 64) (kernels/kernel_relaxed.ts:47-55); for bias 0 four per group, the lanes of kernels/kernel.ts:222-229
 * (lane k: products 2k, 2k+1, 2k+8, 2k+9 of each half of 16). s is [m][rows][K/32] or [m][rows][K/32][4] int32.
 * gemm = 0 uses the GEMV loader, 1 the MFMA GEMM's. */
int32_t hk_group_sums(void *s, const void *xq, const void *w, int32_t m, int32_t rows, int32_t k, int32_t bias,
                      int32_t six, int32_t gemm, void *stream);

/* kernels/kernel.ts:705-719 penalize on device logits (n floats): each distinct token of tokens[0..count) (host,
 * count <= 64, every token in [0, n)) once, value > 0 ? value / penalty : value * penalty. Blocks until done. */
int32_t hk_penalize(void *logits, int32_t n, const int32_t *tokens, int32_t count, float penalty, void *stream);

/* The float64 total of sample()'s kept probabilities (kernels/kernel.ts:845-850: total += p in index order) on device
 * p (n floats, 1 <= n <= 262144) into *total (host), and with checkpoints (host, ceil(n / 256) doubles, or null) the
 * running sum before every 256 values, as the draw's search takes them; nucleus nonzero: by the one block that the
 * draw with a nucleus uses, else as the draw without one takes it (its chunks guessed over the CUs first). The same
 * bits either way. Blocks until done. */
int32_t hk_ordered_sum(const void *p, int32_t n, int32_t nucleus, double *total, double *checkpoints, void *stream);

/* kernels/kernel.ts:803-868 sample on device logits (n floats): the token drawn for random in [0, 1) into *token
 * (host): -1 where the largest logit is not finite, -2 where the nucleus holds more than 8192 tokens. temperature
 * > 0. Blocks until done. */
int32_t hk_sample(const void *logits, int32_t n, float temperature, float topp, double random, int32_t *token,
                  void *stream);

/* No counterpart in the reference: hk_sample for callers that cannot allocate device memory (serving loops and
 * harnesses that forbid hipMalloc). The same draw as hk_sample, token for token, with the
 * sampler's scratch (n probabilities and n token indices, the token and the largest logit, the vocabulary launches'
 * parts for the draw) in a static device array of
 * the library, which every GPU it runs on holds until the process ends; n <= HK_SAMPLE_STATIC_MOST, else HE_E_ARG.
 * It allocates nothing. Every call on one GPU uses that GPU's one array: calls that overlap on one GPU (two streams,
 * two threads) race, and the caller must order them. Blocks until done: it copies the token to the host and waits
 * for the stream, so a stream under graph capture is refused (HE_E_ARG) before anything is launched. */
#define HK_SAMPLE_STATIC_MOST 262144
int32_t hk_sample_static(const void *logits, int32_t n, float temperature, float topp, double random, int32_t *token,
                         void *stream);

/* The memory's read ceiling, kernels/ceilings.ts:9-25 read(p, bytes, passes) on the device: bytes (a multiple of 64)
 * at the device pointer p read by a streaming kernel in each of a few launch shapes (8 to 16 loads of 16 bytes a lane
 * in flight, 256 to 2048 blocks), one untimed pass then passes timed ones a shape. *checksum is read()'s: the xor of
 * the four lanes j of passes times the sum (mod 2^32) of the 32-bit words at p + 16k + 4j (every shape's must agree,
 * else HE_E_HIP). *ms is the fastest shape's mean time of a pass (HIP events on the stream). Blocks until done. */
int32_t hk_read_ceiling(const void *p, int64_t bytes, int32_t passes, int32_t *checksum, double *ms, void *stream);

/* No counterpart in the reference (a measurement beside hk_read_ceiling): the time of one cold streaming read of
 * `bytes` (a multiple of 64), as a decode matmul's launch reads its matrix: launches back to back, each reading the next
 * window of `bytes` within the `span` bytes at the device pointer p (a span larger than the 256 MB MALL keeps every
 * window cold), with hk_read_ceiling's kernel and launch shapes; *us is the fastest shape's mean microseconds a launch
 * over `passes` launches. It allocates a few KiB. Blocks until done. */
int32_t hk_read_floor(const void *p, int64_t span, int64_t bytes, int32_t passes, double *us, void *stream);

/* The float32 multiply-add ceiling, kernels/ceilings.ts:27-50 fma(passes, w, x0, step) in every lane of a launch
 * that fills the device (8192 waves of 64): eight accumulators (starting at 0..7), a pass adds w_j * x and w_j * y
 * (w_j = w + {0, 2^-10, 2^-9, 3 * 2^-10}; x from x0, y from x0 + 0.25, both moving by -step a pass) to them, each
 * product and sum rounded on its own (no FMA, no packed FP32: the form of every step of the exact order). *result is
 * one lane's ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)), which every wave must agree on (else HE_E_HIP); fma()
 * returns the sum of its four equal lanes of it. *ms is the mean time of a launch (three after one untimed), *pairs
 * the multiply + add pairs a launch makes (8 a pass a lane). Blocks until done. */
int32_t hk_valu_ceiling(int32_t passes, float w, float x0, float step, float *result, double *ms, double *pairs,
                        void *stream);

/* The int8 matrix-core ceiling, kernels/ceilings_relaxed.ts:33-50 dotRegisters(passes, first, times, step) on the
 * instruction the prompt GEMM takes (v_mfma_i32_32x32x32_i8), from registers only, in 4096 waves: four 32 x 32 int32
 * accumulators a wave, accumulator n starting at 1000 n + e in element e of every lane; a pass one product into each
 * with every byte of A = first (xor flip after every pass, in place of dotRegisters' moving step) and every byte of
 * B = times. *checksum is a wave's sum (mod 2^32) of the elements of its four accumulators in its 64 lanes, which every
 * wave must agree on (else HE_E_HIP): 4 * 64 * 16 * (mean start) + 4 * 1024 * 32 * times * (the sum of A's byte over
 * the passes) as int8 arithmetic mod 2^32. *ms is the mean time of a launch (three after one untimed), *ops its
 * integer operations (a multiply and an add for each of the 32768 products of every MFMA). Blocks until done. */
int32_t hk_mfma_ceiling(int32_t passes, int32_t first, int32_t times, int32_t flip, int32_t *checksum, double *ms,
                        double *ops, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PYODIDE_LLM_HIP_H */
