// engine.cpp — the C ABI of include/pyodide_llm_hip.h: the forward engine public/forward.js createForward builds
// (public/forward.js:626-1955), for the int8/int6 Llama and Qwen2 forms, on one MI355X.
//
// Device memory: every tensor of the checkpoint in its own 256-byte aligned region of one allocation (the file's
// offsets are only 4-byte aligned), so that the matmuls stream rows with 16-byte loads; a region table maps file
// offsets to device addresses for external().read. The KV cache is allocated for the whole context at start (the
// reference grows it from 256 positions by doubling, public/forward.js:828-848; the values do not depend on it).
// One stream, default priority; every call blocks until its results are on the host, as forward.js's do.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/pyodide_llm_hip.h"
#include "kernels.hpp"

using namespace ple;

namespace {

thread_local std::string g_error;

int32_t fail(int32_t code, const std::string &what) {
  g_error = what;
  return code;
}

#define HIP_TRY(expr)                                                                          \
  do {                                                                                         \
    hipError_t err_ = (expr);                                                                  \
    if (err_ != hipSuccess)                                                                    \
      return fail(HE_E_HIP, std::string(#expr) + ": " + hipGetErrorString(err_));             \
  } while (0)

int32_t group_size(int32_t row_length) {  // public/llama2_convert.py:25-29
  int32_t size = 32;
  while (row_length % size) size /= 2;
  return size;
}

struct Shape {
  int64_t count;  // values in the tensor
  int32_t k;      // the row length (matrices), 0 for float32 vectors
  int32_t rows;   // rows of one layer (matrices)
  int32_t layers;
};

Shape shape_of(const he_config &c, int id) {
  const int64_t L = c.n_layers, dim = c.dim, hidden = c.hidden_dim, vocab = c.vocab_size;
  const int32_t qdim = c.n_heads * c.head_size, kvdim = c.n_kv_heads * c.head_size;
  switch (id) {
    case HE_T_EMBEDDING: return {vocab * dim, c.dim, c.vocab_size, 1};
    case HE_T_RMS_ATT: return {L * dim, 0, 0, c.n_layers};
    case HE_T_WQ: return {L * qdim * dim, c.dim, qdim, c.n_layers};
    case HE_T_WK: return {L * kvdim * dim, c.dim, kvdim, c.n_layers};
    case HE_T_WV: return {L * kvdim * dim, c.dim, kvdim, c.n_layers};
    case HE_T_WO: return {L * dim * qdim, qdim, c.dim, c.n_layers};
    case HE_T_RMS_FFN: return {L * dim, 0, 0, c.n_layers};
    case HE_T_W1: return {L * hidden * dim, c.dim, c.hidden_dim, c.n_layers};
    case HE_T_W2: return {L * dim * hidden, c.hidden_dim, c.dim, c.n_layers};
    case HE_T_W3: return {L * hidden * dim, c.dim, c.hidden_dim, c.n_layers};
    case HE_T_RMS_FINAL: return {dim, 0, 0, 1};
    case HE_T_WCLS: return {vocab * dim, c.dim, c.vocab_size, 1};
    case HE_T_BQ: return {L * qdim, 0, 0, c.n_layers};
    case HE_T_BK: return {L * kvdim, 0, 0, c.n_layers};
    case HE_T_BV: return {L * kvdim, 0, 0, c.n_layers};
    case HE_T_Q_NORM: return {L * c.head_size, 0, 0, c.n_layers};
    case HE_T_K_NORM: return {L * c.head_size, 0, 0, c.n_layers};
    case HE_T_POSITIONS: return {(int64_t)c.seq_len * dim, c.dim, c.seq_len, 1};
    case HE_T_LN_ATT_BIAS: return {L * dim, 0, 0, c.n_layers};
    case HE_T_LN_FFN_BIAS: return {L * dim, 0, 0, c.n_layers};
    case HE_T_LN_FINAL_BIAS: return {dim, 0, 0, 1};
    case HE_T_BO: return {L * dim, 0, 0, c.n_layers};
    case HE_T_B1: return {L * hidden, 0, 0, c.n_layers};
    case HE_T_B2: return {L * dim, 0, 0, c.n_layers};
  }
  return {0, 0, 0, 0};
}

bool layer_norm(const he_config &c) { return c.arch == HE_ARCH_GPT2 || c.arch == HE_ARCH_NEOX; }

// the tensors of the form (public/llama2_convert.py:32-83): Llama's with Qwen2's biases and Qwen3's head norms where
// the form has them; GPT-2's and GPT-NeoX's LayerNorm biases, biases after every matrix, no w3, GPT-2's positions
bool present(const he_config &c, int id) {
  switch (id) {
    case HE_T_WCLS: return !c.shared_classifier;  // else the embedding's
    case HE_T_W3: return !layer_norm(c);
    case HE_T_BQ:
    case HE_T_BK:
    case HE_T_BV: return layer_norm(c) || c.qkv_bias;
    case HE_T_Q_NORM:
    case HE_T_K_NORM: return !layer_norm(c) && c.qk_norm;
    case HE_T_POSITIONS: return c.arch == HE_ARCH_GPT2;
    case HE_T_LN_ATT_BIAS:
    case HE_T_LN_FFN_BIAS:
    case HE_T_LN_FINAL_BIAS:
    case HE_T_BO:
    case HE_T_B1:
    case HE_T_B2: return layer_norm(c);
  }
  return true;
}

// the float32 vectors a synthetic checkpoint fills with 1.0 (norm weights); the others are biases, N(0, 0.02)
bool norm_weight(int id) {
  return id == HE_T_RMS_ATT || id == HE_T_RMS_FFN || id == HE_T_RMS_FINAL || id == HE_T_Q_NORM || id == HE_T_K_NORM;
}

static_assert(HE_OUTLIERS_MOST == 8, "OutlierSet holds 8 channels");

struct Region {
  uint64_t file, bytes, dev;
};

template <typename T>
int32_t dev_alloc(T **p, size_t bytes) {
  void *q = nullptr;
  HIP_TRY(hipMalloc(&q, bytes ? bytes : 1));
  *p = reinterpret_cast<T *>(q);
  return HE_OK;
}

}  // namespace

struct he_engine {
  he_config c{};
  he_tensor t[HE_T_COUNT]{};
  hipStream_t stream = nullptr;
  uint64_t size = 0;
  uint8_t *blob = nullptr;  // the regions
  uint64_t blob_bytes = 0;
  std::vector<Region> regions;
  const uint8_t *values[HE_T_COUNT]{};
  const float *scales[HE_T_COUNT]{};
  float *cos_t = nullptr, *sin_t = nullptr;
  void *keys = nullptr, *vals = nullptr;  // keys [layers][seq_len][kv_dim], values [layers][kv_dim][value_stride]
  int32_t qdim = 0, kvdim = 0, bias = 64, max_block = 1, chunk = 1, xw = 0, widest = 0;
  // activations of `chunk` tokens
  float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *hb = nullptr, *hb2 = nullptr;
  int8_t *xq = nullptr;
  float *xs = nullptr;
  float *scores = nullptr, *tilemax = nullptr;
  float *logits = nullptr;
  int32_t *tokens = nullptr;
  float *amax_v = nullptr;
  int32_t *amax_i = nullptr;
  float *best_v = nullptr;
  int32_t *best_i = nullptr;
  uint64_t device_bytes = 0;
  bool have_logits = false;
  // greedy decode steps replayed from one captured graph of a whole step (embedding to argmax), which reads its token
  // (tokens[0]) and position (state[0]) from device memory and advances them itself
  int32_t *state = nullptr;                           // [0] position, [1] step of the round
  int32_t *step_ids = nullptr;                        // [STEPS_A_ROUND] tokens of a round
  float *step_values = nullptr;                       // their logits
  int32_t *host_ids = nullptr, *host_state = nullptr;  // pinned
  float *host_values = nullptr;                       // pinned
  // the captured step graphs by kind (STEP_GREEDY or STEP_SAMPLED, with STEP_WHOLE and STEP_PENALIZED)
  hipGraphExec_t graph[8] = {};
  bool graph_tried[8] = {};
  // a call's settings (device, and its pinned host copy); the logits of the step that ended the last call, where the
  // round's later replays overwrote its own
  RunParams *run_params = nullptr, *host_params = nullptr;
  float *kept_logits = nullptr;
  bool logits_kept = false;
  // sampled steps: the sampler's scratch, the penalty's window, the token drawn (device); the window (pinned)
  float *sample_probs = nullptr;
  int32_t *sample_index = nullptr, *window = nullptr, *sample_token = nullptr;
  float *sample_best = nullptr;
  DrawParts *sample_parts = nullptr;
  int32_t *host_window = nullptr;
  // the other forms: the layer's input a parallel residual's FFN normalizes (GPT-NeoX); the outlier channels' float32
  // columns of the classifier [n][vocab] and the values taken out of the classifier's input
  float *before = nullptr, *columns = nullptr, *picked = nullptr;
  OutlierSet outliers{};
  bool replayable = false;  // run_chunk is building the graph (positions from state, no host copies)
  // PYODIDE_LLM_HIP_ATTEND=split: decode steps take the separate softmax and weighted-value kernels that contexts
  // past the fused decode kernel's LDS take (a check of that path at any context)
  bool attend_split = false;
  // one-token GEMVs whose first rows extra blocks of the launch before them bring into L2 (L2Fetch); sink: their
  // 64 words
  int64_t fetch_xcd_bytes = 3 << 20;
  uint32_t *sink = nullptr;
  // he_profile_forward: event pairs around every launch while `profiling` is set
  struct Mark {
    int kind;
    double bytes;
    hipEvent_t a, b;
  };
  bool profiling = false;
  std::vector<Mark> marks;

  const uint8_t *mat(int id, int l) const {
    const Shape s = shape_of(c, id == HE_T_WCLS && c.shared_classifier ? HE_T_EMBEDDING : id);
    const int64_t row_bytes = c.six ? (int64_t)s.k / 32 * 24 : s.k;
    return values[id] + (int64_t)l * s.rows * row_bytes;
  }
  const float *mat_scales(int id, int l) const {
    const Shape s = shape_of(c, id == HE_T_WCLS && c.shared_classifier ? HE_T_EMBEDDING : id);
    return scales[id] + (int64_t)l * s.rows * (s.k / 32);
  }
  const float *vec(int id, int64_t at) const { return reinterpret_cast<const float *>(values[id]) + at; }
};

namespace {

constexpr int32_t STEPS_A_ROUND = 64;      // replayed steps between two reads of their tokens
constexpr int32_t STOP_ROUND = 16;         // the same where a stop token may end the call early (the round's later
                                           // replays are then spent for nothing)
constexpr int32_t REPETITION_WINDOW = RUN_WINDOW;  // the penalty's latest tokens (public/llama2_numpy.py:545)
static_assert(STEPS_A_ROUND <= RUN_RANDOMS, "a random number for every step of a round");
// the kinds of replayed step graph
enum { STEP_GREEDY = 0, STEP_PENALIZED = 1, STEP_SAMPLED = 2, STEP_WHOLE = 4 };  // (WHOLE: sampled, no nucleus)

void destroy(he_engine *e) {
  if (!e) return;
  for (hipGraphExec_t g : e->graph)
    if (g) (void)hipGraphExecDestroy(g);
  void *ptrs[] = {e->blob, e->cos_t, e->sin_t, e->keys, e->vals, e->x, e->xb, e->q, e->k, e->v, e->hb, e->hb2,
                  e->xq, e->xs, e->scores, e->tilemax, e->logits, e->tokens, e->amax_v, e->amax_i,
                  e->best_v, e->best_i, e->state, e->step_ids, e->step_values, e->sample_probs, e->sample_index,
                  e->window, e->sample_token, e->sample_best, e->before, e->columns, e->picked, e->sink,
                  e->run_params, e->kept_logits, e->sample_parts};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  void *pinned[] = {e->host_ids, e->host_state, e->host_values, e->host_window, e->host_params};
  for (void *p : pinned)
    if (p) (void)hipHostFree(p);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

int32_t check_config(const he_config &c) {
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
      c.head_size <= 0 || c.vocab_size <= 0 || c.seq_len <= 0)
    return fail(HE_E_ARG, "the plan has a size that is not positive");
  if (c.n_heads % c.n_kv_heads) return fail(HE_E_ARG, "n_heads is not a multiple of n_kv_heads");
  if (c.head_size % 4) return fail(HE_E_ARG, "head_size is not a multiple of 4");
  const int32_t qdim = c.n_heads * c.head_size, kvdim = c.n_kv_heads * c.head_size;
  if (c.dim % 32 || c.hidden_dim % 32 || qdim % 32 || kvdim % 32)
    return fail(HE_E_ARG, "the int8 kernels take rows of whole groups of 32 (dim, hidden, q and kv widths)");
  if (!attention_supported(c.head_size, c.n_heads, c.n_kv_heads))
    return fail(HE_E_ARG, "attention takes head sizes 16, 32, 48, 64, 96, 128, 256 and at most 8 query heads a kv head");
  if (c.seq_len % 4) return fail(HE_E_ARG, "seq_len must be a multiple of 4");
  if (c.seq_len > attention_most_positions())
    return fail(HE_E_ARG, "seq_len is longer than the attention kernels take (" +
                              std::to_string(attention_most_positions()) + " positions)");
  if (c.arch != HE_ARCH_LLAMA && c.arch != HE_ARCH_GPT2 && c.arch != HE_ARCH_NEOX)
    return fail(HE_E_ARG, "arch is not one of llama, gpt2, neox");
  if (layer_norm(c)) {
    if (qdim != c.dim) return fail(HE_E_ARG, "a GPT-2 / GPT-NeoX form has heads of dim / n_heads");
    if (c.qk_norm) return fail(HE_E_ARG, "q/k head norms belong to the llama form (Qwen3)");
    if (c.dim > 16384) return fail(HE_E_ARG, "LayerNorm takes rows of at most 16384");
  } else if (c.parallel_residual) {
    return fail(HE_E_ARG, "a parallel residual belongs to the GPT-NeoX form");
  }
  if (c.arch == HE_ARCH_NEOX && (c.rotary < 0 || c.rotary % 2 || c.rotary > c.head_size))
    return fail(HE_E_ARG, "rotary must be even and at most head_size");
  if (c.arch == HE_ARCH_LLAMA && c.rotary && c.rotary != c.head_size)
    return fail(HE_E_ARG, "the llama form turns every value of a head (rotary 0 or head_size)");
  if (c.qk_norm && c.head_size > 256) return fail(HE_E_ARG, "q/k head norms take heads of at most 256");
  if (c.n_outliers < 0 || c.n_outliers > HE_OUTLIERS_MOST)
    return fail(HE_E_ARG, "at most 8 outlier channels (OUTLIER_CHANNELS)");
  for (int32_t i = 0; i < c.n_outliers; ++i)
    if (c.outliers[i] < 0 || c.outliers[i] >= c.dim || (i > 0 && c.outliers[i] <= c.outliers[i - 1]))
      return fail(HE_E_ARG, "outlier channels must be distinct channels below dim, in increasing order");
  return HE_OK;
}

// the checkpoint's regions: the header, every present tensor's values and scales, and whatever lies between them
int32_t plan_regions(he_engine *e) {
  const he_config &c = e->c;
  std::vector<Region> pieces;
  pieces.push_back({0, 28, 0});
  for (int id = 0; id < HE_T_COUNT; ++id) {
    if (!present(c, id)) continue;
    const Shape s = shape_of(c, id);
    if (s.k) {
      const uint64_t vb = c.six ? (uint64_t)s.count / 32 * 24 : (uint64_t)s.count;
      const uint64_t sb = (uint64_t)s.count / group_size(s.k) * 4;
      if (c.six && s.k % 32) return fail(HE_E_ARG, "int6 matrices need rows of whole groups of 32");
      pieces.push_back({(uint64_t)e->t[id].offset, vb, 0});
      pieces.push_back({(uint64_t)e->t[id].scales, sb, 0});
    } else {
      pieces.push_back({(uint64_t)e->t[id].offset, (uint64_t)s.count * 4, 0});
    }
  }
  std::sort(pieces.begin(), pieces.end(), [](const Region &a, const Region &b) { return a.file < b.file; });
  std::vector<Region> out;
  uint64_t at = 0;
  for (const Region &p : pieces) {
    if (p.file < at) return fail(HE_E_ARG, "the plan's tensors overlap");
    if (p.file > at) out.push_back({at, p.file - at, 0});
    out.push_back(p);
    at = p.file + p.bytes;
  }
  if (at > e->size) return fail(HE_E_ARG, "the plan's tensors run past the checkpoint's size");
  if (at < e->size) out.push_back({at, e->size - at, 0});
  uint64_t dev = 0;
  for (Region &r : out) {
    r.dev = dev;
    dev += (r.bytes + 255) / 256 * 256;
  }
  e->regions = out;
  e->blob_bytes = dev;
  return HE_OK;
}

const uint8_t *device_at(const he_engine *e, uint64_t file) {
  for (const Region &r : e->regions)
    if (file >= r.file && file < r.file + r.bytes) return e->blob + r.dev + (file - r.file);
  return nullptr;
}

int32_t bind_tensors(he_engine *e) {
  for (int id = 0; id < HE_T_COUNT; ++id) {
    const int src = (id == HE_T_WCLS && e->c.shared_classifier) ? HE_T_EMBEDDING : id;
    if (!present(e->c, src)) continue;
    e->values[id] = device_at(e, (uint64_t)e->t[src].offset);
    if (!e->values[id]) return fail(HE_E_ARG, "a tensor is outside the checkpoint");
    if (shape_of(e->c, src).k) {
      e->scales[id] = reinterpret_cast<const float *>(device_at(e, (uint64_t)e->t[src].scales));
      if (!e->scales[id]) return fail(HE_E_ARG, "a tensor's scales are outside the checkpoint");
    }
  }
  return HE_OK;
}

int32_t allocate_state(he_engine *e, const float *rope_cos, const float *rope_sin) {
  const he_config &c = e->c;
  e->qdim = c.n_heads * c.head_size;
  e->kvdim = c.n_kv_heads * c.head_size;
  e->bias = c.relaxed ? 64 : 0;
  e->xw = std::max(c.dim, e->qdim);
  e->widest = std::max(e->xw, c.hidden_dim);
  const int32_t T = e->chunk;
  const size_t table = (size_t)c.seq_len * (c.head_size / 2) * sizeof(float);
  int32_t rc;
#define ALLOC(p, bytes)                                  \
  do {                                                   \
    if ((rc = dev_alloc(&(p), (bytes))) != HE_OK) return rc; \
    e->device_bytes += (bytes);                          \
  } while (0)
  ALLOC(e->cos_t, table);
  ALLOC(e->sin_t, table);
  HIP_TRY(hipMemcpy(e->cos_t, rope_cos, table, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(e->sin_t, rope_sin, table, hipMemcpyHostToDevice));
  const size_t kv = (size_t)c.n_layers * c.seq_len * e->kvdim * (c.half_kv ? 2 : 4);
  const size_t kv_values = (size_t)c.n_layers * value_stride(c.seq_len) * e->kvdim * (c.half_kv ? 2 : 4);
  ALLOC(e->keys, kv);
  ALLOC(e->vals, kv_values);
  HIP_TRY(hipMemset(e->keys, 0, kv));
  HIP_TRY(hipMemset(e->vals, 0, kv_values));
  ALLOC(e->x, sizeof(float) * T * c.dim);
  ALLOC(e->xb, sizeof(float) * T * e->xw);
  ALLOC(e->q, sizeof(float) * T * e->qdim);
  ALLOC(e->k, sizeof(float) * T * e->kvdim);
  ALLOC(e->v, sizeof(float) * T * e->kvdim);
  ALLOC(e->hb, sizeof(float) * T * c.hidden_dim);
  ALLOC(e->hb2, sizeof(float) * T * c.hidden_dim);
  ALLOC(e->xq, (size_t)T * e->widest);
  ALLOC(e->xs, sizeof(float) * T * (e->widest / 32));
  const size_t rows = std::min(T, ATTN_ROWS);  // launch_attention's pieces reuse these rows
  ALLOC(e->scores, sizeof(float) * rows * c.n_heads * (size_t)c.seq_len);
  ALLOC(e->tilemax, sizeof(float) * rows * c.n_heads * (size_t)(c.seq_len / 64 + 1));
  ALLOC(e->logits, sizeof(float) * c.vocab_size);
  ALLOC(e->tokens, sizeof(int32_t) * T);
  ALLOC(e->amax_v, sizeof(float) * 256);
  ALLOC(e->amax_i, sizeof(int32_t) * 256);
  ALLOC(e->best_v, sizeof(float) * 4);
  ALLOC(e->best_i, sizeof(int32_t) * 4);
  ALLOC(e->state, sizeof(int32_t) * STATE_WORDS);
  ALLOC(e->step_ids, sizeof(int32_t) * STEPS_A_ROUND);
  ALLOC(e->step_values, sizeof(float) * STEPS_A_ROUND);
  ALLOC(e->sample_probs, sizeof(float) * sample_probs_floats(c.vocab_size));
  ALLOC(e->sample_index, sizeof(int32_t) * c.vocab_size);
  ALLOC(e->window, sizeof(int32_t) * REPETITION_WINDOW);
  ALLOC(e->sample_token, sizeof(int32_t) * 4);
  ALLOC(e->sample_best, sizeof(float) * 4);
  ALLOC(e->sample_parts, sizeof(DrawParts));
  ALLOC(e->sink, sizeof(uint32_t) * 64);
  ALLOC(e->run_params, sizeof(RunParams));
  ALLOC(e->kept_logits, sizeof(float) * c.vocab_size);
  {
    // the fills pay where a token's weights come from HBM; a checkpoint that the 256 MB MALL holds whole (with room for
    // the cache and activations) finds them there, and the fill blocks would only add latency
    if (e->size < (192ull << 20)) e->fetch_xcd_bytes = 0;
    // PYODIDE_LLM_HIP_L2FETCH: KiB an XCD of the L2 fills ahead of the one-token GEMVs (0: none)
    const char *env = std::getenv("PYODIDE_LLM_HIP_L2FETCH");
    if (env && *env) e->fetch_xcd_bytes = std::max(0L, std::atol(env)) << 10;
    const char *attend = std::getenv("PYODIDE_LLM_HIP_ATTEND");
    e->attend_split = attend && std::strcmp(attend, "split") == 0;
  }
  if (c.parallel_residual) ALLOC(e->before, sizeof(float) * T * c.dim);
  e->outliers.n = c.n_outliers;
  for (int32_t i = 0; i < c.n_outliers; ++i) e->outliers.c[i] = c.outliers[i];
  if (c.n_outliers) {
    ALLOC(e->columns, sizeof(float) * c.n_outliers * (size_t)c.vocab_size);
    ALLOC(e->picked, sizeof(float) * HE_OUTLIERS_MOST);
  }
#undef ALLOC
  HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&e->host_ids), sizeof(int32_t) * STEPS_A_ROUND));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&e->host_values), sizeof(float) * STEPS_A_ROUND));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&e->host_state), sizeof(int32_t) * (STATE_WORDS + 2)));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&e->host_params), sizeof(RunParams)));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&e->host_window), sizeof(int32_t) * REPETITION_WINDOW));
  return HE_OK;
}

// the outlier channels' columns of the classifier (public/forward.js:801-812), once its bytes are on the device
int32_t prepare_outliers(he_engine *e) {
  const he_config &c = e->c;
  if (!c.n_outliers) return HE_OK;
  HIP_TRY(launch_outlier_columns(e->columns, e->values[HE_T_WCLS], e->scales[HE_T_WCLS], c.vocab_size, c.dim,
                                 c.six ? 32 : group_size(c.dim), c.six, e->outliers, e->stream));
  HIP_TRY(hipStreamSynchronize(e->stream));
  return HE_OK;
}

int32_t open_common(const he_config *cfg, const he_tensor *tensors, uint64_t size, const float *rope_cos,
                    const float *rope_sin, int32_t max_block, he_engine **out, he_engine **made) {
  if (!cfg || !tensors || !rope_cos || !rope_sin || !out) return fail(HE_E_ARG, "a required pointer is null");
  if (max_block < 1) return fail(HE_E_ARG, "max_block must be at least 1");
  int32_t rc = check_config(*cfg);
  if (rc) return rc;
  he_engine *e = new he_engine();
  *made = e;
  e->c = *cfg;
  std::memcpy(e->t, tensors, sizeof(e->t));
  e->size = size;
  e->max_block = max_block;
  // the tokens of one pass through the layers: a prompt block up to 1024 (the attention runs them in pieces of
  // ATTN_ROWS; measured at the 8B shape: 512 a pass 19.5k prompt tok/s, 1024 19.6k, 2048 18.5k; with the two-tile
  // GEMM 1024 20.5k, 2048 0.3% more for twice the activations)
  e->chunk = std::min(max_block, e->c.relaxed ? 1024 : 16);
  HIP_TRY(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
  if ((rc = plan_regions(e))) return rc;
  if ((rc = dev_alloc(&e->blob, e->blob_bytes))) return rc;
  e->device_bytes += e->blob_bytes;
  if ((rc = bind_tensors(e))) return rc;
  if ((rc = allocate_state(e, rope_cos, rope_sin))) return rc;
  return HE_OK;
}

// ---- the forward pass of one chunk of tokens (public/forward.js:1011-1090) ----

// a launch (or a few) of one kind, bracketed by events while profiling
template <class F>
hipError_t timed(he_engine *e, int kind, double bytes, F &&launch) {
  if (!e->profiling) return launch();
  he_engine::Mark mk{kind, bytes, nullptr, nullptr};
  hipError_t err = hipEventCreate(&mk.a);
  if (err == hipSuccess) err = hipEventCreate(&mk.b);
  if (err == hipSuccess) err = hipEventRecord(mk.a, e->stream);
  if (err == hipSuccess) err = launch();
  if (err == hipSuccess) err = hipEventRecord(mk.b, e->stream);
  e->marks.push_back(mk);
  return err;
}

// the algorithmic bytes of a matmul of m tokens: every row's values and scales once, the activations and their
// scales, the outputs (read as well where they accumulate)
double matmul_bytes(const he_engine *e, const MatSeg *segs, int nseg, int32_t k, int32_t m) {
  double b = (double)m * k + (double)m * (k / 32) * 4;
  for (int i = 0; i < nseg; ++i) {
    const double row = (e->c.six ? (double)k / 32 * 24 : (double)k) + (double)k / 32 * 4;
    b += segs[i].rows * row + (double)m * segs[i].rows * 4 * (segs[i].accumulate ? 2 : 1);
  }
  return b;
}

// the float32 source of a one-token matmul's activations, quantized in the launch (after rmsnorm with weights norm
// where norm is not null): MatArgs.xf
struct F32Source {
  const float *x;
  const float *norm;
};

hipError_t matmul_launch(he_engine *e, const MatSeg *segs, int nseg, int32_t k, int32_t m, const int8_t *xq,
                         const float *xs, const F32Source *f32 = nullptr, const QkvFuse *qkv = nullptr,
                         bool persistent = false) {
  const int32_t xq_stride = e->widest, xs_stride = e->widest / 32;
  const int32_t step = gemv_tokens(k, e->c.relaxed);
  if (step < 1) return hipErrorInvalidValue;
  for (int32_t t0 = 0; t0 < m; t0 += step) {
    MatArgs a{};
    a.nseg = nseg;
    a.total_rows = 0;
    for (int i = 0; i < nseg; ++i) {
      a.seg[i] = segs[i];
      a.seg[i].y = segs[i].y + (int64_t)t0 * segs[i].y_stride;
      a.total_rows += segs[i].rows;
    }
    a.xq = xq + (int64_t)t0 * xq_stride;
    a.xs = xs + (int64_t)t0 * xs_stride;
    a.xq_stride = xq_stride;
    a.xs_stride = xs_stride;
    a.k = k;
    a.m = std::min(step, m - t0);
    a.sums = nullptr;
    if (f32) {
      a.xf = f32->x;
      a.xnorm = f32->norm;
      a.eps = e->c.rms_norm_eps;
    }
    if (qkv) a.qkv = *qkv;
    a.persistent = persistent && a.m == 1 && decode_persistent(k, e->c.six != 0, e->c.relaxed != 0);
    hipError_t err = launch_gemv(a, e->c.six, e->c.relaxed, e->stream);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

// more tokens than one GEMV launch takes go to the MFMA GEMM (the same bits per token and row)
bool use_gemm(const he_engine *e, int32_t k, int32_t m) {
  return m > GEMV_MOST && gemm_supported(k, e->c.relaxed != 0);
}

hipError_t gemm_launch(he_engine *e, const MatSeg *segs, int nseg, int32_t k, int32_t m, const int8_t *xq,
                       const float *xs) {
  MatArgs a{};
  a.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    a.seg[i] = segs[i];
    a.total_rows += segs[i].rows;
  }
  a.xq = xq;
  a.xs = xs;
  a.xq_stride = e->widest;
  a.xs_stride = e->widest / 32;
  a.k = k;
  a.m = m;
  return launch_gemm(a, e->c.six, e->c.relaxed, e->stream);
}

// the prompt's w1 / w3 GEMM with the SwiGLU in its epilogue, writing quantize_x of its output to gq / gs
// ([m][widest] bytes, [m][widest / 32] scales)
hipError_t gemm_glu_launch(he_engine *e, const MatSeg *w13, int32_t k, int32_t m, const int8_t *xq, const float *xs,
                           int8_t *gq, float *gs) {
  MatArgs a{};
  a.nseg = 2;
  a.seg[0] = w13[0];
  a.seg[1] = w13[1];
  a.total_rows = w13[0].rows + w13[1].rows;
  a.xq = xq;
  a.xs = xs;
  a.xq_stride = e->widest;
  a.xs_stride = e->widest / 32;
  a.k = k;
  a.m = m;
  a.glu = GluOut{gq, gs, e->widest, e->widest / 32, e->bias};
  return launch_gemm_glu(a, e->c.six, e->stream);
}

// whether a chunk of m tokens takes the GEMM's SwiGLU epilogue: the w1 / w3 matmul on the GEMM, hidden units in whole
// groups, and the float32 buffers of h1 / h3 large enough for the quantized output ([chunk][widest] bytes in hb,
// [chunk][widest / 32] floats in hb2)
bool glu_in_gemm(const he_engine *e, int32_t m) {
  const int32_t hidden = e->c.hidden_dim;
  return use_gemm(e, e->c.dim, m) && hidden % 32 == 0 && e->widest % 4 == 0 && e->widest <= 4 * (int64_t)hidden;
}

hipError_t matmul(he_engine *e, const MatSeg *segs, int nseg, int32_t k, int32_t m, const int8_t *xq, const float *xs,
                  const F32Source *f32 = nullptr, const QkvFuse *qkv = nullptr, bool persistent = false) {
  if (use_gemm(e, k, m))
    return timed(e, HE_K_GEMM, matmul_bytes(e, segs, nseg, k, m),
                 [&] { return gemm_launch(e, segs, nseg, k, m, xq, xs); });
  return timed(e, HE_K_GEMV, matmul_bytes(e, segs, nseg, k, m),
               [&] { return matmul_launch(e, segs, nseg, k, m, xq, xs, f32, qkv, persistent); });
}

// one token whose rows of k the decode GEMV quantizes itself: it saves a launch where the GEMV is about one block a
// CU (wo), and would cost more than it saves on the larger ones (each block repeats it). (Measured: rmsnorm in the
// q/k/v GEMV's blocks costs as much as its own launch, which is latency inside the norm, not the launch.)
bool quantizes_itself(const he_engine *e, int32_t k, int32_t m, int32_t rows) {
  return m == 1 && rows <= 8192 && decode_takes_f32(k, e->c.six != 0, e->c.relaxed != 0);
}

// The L2Fetch of a one-token GEMV over segs (rows of k): the rows of its first blocks, at most fetch_xcd_bytes an XCD
// (of its 4 MiB L2), fetched by `blocks` extra blocks of the launch before it. None (blocks = 0) for more tokens, where
// the GEMV is not the one-token path, or where a segment's rows are not whole GEMV blocks.
L2Fetch fetch_for(const he_engine *e, const MatSeg *segs, int nseg, int32_t k, int32_t m, int32_t blocks,
                  bool qkv_on = false) {
  L2Fetch f{};
  if (e->fetch_xcd_bytes <= 0 || m != 1 || blocks < 8 || blocks % 8) return f;
  int32_t total = 0;
  for (int i = 0; i < nseg; ++i) total += segs[i].rows;
  const int32_t br = decode_block_rows(k, total, e->c.six != 0, e->c.relaxed != 0, false, qkv_on);
  if (br <= 0) return f;
  const int32_t row_bytes = e->c.six ? k / 32 * 24 : k, scale_bytes = k / 32 * 4;
  for (int i = 0; i < nseg; ++i) {
    // whole GEMV blocks a segment, and every block's values and scales on 16-byte boundaries
    if (segs[i].rows % br || (br * row_bytes) % 16 || (br * scale_bytes) % 16 ||
        reinterpret_cast<uintptr_t>(segs[i].w) % 16 || reinterpret_cast<uintptr_t>(segs[i].ws) % 16)
      return L2Fetch{};
    f.w[i] = segs[i].w;
    f.ws[i] = reinterpret_cast<const uint8_t *>(segs[i].ws);
    f.rows[i] = segs[i].rows;
  }
  f.nseg = nseg;
  f.row_bytes = row_bytes;
  f.scale_bytes = scale_bytes;
  f.block_rows = br;
  const int64_t per_block = (int64_t)br * (f.row_bytes + f.scale_bytes);
  f.gemv_blocks = (int32_t)std::min<int64_t>(total / br, 8 * (e->fetch_xcd_bytes / per_block));
  if (f.gemv_blocks < 1) return L2Fetch{};
  f.blocks = blocks;
  f.sink = e->sink;
  return f;
}

int32_t run_chunk(he_engine *e, const int32_t *tokens, int32_t m, int32_t pos0, bool need_logits) {
  const he_config &c = e->c;
  hipStream_t s = e->stream;
  const int32_t dim = c.dim, hidden = c.hidden_dim, qdim = e->qdim, kvdim = e->kvdim, hs = c.head_size;
  const int32_t W = e->widest;
  const size_t esz = c.half_kv ? 2 : 4;
  const int32_t *dpos = e->replayable ? e->state : nullptr;  // a replayed step: the position in device memory
  if (!e->replayable) HIP_TRY(hipMemcpyAsync(e->tokens, tokens, sizeof(int32_t) * m, hipMemcpyHostToDevice, s));
  const bool ln = layer_norm(c);  // GPT-2 / GPT-NeoX: LayerNorm, GELU, biases after every matrix
  Positions positions{};
  if (c.arch == HE_ARCH_GPT2)
    positions = {e->values[HE_T_POSITIONS], e->scales[HE_T_POSITIONS], c.six ? 32 : group_size(dim), pos0, dpos};
  HIP_TRY(timed(e, HE_K_ELEMENTWISE, (double)m * dim * (c.six ? 0.75 + 0.125 + 4 : 1 + 0.125 + 4), [&] {
    return launch_embed(e->x, e->tokens, e->values[HE_T_EMBEDDING], e->scales[HE_T_EMBEDDING], m, dim, dim,
                        c.six ? 32 : group_size(dim), c.six, positions, s);
  }));
  for (int32_t l = 0; l < c.n_layers; ++l) {
    const MatSeg qkv[3] = {
        {e->mat(HE_T_WQ, l), e->mat_scales(HE_T_WQ, l), e->q, qdim, qdim, 0},
        {e->mat(HE_T_WK, l), e->mat_scales(HE_T_WK, l), e->k, kvdim, kvdim, 0},
        {e->mat(HE_T_WV, l), e->mat_scales(HE_T_WV, l), e->v, kvdim, kvdim, 0}};
    QkvPost qp{};
    qp.q = e->q;
    qp.k = e->k;
    qp.v = e->v;
    qp.q_stride = qdim;
    qp.kv_stride = kvdim;
    const bool biases = c.qkv_bias || ln;
    qp.bq = biases ? e->vec(HE_T_BQ, (int64_t)l * qdim) : nullptr;
    qp.bk = biases ? e->vec(HE_T_BK, (int64_t)l * kvdim) : nullptr;
    qp.bv = biases ? e->vec(HE_T_BV, (int64_t)l * kvdim) : nullptr;
    qp.cos_t = e->cos_t;
    qp.sin_t = e->sin_t;
    qp.kcache = reinterpret_cast<uint8_t *>(e->keys) + (size_t)l * c.seq_len * kvdim * esz;
    qp.vcache = reinterpret_cast<uint8_t *>(e->vals) + (size_t)l * value_stride(c.seq_len) * kvdim * esz;
    qp.nh = c.n_heads;
    qp.nkv = c.n_kv_heads;
    qp.hs = hs;
    qp.pos0 = pos0;
    qp.m = m;
    qp.half = c.half_kv;
    qp.vstride = value_stride(c.seq_len);
    qp.dpos = dpos;
    qp.rot = c.arch == HE_ARCH_GPT2 ? 0 : (c.rotary > 0 && c.rotary < hs ? c.rotary : hs);
    if (ln) {
      HIP_TRY(timed(e, HE_K_NORM, (double)m * dim * (8 + 1 + 0.125) + dim * 8.0, [&] {
        return launch_layernorm_quant(e->xq, e->xs, nullptr, c.parallel_residual ? e->before : nullptr, e->x,
                                      e->vec(HE_T_RMS_ATT, (int64_t)l * dim), e->vec(HE_T_LN_ATT_BIAS, (int64_t)l * dim),
                                      m, dim, dim, W, W / 32, 0, e->bias, s);
      }));
    }
    const bool fuse_qkv = c.arch == HE_ARCH_LLAMA && !c.qk_norm && m == 1 &&
                          decode_fuses_qkv(dim, c.six != 0, c.relaxed != 0);
    // one token of a small model (dim <= 1024): the q/k/v and w1/w3 GEMVs take the float32 token and run rmsnorm and
    // quantize_x in each block (an ordered sum of 256 steps at most), two launches a layer fewer. (At dim 4096 each
    // block repeating the 1024-step sum costs more than the launch.)
    const bool norm_in_gemv = !ln && m == 1 && dim <= 1024 && decode_takes_f32(dim, c.six != 0, c.relaxed != 0);
    const F32Source att_src{e->x, e->vec(HE_T_RMS_ATT, (int64_t)l * dim)};
    if (!ln && !norm_in_gemv) {
      const L2Fetch fq = fetch_for(e, qkv, 3, dim, m, 256, fuse_qkv);
      HIP_TRY(timed(e, HE_K_NORM, (double)m * dim * (8 + 1 + 0.125) + dim * 4.0, [&] {
        return launch_rmsnorm_quant(e->xq, e->xs, nullptr, e->x, e->vec(HE_T_RMS_ATT, (int64_t)l * dim), m, dim, dim,
                                    W, W / 32, 0, c.rms_norm_eps, e->bias, s, &fq);
      }));
    }
    if (fuse_qkv) {
      // one token: the q/k/v GEMV adds the biases, rotates q and k and writes k and v into the cache itself
      const QkvFuse fuse{1, qp.bq, qp.bk, qp.bv, e->cos_t, e->sin_t, qp.kcache, qp.vcache, pos0, hs, kvdim, c.half_kv,
                         qp.vstride, dpos};
      HIP_TRY(matmul(e, qkv, 3, dim, m, e->xq, e->xs, norm_in_gemv ? &att_src : nullptr, &fuse));
    } else {
      HIP_TRY(matmul(e, qkv, 3, dim, m, e->xq, e->xs, norm_in_gemv ? &att_src : nullptr));
      if (c.qk_norm) {
        // Qwen3: the q/k biases, then every head normalized, before RoPE
        HIP_TRY(timed(e, HE_K_NORM, (double)m * (qdim + kvdim) * 8, [&] {
          return launch_head_norm(e->q, e->k, qp.bq, qp.bk, e->vec(HE_T_Q_NORM, (int64_t)l * hs),
                                  e->vec(HE_T_K_NORM, (int64_t)l * hs), m, c.n_heads, c.n_kv_heads, hs, qdim, kvdim,
                                  c.rms_norm_eps, s);
        }));
        qp.bq = qp.bk = nullptr;
      }
      HIP_TRY(timed(e, HE_K_ELEMENTWISE, (double)m * (qdim + 2 * kvdim) * 8 + (double)m * 2 * kvdim * esz,
                    [&] { return launch_qkv_post(qp, s); }));
    }
    AttnArgs at{};
    at.q = e->q;
    at.q_stride = qdim;
    at.kcache = qp.kcache;
    at.vcache = qp.vcache;
    at.out = e->xb;
    at.out_stride = e->xw;
    at.scores = e->scores;
    at.tilemax = e->tilemax;
    at.nh = c.n_heads;
    at.nkv = c.n_kv_heads;
    at.hs = hs;
    at.pos0 = pos0;
    at.m = m;
    at.seq_len = c.seq_len;
    at.half = c.half_kv;
    at.vstride = qp.vstride;
    at.dpos = dpos;
    at.xq = e->xq;
    at.xs = e->xs;
    at.xq_stride = W;
    at.xs_stride = W / 32;
    at.bias = e->bias;
    at.split = e->attend_split;
    // wo quantizes the attention's float32 output itself where its decode GEMV takes a float32 token (then the
    // attention runs blocks of 16 columns); else the attention writes quantize_x of its output too where it can
    const bool wo_quantizes = quantizes_itself(e, qdim, m, dim);
    if (wo_quantizes) at.xq = nullptr;
    const bool quantized = at.xq && attention_quantizes(at);
    if (!quantized) at.xq = nullptr;
    double kv_rows = 0;
    for (int32_t t = 0; t < m; ++t) kv_rows += pos0 + t + 1;
    const MatSeg wo[1] = {{e->mat(HE_T_WO, l), e->mat_scales(HE_T_WO, l), e->x, dim, dim, 1}};
    HIP_TRY(timed(e, HE_K_ATTENTION, kv_rows * 2 * kvdim * esz + (double)m * qdim * 8,
                  [&] { return launch_attention(at, s); }));
    if (quantized) {
      HIP_TRY(matmul(e, wo, 1, qdim, m, e->xq, e->xs));
    } else if (wo_quantizes) {
      // the wide models' output projection on the persistent GEMV (each block quantizes the token once)
      const F32Source src{e->xb, nullptr};
      HIP_TRY(matmul(e, wo, 1, qdim, m, e->xq, e->xs, &src, nullptr, true));
    } else {
      HIP_TRY(timed(e, HE_K_NORM, (double)m * qdim * (4 + 1 + 0.125),
                    [&] { return launch_quantize(e->xq, e->xs, e->xb, m, qdim, e->xw, W, W / 32, e->bias, s); }));
      HIP_TRY(matmul(e, wo, 1, qdim, m, e->xq, e->xs));
    }
    if (ln) {
      // x += bo; LayerNorm of x (or of the layer's input: parallel residual); w1; gelu(+ b1); w2; x += b2
      HIP_TRY(timed(e, HE_K_ELEMENTWISE, (double)m * dim * 12,
                    [&] { return launch_add_rows(e->x, e->vec(HE_T_BO, (int64_t)l * dim), m, dim, dim, s); }));
      HIP_TRY(timed(e, HE_K_NORM, (double)m * dim * (8 + 1 + 0.125) + dim * 8.0, [&] {
        return launch_layernorm_quant(e->xq, e->xs, nullptr, nullptr, c.parallel_residual ? e->before : e->x,
                                      e->vec(HE_T_RMS_FFN, (int64_t)l * dim), e->vec(HE_T_LN_FFN_BIAS, (int64_t)l * dim),
                                      m, dim, dim, W, W / 32, 0, e->bias, s);
      }));
      const MatSeg w1[1] = {{e->mat(HE_T_W1, l), e->mat_scales(HE_T_W1, l), e->hb, hidden, hidden, 0}};
      HIP_TRY(matmul(e, w1, 1, dim, m, e->xq, e->xs));
      HIP_TRY(timed(e, HE_K_ELEMENTWISE, (double)m * hidden * (8 + 1 + 0.125), [&] {
        return launch_gelu_quant(e->xq, e->xs, nullptr, e->hb, e->vec(HE_T_B1, (int64_t)l * hidden), m, hidden,
                                 hidden, W, W / 32, e->bias, s);
      }));
      const MatSeg w2g[1] = {{e->mat(HE_T_W2, l), e->mat_scales(HE_T_W2, l), e->x, dim, dim, 1}};
      HIP_TRY(matmul(e, w2g, 1, hidden, m, e->xq, e->xs));
      HIP_TRY(timed(e, HE_K_ELEMENTWISE, (double)m * dim * 12,
                    [&] { return launch_add_rows(e->x, e->vec(HE_T_B2, (int64_t)l * dim), m, dim, dim, s); }));
      continue;
    }
    const MatSeg w13[2] = {{e->mat(HE_T_W1, l), e->mat_scales(HE_T_W1, l), e->hb, hidden, hidden, 0},
                           {e->mat(HE_T_W3, l), e->mat_scales(HE_T_W3, l), e->hb2, hidden, hidden, 0}};
    const L2Fetch f13 = fetch_for(e, w13, 2, dim, m, 256);
    if (!norm_in_gemv) {
      HIP_TRY(timed(e, HE_K_NORM, (double)m * dim * (8 + 1 + 0.125) + dim * 4.0, [&] {
        return launch_rmsnorm_quant(e->xq, e->xs, nullptr, e->x, e->vec(HE_T_RMS_FFN, (int64_t)l * dim), m, dim, dim,
                                    W, W / 32, 0, c.rms_norm_eps, e->bias, s, &f13);
      }));
    }
    const MatSeg w2[1] = {{e->mat(HE_T_W2, l), e->mat_scales(HE_T_W2, l), e->x, dim, dim, 1}};
    if (glu_in_gemm(e, m)) {
      // the GEMM finishes the SwiGLU and its quantize_x itself; its bytes and scales go where h1 and h3 would (hb and
      // hb2 hold [chunk][W] bytes and [chunk][W / 32] floats: glu_in_gemm checks), apart from the w1 / w3 GEMM's
      // input in xq / xs
      int8_t *gq = reinterpret_cast<int8_t *>(e->hb);
      HIP_TRY(timed(e, HE_K_GEMM, matmul_bytes(e, w13, 2, dim, m),
                    [&] { return gemm_glu_launch(e, w13, dim, m, e->xq, e->xs, gq, e->hb2); }));
      HIP_TRY(matmul(e, w2, 1, hidden, m, gq, e->hb2));
      continue;
    }
    const F32Source ffn_src{e->x, e->vec(HE_T_RMS_FFN, (int64_t)l * dim)};
    HIP_TRY(matmul(e, w13, 2, dim, m, e->xq, e->xs, norm_in_gemv ? &ffn_src : nullptr));
    HIP_TRY(timed(e, HE_K_ELEMENTWISE, (double)m * hidden * (8 + 1 + 0.125), [&] {
      return launch_swiglu_quant(e->xq, e->xs, nullptr, e->hb, e->hb2, m, hidden, hidden, W, W / 32, e->bias, s);
    }));
    HIP_TRY(matmul(e, w2, 1, hidden, m, e->xq, e->xs));
  }
  if (need_logits) {
    // the final norm; with outlier channels its float32 output too, whose channels are taken out and the rest
    // quantized again (public/forward.js:1082-1089)
    const bool apart = c.n_outliers > 0;
    const float *last = e->x + (int64_t)(m - 1) * dim;
    const MatSeg cls[1] = {{e->mat(HE_T_WCLS, 0), e->mat_scales(HE_T_WCLS, 0), e->logits, c.vocab_size, 0, 0}};
    const L2Fetch fc = fetch_for(e, cls, 1, dim, 1, apart ? 0 : 256);
    HIP_TRY(timed(e, HE_K_NORM, (double)dim * (8 + 1 + 0.125), [&] {
      return ln ? launch_layernorm_quant(e->xq, e->xs, apart ? e->xb : nullptr, nullptr, last,
                                         e->vec(HE_T_RMS_FINAL, 0), e->vec(HE_T_LN_FINAL_BIAS, 0), 1, dim, dim, W,
                                         W / 32, e->xw, e->bias, s)
                : launch_rmsnorm_quant(e->xq, e->xs, apart ? e->xb : nullptr, last, e->vec(HE_T_RMS_FINAL, 0), 1,
                                       dim, dim, W, W / 32, e->xw, c.rms_norm_eps, e->bias, s, &fc);
    }));
    if (apart) {
      HIP_TRY(timed(e, HE_K_ELEMENTWISE, 64.0, [&] { return launch_pick(e->xb, e->picked, e->outliers, s); }));
      HIP_TRY(timed(e, HE_K_NORM, (double)dim * (4 + 1 + 0.125), [&] {
        return launch_quantize(e->xq, e->xs, e->xb, 1, dim, e->xw, W, W / 32, e->bias, s);
      }));
    }
    HIP_TRY(matmul(e, cls, 1, dim, 1, e->xq, e->xs));
    if (apart)
      HIP_TRY(timed(e, HE_K_ELEMENTWISE, (double)c.vocab_size * (8 + 4 * c.n_outliers), [&] {
        return launch_add_columns(e->logits, e->columns, e->picked, c.n_outliers, c.vocab_size, s);
      }));
    e->have_logits = true;
    e->logits_kept = false;
  }
  return HE_OK;
}

int32_t run_tokens(he_engine *e, const int32_t *tokens, int32_t count, int32_t pos0, bool need_logits) {
  if (count < 1) return fail(HE_E_ARG, "no tokens");
  if (pos0 < 0 || (int64_t)pos0 + count > e->c.seq_len)
    return fail(HE_E_STATE, "the positions run past the context (seq_len)");
  for (int32_t i = 0; i < count; ++i)
    if (tokens[i] < 0 || tokens[i] >= e->c.vocab_size) return fail(HE_E_ARG, "a token is outside the vocabulary");
  for (int32_t at = 0; at < count; at += e->chunk) {
    const int32_t m = std::min(e->chunk, count - at);
    const int32_t rc = run_chunk(e, tokens + at, m, pos0 + at, need_logits && at + m == count);
    if (rc) return rc;
  }
  return HE_OK;
}

}  // namespace

extern "C" {

const char *he_last_error(void) { return g_error.c_str(); }

int32_t he_open(const he_config *cfg, const he_tensor *tensors, const void *checkpoint, uint64_t size,
                const float *rope_cos, const float *rope_sin, int32_t max_block, he_engine **out) {
  if (!checkpoint) return fail(HE_E_ARG, "checkpoint is null");
  he_engine *e = nullptr;
  int32_t rc = open_common(cfg, tensors, size, rope_cos, rope_sin, max_block, out, &e);
  if (rc == HE_OK) {
    const uint8_t *src = reinterpret_cast<const uint8_t *>(checkpoint);
    for (const Region &r : e->regions) {
      hipError_t err = hipMemcpy(e->blob + r.dev, src + r.file, r.bytes, hipMemcpyHostToDevice);
      if (err != hipSuccess) {
        rc = fail(HE_E_HIP, std::string("uploading the checkpoint: ") + hipGetErrorString(err));
        break;
      }
    }
  }
  if (rc == HE_OK) rc = prepare_outliers(e);
  if (rc != HE_OK) {
    destroy(e);
    return rc;
  }
  *out = e;
  return HE_OK;
}

int32_t he_open_synthetic(const he_config *cfg, const he_tensor *tensors, uint64_t size, uint64_t seed,
                          const float *rope_cos, const float *rope_sin, int32_t max_block, he_engine **out) {
  he_engine *e = nullptr;
  int32_t rc = open_common(cfg, tensors, size, rope_cos, rope_sin, max_block, out, &e);
  const float factor = (float)(0.02 / std::sqrt(4.0 * (65536.0 * 65536.0 - 1.0) / 12.0));
  if (rc == HE_OK) {
    const he_config &c = e->c;
    const int32_t header[7] = {c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads,
                               c.shared_classifier ? c.vocab_size : -c.vocab_size, c.seq_len};
    hipError_t err = hipMemcpy(e->blob, header, 28, hipMemcpyHostToDevice);
    for (int id = 0; id < HE_T_COUNT && err == hipSuccess; ++id) {
      if (!present(c, id)) continue;
      const Shape s = shape_of(c, id);
      uint8_t *vals = const_cast<uint8_t *>(e->values[id]);
      if (s.k) {
        if (s.k % 32) {
          rc = fail(HE_E_ARG, "synthetic checkpoints take rows of whole groups of 32");
          break;
        }
        err = launch_synth_matrix(vals, const_cast<float *>(e->scales[id]), s.count / s.k, s.k, seed, id, factor,
                                  c.six, e->stream);
      } else {
        err = launch_synth_vector(reinterpret_cast<float *>(vals), s.count, seed, id, factor, norm_weight(id),
                                e->stream);
      }
    }
    if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
    if (err != hipSuccess && rc == HE_OK) rc = fail(HE_E_HIP, std::string("synthesis: ") + hipGetErrorString(err));
    if (rc == HE_OK) rc = prepare_outliers(e);
  }
  if (rc != HE_OK) {
    destroy(e);
    return rc;
  }
  *out = e;
  return HE_OK;
}

int32_t he_forward(he_engine *e, int32_t token, int32_t pos, int32_t need_logits, float *logits) {
  if (!e) return fail(HE_E_ARG, "engine is null");
  int32_t rc = run_tokens(e, &token, 1, pos, need_logits != 0);
  if (rc) return rc;
  if (need_logits && logits)
    HIP_TRY(hipMemcpyAsync(logits, e->logits, sizeof(float) * e->c.vocab_size, hipMemcpyDeviceToHost, e->stream));
  HIP_TRY(hipStreamSynchronize(e->stream));
  return HE_OK;
}

int32_t he_forward_many(he_engine *e, const int32_t *tokens, int32_t count, int32_t pos) {
  if (!e || !tokens) return fail(HE_E_ARG, "engine or tokens is null");
  if (count > e->max_block) return fail(HE_E_ARG, "more tokens than the prompt block");
  int32_t rc = run_tokens(e, tokens, count, pos, false);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(e->stream));
  return HE_OK;
}

namespace {
// the graph of one decode step of a kind (the caller has run at least one step eagerly, so that every launch's one-time
// set-up is done): captured with positions bounded by seq_len - 1 and read from state[STATE_POS]: the forward pass with
// logits, the penalty over the window in device memory (STEP_PENALIZED), the greedy choice or the draw with the call's
// settings and the round's random number (STEP_SAMPLED), then the step's end (launch_step_end)
void build_graph(he_engine *e, int kind) {
  e->graph_tried[kind] = true;
  // PYODIDE_LLM_HIP_GRAPH=0 keeps every step eager (a kernel-trace profiler that does not follow graph launches)
  const char *env = std::getenv("PYODIDE_LLM_HIP_GRAPH");
  if (env && env[0] == '0') return;
  hipGraph_t g = nullptr;
  e->replayable = true;
  hipError_t err = hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal);
  int32_t rc = HE_OK;
  if (err == hipSuccess) {
    rc = run_chunk(e, nullptr, 1, e->c.seq_len - 1, true);
    if (rc == HE_OK) {
      const int32_t n = e->c.vocab_size;
      hipError_t le = hipSuccess;
      const bool drawn = (kind & STEP_SAMPLED) != 0, penalized = (kind & STEP_PENALIZED) != 0;
      // (a drawn step takes the penalty in the draw's first launch)
      if (penalized && !drawn) le = launch_penalize_steps(e->logits, e->window, e->state, e->run_params, e->stream);
      if (le == hipSuccess)
        le = drawn ? launch_sample_steps(e->logits, n, e->run_params, e->state, penalized ? e->window : nullptr,
                                         (kind & STEP_WHOLE) != 0, e->sample_probs, e->sample_index,
                                         e->sample_parts, e->sample_token, e->sample_best, e->stream)
                   : launch_argmax(e->best_i, e->best_v, e->logits, n, e->amax_v, e->amax_i, e->stream);
      if (le == hipSuccess)
        le = launch_step_end(e->logits, n, e->kept_logits, e->tokens, e->state, drawn ? e->sample_token : e->best_i,
                             drawn ? e->sample_best : e->best_v, e->step_ids, e->step_values, e->window,
                             e->run_params, e->stream);
      if (le != hipSuccess) rc = HE_E_HIP;
    }
    const hipError_t end = hipStreamEndCapture(e->stream, &g);
    if (err == hipSuccess) err = end;
  }
  e->replayable = false;
  if (err == hipSuccess && rc == HE_OK && g) err = hipGraphInstantiate(&e->graph[kind], g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (err != hipSuccess || rc != HE_OK) {
    e->graph[kind] = nullptr;  // the steps stay eager
    (void)hipGetLastError();
  }
}

// one eager greedy step: its token into *best and the largest logit into *value
int32_t eager_step(he_engine *e, int32_t token, int32_t pos, int32_t *best, float *value) {
  int32_t rc = run_tokens(e, &token, 1, pos, true);
  if (rc) return rc;
  HIP_TRY(launch_argmax(e->best_i, e->best_v, e->logits, e->c.vocab_size, e->amax_v, e->amax_i, e->stream));
  HIP_TRY(hipMemcpyAsync(best, e->best_i, sizeof(int32_t), hipMemcpyDeviceToHost, e->stream));
  HIP_TRY(hipMemcpyAsync(value, e->best_v, sizeof(float), hipMemcpyDeviceToHost, e->stream));
  HIP_TRY(hipStreamSynchronize(e->stream));
  return HE_OK;
}
}  // namespace

namespace {
// sampled (or penalized greedy) steps, one at a time: forward, penalty, the draw, the token read back
int32_t sampled_steps(he_engine *e, int32_t token, int32_t pos, const int32_t *history, int32_t n_history,
                      int32_t count, float temperature, float topp, float penalty, const double *randoms,
                      const std::function<bool(int32_t)> &is_stop, int32_t *ids, int32_t *n_ids) {
  std::vector<int32_t> window(history + std::max(0, n_history - REPETITION_WINDOW), history + n_history);
  for (int32_t i = 0; i < count; ++i) {
    int32_t rc = run_tokens(e, &token, 1, pos + i, true);
    if (rc) return rc;
    if (penalty != 1.0f && !window.empty()) {
      const int32_t w = (int32_t)window.size();
      std::memcpy(e->host_window, window.data(), sizeof(int32_t) * w);
      HIP_TRY(hipMemcpyAsync(e->window, e->host_window, sizeof(int32_t) * w, hipMemcpyHostToDevice, e->stream));
      HIP_TRY(launch_penalize(e->logits, e->window, w, penalty, e->stream));
    }
    if (temperature == 0.0f) {
      HIP_TRY(launch_argmax(e->best_i, e->best_v, e->logits, e->c.vocab_size, e->amax_v, e->amax_i, e->stream));
      HIP_TRY(hipMemcpyAsync(e->host_ids, e->best_i, sizeof(int32_t), hipMemcpyDeviceToHost, e->stream));
      HIP_TRY(hipMemcpyAsync(e->host_values, e->best_v, sizeof(float), hipMemcpyDeviceToHost, e->stream));
    } else {
      HIP_TRY(launch_sample(e->logits, e->c.vocab_size, temperature, topp, randoms[i], e->sample_probs,
                            e->sample_index, e->sample_parts, e->sample_token, e->sample_best, e->stream));
      HIP_TRY(hipMemcpyAsync(e->host_ids, e->sample_token, sizeof(int32_t), hipMemcpyDeviceToHost, e->stream));
      HIP_TRY(hipMemcpyAsync(e->host_values, e->sample_best, sizeof(float), hipMemcpyDeviceToHost, e->stream));
    }
    HIP_TRY(hipStreamSynchronize(e->stream));
    const int32_t chosen = e->host_ids[0];
    if (!std::isfinite(e->host_values[0]) || chosen == SAMPLE_NOT_FINITE)
      return fail(HE_E_NOTFINITE, "the largest logit is not finite");
    if (chosen == SAMPLE_DECLINED) return HE_OK;  // the caller takes this step (nothing of it in ids)
    ids[(*n_ids)++] = chosen;
    token = chosen;
    window.push_back(chosen);
    if ((int32_t)window.size() > REPETITION_WINDOW) window.erase(window.begin());
    if (is_stop(chosen)) return HE_OK;
  }
  return HE_OK;
}
}  // namespace

int32_t he_generate_many(he_engine *e, int32_t token, int32_t pos, const int32_t *history, int32_t n_history,
                         int32_t length, int32_t count, float temperature, float topp, float penalty,
                         const double *randoms, int32_t n_randoms, const int32_t *stops, int32_t n_stops, int32_t *ids,
                         int32_t *n_ids) {
  (void)length;
  if (!e || !ids || !n_ids) return fail(HE_E_ARG, "a required pointer is null");
  if (count < 1) return fail(HE_E_ARG, "count must be at least 1");
  if ((int64_t)pos + count > e->c.seq_len) return fail(HE_E_STATE, "the steps run past the context (seq_len)");
  if (token < 0 || token >= e->c.vocab_size) return fail(HE_E_ARG, "a token is outside the vocabulary");
  if (n_history < 0 || (n_history > 0 && !history)) return fail(HE_E_ARG, "history is null");
  for (int32_t i = std::max(0, n_history - REPETITION_WINDOW); i < n_history; ++i)
    if (history[i] < 0 || history[i] >= e->c.vocab_size) return fail(HE_E_ARG, "a history token is outside the vocabulary");
  if (!(temperature >= 0.0f) || !std::isfinite(temperature)) return fail(HE_E_ARG, "temperature must be finite, >= 0");
  if (!(penalty > 0.0f) || !std::isfinite(penalty)) return fail(HE_E_ARG, "penalty must be finite, > 0");
  if (temperature > 0.0f && (!randoms || n_randoms < count)) return fail(HE_E_ARG, "a random number for every step");
  if (n_stops > 0 && !stops) return fail(HE_E_ARG, "stops is null");
  *n_ids = 0;
  auto is_stop = [&](int32_t id) {
    for (int32_t j = 0; j < n_stops; ++j)
      if (stops[j] == id) return true;
    return false;
  };
  // more stop tokens than a replayed call takes (public/forward.js STOPS_MOST): every step eager
  if (n_stops > RUN_STOPS_MOST)
    return sampled_steps(e, token, pos, history, n_history, count, temperature, topp, penalty, randoms, is_stop, ids,
                         n_ids);
  const bool nucleus = topp > 0.0f && topp < 1.0f;  // (as the draw decides it on the device)
  const int kind = (temperature > 0.0f ? (nucleus ? STEP_SAMPLED : STEP_SAMPLED | STEP_WHOLE) : STEP_GREEDY) |
                   (penalty != 1.0f ? STEP_PENALIZED : 0);
  // the penalty's window: the latest of history, then the tokens this call chooses
  std::vector<int32_t> window(history + std::max(0, n_history - REPETITION_WINDOW), history + n_history);
  int32_t done = 0;
  // eager steps until the kind's graph exists (the first step of an engine's first call of a kind builds it)
  while (done < count && !e->graph[kind]) {
    const int32_t before = *n_ids;
    const int32_t rc = sampled_steps(e, token, pos + done, window.data(), (int32_t)window.size(), 1, temperature,
                                     topp, penalty, randoms ? randoms + done : nullptr, is_stop, ids, n_ids);
    if (rc) return rc;
    if (*n_ids == before) return HE_OK;  // declined: the caller takes the step
    token = ids[*n_ids - 1];
    window.push_back(token);
    if ((int32_t)window.size() > REPETITION_WINDOW) window.erase(window.begin());
    ++done;
    if (is_stop(token)) return HE_OK;
    if (!e->graph_tried[kind]) build_graph(e, kind);
  }
  if (done == count) return HE_OK;
  // replayed steps, a round at a time, with the call's settings, stop tokens and window in device memory: the round's
  // tokens are read once at its end, and the first step that ends the call (a stop token, a declined draw, a largest
  // logit that is not finite) is known from state[STATE_HALTED]; the round's replays after it are spent for nothing
  // (their cache rows lie past the call's positions, rewritten by whatever step takes those positions next), its
  // logits kept apart for he_logits. Rounds are shorter where stop tokens may end the call.
  RunParams &hp = *e->host_params;
  hp.temperature = temperature;
  hp.topp = topp;
  hp.penalty = penalty;
  hp.n_stops = n_stops;
  for (int32_t j = 0; j < RUN_STOPS_MOST; ++j) hp.stops[j] = j < n_stops ? stops[j] : -1;
  const int32_t w = (int32_t)window.size();
  if (w > 0) {
    std::memcpy(e->host_window, window.data(), sizeof(int32_t) * w);
    HIP_TRY(hipMemcpyAsync(e->window, e->host_window, sizeof(int32_t) * w, hipMemcpyHostToDevice, e->stream));
  }
  const int32_t round = n_stops > 0 ? STOP_ROUND : STEPS_A_ROUND;
  int32_t *hs = e->host_state;
  for (bool first = true; done < count; first = false) {
    const int32_t n = std::min(round, count - done);
    for (int32_t i = 0; i < RUN_RANDOMS; ++i) hp.randoms[i] = temperature > 0.0f && i < n ? randoms[done + i] : 0.0;
    hs[STATE_WORDS] = token;
    hs[STATE_POS] = pos + done;
    hs[STATE_STEP] = 0;
    hs[STATE_HALTED] = 0;
    hs[STATE_WINDOW] = w;  // (uploaded with the first round only: the device appends to the window from then on)
    hs[STATE_HEAD] = 0;
    HIP_TRY(hipMemcpyAsync(e->tokens, hs + STATE_WORDS, sizeof(int32_t), hipMemcpyHostToDevice, e->stream));
    HIP_TRY(hipMemcpyAsync(e->state, hs, sizeof(int32_t) * (first ? STATE_HEAD + 1 : STATE_HALTED + 1),
                           hipMemcpyHostToDevice, e->stream));
    HIP_TRY(hipMemcpyAsync(e->run_params, &hp, sizeof(RunParams), hipMemcpyHostToDevice, e->stream));
    for (int32_t i = 0; i < n; ++i) HIP_TRY(hipGraphLaunch(e->graph[kind], e->stream));
    HIP_TRY(hipMemcpyAsync(e->host_ids, e->step_ids, sizeof(int32_t) * n, hipMemcpyDeviceToHost, e->stream));
    HIP_TRY(hipMemcpyAsync(e->host_values, e->step_values, sizeof(float) * n, hipMemcpyDeviceToHost, e->stream));
    HIP_TRY(hipMemcpyAsync(hs + STATE_WORDS + 1, e->state + STATE_HALTED, sizeof(int32_t), hipMemcpyDeviceToHost,
                           e->stream));
    HIP_TRY(hipStreamSynchronize(e->stream));
    const int32_t halted = hs[STATE_WORDS + 1];
    for (int32_t j = 0; j < (halted ? halted : n); ++j) {
      const int32_t id = e->host_ids[j];
      if (halted && j == halted - 1) {
        e->logits_kept = true;
        if (id == SAMPLE_NOT_FINITE || !std::isfinite(e->host_values[j]))
          return fail(HE_E_NOTFINITE, "the largest logit is not finite");
        if (id != SAMPLE_DECLINED) ids[(*n_ids)++] = id;  // the stop token, last
        return HE_OK;  // (declined: the caller takes that step)
      }
      ids[(*n_ids)++] = id;
    }
    token = ids[*n_ids - 1];
    done += n;
  }
  e->logits_kept = false;
  return HE_OK;
}

namespace {
// run_tokens with a HIP event pair around every launch, summed by kind; the greedy choice timed too where logits are
int32_t profile_tokens(he_engine *e, const int32_t *tokens, int32_t count, int32_t pos, bool need_logits, double *ms,
                       double *bytes, int32_t *launches) {
  if (!e || !tokens || !ms || !bytes || !launches) return fail(HE_E_ARG, "a required pointer is null");
  for (int k = 0; k < HE_K_COUNT; ++k) {
    ms[k] = 0;
    bytes[k] = 0;
    launches[k] = 0;
  }
  HIP_TRY(hipStreamSynchronize(e->stream));
  e->profiling = true;
  e->marks.clear();
  int32_t rc = run_tokens(e, tokens, count, pos, need_logits);
  if (rc == HE_OK && need_logits)
    rc = timed(e, HE_K_ARGMAX, (double)e->c.vocab_size * 4, [&] {
           return launch_argmax(e->best_i, e->best_v, e->logits, e->c.vocab_size, e->amax_v, e->amax_i, e->stream);
         }) == hipSuccess ? HE_OK : fail(HE_E_HIP, "argmax launch failed");
  e->profiling = false;
  hipError_t err = hipStreamSynchronize(e->stream);
  for (auto &mk : e->marks) {
    float t = 0;
    if (err == hipSuccess && mk.a && mk.b) err = hipEventElapsedTime(&t, mk.a, mk.b);
    ms[mk.kind] += t;
    bytes[mk.kind] += mk.bytes;
    launches[mk.kind] += 1;
    if (mk.a) (void)hipEventDestroy(mk.a);
    if (mk.b) (void)hipEventDestroy(mk.b);
  }
  e->marks.clear();
  if (rc) return rc;
  if (err != hipSuccess) return fail(HE_E_HIP, std::string("profile: ") + hipGetErrorString(err));
  return HE_OK;
}
}  // namespace

int32_t he_profile_forward(he_engine *e, int32_t token, int32_t pos, int32_t need_logits, double *ms, double *bytes,
                           int32_t *launches) {
  return profile_tokens(e, &token, 1, pos, need_logits != 0, ms, bytes, launches);
}

int32_t he_profile_forward_many(he_engine *e, const int32_t *tokens, int32_t count, int32_t pos, double *ms,
                                double *bytes, int32_t *launches) {
  if (e && count > e->max_block) return fail(HE_E_ARG, "more tokens than the prompt block");
  return profile_tokens(e, tokens, count, pos, false, ms, bytes, launches);
}

int32_t he_profile_matmul(he_engine *e, int32_t which, int32_t rounds, double *ms, double *bytes, int32_t *launches) {
  if (!e || !ms || !bytes || !launches) return fail(HE_E_ARG, "a required pointer is null");
  if (which < -1 || which > 4 || rounds < 1) return fail(HE_E_ARG, "he_profile_matmul: which in -1..4, rounds >= 1");
  const he_config &c = e->c;
  const int32_t dim = c.dim, hidden = c.hidden_dim, qdim = e->qdim, kvdim = e->kvdim;
  // the outputs go to scratch rows (the engine's activations, cache and logits are not touched)
  const int64_t out_floats = std::max<int64_t>({(int64_t)c.vocab_size, 2LL * hidden, (int64_t)qdim + 2LL * kvdim,
                                                (int64_t)dim});
  float *out = nullptr;
  if (dev_alloc(&out, sizeof(float) * out_floats)) return HE_E_HIP;
  struct Launch {
    MatSeg seg[3];
    int nseg;
    int32_t k;
    bool persistent;  // the output projection: as the step launches it
  };
  std::vector<Launch> seq;
  for (int32_t l = 0; l < c.n_layers; ++l) {
    if (which == -1 || which == 0)
      seq.push_back({{{e->mat(HE_T_WQ, l), e->mat_scales(HE_T_WQ, l), out, qdim, qdim, 0},
                      {e->mat(HE_T_WK, l), e->mat_scales(HE_T_WK, l), out + qdim, kvdim, kvdim, 0},
                      {e->mat(HE_T_WV, l), e->mat_scales(HE_T_WV, l), out + qdim + kvdim, kvdim, kvdim, 0}},
                     3, dim, false});
    if (which == -1 || which == 1)
      seq.push_back({{{e->mat(HE_T_WO, l), e->mat_scales(HE_T_WO, l), out, dim, dim, 1}}, 1, qdim, true});
    if ((which == -1 || which == 2) && present(c, HE_T_W3))
      seq.push_back({{{e->mat(HE_T_W1, l), e->mat_scales(HE_T_W1, l), out, hidden, hidden, 0},
                      {e->mat(HE_T_W3, l), e->mat_scales(HE_T_W3, l), out + hidden, hidden, hidden, 0}},
                     2, dim, false});
    else if (which == -1 || which == 2)
      seq.push_back({{{e->mat(HE_T_W1, l), e->mat_scales(HE_T_W1, l), out, hidden, hidden, 0}}, 1, dim, false});
    if (which == -1 || which == 3)
      seq.push_back({{{e->mat(HE_T_W2, l), e->mat_scales(HE_T_W2, l), out, dim, dim, 1}}, 1, hidden, false});
  }
  if (which == -1 || which == 4)
    seq.push_back({{{e->mat(HE_T_WCLS, 0), e->mat_scales(HE_T_WCLS, 0), out, c.vocab_size, 0, 0}}, 1, dim, false});
  double pass_bytes = 0;
  for (const Launch &l : seq) pass_bytes += matmul_bytes(e, l.seg, l.nseg, l.k, 1);
  hipEvent_t a = nullptr, b = nullptr;
  hipError_t err = hipEventCreate(&a);
  if (err == hipSuccess) err = hipEventCreate(&b);
  if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
  if (err == hipSuccess) err = hipEventRecord(a, e->stream);
  for (int32_t r = 0; r < rounds && err == hipSuccess; ++r)
    for (const Launch &l : seq) {
      err = matmul_launch(e, l.seg, l.nseg, l.k, 1, e->xq, e->xs, nullptr, nullptr, l.persistent);
      if (err != hipSuccess) break;
    }
  if (err == hipSuccess) err = hipEventRecord(b, e->stream);
  if (err == hipSuccess) err = hipEventSynchronize(b);
  float t = 0;
  if (err == hipSuccess) err = hipEventElapsedTime(&t, a, b);
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  (void)hipFree(out);
  if (err != hipSuccess) return fail(HE_E_HIP, std::string("he_profile_matmul: ") + hipGetErrorString(err));
  *ms = (double)t / rounds;
  *bytes = pass_bytes;
  *launches = (int32_t)seq.size();
  return HE_OK;
}

int32_t he_logits(he_engine *e, float *out) {
  if (!e || !out) return fail(HE_E_ARG, "a required pointer is null");
  if (!e->have_logits) return fail(HE_E_STATE, "no step with logits has run");
  HIP_TRY(hipMemcpyAsync(out, e->logits_kept ? e->kept_logits : e->logits, sizeof(float) * e->c.vocab_size,
                         hipMemcpyDeviceToHost, e->stream));
  HIP_TRY(hipStreamSynchronize(e->stream));
  return HE_OK;
}

int32_t he_kv_read(he_engine *e, int32_t from, int32_t count, float *keys, float *values) {
  if (!e || !keys || !values) return fail(HE_E_ARG, "a required pointer is null");
  if (from < 0 || count < 0 || (int64_t)from + count > e->c.seq_len) return fail(HE_E_ARG, "positions out of range");
  const size_t esz = e->c.half_kv ? 2 : 4, kvdim = e->kvdim, vs = value_stride(e->c.seq_len);
  std::vector<uint8_t> rows((size_t)count * kvdim * esz);
  auto widen = [&](size_t i) {  // element i of rows as float32
    if (esz == 4) {
      float f;
      std::memcpy(&f, &rows[i * 4], 4);
      return f;
    }
    // public/forward.js:593-597 halfToFloat: exact for finite halves; an infinity stays infinite, a NaN is NaN (the
    // kernels' widening, which attention uses, reads an infinity as 65536)
    uint16_t h;
    std::memcpy(&h, &rows[i * 2], 2);
    if ((h & 0x7c00) == 0x7c00)
      return (h & 0x3ff) ? std::numeric_limits<float>::quiet_NaN()
                         : ((h & 0x8000) ? -std::numeric_limits<float>::infinity()
                                         : std::numeric_limits<float>::infinity());
    int32_t bits = ((int32_t)(int16_t)h << 13) & (int32_t)0x8fffffff;
    float f;
    std::memcpy(&f, &bits, 4);
    return f * 5.192296858534828e33f;
  };
  for (int32_t l = 0; l < e->c.n_layers; ++l) {
    // keys: the positions' rows as they lie
    const uint8_t *k = reinterpret_cast<const uint8_t *>(e->keys) + ((size_t)l * e->c.seq_len + from) * kvdim * esz;
    HIP_TRY(hipMemcpy(rows.data(), k, rows.size(), hipMemcpyDeviceToHost));
    float *ko = keys + (size_t)l * count * kvdim;
    for (size_t i = 0; i < (size_t)count * kvdim; ++i) ko[i] = widen(i);
    if (count == 0) continue;
    // values: kv_dim columns of count positions each, turned into the positions' rows
    const uint8_t *v = reinterpret_cast<const uint8_t *>(e->vals) + ((size_t)l * kvdim * vs + from) * esz;
    HIP_TRY(hipMemcpy2D(rows.data(), (size_t)count * esz, v, vs * esz, (size_t)count * esz, kvdim,
                        hipMemcpyDeviceToHost));
    float *vo = values + (size_t)l * count * kvdim;
    for (size_t col = 0; col < kvdim; ++col)
      for (size_t p = 0; p < (size_t)count; ++p) vo[p * kvdim + col] = widen(col * count + p);
  }
  return HE_OK;
}

int32_t he_checkpoint_read(he_engine *e, uint64_t offset, uint64_t length, void *out) {
  if (!e || !out) return fail(HE_E_ARG, "a required pointer is null");
  if (offset + length > e->size) return fail(HE_E_ARG, "the bytes run past the checkpoint");
  uint8_t *o = reinterpret_cast<uint8_t *>(out);
  while (length) {
    const Region *hit = nullptr;
    for (const Region &r : e->regions)
      if (offset >= r.file && offset < r.file + r.bytes) hit = &r;
    if (!hit) return fail(HE_E_ARG, "offset outside the checkpoint");
    const uint64_t n = std::min(length, hit->file + hit->bytes - offset);
    HIP_TRY(hipMemcpy(o, e->blob + hit->dev + (offset - hit->file), n, hipMemcpyDeviceToHost));
    o += n;
    offset += n;
    length -= n;
  }
  return HE_OK;
}

int32_t he_prompt_block(he_engine *e) { return e ? e->max_block : 0; }

uint64_t he_device_bytes(he_engine *e) { return e ? e->device_bytes : 0; }

int32_t he_close(he_engine *e) {
  if (!e) return HE_OK;
  (void)hipStreamSynchronize(e->stream);
  destroy(e);
  return HE_OK;
}

// ---- kernel level ----

int32_t hk_quantize_x(void *xq, void *xs, const void *x, int32_t m, int32_t n, int32_t bias, void *stream) {
  if (!xq || !xs || !x || m < 1 || n < 32 || n % 32) return fail(HE_E_ARG, "hk_quantize_x: bad arguments");
  if (bias != 0 && bias != 64) return fail(HE_E_ARG, "bias must be 0 or 64");
  HIP_TRY(launch_quantize(reinterpret_cast<int8_t *>(xq), reinterpret_cast<float *>(xs),
                          reinterpret_cast<const float *>(x), m, n, n, n, n / 32, bias,
                          reinterpret_cast<hipStream_t>(stream)));
  return HE_OK;
}

namespace {
int32_t matmul_args(MatArgs &a, void *y, const void *xq, const void *xs, const void *w, const void *ws, int32_t m,
                    int32_t rows, int32_t k, int32_t bias) {
  if (!xq || !w || m < 1 || rows < 1 || k < 32 || k % 32) return fail(HE_E_ARG, "matmul: bad arguments");
  if (bias != 0 && bias != 64) return fail(HE_E_ARG, "bias must be 0 or 64");
  a = MatArgs{};
  a.nseg = 1;
  a.seg[0] = {reinterpret_cast<const uint8_t *>(w), reinterpret_cast<const float *>(ws), reinterpret_cast<float *>(y),
              rows, rows, 0};
  a.total_rows = rows;
  a.xq = reinterpret_cast<const int8_t *>(xq);
  a.xs = reinterpret_cast<const float *>(xs);
  a.xq_stride = k;
  a.xs_stride = k / 32;
  a.k = k;
  return HE_OK;
}
}  // namespace

int32_t hk_matmul(void *y, const void *xq, const void *xs, const void *w, const void *ws, int32_t m, int32_t rows,
                  int32_t k, int32_t bias, int32_t six, void *stream) {
  MatArgs base;
  int32_t rc = matmul_args(base, y, xq, xs, w, ws, m, rows, k, bias);
  if (rc) return rc;
  if (!y || !xs || !ws) return fail(HE_E_ARG, "matmul: a required pointer is null");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (m > GEMV_MOST && gemm_supported(k, bias == 64)) {
    base.m = m;
    HIP_TRY(launch_gemm(base, six != 0, bias == 64, s));
    return HE_OK;
  }
  const int32_t step = gemv_tokens(k, bias == 64);
  if (step < 1) return fail(HE_E_ARG, "matmul: rows too long for the GEMV");
  for (int32_t t0 = 0; t0 < m; t0 += step) {
    MatArgs a = base;
    a.m = std::min(step, m - t0);
    a.xq = base.xq + (int64_t)t0 * k;
    a.xs = base.xs + (int64_t)t0 * (k / 32);
    a.seg[0].y = base.seg[0].y + (int64_t)t0 * rows;
    HIP_TRY(launch_gemv(a, six != 0, bias == 64, s));
  }
  return HE_OK;
}

int32_t hk_group_sums(void *s, const void *xq, const void *w, int32_t m, int32_t rows, int32_t k, int32_t bias,
                      int32_t six, int32_t gemm, void *stream) {
  MatArgs base;
  int32_t rc = matmul_args(base, nullptr, xq, nullptr, w, nullptr, m, rows, k, bias);
  if (rc) return rc;
  if (!s) return fail(HE_E_ARG, "sums is null");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (gemm) {
    if (!gemm_supported(k, bias == 64)) return fail(HE_E_ARG, "the MFMA GEMM takes bias 64 only");
    base.m = m;
    base.sums = reinterpret_cast<int32_t *>(s);
    HIP_TRY(launch_gemm(base, six != 0, true, st));
    return HE_OK;
  }
  const int64_t per_token = (int64_t)rows * (k / 32) * (bias ? 1 : 4);
  for (int32_t t0 = 0; t0 < m; t0 += 8) {
    MatArgs a = base;
    a.m = std::min(8, m - t0);
    a.xq = base.xq + (int64_t)t0 * k;
    a.sums = reinterpret_cast<int32_t *>(s) + t0 * per_token;
    HIP_TRY(launch_gemv(a, six != 0, bias == 64, st));
  }
  return HE_OK;
}


int32_t hk_penalize(void *logits, int32_t n, const int32_t *tokens, int32_t count, float penalty, void *stream) {
  if (!logits || n < 1 || count < 0 || count > REPETITION_WINDOW || (count > 0 && !tokens))
    return fail(HE_E_ARG, "hk_penalize: bad arguments");
  for (int32_t i = 0; i < count; ++i)
    if (tokens[i] < 0 || tokens[i] >= n) return fail(HE_E_ARG, "hk_penalize: a token is outside the logits");
  if (count == 0) return HE_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int32_t *d = nullptr;
  int32_t rc = dev_alloc(&d, sizeof(int32_t) * count);
  if (rc) return rc;
  hipError_t err = hipMemcpyAsync(d, tokens, sizeof(int32_t) * count, hipMemcpyHostToDevice, s);
  if (err == hipSuccess) err = launch_penalize(reinterpret_cast<float *>(logits), d, count, penalty, s);
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  (void)hipFree(d);
  if (err != hipSuccess) return fail(HE_E_HIP, std::string("hk_penalize: ") + hipGetErrorString(err));
  return HE_OK;
}

int32_t hk_ordered_sum(const void *p, int32_t n, int32_t nucleus, double *total, double *checkpoints, void *stream) {
  if (!p || !total || n < 1 || n > SAMPLE_MOST) return fail(HE_E_ARG, "hk_ordered_sum: bad arguments");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int32_t ncp = (n + SAMPLE_CHECKPOINT - 1) / SAMPLE_CHECKPOINT;
  float *padded = nullptr;
  double *out = nullptr;
  DrawParts *parts = nullptr;
  int32_t rc = dev_alloc(&padded, sizeof(float) * sample_probs_floats(n));  // whole chunks, as the draw's buffers
  if (!rc) rc = dev_alloc(&out, sizeof(double) * (1 + (size_t)ncp));
  if (!rc && !nucleus) rc = dev_alloc(&parts, sizeof(DrawParts));
  hipError_t err = hipSuccess;
  if (!rc) {
    err = hipMemcpyAsync(padded, p, sizeof(float) * (size_t)n, hipMemcpyDeviceToDevice, s);
    if (err == hipSuccess)  // +0.0 to the chunk's end, as the draw leaves its buffer
      err = hipMemsetAsync(padded + n, 0, sizeof(float) * (sample_probs_floats(n) - (size_t)n), s);
    if (err == hipSuccess) err = launch_ordered_sum(padded, n, out, out + 1, parts, s);
    if (err == hipSuccess) err = hipMemcpyAsync(total, out, sizeof(double), hipMemcpyDeviceToHost, s);
    if (err == hipSuccess && checkpoints)
      err = hipMemcpyAsync(checkpoints, out + 1, sizeof(double) * (size_t)ncp, hipMemcpyDeviceToHost, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
  }
  if (padded) (void)hipFree(padded);
  if (out) (void)hipFree(out);
  if (parts) (void)hipFree(parts);
  if (rc) return rc;
  if (err != hipSuccess) return fail(HE_E_HIP, std::string("hk_ordered_sum: ") + hipGetErrorString(err));
  return HE_OK;
}

int32_t hk_sample(const void *logits, int32_t n, float temperature, float topp, double random, int32_t *token,
                  void *stream) {
  if (!logits || !token || n < 1 || !(temperature > 0.0f)) return fail(HE_E_ARG, "hk_sample: bad arguments");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float *probs = nullptr, *best = nullptr;
  int32_t *index = nullptr, *out = nullptr;
  DrawParts *parts = nullptr;
  int32_t rc = dev_alloc(&probs, sizeof(float) * sample_probs_floats(n));
  if (!rc) rc = dev_alloc(&index, sizeof(int32_t) * n);
  if (!rc) rc = dev_alloc(&out, sizeof(int32_t) * 4);
  if (!rc) rc = dev_alloc(&best, sizeof(float) * 4);
  if (!rc) rc = dev_alloc(&parts, sizeof(DrawParts));
  hipError_t err = hipSuccess;
  if (!rc) {
    err = launch_sample(reinterpret_cast<const float *>(logits), n, temperature, topp, random, probs, index, parts, out,
                        best, s);
    if (err == hipSuccess) err = hipMemcpyAsync(token, out, sizeof(int32_t), hipMemcpyDeviceToHost, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
  }
  void *ptrs[] = {probs, index, out, best, parts};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  if (rc) return rc;
  if (err != hipSuccess) return fail(HE_E_HIP, std::string("hk_sample: ") + hipGetErrorString(err));
  return HE_OK;
}

}  // extern "C"

// hk_sample_static's scratch: probabilities [HK_SAMPLE_STATIC_MOST] float32, token indices [HK_SAMPLE_STATIC_MOST]
// int32, then the drawn token and the largest logit, 256 bytes apart, then the draw's parts (DrawParts: 277 KiB), in
// all 2 MiB and 278 KiB. Every GPU holds its own
// copy at its own address, found once a device with hipGetSymbolAddress: in host code the array's name is a stand-in,
// not a device address, and is never passed to a kernel or a copy.
namespace ple {
constexpr size_t SAMPLE_INDEX_AT = 4 * (size_t)HK_SAMPLE_STATIC_MOST, SAMPLE_TOKEN_AT = 8 * (size_t)HK_SAMPLE_STATIC_MOST;
constexpr size_t SAMPLE_BEST_AT = SAMPLE_TOKEN_AT + 256, SAMPLE_PARTS_AT = SAMPLE_BEST_AT + 256;
constexpr size_t SAMPLE_SCRATCH_BYTES = SAMPLE_PARTS_AT + sizeof(DrawParts);
__device__ __align__(256) uint8_t scratch[SAMPLE_SCRATCH_BYTES];
static_assert(SAMPLE_SCRATCH_BYTES <= (2u << 20) + 278u * 1024, "the static scratch's stated size");
static_assert(sample_probs_floats(HK_SAMPLE_STATIC_MOST) == (size_t)HK_SAMPLE_STATIC_MOST,
              "the probabilities' region holds the sampler's whole chunks");
}  // namespace ple

namespace {
constexpr int MOST_DEVICES = 64;
std::mutex g_scratch_lock;
uint8_t *g_scratch[MOST_DEVICES] = {};

// the current device's copy of `scratch`
int32_t sample_scratch(uint8_t **out) {
  int device = -1;
  HIP_TRY(hipGetDevice(&device));
  if (device < 0 || device >= MOST_DEVICES) return fail(HE_E_HIP, "hk_sample_static: a device index past 63");
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch[device]) {
    void *p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(HE_E_HIP, "hk_sample_static: no address for the scratch array");
    g_scratch[device] = reinterpret_cast<uint8_t *>(p);
  }
  *out = g_scratch[device];
  return HE_OK;
}

// the mean time of three launches of one ceiling loop between an event pair (after one untimed launch), and the
// output words (one a wave) of the last
template <class T, class F>
int32_t time_ceiling(const char *what, int32_t waves, hipStream_t s, std::vector<T> &host, double *ms, F &&launch) {
  T *out = nullptr;
  int32_t rc = dev_alloc(&out, sizeof(T) * waves);
  if (rc) return rc;
  hipEvent_t a = nullptr, b = nullptr;
  hipError_t err = hipEventCreate(&a);
  if (err == hipSuccess) err = hipEventCreate(&b);
  if (err == hipSuccess) err = launch(out);
  if (err == hipSuccess) err = hipEventRecord(a, s);
  const int reps = 3;
  for (int r = 0; r < reps && err == hipSuccess; ++r) err = launch(out);
  if (err == hipSuccess) err = hipEventRecord(b, s);
  if (err == hipSuccess) err = hipEventSynchronize(b);
  float t = 0;
  if (err == hipSuccess) err = hipEventElapsedTime(&t, a, b);
  host.assign(waves, T{});
  if (err == hipSuccess) err = hipMemcpy(host.data(), out, sizeof(T) * waves, hipMemcpyDeviceToHost);
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  (void)hipFree(out);
  if (err != hipSuccess) return fail(HE_E_HIP, std::string(what) + ": " + hipGetErrorString(err));
  *ms = (double)t / reps;
  return HE_OK;
}

}  // namespace

extern "C" {

int32_t hk_sample_static(const void *logits, int32_t n, float temperature, float topp, double random, int32_t *token,
                         void *stream) {
  if (!logits || !token || n < 1 || !(temperature > 0.0f)) return fail(HE_E_ARG, "hk_sample_static: bad arguments");
  if (n > HK_SAMPLE_STATIC_MOST)
    return fail(HE_E_ARG, "hk_sample_static takes at most HK_SAMPLE_STATIC_MOST (262144) logits");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // the token comes back to the host and the stream is waited for: neither may be recorded into a graph
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(s, &capture));
  if (capture != hipStreamCaptureStatusNone)
    return fail(HE_E_ARG, "hk_sample_static: the stream is under graph capture (the token is copied to the host)");
  uint8_t *base = nullptr;
  const int32_t rc = sample_scratch(&base);
  if (rc) return rc;
  int32_t *out = reinterpret_cast<int32_t *>(base + SAMPLE_TOKEN_AT);
  HIP_TRY(launch_sample(reinterpret_cast<const float *>(logits), n, temperature, topp, random,
                        reinterpret_cast<float *>(base), reinterpret_cast<int32_t *>(base + SAMPLE_INDEX_AT),
                        reinterpret_cast<DrawParts *>(base + SAMPLE_PARTS_AT), out,
                        reinterpret_cast<float *>(base + SAMPLE_BEST_AT), s));
  HIP_TRY(hipMemcpyAsync(token, out, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return HE_OK;
}

int32_t hk_read_ceiling(const void *p, int64_t bytes, int32_t passes, int32_t *checksum, double *ms, void *stream) {
  if (!p || !checksum || !ms || bytes < 64 || bytes % 64 || passes < 1)
    return fail(HE_E_ARG, "hk_read_ceiling: bad arguments");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int32_t most = 1;
  for (int32_t i = 0; i < read_ceiling_shapes(); ++i) most = std::max(most, read_ceiling_blocks(bytes, i));
  uint32_t *partial = nullptr;
  int32_t rc = dev_alloc(&partial, sizeof(uint32_t) * 4 * most);
  if (rc) return rc;
  hipEvent_t a = nullptr, b = nullptr;
  hipError_t err = hipEventCreate(&a);
  if (err == hipSuccess) err = hipEventCreate(&b);
  std::vector<uint32_t> h(4 * (size_t)most);
  double best = 0;
  int64_t sum = -1;
  bool agree = true;
  // each launch shape: one untimed pass, then `passes` between an event pair; the fastest shape's mean pass
  for (int32_t shape = 0; shape < read_ceiling_shapes() && err == hipSuccess; ++shape) {
    err = launch_read_ceiling(p, bytes, shape, partial, s);
    if (err == hipSuccess) err = hipEventRecord(a, s);
    for (int32_t r = 0; r < passes && err == hipSuccess; ++r) err = launch_read_ceiling(p, bytes, shape, partial, s);
    if (err == hipSuccess) err = hipEventRecord(b, s);
    if (err == hipSuccess) err = hipEventSynchronize(b);
    float t = 0;
    if (err == hipSuccess) err = hipEventElapsedTime(&t, a, b);
    const int32_t blocks = read_ceiling_blocks(bytes, shape);
    if (err == hipSuccess)
      err = hipMemcpy(h.data(), partial, sizeof(uint32_t) * 4 * blocks, hipMemcpyDeviceToHost);
    if (err != hipSuccess) break;
    // every pass reads the same words: passes times one pass's lane sums (mod 2^32)
    uint32_t lane[4] = {0, 0, 0, 0};
    for (int32_t i = 0; i < blocks; ++i)
      for (int j = 0; j < 4; ++j) lane[j] += h[4 * (size_t)i + j];
    for (int j = 0; j < 4; ++j) lane[j] *= (uint32_t)passes;
    const int64_t x = (int64_t)(lane[0] ^ lane[1] ^ lane[2] ^ lane[3]);
    if (sum >= 0 && x != sum) agree = false;
    sum = x;
    const double pass_ms = (double)t / passes;
    if (best == 0 || pass_ms < best) best = pass_ms;
  }
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  (void)hipFree(partial);
  if (err != hipSuccess) return fail(HE_E_HIP, std::string("hk_read_ceiling: ") + hipGetErrorString(err));
  if (!agree) return fail(HE_E_HIP, "hk_read_ceiling: the launch shapes' checksums differ");
  *checksum = (int32_t)(uint32_t)sum;
  *ms = best;
  return HE_OK;
}

int32_t hk_read_floor(const void *p, int64_t span, int64_t bytes, int32_t passes, double *us, void *stream) {
  if (!p || !us || bytes < 64 || bytes % 64 || span < bytes || passes < 1)
    return fail(HE_E_ARG, "hk_read_floor: bad arguments");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t windows = span / bytes;  // launch i reads window i % windows
  int32_t most = 1;
  for (int32_t i = 0; i < read_ceiling_shapes(); ++i) most = std::max(most, read_ceiling_blocks(bytes, i));
  uint32_t *partial = nullptr;
  int32_t rc = dev_alloc(&partial, sizeof(uint32_t) * 4 * most);
  if (rc) return rc;
  hipEvent_t a = nullptr, b = nullptr;
  hipError_t err = hipEventCreate(&a);
  if (err == hipSuccess) err = hipEventCreate(&b);
  const uint8_t *base = reinterpret_cast<const uint8_t *>(p);
  double best = 0;
  int64_t window = 0;
  auto next = [&]() { return base + (window++ % windows) * bytes; };
  // each launch shape: three untimed launches, then `passes` back to back between an event pair, each on the next
  // window; the fastest shape's mean launch
  for (int32_t shape = 0; shape < read_ceiling_shapes() && err == hipSuccess; ++shape) {
    for (int r = 0; r < 3 && err == hipSuccess; ++r) err = launch_read_ceiling(next(), bytes, shape, partial, s);
    if (err == hipSuccess) err = hipEventRecord(a, s);
    for (int32_t r = 0; r < passes && err == hipSuccess; ++r) err = launch_read_ceiling(next(), bytes, shape, partial, s);
    if (err == hipSuccess) err = hipEventRecord(b, s);
    if (err == hipSuccess) err = hipEventSynchronize(b);
    float t = 0;
    if (err == hipSuccess) err = hipEventElapsedTime(&t, a, b);
    if (err != hipSuccess) break;
    const double launch_us = 1e3 * (double)t / passes;
    if (best == 0 || launch_us < best) best = launch_us;
  }
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  (void)hipStreamSynchronize(s);
  (void)hipFree(partial);
  if (err != hipSuccess) return fail(HE_E_HIP, std::string("hk_read_floor: ") + hipGetErrorString(err));
  *us = best;
  return HE_OK;
}

int32_t hk_valu_ceiling(int32_t passes, float w, float x0, float step, float *result, double *ms, double *pairs,
                        void *stream) {
  if (!result || !ms || !pairs || passes < 1) return fail(HE_E_ARG, "hk_valu_ceiling: bad arguments");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int32_t waves = valu_ceiling_waves();
  std::vector<float> h;
  const int32_t rc = time_ceiling("hk_valu_ceiling", waves, s, h, ms, [&](float *out) {
    return launch_valu_ceiling(passes, w, x0, step, 0.0f, out, s);
  });
  if (rc) return rc;
  for (int32_t i = 1; i < waves; ++i)
    if (std::memcmp(&h[i], &h[0], sizeof(float)))
      return fail(HE_E_HIP, "hk_valu_ceiling: the waves' sums differ");
  *result = h[0];
  *pairs = (double)waves * 64 * passes * 8;
  return HE_OK;
}

int32_t hk_mfma_ceiling(int32_t passes, int32_t first, int32_t times, int32_t flip, int32_t *checksum, double *ms,
                        double *ops, void *stream) {
  if (!checksum || !ms || !ops || passes < 1) return fail(HE_E_ARG, "hk_mfma_ceiling: bad arguments");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int32_t waves = mfma_ceiling_waves();
  std::vector<uint32_t> h;
  const int32_t rc = time_ceiling("hk_mfma_ceiling", waves, s, h, ms, [&](uint32_t *out) {
    return launch_mfma_ceiling(passes, first, times, flip, out, s);
  });
  if (rc) return rc;
  for (int32_t i = 1; i < waves; ++i)
    if (h[i] != h[0]) return fail(HE_E_HIP, "hk_mfma_ceiling: the waves' sums differ");
  *checksum = (int32_t)h[0];
  // 4 products of 32 x 32 x 32 a pass, a multiply and an add each
  *ops = (double)waves * passes * 4 * 32768.0 * 2;
  return HE_OK;
}

}  // extern "C"
