/*
 * napi_addon.c — hip_engine.node: the N-API addon that gives JavaScript the C ABI of include/pyodide_llm_hip.h.
 *
 * Thin on purpose: every function checks its arguments' JavaScript types, calls one he_* function and turns a
 * negative return into a thrown Error (message: he_last_error(), property `code`: the HE_E_* value), as
 * public/forward.js throws to its Python caller. The engine handle is a JavaScript external; pyodide-llm_amd/
 * forward_hip.mjs builds the forward.js interface on top. Built with gcc against Node's N-API headers (version 8).
 */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "include/pyodide_llm_hip.h"

#define MAX_ARGS 16 /* the most any function here takes (generateMany: 12) */

/* a failed N-API call: throw (if nothing is pending yet) and return NULL from the callback */
#define NAPI_TRY(env, call)                                                      \
  do {                                                                           \
    if ((call) != napi_ok) {                                                     \
      bool pending_ = false;                                                     \
      napi_is_exception_pending((env), &pending_);                               \
      if (!pending_) napi_throw_error((env), NULL, "hip_engine: N-API failure"); \
      return NULL;                                                               \
    }                                                                            \
  } while (0)

static napi_value throw_engine(napi_env env, int32_t code) {
  char message[1024];
  snprintf(message, sizeof message, "%s", he_last_error());
  if (!message[0]) snprintf(message, sizeof message, "engine call failed (%d)", (int)code);
  napi_value msg, err, code_value;
  if (napi_create_string_utf8(env, message, NAPI_AUTO_LENGTH, &msg) != napi_ok) return NULL;
  if (napi_create_error(env, NULL, msg, &err) != napi_ok) return NULL;
  if (napi_create_int32(env, code, &code_value) == napi_ok) napi_set_named_property(env, err, "code", code_value);
  napi_throw(env, err);
  return NULL;
}

static napi_value throw_type(napi_env env, const char *what) {
  napi_throw_type_error(env, NULL, what);
  return NULL;
}

static napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

static int args_of(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = MAX_ARGS;
  napi_value all[MAX_ARGS];
  if (want > MAX_ARGS) {
    napi_throw_error(env, NULL, "hip_engine: a function takes more arguments than MAX_ARGS");
    return 0;
  }
  if (napi_get_cb_info(env, info, &argc, all, NULL, NULL) != napi_ok) return 0;
  if (argc < want) {
    napi_throw_type_error(env, NULL, "hip_engine: too few arguments");
    return 0;
  }
  for (size_t i = 0; i < want; ++i) argv[i] = all[i];
  return 1;
}

static int get_i32(napi_env env, napi_value v, int32_t *out) {
  double d;
  if (napi_get_value_double(env, v, &d) != napi_ok || d != d || d < -2147483648.0 || d > 2147483647.0 ||
      d != (double)(int32_t)d) {
    napi_throw_type_error(env, NULL, "hip_engine: an argument is not a 32-bit integer");
    return 0;
  }
  *out = (int32_t)d;
  return 1;
}

/* a non-negative integer below 2^53 (offsets and sizes), from a Number or a BigInt */
static int get_u64(napi_env env, napi_value v, uint64_t *out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return 0;
  if (t == napi_bigint) {
    bool lossless = false;
    if (napi_get_value_bigint_uint64(env, v, out, &lossless) != napi_ok || !lossless) {
      napi_throw_type_error(env, NULL, "hip_engine: a BigInt argument is not an unsigned 64-bit integer");
      return 0;
    }
    return 1;
  }
  double d;
  if (napi_get_value_double(env, v, &d) != napi_ok || !(d >= 0) || d > 9007199254740992.0 || d != (double)(uint64_t)d) {
    napi_throw_type_error(env, NULL, "hip_engine: an argument is not a non-negative integer");
    return 0;
  }
  *out = (uint64_t)d;
  return 1;
}

/* what a JavaScript engine external points to: the handle (NULL once closed) and the sizes its output arrays are
 * checked against, so that a short typed array is a TypeError instead of a write past its end */
typedef struct engine_slot {
  he_engine *e;
  int64_t vocab;  /* floats of the logits */
  int64_t layers; /* keysAndValues: layers * count * kv_dim floats of keys, and of values */
  int64_t kv_dim;
} engine_slot;

static engine_slot *slot_of(napi_env env, napi_value v) {
  void *p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "hip_engine: not an engine (or one already closed)");
    return NULL;
  }
  engine_slot *slot = (engine_slot *)p;
  if (!slot->e) {
    napi_throw_error(env, NULL, "hip_engine: the engine was released");
    return NULL;
  }
  return slot;
}

static he_engine *engine_of(napi_env env, napi_value v) {
  engine_slot *slot = slot_of(env, v);
  return slot ? slot->e : NULL;
}

/* the bytes of a TypedArray (of the given type, or any if type < 0) or a DataView-less ArrayBuffer */
static int bytes_of(napi_env env, napi_value v, int type, void **data, size_t *length) {
  bool is_typed = false, is_buffer = false;
  napi_is_typedarray(env, v, &is_typed);
  if (is_typed) {
    napi_typedarray_type t;
    size_t count = 0, offset = 0;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &t, &count, data, &ab, &offset) != napi_ok) return 0;
    if (type >= 0 && (int)t != type) {
      napi_throw_type_error(env, NULL, "hip_engine: a typed array of the wrong type");
      return 0;
    }
    static const size_t sizes[] = {1, 1, 1, 2, 2, 4, 4, 4, 8, 8, 8};
    *length = count * ((size_t)t < sizeof sizes / sizeof sizes[0] ? sizes[t] : 1);
    return 1;
  }
  napi_is_arraybuffer(env, v, &is_buffer);
  if (is_buffer && type < 0) return napi_get_arraybuffer_info(env, v, data, length) == napi_ok;
  napi_throw_type_error(env, NULL, "hip_engine: expected a typed array or an ArrayBuffer");
  return 0;
}

static int field_i32(napi_env env, napi_value obj, const char *name, int32_t *out) {
  napi_value v;
  if (napi_get_named_property(env, obj, name, &v) != napi_ok) return 0;
  if (!get_i32(env, v, out)) return 0;
  return 1;
}

/* he_config from {dim, hidden_dim, ..., rms_norm_eps, arch, rotary, parallel_residual, qk_norm, outliers: [...]} (the
 * names of include/pyodide_llm_hip.h) */
static int config_of(napi_env env, napi_value obj, he_config *c) {
  memset(c, 0, sizeof *c);
  static const char *names[] = {"dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_size", "vocab_size",
                                "seq_len", "shared_classifier", "six", "qkv_bias", "relaxed", "half_kv"};
  int32_t *fields[] = {&c->dim, &c->hidden_dim, &c->n_layers, &c->n_heads, &c->n_kv_heads, &c->head_size,
                       &c->vocab_size, &c->seq_len, &c->shared_classifier, &c->six, &c->qkv_bias, &c->relaxed,
                       &c->half_kv};
  for (size_t i = 0; i < sizeof names / sizeof names[0]; ++i)
    if (!field_i32(env, obj, names[i], fields[i])) return 0;
  napi_value v;
  double eps;
  if (napi_get_named_property(env, obj, "rms_norm_eps", &v) != napi_ok || napi_get_value_double(env, v, &eps) != napi_ok) {
    napi_throw_type_error(env, NULL, "hip_engine: config.rms_norm_eps is not a number");
    return 0;
  }
  c->rms_norm_eps = (float)eps;
  static const char *forms[] = {"arch", "rotary", "parallel_residual", "qk_norm"};
  int32_t *form_fields[] = {&c->arch, &c->rotary, &c->parallel_residual, &c->qk_norm};
  for (size_t i = 0; i < sizeof forms / sizeof forms[0]; ++i)
    if (!field_i32(env, obj, forms[i], form_fields[i])) return 0;
  /* outliers: an array of at most HE_OUTLIERS_MOST channels */
  uint32_t n = 0;
  if (napi_get_named_property(env, obj, "outliers", &v) != napi_ok || napi_get_array_length(env, v, &n) != napi_ok ||
      n > HE_OUTLIERS_MOST) {
    napi_throw_type_error(env, NULL, "hip_engine: config.outliers is not an array of at most 8 channels");
    return 0;
  }
  c->n_outliers = (int32_t)n;
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    if (napi_get_element(env, v, i, &e) != napi_ok || !get_i32(env, e, &c->outliers[i])) return 0;
  }
  return 1;
}

/* he_tensor[HE_T_COUNT] from an array of HE_T_COUNT [offset, scales] pairs (BigInt or Number) */
static int tensors_of(napi_env env, napi_value arr, he_tensor *t) {
  uint32_t n = 0;
  if (napi_get_array_length(env, arr, &n) != napi_ok || n != HE_T_COUNT) {
    napi_throw_type_error(env, NULL, "hip_engine: tensors must be an array of HE_T_COUNT (24) [offset, scales] pairs");
    return 0;
  }
  for (uint32_t i = 0; i < n; ++i) {
    napi_value pair, a, b;
    uint64_t offset, scales;
    if (napi_get_element(env, arr, i, &pair) != napi_ok || napi_get_element(env, pair, 0, &a) != napi_ok ||
        napi_get_element(env, pair, 1, &b) != napi_ok)
      return 0;
    if (!get_u64(env, a, &offset) || !get_u64(env, b, &scales)) return 0;
    t[i].offset = (int64_t)offset;
    t[i].scales = (int64_t)scales;
  }
  return 1;
}

static void finalize_engine(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  engine_slot *slot = (engine_slot *)data;
  if (slot->e) he_close(slot->e);
  free(slot);
}

static napi_value wrap_engine(napi_env env, he_engine *e, const he_config *c) {
  engine_slot *slot = (engine_slot *)malloc(sizeof *slot);
  if (!slot) {
    he_close(e);
    napi_throw_error(env, NULL, "hip_engine: out of host memory");
    return NULL;
  }
  slot->e = e;
  slot->vocab = c->vocab_size;
  slot->layers = c->n_layers;
  slot->kv_dim = (int64_t)c->n_kv_heads * c->head_size;
  napi_value out;
  if (napi_create_external(env, slot, finalize_engine, NULL, &out) != napi_ok) {
    he_close(e);
    free(slot);
    return NULL;
  }
  return out;
}

/* open(config, tensors, checkpoint: ArrayBuffer|TypedArray, base, size, cos: Float32Array, sin: Float32Array,
 *      maxBlock) -> engine: he_open on the `size` bytes at `base` of the checkpoint's buffer */
static napi_value js_open(napi_env env, napi_callback_info info) {
  napi_value argv[8];
  if (!args_of(env, info, 8, argv)) return NULL;
  he_config c;
  he_tensor t[HE_T_COUNT];
  void *data, *cos_d, *sin_d;
  size_t length, cos_n, sin_n;
  uint64_t base, size;
  int32_t max_block;
  if (!config_of(env, argv[0], &c) || !tensors_of(env, argv[1], t) || !bytes_of(env, argv[2], -1, &data, &length) ||
      !get_u64(env, argv[3], &base) || !get_u64(env, argv[4], &size) ||
      !bytes_of(env, argv[5], napi_float32_array, &cos_d, &cos_n) ||
      !bytes_of(env, argv[6], napi_float32_array, &sin_d, &sin_n) || !get_i32(env, argv[7], &max_block))
    return NULL;
  if (base > length || size > length - base) return throw_type(env, "hip_engine: the checkpoint is not in the buffer");
  const uint64_t table = (uint64_t)c.seq_len * (uint64_t)(c.head_size / 2) * 4;
  if (c.seq_len < 1 || c.head_size < 2 || cos_n < table || sin_n < table)
    return throw_type(env, "hip_engine: the RoPE tables are smaller than [seq_len][head_size/2]");
  he_engine *e = NULL;
  const int32_t rc = he_open(&c, t, (const uint8_t *)data + base, size, (const float *)cos_d, (const float *)sin_d,
                             max_block, &e);
  if (rc) return throw_engine(env, rc);
  return wrap_engine(env, e, &c);
}

/* openSynthetic(config, tensors, size, seed, cos, sin, maxBlock) -> engine (he_open_synthetic) */
static napi_value js_open_synthetic(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!args_of(env, info, 7, argv)) return NULL;
  he_config c;
  he_tensor t[HE_T_COUNT];
  void *cos_d, *sin_d;
  size_t cos_n, sin_n;
  uint64_t size, seed;
  int32_t max_block;
  if (!config_of(env, argv[0], &c) || !tensors_of(env, argv[1], t) || !get_u64(env, argv[2], &size) ||
      !get_u64(env, argv[3], &seed) || !bytes_of(env, argv[4], napi_float32_array, &cos_d, &cos_n) ||
      !bytes_of(env, argv[5], napi_float32_array, &sin_d, &sin_n) || !get_i32(env, argv[6], &max_block))
    return NULL;
  const uint64_t table = (uint64_t)c.seq_len * (uint64_t)(c.head_size / 2) * 4;
  if (c.seq_len < 1 || c.head_size < 2 || cos_n < table || sin_n < table)
    return throw_type(env, "hip_engine: the RoPE tables are smaller than [seq_len][head_size/2]");
  he_engine *e = NULL;
  const int32_t rc = he_open_synthetic(&c, t, size, seed, (const float *)cos_d, (const float *)sin_d, max_block, &e);
  if (rc) return throw_engine(env, rc);
  return wrap_engine(env, e, &c);
}

/* forward(engine, token, pos, needLogits, logits: Float32Array|null) */
static napi_value js_forward(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!args_of(env, info, 5, argv)) return NULL;
  engine_slot *slot = slot_of(env, argv[0]);
  int32_t token, pos;
  bool need = false;
  if (!slot || !get_i32(env, argv[1], &token) || !get_i32(env, argv[2], &pos)) return NULL;
  he_engine *e = slot->e;
  NAPI_TRY(env, napi_get_value_bool(env, argv[3], &need));
  napi_valuetype tt;
  NAPI_TRY(env, napi_typeof(env, argv[4], &tt));
  float *logits = NULL;
  if (need && tt != napi_null && tt != napi_undefined) {
    void *d;
    size_t n;
    if (!bytes_of(env, argv[4], napi_float32_array, &d, &n)) return NULL;
    if (n < 4 * (size_t)slot->vocab) return throw_type(env, "hip_engine: logits holds fewer than vocab_size floats");
    logits = (float *)d;
  }
  const int32_t rc = he_forward(e, token, pos, need ? 1 : 0, logits);
  if (rc) return throw_engine(env, rc);
  return undefined(env);
}

/* forwardMany(engine, tokens: Int32Array, pos) */
static napi_value js_forward_many(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args_of(env, info, 3, argv)) return NULL;
  he_engine *e = engine_of(env, argv[0]);
  void *d;
  size_t n;
  int32_t pos;
  if (!e || !bytes_of(env, argv[1], napi_int32_array, &d, &n) || !get_i32(env, argv[2], &pos)) return NULL;
  const int32_t rc = he_forward_many(e, (const int32_t *)d, (int32_t)(n / 4), pos);
  if (rc) return throw_engine(env, rc);
  return undefined(env);
}

static int get_f64(napi_env env, napi_value v, double *out) {
  if (napi_get_value_double(env, v, out) != napi_ok) {
    napi_throw_type_error(env, NULL, "hip_engine: an argument is not a number");
    return 0;
  }
  return 1;
}

/* generateMany(engine, token, pos, history: Int32Array, length, count, temperature, topp, penalty,
 * randoms: Float64Array, stops: Int32Array, ids: Int32Array) -> the number of ids (0: the engine did not take the
 * first step), or -1 where a step's largest logit was not finite */
static napi_value js_generate_many(napi_env env, napi_callback_info info) {
  napi_value argv[12];
  if (!args_of(env, info, 12, argv)) return NULL;
  he_engine *e = engine_of(env, argv[0]);
  int32_t token, pos, length, count;
  double temperature, topp, penalty;
  void *history, *randoms, *stops, *ids;
  size_t n_history, n_randoms, n_stops, n_ids;
  if (!e || !get_i32(env, argv[1], &token) || !get_i32(env, argv[2], &pos) ||
      !bytes_of(env, argv[3], napi_int32_array, &history, &n_history) || !get_i32(env, argv[4], &length) ||
      !get_i32(env, argv[5], &count) || !get_f64(env, argv[6], &temperature) || !get_f64(env, argv[7], &topp) ||
      !get_f64(env, argv[8], &penalty) || !bytes_of(env, argv[9], napi_float64_array, &randoms, &n_randoms) ||
      !bytes_of(env, argv[10], napi_int32_array, &stops, &n_stops) ||
      !bytes_of(env, argv[11], napi_int32_array, &ids, &n_ids))
    return NULL;
  if (count < 1 || (size_t)count > n_ids / 4) return throw_type(env, "hip_engine: ids holds fewer than count ids");
  int32_t got = 0;
  const int32_t rc = he_generate_many(e, token, pos, (const int32_t *)history, (int32_t)(n_history / 4), length, count,
                                      (float)temperature, (float)topp, (float)penalty, (const double *)randoms,
                                      (int32_t)(n_randoms / 8), (const int32_t *)stops, (int32_t)(n_stops / 4),
                                      (int32_t *)ids, &got);
  napi_value out;
  if (rc == HE_E_NOTFINITE) got = -1;
  else if (rc) return throw_engine(env, rc);
  NAPI_TRY(env, napi_create_int32(env, got, &out));
  return out;
}

/* logits(engine, out: Float32Array) */
static napi_value js_logits(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args_of(env, info, 2, argv)) return NULL;
  engine_slot *slot = slot_of(env, argv[0]);
  void *d;
  size_t n;
  if (!slot || !bytes_of(env, argv[1], napi_float32_array, &d, &n)) return NULL;
  if (n < 4 * (size_t)slot->vocab) return throw_type(env, "hip_engine: out holds fewer than vocab_size floats");
  const int32_t rc = he_logits(slot->e, (float *)d);
  if (rc) return throw_engine(env, rc);
  return undefined(env);
}

/* kvRead(engine, from, count, keys: Float32Array, values: Float32Array) */
static napi_value js_kv_read(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!args_of(env, info, 5, argv)) return NULL;
  engine_slot *slot = slot_of(env, argv[0]);
  int32_t from, count;
  void *k, *v;
  size_t nk, nv;
  if (!slot || !get_i32(env, argv[1], &from) || !get_i32(env, argv[2], &count) ||
      !bytes_of(env, argv[3], napi_float32_array, &k, &nk) || !bytes_of(env, argv[4], napi_float32_array, &v, &nv))
    return NULL;
  if (count < 0) return throw_type(env, "hip_engine: count is negative");
  const uint64_t need = 4 * (uint64_t)slot->layers * (uint64_t)count * (uint64_t)slot->kv_dim;
  if (nk < need || nv < need)
    return throw_type(env, "hip_engine: keys or values holds fewer than layers * count * kv_dim floats");
  const int32_t rc = he_kv_read(slot->e, from, count, (float *)k, (float *)v);
  if (rc) return throw_engine(env, rc);
  return undefined(env);
}

/* checkpointRead(engine, offset, length, out: Uint8Array) */
static napi_value js_checkpoint_read(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!args_of(env, info, 4, argv)) return NULL;
  he_engine *e = engine_of(env, argv[0]);
  uint64_t offset, length;
  void *d;
  size_t n;
  if (!e || !get_u64(env, argv[1], &offset) || !get_u64(env, argv[2], &length) ||
      !bytes_of(env, argv[3], napi_uint8_array, &d, &n))
    return NULL;
  if (length > n) return throw_type(env, "hip_engine: out is shorter than length");
  const int32_t rc = he_checkpoint_read(e, offset, length, d);
  if (rc) return throw_engine(env, rc);
  return undefined(env);
}

static napi_value js_prompt_block(napi_env env, napi_callback_info info) {
  napi_value argv[1], out;
  if (!args_of(env, info, 1, argv)) return NULL;
  he_engine *e = engine_of(env, argv[0]);
  if (!e) return NULL;
  NAPI_TRY(env, napi_create_int32(env, he_prompt_block(e), &out));
  return out;
}

static napi_value js_device_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1], out;
  if (!args_of(env, info, 1, argv)) return NULL;
  he_engine *e = engine_of(env, argv[0]);
  if (!e) return NULL;
  NAPI_TRY(env, napi_create_double(env, (double)he_device_bytes(e), &out));
  return out;
}

/* close(engine): frees the device memory now (the external's finalizer would later) */
static napi_value js_close(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return NULL;
  void *p = NULL;
  NAPI_TRY(env, napi_get_value_external(env, argv[0], &p));
  engine_slot *slot = (engine_slot *)p;
  if (slot && slot->e) {
    he_engine *e = slot->e;
    slot->e = NULL;
    const int32_t rc = he_close(e);
    if (rc) return throw_engine(env, rc);
  }
  return undefined(env);
}

/* profile(engine, token, pos, needLogits, ms: Float64Array, bytes: Float64Array, launches: Int32Array) */
static napi_value js_profile(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!args_of(env, info, 7, argv)) return NULL;
  he_engine *e = engine_of(env, argv[0]);
  int32_t token, pos;
  bool need = false;
  void *ms, *bytes, *launches;
  size_t n1, n2, n3;
  if (!e || !get_i32(env, argv[1], &token) || !get_i32(env, argv[2], &pos)) return NULL;
  NAPI_TRY(env, napi_get_value_bool(env, argv[3], &need));
  if (!bytes_of(env, argv[4], napi_float64_array, &ms, &n1) || !bytes_of(env, argv[5], napi_float64_array, &bytes, &n2) ||
      !bytes_of(env, argv[6], napi_int32_array, &launches, &n3))
    return NULL;
  if (n1 < 8 * HE_K_COUNT || n2 < 8 * HE_K_COUNT || n3 < 4 * HE_K_COUNT)
    return throw_type(env, "hip_engine: profile arrays are shorter than the kinds of kernel");
  const int32_t rc = he_profile_forward(e, token, pos, need ? 1 : 0, (double *)ms, (double *)bytes, (int32_t *)launches);
  if (rc) return throw_engine(env, rc);
  return undefined(env);
}

static napi_value init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"open", NULL, js_open, NULL, NULL, NULL, napi_enumerable, NULL},
      {"openSynthetic", NULL, js_open_synthetic, NULL, NULL, NULL, napi_enumerable, NULL},
      {"forward", NULL, js_forward, NULL, NULL, NULL, napi_enumerable, NULL},
      {"forwardMany", NULL, js_forward_many, NULL, NULL, NULL, napi_enumerable, NULL},
      {"generateMany", NULL, js_generate_many, NULL, NULL, NULL, napi_enumerable, NULL},
      {"logits", NULL, js_logits, NULL, NULL, NULL, napi_enumerable, NULL},
      {"kvRead", NULL, js_kv_read, NULL, NULL, NULL, napi_enumerable, NULL},
      {"checkpointRead", NULL, js_checkpoint_read, NULL, NULL, NULL, napi_enumerable, NULL},
      {"promptBlock", NULL, js_prompt_block, NULL, NULL, NULL, napi_enumerable, NULL},
      {"deviceBytes", NULL, js_device_bytes, NULL, NULL, NULL, napi_enumerable, NULL},
      {"close", NULL, js_close, NULL, NULL, NULL, napi_enumerable, NULL},
      {"profile", NULL, js_profile, NULL, NULL, NULL, napi_enumerable, NULL},
  };
  NAPI_TRY(env, napi_define_properties(env, exports, sizeof props / sizeof props[0], props));
  napi_value kinds;
  NAPI_TRY(env, napi_create_int32(env, HE_K_COUNT, &kinds));
  NAPI_TRY(env, napi_set_named_property(env, exports, "KIND_COUNT", kinds));
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
