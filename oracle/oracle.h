/*
 * oracle.h — TEST INFRASTRUCTURE, NOT PART OF THE PRODUCT.
 *
 * A plain-C restatement of the arithmetic of pyodide-llm's CPU path (kernels/kernel.ts, kernels/kernel_relaxed.ts,
 * kernels/six.ts, public/forward.js run(), public/llama2_convert.py quantize(), public/llama2_numpy.py
 * quantize6/pack6/Places), in the reference's exact float32 order. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, as the parity reference or the CPU baseline, never as the thing measured on the GPU.
 * Every function cites the reference lines it follows; oracle/oracle.c's header lists how each one is pinned.
 */
#ifndef PYODIDE_LLM_ORACLE_H
#define PYODIDE_LLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/pyodide_llm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic inputs (the same bits as the device generator) ---- */
uint64_t or_mix64(uint64_t z);
float or_synth_factor(double sigma);
float or_synth_value(uint64_t seed, int32_t stream, uint64_t index, float factor);
void or_synth_fill(float *out, uint64_t n, uint64_t seed, int32_t stream, uint64_t first, double sigma);

/* ---- weight formats ---- */
int32_t or_group_size(int32_t row_length);
void or_quantize(int8_t *q, float *scales, const float *x, int64_t count, int32_t group);
void or_quantize6(int8_t *q, float *scales, const float *x, int64_t groups);
void or_pack6(uint8_t *out, const int8_t *q, int64_t groups);
void or_unpack6(int8_t *out, const uint8_t *packed, int64_t groups);

/* ---- the kernels ---- */
void or_quantize_x(int8_t *xq, float *xs, const float *x, int32_t n, int32_t bias);
void or_matmul_q8r(float *y, const int8_t *xq, const float *xs, const int8_t *w, const float *ws, int32_t k,
                   int32_t r0, int32_t r1);
void or_matmul_q8(float *y, const int8_t *xq, const float *xs, const int8_t *w, const float *ws, int32_t k,
                  int32_t r0, int32_t r1);
void or_matmul_q6r(float *y, const int8_t *xq, const float *xs, const uint8_t *w, const float *ws, int32_t k,
                   int32_t r0, int32_t r1);
void or_matmul_q6(float *y, const int8_t *xq, const float *xs, const uint8_t *w, const float *ws, int32_t k,
                  int32_t r0, int32_t r1);
void or_group_sums(int32_t *s, const int8_t *xq, const void *w, int32_t rows, int32_t k, int32_t bias, int32_t six);
void or_matmul(float *y, const int8_t *xq, const float *xs, const void *w, const float *ws, int32_t m, int32_t rows,
               int32_t k, int32_t bias, int32_t six);
void or_rmsnorm(float *out, const float *x, const float *w, int32_t n, float eps);
void or_rope(float *v, const float *fcr, const float *fci, int32_t nh, int32_t hs, int32_t rot);
void or_attention(float *out, const float *q, const void *kc, const void *vc, float *att, int32_t pos, int32_t nh,
                  int32_t nkv, int32_t hs, int32_t h0, int32_t h1, int32_t half);
void or_to_f16(uint16_t *out, const float *x, int32_t n);
void or_from_f16(float *out, const uint16_t *x, int32_t n);
float or_fexp(float x);
void or_vexp(float *x, int32_t n);
void or_swiglu(float *out, const float *h1, const float *h3, int32_t n);
void or_layernorm(float *out, const float *x, const float *w, const float *b, int32_t n);
void or_gelu(float *out, const float *x, const float *b, int32_t n);
void or_add_columns(float *y, const float *rows, const float *a, int32_t count, int32_t n);
void or_add(float *x, const float *y, int32_t n);
int32_t or_argmax(const float *x, int32_t n);
void or_penalize(float *logits, const int32_t *tokens, int32_t count, float penalty);
int32_t or_sample(const float *logits, int32_t n, float temperature, float topp, double random, float *probs,
                  int32_t *index, int32_t *order);

/* ---- the checkpoint ---- */
int64_t or_places(const he_config *cfg, he_tensor *tensors);
void or_synth_checkpoint(const he_config *cfg, const he_tensor *tensors, uint8_t *out, int64_t size, uint64_t seed);
void or_rope_tables(float *cos_out, float *sin_out, int32_t seq_len, int32_t hs, double theta);

/* ---- the forward pass: public/forward.js createForward + run() ---- */
typedef struct or_model or_model;
or_model *or_model_open(const he_config *cfg, const he_tensor *tensors, const uint8_t *checkpoint,
                        const float *rope_cos, const float *rope_sin, int32_t max_block);
int32_t or_model_run(or_model *m, const int32_t *tokens, int32_t count, int32_t pos0, int32_t need_logits);
const float *or_model_logits(const or_model *m);
void or_model_kv(const or_model *m, int32_t from, int32_t count, float *keys, float *values);
void or_model_close(or_model *m);
int32_t or_generate(or_model *m, const int32_t *prompt, int32_t n_prompt, int32_t steps, int32_t block,
                    int32_t *out_tokens, float *last_logits);
void or_abi_layout(int64_t *out);
void or_set_threads(int32_t n);
int32_t or_get_threads(void);

#ifdef __cplusplus
}
#endif

#endif
