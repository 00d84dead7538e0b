// forward_hip.mjs — the JavaScript host of the MI355X forward engine: the interface public/forward.js gives its
// Python caller (Llama(external=...), public/llama2_numpy.py:1248-1298), over the N-API addon hip_engine.node and the
// C ABI of include/pyodide_llm_hip.h.
//
// A caller of forward.js switches by importing this module instead: external({memory, base, size, kernels}) returns
// {size, read, start(plan)} (public/forward.js:571-590), and start(plan) returns the engine object with bind, forward,
// forwardMany, promptBlock, tokenBlock, generateMany, logits, keysAndValues, memoryBytes and release
// (public/forward.js:1676-1955). The arithmetic is the reference's CPU path to the bit (int8 activations, exact int32
// group sums, the float32 order of kernels/kernel_relaxed.ts and kernels/kernel.ts) on the GPU. There is no CPU path
// here: without the built addon (or without a GPU) the import or start() throws.
//
// Node 12 or later (ES modules, BigInt, N-API 8); no top-level await.
import { createRequire } from "module";

const require = createRequire(import.meta.url);
const addon = require("./hip_engine.node");

// public/jobs.js:22 (the CPU's prompt block) and public/forward.js:33 (a GPU's): the constants callers read
export const BATCH = 16;
export const GPU_BLOCK = 64;
// the tokens one forwardMany call takes here: the whole prompt block goes through each matrix at once
export const PROMPT_BLOCK = 512;
// the steps one generateMany call takes (greedy steps replayed from one captured step; sampled ones a step at a time)
export const TOKEN_BLOCK = 16;
// include/pyodide_llm_hip.h HE_T_*: the tensors the forward reads, by their plan names
const TENSORS = ["token_embedding_table", "rms_att_weight", "wq", "wk", "wv", "wo", "rms_ffn_weight", "w1", "w2", "w3",
  "rms_final_weight", "wcls", "bq", "bk", "bv", "q_norm", "k_norm", "positions", "ln_att_bias", "ln_ffn_bias",
  "ln_final_bias", "bo", "b1", "b2"];
// include/pyodide_llm_hip.h HE_ARCH_*, HE_OUTLIERS_MOST
const ARCHS = { llama: 0, gpt2: 1, neox: 2 };
const OUTLIERS_MOST = 8;
// include/pyodide_llm_hip.h HE_K_*
const KINDS = ["gemv", "gemm", "attention", "norm", "elementwise", "argmax"];

/** compileKernels (public/forward.js:226): the WASM modules of the CPU path are not used here; what stays is whether the
 * caller has the relaxed kernels (activations with bias 64 and matmul_q8r's order) or only the plain ones (bias 0,
 * matmul_q8's lanes), which decides the engine's arithmetic as it decides the reference's (public/forward.js:650-652). */
export function compileKernels(plain, relaxed, wide = false) {
  return { plain: or(plain, null), relaxed: relaxed ? true : null, wide: Boolean(wide), hip: true };
}

/** needsWide (public/forward.js:521): whether a checkpoint needs a 64-bit WebAssembly memory. The engine's weights are
 * in HBM and its host buffer is a plain ArrayBuffer: never. */
export const needsWide = (size, after) => false;

/** weightsMemory (public/forward.js:539): where the caller writes the checkpoint's bytes, at base. A plain
 * ArrayBuffer: the engine copies the bytes to the device at start(plan) and reads nothing else of it. */
export function weightsMemory(size, { shared = false } = {}) {
  const base = 64;
  const buffer = shared && typeof SharedArrayBuffer !== "undefined" ? new SharedArrayBuffer(base + size)
    : new ArrayBuffer(base + size);
  return { memory: { buffer }, base };
}

/** footprint (public/forward.js:270): the bytes the forward pass holds besides the checkpoint. Here they are device
 * bytes: the keys and values of the whole context (no growth steps), the RoPE tables, one pass's activations (up to
 * 1024 prompt tokens with relaxed matmuls, 16 without) and the scores of up to 512 of its tokens (the attention's
 * pieces), the logits and the sampler's buffers. header: [dim, hidden, layers, heads, kvHeads, signedVocab, seqLen] as the file's. */
export function footprint(header, size, { relaxed = true, halfKV = false, head_dim = 0, promptBlock = PROMPT_BLOCK } = {}) {
  const [dim, hidden, layers, heads, kvHeads, signedVocab, seqLen] = header;
  const vocab = Math.abs(signedVocab), headSize = head_dim || dim / heads;
  const kvDim = kvHeads * headSize, qDim = heads * headSize, wide = Math.max(dim, qDim, hidden);
  const half = halfKV && kvHeads >= heads;
  // keys by position, values by column (each column's positions rounded up to 64)
  const keys = layers * (seqLen + Math.ceil(seqLen / 64) * 64) * kvDim * (half ? 2 : 4);
  const chunk = Math.min(promptBlock, relaxed ? 1024 : 16), rows = Math.min(chunk, 512);
  const frames = chunk * (4 * (dim + Math.max(dim, qDim) + qDim + 2 * kvDim + 2 * hidden) + wide + wide / 8) +
    rows * 4 * heads * (seqLen + Math.floor(seqLen / 64) + 1);
  // the logits, the sampler's probabilities and indices; 1 MiB for the small buffers and the regions' alignment
  return keys + 2 * seqLen * headSize * 2 + frames + vocab * 12 + 2 ** 20;
}

/** keysInHalf (public/forward.js:326): float16 keys and values where every head has its own (a grouped-query model's
 * stay float32, as the reference keeps them where the model fits its memory) */
export const keysInHalf = (header, size, options = {}) => Boolean(options.halfKV) && header[4] >= header[3];

const or = (v, d) => (v === undefined || v === null ? d : v);
const fromJs = (x) => (x && x.toJs ? x.toJs({ dict_converter: Object.fromEntries }) : x);

function floats(bytes, count, name) {
  const b = fromJs(bytes);
  const u8 = b instanceof Uint8Array ? b : ArrayBuffer.isView(b) ? new Uint8Array(b.buffer, b.byteOffset, b.byteLength)
    : new Uint8Array(b);
  if (u8.byteLength < count * 4) throw new Error(`plan.derived.${name} holds ${u8.byteLength} bytes, not ${count * 4}`);
  // a copy of its own (a Node Buffer's slice() shares a larger pooled ArrayBuffer at some offset)
  const copy = new Uint8Array(count * 4);
  copy.set(u8.subarray(0, count * 4));
  return new Float32Array(copy.buffer);
}

/** The engine's config and tensor places from a plan (public/llama2_numpy.py:1261-1270): the llama form (Qwen2's
 * biases and Qwen3's head norms where the plan has those tensors), gpt2 and neox (public/forward.js:636). The forms the
 * engine does not run are refused by name, as public/forward.js refuses what its kernels cannot take. */
export function planToConfig(plan, { relaxedKernels = true, halfKeys } = {}) {
  const arch = or(plan.arch, "llama");
  if (!(arch in ARCHS)) throw new Error(`the HIP engine runs the llama, gpt2 and neox forms, not ${arch}`);
  if (!plan.int8) throw new Error("the HIP engine multiplies int8/int6 matrices only (plan.int8)");
  const T = plan.tensors, layerNorm = arch !== "llama";
  const names = ["wq", "wk", "wv", "wo", "w1", "w2", "token_embedding_table", ...(layerNorm ? [] : ["w3"]),
    ...(arch === "gpt2" ? ["positions"] : [])];
  const kinds = new Set(names.map((n) => T[n] && T[n].kind));
  if (kinds.size !== 1 || !(kinds.has("int8") || kinds.has("int6"))) {
    throw new Error(`the HIP engine takes int8 or int6 matrices, not ${[...kinds].join(", ")}`);
  }
  const rotary = Number(plan.rotary || 0);
  if (arch === "llama" && rotary && rotary !== plan.head_size) {
    throw new Error("partial rotary embeddings belong to the neox form");
  }
  const outliers = [...or(fromJs(plan.outliers), [])].map(Number).sort((a, b) => a - b);
  if (outliers.length > OUTLIERS_MOST) throw new Error(`at most ${OUTLIERS_MOST} outlier channels`);
  const heads = plan.n_heads, kvHeads = plan.n_kv_heads;
  const config = {
    dim: plan.dim, hidden_dim: plan.hidden_dim, n_layers: plan.n_layers, n_heads: heads, n_kv_heads: kvHeads,
    head_size: plan.head_size, vocab_size: plan.vocab_size, seq_len: plan.seq_len,
    shared_classifier: plan.shared_classifier ? 1 : 0, six: kinds.has("int6") ? 1 : 0, qkv_bias: T.bq ? 1 : 0,
    // public/forward.js:650-652: bias 64 where the plan and the kernels allow relaxed SIMD
    relaxed: plan.relaxed !== false && relaxedKernels ? 1 : 0,
    // public/forward.js:762
    half_kv: plan.half_kv && or(halfKeys, kvHeads >= heads) ? 1 : 0,
    rms_norm_eps: or(plan.rms_norm_eps, 1e-5),
    arch: ARCHS[arch], rotary: arch === "neox" ? rotary : 0,
    parallel_residual: layerNorm && plan.parallel_residual ? 1 : 0,
    qk_norm: T.q_norm && T.k_norm ? 1 : 0, outliers,
  };
  const tensors = TENSORS.map((name) => {
    const t = name === "wcls" && config.shared_classifier ? T.token_embedding_table : T[name];
    return t ? [Number(t.offset), Number(t.scales || 0)] : [0, 0];
  });
  return { config, tensors };
}

function engineObject(handle, config) {
  const vocab = config.vocab_size, kvDim = config.n_kv_heads * config.head_size, layers = config.n_layers;
  const logits = new Float32Array(vocab);
  let bound = null, haveLogits = false, live = true;
  const ids = new Int32Array(TOKEN_BLOCK);
  const toBound = () => {
    if (!bound) return;
    const view = bound.getBuffer ? bound.getBuffer("f32") : { data: bound, release() {} };
    view.data.set(logits);
    view.release();
  };
  const promptBlock = addon.promptBlock(handle);
  return {
    backend: `MI355X HIP kernels (gfx950), ${config.six ? "int6" : "int8"}${config.relaxed ? ", relaxed order" : ""}`,
    // the thread controls of the CPU path (public/forward.js:1677-1750) have nothing to do on one GPU
    async setThreads() { return 1; },
    async findThreads() { return 1; },
    newGeneration() {},
    get searching() { return false; },
    searchLog: [],
    get threads() { return 1; },
    stopThreads() {},
    get lostThreads() { return false; },
    gpu: Promise.resolve("MI355X (HIP)"),
    get gpuStatus() { return "MI355X (HIP)"; },
    get gpuReady() { return { matrices: "hip", attention: "hip" }; },
    get gpuWhyNot() { return null; },
    get gpuTokensWhyNot() { return null; },
    get gpuTokensPlanned() { return true; },
    get gpuTokens() { return 0; },
    get gpuSampled() { return 0; },
    /** the float32 array of the caller's that forward() fills with the logits (public/forward.js:1744-1746) */
    bind(array) {
      bound = array && array.copy ? array.copy() : array;
    },
    /** forwardMany (public/forward.js:1755-1769): tokens at pos, pos + 1, ... without logits; each token's numbers are
     * those forward() gives it alone */
    forwardMany(tokens, pos) {
      const list = Int32Array.from(fromJs(tokens));
      for (let at = 0; at < list.length; at += promptBlock) {
        addon.forwardMany(handle, list.subarray(at, at + promptBlock), pos + at);
      }
    },
    get promptBlock() { return promptBlock; },
    get tokenBlock() { return TOKEN_BLOCK; },
    /** generateMany (public/forward.js:1837-1890): count steps on the device, each the forward pass, the repetition
     * penalty over history (the latest 64 of the generation's tokens, then the ids chosen; where penalty != 1) and the
     * choice of the next token: the first index of the largest logit (temperature 0, kernels/kernel.ts:695-699) or a
     * draw with randoms[i] (kernels/kernel.ts:803-868). Returns the ids (a stop token last). undefined where the engine
     * does not take the first step: more steps than tokenBlock, too few random numbers, a nucleus larger than the
     * device sorts (8192 tokens), or logits that are not finite (the caller's own step then stops on NOT_FINITE) */
    generateMany(token, pos, history, length, count, temperature, topp, penalty, randoms, stops) {
      if (!(count >= 1 && count <= TOKEN_BLOCK)) return undefined;
      const t = Number(or(temperature, 0)), p = Number(or(penalty, 1));
      const draws = Float64Array.from(or(fromJs(randoms), []));
      if (t !== 0 && draws.length < count) return undefined;
      const past = Int32Array.from(or(fromJs(history), []));
      const stopList = Int32Array.from(or(fromJs(stops), []));
      const got = addon.generateMany(handle, token, pos, past, Number(or(length, past.length)), count, t,
        Number(or(topp, 0.9)), p, draws, stopList, ids);
      // -1: a largest logit that is not finite; 0: the engine did not take the first step (its nucleus is larger than
      // the device sorts): the caller takes the step, as the reference's undefined says
      if (got <= 0) return undefined;
      addon.logits(handle, logits);
      haveLogits = true;
      toBound();
      return Array.from(ids.subarray(0, got));
    },
    forward(token, pos, needLogits = true) {
      addon.forward(handle, token, pos, Boolean(needLogits), needLogits ? logits : null);
      if (!needLogits) return;
      haveLogits = true;
      toBound();
    },
    /** the logits of the last step with logits (tests) */
    logits() {
      if (!haveLogits) addon.logits(handle, logits);
      return logits;
    },
    /** the cache at positions from .. from + count - 1 as float32 [layers][count][kvDim] each
     * (public/forward.js:1939-1953) */
    keysAndValues(from, count) {
      const keys = new Float32Array(layers * count * kvDim), values = new Float32Array(layers * count * kvDim);
      addon.kvRead(handle, from, count, keys, values);
      return { keys, values };
    },
    memoryBytes: () => addon.deviceBytes(handle),
    /** one forward step timed by kind of kernel: {kind: [ms, algorithmic bytes, launches]} */
    profile(token, pos, needLogits = true) {
      const ms = new Float64Array(KINDS.length), bytes = new Float64Array(KINDS.length);
      const launches = new Int32Array(KINDS.length);
      addon.profile(handle, token, pos, Boolean(needLogits), ms, bytes, launches);
      return Object.fromEntries(KINDS.map((k, i) => [k, [ms[i], bytes[i], launches[i]]]));
    },
    /** frees the device memory (public/forward.js:1918-1935); resolves to true */
    release() {
      if (bound && bound.destroy) bound.destroy();
      bound = null;
      if (live) addon.close(handle);
      live = false;
      return Promise.resolve(true);
    },
  };
}

function ropeOf(plan, config) {
  const derived = or(plan.derived, {});
  if (!derived.freq_cis_real || !derived.freq_cis_imag) {
    throw new Error("the HIP engine takes the RoPE tables from plan.derived (freq_cis_real, freq_cis_imag)");
  }
  const count = config.seq_len * (config.head_size / 2);
  return [floats(derived.freq_cis_real, count, "freq_cis_real"), floats(derived.freq_cis_imag, count, "freq_cis_imag")];
}

/** createForward (public/forward.js:626): the engine for a plan over a checkpoint of size bytes at base of memory */
export function createForward({ memory, base, size, kernels, plan, halfKeys, promptBlock = PROMPT_BLOCK }) {
  plan = fromJs(plan);
  const { config, tensors } = planToConfig(plan, { relaxedKernels: !kernels || Boolean(kernels.relaxed), halfKeys });
  const [cos, sin] = ropeOf(plan, config);
  const handle = addon.open(config, tensors, memory.buffer, base, size, cos, sin, promptBlock);
  return engineObject(handle, config);
}

/** The engine over a checkpoint made on the device from a seed (weights N(0, 0.02) quantized by the reference's rules,
 * norm weights 1.0) instead of uploaded: for measurements of models too large to make on the host. plan.tensors must
 * place every tensor as the file would (public/llama2_numpy.py:778-795, external_tensors). */
export function syntheticForward({ plan, size, seed = 0, halfKeys, promptBlock = PROMPT_BLOCK }) {
  plan = fromJs(plan);
  const { config, tensors } = planToConfig(plan, { halfKeys });
  const [cos, sin] = ropeOf(plan, config);
  const handle = addon.openSynthetic(config, tensors, size, BigInt(seed), cos, sin, promptBlock);
  return engineObject(handle, config);
}

/** external (public/forward.js:571-590): what Llama(external=) takes: the checkpoint's size, read() for the bytes
 * Python looks at itself, and start(plan), which makes the engine */
export function external({ memory, base, size, kernels, halfKeys, promptBlock }) {
  const outside = {
    size,
    read: (offset, length) => new Uint8Array(memory.buffer, base + offset, length).slice(),
    start: (plan) => {
      outside.engine = createForward({ memory, base, size, kernels, plan, halfKeys, promptBlock });
      return outside.engine;
    },
  };
  return outside;
}
