// decode_bench.mjs — greedy decode timed through the JavaScript host (forward_hip.mjs over hip_engine.node), the
// way tests/profile.mjs times the reference's engine in Node: a synthetic checkpoint made on the device, the prompt
// [BOS] + prompt[:-1] through forwardMany, then warmup + steps greedy tokens through generateMany (each call returns
// its ids, so the clock stops when the device is done). Prints one JSON line: prompt tokens/s, decode tokens/s and
// the ids, which a caller can hold against another host's run of the same seed and prompt.
//
//     node pyodide-llm_amd/decode_bench.mjs job.json
//
// job.json: {plan (without derived), size, seed, prompt: [ids], warmup, steps, promptBlock}; cos.bin and sin.bin
// (the RoPE tables, float32) beside it.
import fs from "fs";
import path from "path";
import { performance } from "perf_hooks";
import { syntheticForward } from "./forward_hip.mjs";

const jobPath = process.argv[2];
const job = JSON.parse(fs.readFileSync(jobPath, "utf8"));
const dir = path.dirname(jobPath);
const table = (name) => new Float32Array(new Uint8Array(fs.readFileSync(path.join(dir, name))).buffer);
const plan = { ...job.plan, derived: { freq_cis_real: table("cos.bin"), freq_cis_imag: table("sin.bin") } };

const opened = performance.now();
const engine = syntheticForward({ plan, size: job.size, seed: job.seed, promptBlock: job.promptBlock });
const setupMs = performance.now() - opened;

const prompt = job.prompt, P = prompt.length;
let began = performance.now();
engine.forwardMany([1, ...prompt.slice(0, P - 1)], 0);
const prefillMs = performance.now() - began;

const ids = [];
let token = prompt[P - 1], pos = P;
function decode(n) {
  for (let done = 0; done < n;) {
    const got = engine.generateMany(token, pos, [], 0, Math.min(engine.tokenBlock, n - done), 0, 0.9, 1, [], []);
    if (got === undefined) throw new Error(`generateMany refused the step at ${pos}`);
    ids.push(...got);
    token = got[got.length - 1];
    pos += got.length;
    done += got.length;
  }
}
decode(job.warmup);
began = performance.now();
decode(job.steps);
const decodeMs = performance.now() - began;
engine.release();
console.log(JSON.stringify({
  prefill_tok_s: P / (prefillMs / 1000), decode_tok_s: job.steps / (decodeMs / 1000),
  ms_per_step: decodeMs / job.steps, setup_ms: setupMs, ids,
}));
