// Runs the JavaScript host (pyodide-llm_amd/forward_hip.mjs) the way Llama.generate() drives forward.js
// (public/llama2_numpy.py:1586-1612): the checkpoint written into weightsMemory(), external().start(plan), the prompt
// [BOS] + prompt[:-1] through forwardMany, then greedy steps and two sampled ones through generateMany; and a second
// engine fed one token at a time through forward() with a bound logits array. Writes what it got for the test to
// compare with the oracle.
//
//     node tests/node/run_engine.mjs job.json
import fs from "fs";
import path from "path";
import { createRequire } from "module";
import * as F from "../../pyodide-llm_amd/forward_hip.mjs";

const addon = createRequire(import.meta.url)("../../pyodide-llm_amd/hip_engine.node");

const job = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
const dir = path.dirname(process.argv[2]);
const read = (name) => fs.readFileSync(path.join(dir, name));
const write = (name, array) => fs.writeFileSync(path.join(dir, name), Buffer.from(array.buffer, array.byteOffset, array.byteLength));

const { memory, base } = F.weightsMemory(job.size);
new Uint8Array(memory.buffer, base, job.size).set(read("checkpoint.bin"));
const kernels = F.compileKernels(null, job.relaxed ? new Uint8Array(8) : null);
const plan = { ...job.plan, derived: { freq_cis_real: read("cos.bin"), freq_cis_imag: read("sin.bin") } };
const outside = F.external({ memory, base, size: job.size, kernels });
const header = outside.read(0, 28);
const engine = outside.start(plan);
const bound = new Float32Array(plan.vocab_size);
engine.bind(bound);

const prompt = job.prompt, P = prompt.length;
engine.forwardMany([1, ...prompt.slice(0, P - 1)], 0);
const ids = [];
let token = prompt[P - 1], pos = P;
while (pos < job.steps) {
  const got = engine.generateMany(token, pos, [], 0, Math.min(engine.tokenBlock, job.steps - pos), 0, 0.9, 1, [], []);
  if (got === undefined) throw new Error(`generateMany refused at ${pos}`);
  ids.push(...got);
  token = got[got.length - 1];
  pos += got.length;
}
write("greedy_logits.bin", engine.logits());
write("bound_logits.bin", bound);
const kv = engine.keysAndValues(0, job.steps);
write("keys.bin", kv.keys);
write("values.bin", kv.values);
// two sampled steps (temperature 0.8, top-p 0.9, penalty 1.3 over the last 64 of the history), as generate() asks them
const history = [1, ...prompt, ...ids];
const sampled = engine.generateMany(token, pos, history.slice(-64), history.length, 2, 0.8, 0.9, 1.3, [0.5, 0.25], []);
const memoryBytes = engine.memoryBytes();
const footprint = F.footprint(Array.from(new Int32Array(header.buffer, header.byteOffset, 7)), job.size,
  { relaxed: job.relaxed, halfKV: !!plan.half_kv, promptBlock: engine.promptBlock });

// one token at a time through forward(), the logits of the last into the bound array
const second = outside.start(plan);
const one = new Float32Array(plan.vocab_size);
second.bind(one);
const fed = [1, ...prompt.slice(0, P - 1)];
fed.forEach((t, i) => second.forward(t, i, false));
second.forward(prompt[P - 1], P, true);
write("forward_logits.bin", one);
let threw = "";
try {
  second.forward(0, plan.seq_len, true);
} catch (e) {
  threw = e.message;
}

// the addon itself refuses output arrays shorter than what it would write (a TypeError, nothing written)
const { config, tensors } = F.planToConfig(plan, { relaxedKernels: job.relaxed });
const f32 = (bytes) => new Float32Array(Uint8Array.from(bytes).buffer);  // a copy of exactly the file's floats
const raw = addon.open(config, tensors, memory.buffer, base, job.size, f32(read("cos.bin")), f32(read("sin.bin")), 16);
const kvDim = config.n_kv_heads * config.head_size;
const short = [];
const refuses = (what, call) => {
  try {
    call();
    short.push(`${what}: no error`);
  } catch (e) {
    short.push(e instanceof TypeError ? "TypeError" : `${what}: ${e.message}`);
  }
};
refuses("forward", () => addon.forward(raw, 1, 0, true, new Float32Array(plan.vocab_size - 1)));
refuses("logits", () => addon.logits(raw, new Float32Array(plan.vocab_size - 1)));
refuses("kvRead keys", () => addon.kvRead(raw, 0, 1, new Float32Array(config.n_layers * kvDim - 1),
  new Float32Array(config.n_layers * kvDim)));
refuses("kvRead values", () => addon.kvRead(raw, 0, 2, new Float32Array(2 * config.n_layers * kvDim),
  new Float32Array(2 * config.n_layers * kvDim - 1)));
addon.close(raw);

Promise.all([engine.release(), second.release()]).then((released) => {
  console.log(JSON.stringify({ ids, backend: engine.backend, promptBlock: engine.promptBlock, tokenBlock: engine.tokenBlock,
    memoryBytes, footprint, sampled: sampled === undefined ? null : Array.from(sampled), released, threw, short,
    header: Array.from(header) }));
});
