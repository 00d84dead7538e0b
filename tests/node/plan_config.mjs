// Prints, as JSON, what the JavaScript host makes of plans (planToConfig) and of its small exports, for the CPU tests:
//     node tests/node/plan_config.mjs plans.json
import fs from "fs";
import * as F from "../../pyodide-llm_amd/forward_hip.mjs";

const plans = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
const out = { exports: Object.keys(F).sort(), configs: [], refused: [] };
for (const plan of plans.take) out.configs.push(F.planToConfig(plan, plan._options || {}));
for (const plan of plans.refuse) {
  try {
    F.planToConfig(plan);
    out.refused.push(null);
  } catch (e) {
    out.refused.push(e.message);
  }
}
out.kernels = [F.compileKernels(null, null).relaxed, F.compileKernels(null, new Uint8Array(1)).relaxed];
out.keysInHalf = [F.keysInHalf([288, 768, 6, 6, 6, 32000, 256], 0, { halfKV: true }),
  F.keysInHalf([4096, 14336, 32, 32, 8, -128256, 4096], 0, { halfKV: true })];
const { memory, base } = F.weightsMemory(1000);
out.memory = [memory.buffer.byteLength, base];
console.log(JSON.stringify(out));
