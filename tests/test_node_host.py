"""The JavaScript host (pyodide-llm_amd/forward_hip.mjs over hip_engine.node) without a GPU: the module loads with its
addon, exports forward.js's names, and turns the reference's plans into the same engine config as the Python host,
refusing the same forms."""
import json
import os
import shutil
import subprocess

import pytest

from paths import REPO, package
from plans import plan_of
import oracle_lib as ol

NODE = shutil.which("node")
pytestmark = pytest.mark.skipif(NODE is None, reason="no node here")


def run_node(script, *args):
    proc = subprocess.run([NODE, os.path.join(REPO, "tests", "node", script), *args], stdout=subprocess.PIPE,
                          stderr=subprocess.PIPE, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    return json.loads(proc.stdout.strip().splitlines()[-1])


def golden_plans():
    with open(os.path.join(REPO, "tests", "golden", "plans.json")) as f:
        golden = json.load(f)
    out = []
    for name, g in golden.items():
        dim, hidden, layers, heads, kv_heads, vocab, seq_len = g["header"]
        plan = {"arch": "llama", "dim": dim, "hidden_dim": hidden, "n_layers": layers, "n_heads": heads,
                "n_kv_heads": kv_heads, "head_size": dim // heads, "vocab_size": abs(vocab), "seq_len": seq_len,
                "rotary": 0, "parallel_residual": False, "kv_start": 256, "rms_norm_eps": 1e-5,
                "shared_classifier": vocab > 0, "int8": True, "relaxed": True, "tensors": g["tensors"],
                "outliers": [], "half_kv": True, "form": {}}
        out.append(plan)
    return out


def test_module_exports_and_plan_conversion_match_the_python_host(tmp_path):
    pk = package()
    take = golden_plans()
    cfg = ol.config(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2, head_size=16, vocab_size=320,
                    seq_len=48, shared_classifier=0, six=1, qkv_bias=1, relaxed=0, half_kv=1)
    tensors, _ = ol.places(cfg)
    take.append(plan_of(cfg, tensors))
    base = take[-1]
    norms = {name: {"kind": "f32", "offset": 1000 + i, "shape": [2, 16], "group": 0, "scales": 0}
             for i, name in enumerate(("q_norm", "k_norm"))}
    positions = dict(base["tensors"]["wq"], offset=7000, scales=7500)
    take += [{**base, "outliers": [40, 3, 17]}, {**base, "tensors": {**base["tensors"], **norms}},
             {**base, "arch": "gpt2", "tensors": {**base["tensors"], "positions": positions}},
             {**base, "arch": "neox", "rotary": 8, "parallel_residual": True}]
    refuse = [{**base, "arch": "qwen35"}, {**base, "outliers": list(range(9))}, {**base, "int8": False},
              {**base, "rotary": 8}]
    job = tmp_path / "plans.json"
    job.write_text(json.dumps({"take": take, "refuse": refuse}))
    out = run_node("plan_config.mjs", str(job))
    for name in ("external", "createForward", "compileKernels", "weightsMemory", "footprint", "keysInHalf",
                 "needsWide", "BATCH", "GPU_BLOCK"):
        assert name in out["exports"], name
    for plan, js in zip(take, out["configs"]):
        c, t = pk.plan_to_config(plan)
        for field, _ in c._fields_:
            want = getattr(c, field)
            if field == "n_outliers":
                assert len(js["config"]["outliers"]) == want
            elif field == "outliers":
                assert js["config"]["outliers"] == list(want)[:c.n_outliers]
            else:
                assert js["config"][field] == pytest.approx(want, rel=1e-7), (field, plan["dim"])
        assert [list(p) for p in js["tensors"]] == [[t[i].offset, t[i].scales] for i in range(len(t))]
    assert all(message for message in out["refused"]), out["refused"]
    assert out["kernels"] == [None, True]
    assert out["keysInHalf"] == [True, False]
    assert out["memory"] == [1064, 64]
