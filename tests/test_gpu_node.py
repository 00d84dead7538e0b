"""The JavaScript host on the GPU: Node drives pyodide-llm_amd/forward_hip.mjs (over hip_engine.node and the C ABI)
the way Llama.generate() drives forward.js, and everything it gets is the oracle's to the bit: greedy tokens, the logits
of forward() in the bound array, the last step's logits, the KV cache, and two sampled steps."""
import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

import oracle_lib as ol
from paths import REPO
from plans import plan_of

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="no node here")]

CASES = {
    "tiny_gqa": (dict(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2, head_size=16, vocab_size=320,
                      seq_len=64, shared_classifier=1), 10000.0, 12, 40),
    "tiny_qwen_int6_plain": (dict(dim=128, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=1, head_size=32,
                                  vocab_size=288, seq_len=64, shared_classifier=0, six=1, qkv_bias=1, relaxed=0),
                             1000000.0, 9, 30),
    "stories15m_f16": (dict(dim=288, hidden_dim=768, n_layers=6, n_heads=6, n_kv_heads=6, head_size=48,
                            vocab_size=32000, seq_len=256, shared_classifier=1, half_kv=1), 10000.0, 32, 96),
}


def nucleus_size(logits, temperature, topp):
    """how many tokens the nucleus sort takes (float64 NumPy: the cases here lie far from the device's 8192)"""
    best = float(logits.max())
    kept = logits[logits >= best - temperature * 16.118095].astype(np.float64)
    p = np.exp((kept - best) / temperature)
    return int((p >= min((1 - topp) / max(p.size - 1, 1) * p.sum(), p.max())).sum())


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", sorted(CASES))
def test_node_host_matches_the_oracle(name, tmp_path):
    fields, theta, prompt_len, steps = CASES[name]
    cfg = ol.config(**fields)
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=3)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, theta)
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg.vocab_size, size=prompt_len)]
    ck.tofile(tmp_path / "checkpoint.bin")
    np.asarray(cos, np.float32).tofile(tmp_path / "cos.bin")
    np.asarray(sin, np.float32).tofile(tmp_path / "sin.bin")
    job = {"size": int(size), "plan": plan_of(cfg, tensors), "prompt": prompt, "steps": steps,
           "relaxed": bool(cfg.relaxed)}
    (tmp_path / "job.json").write_text(json.dumps(job))
    print(f"node host: {name}", flush=True)
    sys.stdout.flush()
    proc = subprocess.run(["node", os.path.join(REPO, "tests", "node", "run_engine.mjs"), str(tmp_path / "job.json")],
                          stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-3000:]
    out = json.loads(proc.stdout.strip().splitlines()[-1])

    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    want, want_logits = ref.generate(prompt, steps)
    assert out["ids"] == [int(t) for t in want]
    got = np.fromfile(tmp_path / "greedy_logits.bin", dtype=np.float32)
    assert np.array_equal(bits(got), bits(want_logits))
    assert np.array_equal(bits(np.fromfile(tmp_path / "bound_logits.bin", dtype=np.float32)), bits(want_logits))
    k, v = ref.kv(0, steps)
    assert np.array_equal(bits(np.fromfile(tmp_path / "keys.bin", dtype=np.float32)), bits(k.reshape(-1)))
    assert np.array_equal(bits(np.fromfile(tmp_path / "values.bin", dtype=np.float32)), bits(v.reshape(-1)))

    one = ol.Model(cfg, tensors, ck, cos, sin, max_block=1)
    for i, t in enumerate([1] + prompt[:-1]):
        one.run([t], i, False)
    one.run([prompt[-1]], prompt_len, True)
    got = np.fromfile(tmp_path / "forward_logits.bin", dtype=np.float32)
    assert np.array_equal(bits(got), bits(one.logits()))

    # the two sampled steps: the oracle's penalty over the last 64 of [BOS, prompt, ids], its draw for 0.5 then 0.25
    # (undefined where the nucleus is larger than the device sorts: the caller takes the step)
    history = [1] + prompt + [int(t) for t in want]
    expect, token = [], int(want[-1])
    for i, u in enumerate((0.5, 0.25)):
        ref.run([token], steps + i, True)
        logits = ol.penalize(ref.logits(), set(history[-64:]), 1.3)
        if nucleus_size(logits, 0.8, 0.9) > 8192:
            expect = None if i == 0 else expect
            break
        token = ol.sample(logits, 0.8, 0.9, u)
        expect.append(token)
        history.append(token)
    assert out["sampled"] == expect
    assert out["released"] == [True, True]
    assert "context" in out["threw"]  # a position past seq_len throws, as forward.js does
    assert out["short"] == ["TypeError"] * 4  # the addon refuses output arrays shorter than it writes
    assert out["header"] == list(ck[:28])
    assert out["memoryBytes"] > size
    # footprint() (public/forward.js:270) bounds what the engine holds besides the checkpoint, to within 2 MiB
    assert size + out["footprint"] >= out["memoryBytes"] > size + out["footprint"] - (2 << 20)
