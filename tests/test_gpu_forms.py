"""The engine's other forms against the oracle, to the bit: GPT-2 (LayerNorm, learned positions, GELU, biases after every
matrix), GPT-NeoX (partial RoPE, parallel residual), Qwen3 (q/k head norms, heads wider than dim / n_heads) and the
outlier channels of the classifier's input (public/forward.js:1011-1090, 801-812). Every token's logits and the KV
cache, prompt blocks then greedy steps (replayed from the captured step graph: GPT-2's position row comes from device
memory there), sampled steps, and the device-made checkpoint, on tiny models and on larger shapes of each form."""
import ctypes

import numpy as np
import pytest

import oracle_lib as ol
from forms import FORM_TINY, form_model
from paths import package

pytestmark = pytest.mark.gpu

LARGER = {
    # name: (he_config fields, rope theta, outlier channels of the final norm)
    "gpt2_small_shape": (dict(dim=768, hidden_dim=3072, n_layers=2, n_heads=12, n_kv_heads=12, head_size=64,
                              vocab_size=50257, seq_len=96, shared_classifier=1, arch=1), 10000.0, {5: 9.0, 700: -8.0}),
    "neox_parallel": (dict(dim=512, hidden_dim=2048, n_layers=2, n_heads=8, n_kv_heads=8, head_size=64,
                           vocab_size=4096, seq_len=96, shared_classifier=0, arch=2, rotary=16, parallel_residual=1),
                      10000.0, {}),
    "qwen3_0p6b_shape": (dict(dim=1024, hidden_dim=3072, n_layers=2, n_heads=16, n_kv_heads=8, head_size=128,
                              vocab_size=8192, seq_len=96, shared_classifier=1, qk_norm=1, rms_norm_eps=1e-6),
                         1000000.0, {}),
}


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def larger(name, **extra):
    fields, theta, outliers = LARGER[name]
    cfg = ol.config(**fields)
    tensors, size = ol.places(cfg)
    ck = ol.vary_vectors(cfg, tensors, ol.synth_checkpoint(cfg, tensors, size, seed=9), seed=13)
    final = tensors[package().T["rms_final_weight"]].offset
    for channel, value in outliers.items():
        ck[final + 4 * channel:final + 4 * channel + 4] = np.frombuffer(np.float32(value).tobytes(), dtype=np.uint8)
    weight = np.frombuffer(ck.tobytes(), dtype=np.float32, count=cfg.dim, offset=final)
    cfg = ol.config(**{**fields, **extra, "outliers": ol.outlier_channels(weight)})
    cos, sin = package().rope_tables(cfg.seq_len, cfg.head_size, theta, cfg.rotary if cfg.arch == 2 else 0)
    return cfg, tensors, ck, cos, sin


def model(name, **extra):
    if name in FORM_TINY:
        return form_model(name, **extra)[:5]
    return larger(name, **extra)


@pytest.mark.parametrize("name", sorted(FORM_TINY))
@pytest.mark.parametrize("relaxed", [1, 0])
@pytest.mark.parametrize("half_kv", [0, 1])
def test_forward_logits_and_cache_bits(name, relaxed, half_kv):
    cfg, tensors, ck, cos, sin = model(name, relaxed=relaxed, half_kv=half_kv)
    print(f"forms: forward {name} relaxed={relaxed} half_kv={half_kv} outliers={cfg.n_outliers}", flush=True)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=64)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    tokens = np.random.default_rng(5).integers(0, cfg.vocab_size, size=12)
    for pos, tok in enumerate(tokens):
        ref.run([int(tok)], pos, True)
        eng.forward(int(tok), pos, True)
        assert same_bits(eng.logits(), ref.logits()), pos
    k_ref, v_ref = ref.kv(0, len(tokens))
    kv = eng.keysAndValues(0, len(tokens))
    assert same_bits(kv["keys"], k_ref.reshape(-1)) and same_bits(kv["values"], v_ref.reshape(-1))
    eng.release()


@pytest.mark.parametrize("name", sorted(FORM_TINY) + sorted(LARGER))
def test_prompt_blocks_then_greedy_steps(name):
    """[BOS] + prompt[:-1] through forwardMany, then greedy steps through generateMany (the replayed step graph after
    its first step), against the oracle's generate(); the last logits and the cache to the bit"""
    cfg, tensors, ck, cos, sin = model(name)
    prompt_len = 40 if name in LARGER else 14
    steps = min(cfg.seq_len, prompt_len + 40)
    print(f"forms: greedy {name} prompt={prompt_len} steps={steps} outliers={cfg.n_outliers}", flush=True)
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, cfg.vocab_size, size=prompt_len)]
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    want, want_logits = ref.generate(prompt, steps)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany([1] + prompt[:-1], 0)
    got, token, pos = [], prompt[-1], prompt_len
    while pos < steps:
        ids = eng.generateMany(token, pos, [], 0, min(16, steps - pos), 0.0, 0.9, 1.0, [], [])
        got += ids
        token, pos = ids[-1], pos + len(ids)
    assert got == [int(t) for t in want]
    assert same_bits(eng.logits(), want_logits)
    k_ref, v_ref = ref.kv(0, steps)
    kv = eng.keysAndValues(0, steps)
    assert same_bits(kv["keys"], k_ref.reshape(-1)) and same_bits(kv["values"], v_ref.reshape(-1))
    eng.release()


@pytest.mark.parametrize("name", sorted(FORM_TINY))
def test_sampled_steps(name):
    """temperature 0.8, top-p 0.9, penalty 1.3 over the latest 64 of the history: generateMany's draws against the
    oracle's forward, or_penalize and or_sample with the same random numbers"""
    cfg, tensors, ck, cos, sin = model(name)
    print(f"forms: sampled {name}", flush=True)
    rng = np.random.default_rng(21)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=10)]
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    ref.run([1] + prompt[:-1], 0, False)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany([1] + prompt[:-1], 0)
    history, token, pos = [1] + prompt, prompt[-1], len(prompt)
    while pos < cfg.seq_len:
        count = min(8, cfg.seq_len - pos)
        randoms = list(rng.random(count))
        got = eng.generateMany(token, pos, history[-64:], len(history), count, 0.8, 0.9, 1.3, randoms, [])
        assert got is not None and len(got) == count  # tiny vocabularies: every nucleus fits the device's sort
        for i, t in enumerate(got):
            ref.run([token], pos, True)
            want = ol.sample(ol.penalize(ref.logits(), set(history[-64:]), 1.3), 0.8, 0.9, randoms[i])
            assert t == want, (pos, i)
            history.append(t)
            token, pos = t, pos + 1
    eng.release()


@pytest.mark.parametrize("name", sorted(LARGER))
def test_device_checkpoint_equals_host_checkpoint(name):
    fields, theta, _ = LARGER[name]
    cfg = ol.config(**fields)
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=7)
    cos, sin = package().rope_tables(cfg.seq_len, cfg.head_size, theta, cfg.rotary if cfg.arch == 2 else 0)
    print(f"forms: device checkpoint {name}", flush=True)
    pk = package()
    eng = pk.open_synthetic(cfg, tensors, size, 7, cos, sin, max_block=8)
    out = np.zeros(size, dtype=np.uint8)
    pk.hip_engine.check(pk.library().he_checkpoint_read(eng._h, 0, size, ctypes.c_void_p(out.ctypes.data)))
    assert np.array_equal(out, ck)
    eng.release()
