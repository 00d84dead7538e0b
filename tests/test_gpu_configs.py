"""The engine at the widths of the workloads it is measured on, against the oracle to the bit.

- Llama-3-8B shape (hidden 4096, 32 q / 8 kv heads of 128, SwiGLU 14336, vocab 128256, theta 5e5, float32 cache):
  two of its layers against the oracle over a 2048-token prompt and 256 replayed greedy steps (every step's token,
  the last logits, the cache), with the L2 fills ahead of the q/k/v, w1/w3 and classifier GEMVs on; all 32 layers
  against the engine itself: the device-made checkpoint's tensors equal the host's synthesis, the 2048-token prompt
  through the MFMA GEMM equals one token at a time through the GEMV, replayed steps equal eager ones.
- Qwen2.5-7B shape, int6 (hidden 3584, 28 q / 4 kv heads, q/k/v biases, SwiGLU 18944, vocab 152064): two layers
  against the oracle over a 1024-token prompt and 256 greedy steps; all 28 layers against the engine itself.
- Both whole models (all 32 / 28 layers) against the oracle too: a 128-token prompt and 32 replayed greedy steps, so
  that every tensor of the checkpoint, past 2 GiB and up to the classifier near its end, is checked to the bit.
- The 150M shape (hidden 512, 12 layers, 8 heads, SwiGLU 2048, vocab 99487, float16 cache): the whole model against
  the oracle, a 512-token prompt and 256 greedy steps.
- A Llama form wider than 1024 (the width where rmsnorm runs as its own launch and carries the L2 fills) with no,
  part and all of the fills.

The prompt goes in as generate() feeds it ([BOS] + prompt[:-1] through forwardMany, public/llama2_numpy.py:1580-1606)
and the oracle's or_generate runs the same steps (stop tokens off). The reference holds prompt blocks equal to one
token at a time at full model size (tests/forward-check.mjs:422-462); these are its counterparts at these widths.
The checkpoints of the wide models come from the device's synthesis (read back with he_checkpoint_read, its bytes
checked against the host's for sampled tensors) with the norm weights and biases varied, so that a dropped or
misplaced one shows; the engine under test opens those bytes through he_open like any caller's file."""
import ctypes

import numpy as np
import pytest

import oracle_lib as ol
from paths import package

pytestmark = pytest.mark.gpu

LLAMA3_8B = dict(dim=4096, hidden_dim=14336, n_layers=32, n_heads=32, n_kv_heads=8, head_size=128, vocab_size=128256,
                 seq_len=4096, shared_classifier=0, half_kv=0)
QWEN25_7B_INT6 = dict(dim=3584, hidden_dim=18944, n_layers=28, n_heads=28, n_kv_heads=4, head_size=128,
                      vocab_size=152064, seq_len=2048, shared_classifier=0, six=1, qkv_bias=1, half_kv=0,
                      rms_norm_eps=1e-6)
LLM_150M = dict(dim=512, hidden_dim=2048, n_layers=12, n_heads=8, n_kv_heads=8, head_size=64, vocab_size=99487,
                seq_len=1024, shared_classifier=1, half_kv=1)
THETA = {"llama3-8b": 500000.0, "qwen25-7b-int6": 1000000.0, "llm150m": 10000.0}


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def read_checkpoint(eng, size):
    out = np.zeros(size, dtype=np.uint8)
    pk = package()
    pk.hip_engine.check(pk.library().he_checkpoint_read(eng._h, 0, size, ctypes.c_void_p(out.ctypes.data)))
    return out


def model(fields, theta, seed, **extra):
    """a config, its places, the device-made checkpoint's bytes with varied norm weights and biases, RoPE tables"""
    cfg = ol.config(**{**fields, **extra})
    tensors, size = ol.places(cfg)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, theta)
    eng = package().open_synthetic(cfg, tensors, size, seed, cos, sin, max_block=1)
    ck = read_checkpoint(eng, size)
    eng.release()
    ol.vary_vectors(cfg, tensors, ck, seed)
    return cfg, tensors, ck, cos, sin


def generate(eng, prompt, steps, per_call=64):
    """generate()'s greedy steps through forwardMany and generateMany (replayed step graphs)"""
    eng.forwardMany([1] + prompt[:-1], 0)
    got, token, pos = [], prompt[-1], len(prompt)
    while pos < steps:
        ids = eng.generateMany(token, pos, [], 0, min(per_call, steps - pos), 0.0, 0.9, 1.0, [], [])
        got += ids
        token, pos = ids[-1], pos + len(ids)
    return got


def against_the_oracle(cfg, tensors, ck, cos, sin, prompt_len, decode, seed, max_block=2048):
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=prompt_len)]
    steps = prompt_len + decode
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=512)
    want, want_logits = ref.generate(prompt, steps)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=max_block)
    got = generate(eng, prompt, steps)
    assert got == [int(t) for t in want]
    assert same_bits(eng.logits(), want_logits)
    kv = eng.keysAndValues(0, steps)
    k, v = ref.kv(0, steps)
    assert same_bits(kv["keys"], k.reshape(-1)), "keys"
    assert same_bits(kv["values"], v.reshape(-1)), "values"
    eng.release()
    ref.close()


def test_llama3_8b_widths_two_layers_against_the_oracle():
    """two layers of the Llama-3-8B shape: a 2048-token prompt (four 512-token GEMM passes at K = 4096 and 14336,
    prompt attention past 2048 positions), then 256 replayed greedy steps (the fused q/k/v epilogue at 32 q / 8 kv
    heads, wo, w1/w3 with its L2 fill, w2 at K = 14336, decode attention past 2048 positions, the 128256-row
    classifier with its fill)"""
    cfg, tensors, ck, cos, sin = model(LLAMA3_8B, THETA["llama3-8b"], seed=3, n_layers=2)
    against_the_oracle(cfg, tensors, ck, cos, sin, 2048, 256, seed=21)


def test_qwen25_7b_int6_widths_two_layers_against_the_oracle():
    """two layers of the Qwen2.5-7B shape in int6: a 1024-token prompt (the GEMM widening six.ts groups while it
    stages them), then 256 greedy steps (the int6 GEMV at K = 3584 and 18944, the q/k/v biases in the fused epilogue,
    seven q heads a kv head)"""
    cfg, tensors, ck, cos, sin = model(QWEN25_7B_INT6, THETA["qwen25-7b-int6"], seed=4, n_layers=2)
    against_the_oracle(cfg, tensors, ck, cos, sin, 1024, 256, seed=22)


def test_llama3_8b_whole_model_against_the_oracle():
    """all 32 layers of the Llama-3-8B shape (8.45 GB: every layer's tensors past 2 GiB, the classifier near 7.9 GB)
    against the oracle: a 128-token prompt through forwardMany (the MFMA GEMM), then 32 replayed greedy steps; every
    token, the last logits and the whole cache to the bit (tests/forward-check.mjs:422-462 holds whole models the
    same way)"""
    cfg, tensors, ck, cos, sin = model(LLAMA3_8B, THETA["llama3-8b"], seed=7)
    against_the_oracle(cfg, tensors, ck, cos, sin, 128, 32, seed=25)


def test_qwen25_7b_int6_whole_model_against_the_oracle():
    """all 28 layers of the Qwen2.5-7B shape in int6 (6.2 GB) against the oracle: a 128-token prompt, then 32
    replayed greedy steps; tokens, last logits and cache to the bit"""
    cfg, tensors, ck, cos, sin = model(QWEN25_7B_INT6, THETA["qwen25-7b-int6"], seed=8)
    against_the_oracle(cfg, tensors, ck, cos, sin, 128, 32, seed=26)


def test_llama3_8b_widths_replayed_draws_with_a_stop_token():
    """two layers of the Llama-3-8B shape, sampled steps on the device over the 128256-token vocabulary (temperature 0.8,
    no nucleus, penalty 1.1) and greedy steps with the penalty, each in replayed calls that a stop token ends: every
    token and the halting step's logits against the oracle's steps"""
    from steps import oracle_steps
    cfg, tensors, ck, cos, sin = model(LLAMA3_8B, THETA["llama3-8b"], seed=9, n_layers=2)
    rng = np.random.default_rng(27)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=64)]
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=64)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    for temperature, topp, penalty in ((0.8, 1.0, 1.1), (0.0, 0.9, 1.1)):
        eng.forwardMany([1] + prompt[:-1], 0)
        ref.run([1] + prompt[:-1], 0, False)
        history = [1] + prompt
        randoms = list(rng.random(40))
        want, logits = oracle_steps(ref, list(history), len(prompt), 40, temperature, topp, penalty, randoms)
        stop = want[25]
        first = want.index(stop)
        got = eng.generateMany(history[-1], len(prompt), history[-64:], len(history), 40, temperature, topp, penalty,
                               randoms if temperature > 0.0 else [], [stop, 1])
        assert got == want[:want.index(1) + 1 if 1 in want[:first] else first + 1]
        assert same_bits(eng.logits(), logits[len(got) - 1])
    eng.release()
    ref.close()


def test_150m_whole_model_against_the_oracle():
    """the 150M shape, every layer: a 512-token prompt and 256 greedy steps, float16 cache"""
    cfg, tensors, ck, cos, sin = model(LLM_150M, THETA["llm150m"], seed=5)
    against_the_oracle(cfg, tensors, ck, cos, sin, 512, 256, seed=23, max_block=512)


@pytest.mark.parametrize("fill_kib", ["0", "16", "3072"])
def test_l2_fills_at_width_2048_change_no_bits(fill_kib, monkeypatch):
    """a Llama form of width 2048 (over 1024: rmsnorm runs as its own launch before q/k/v and w1/w3 and carries their
    L2 fills, and the classifier's): no fill, part of the first GEMV blocks (16 KiB an XCD) and all of them give the
    oracle's tokens, logits and cache"""
    monkeypatch.setenv("PYODIDE_LLM_HIP_L2FETCH", fill_kib)
    fields = dict(dim=2048, hidden_dim=5632, n_layers=2, n_heads=16, n_kv_heads=4, head_size=128, vocab_size=32000,
                  seq_len=256, shared_classifier=0, half_kv=0)
    cfg, tensors, ck, cos, sin = model(fields, 10000.0, seed=6)
    against_the_oracle(cfg, tensors, ck, cos, sin, 64, 48, seed=24, max_block=64)


def host_rows(cfg, tensors, name, layer, r0, rows, seed):
    """the bytes of rows r0.. of a matrix of the synthetic checkpoint as the host makes them (or_synth_fill, then
    quantize() / quantize6() + pack6()): (values, scales)"""
    pk = package()
    shape = {"wq": (cfg.n_heads * cfg.head_size, cfg.dim), "w2": (cfg.dim, cfg.hidden_dim),
             "wcls": (cfg.vocab_size, cfg.dim), "token_embedding_table": (cfg.vocab_size, cfg.dim)}[name]
    n_rows, k = shape
    first = (layer * n_rows + r0) * k
    x = ol.synth(rows * k, seed, pk.T[name], 0.02, first).reshape(rows, k)
    if cfg.six:
        q, s = ol.quantize6(x)
        values = ol.pack6(q).reshape(-1)
    else:
        q, s = ol.quantize(x)
        values = q.reshape(-1).view(np.uint8)
    return values, s.reshape(-1).view(np.uint8), first


def check_synthesis(eng, cfg, tensors, seed, samples):
    pk = package()
    lib = pk.library()
    for name, layer, r0, rows in samples:
        values, scales, first = host_rows(cfg, tensors, name, layer, r0, rows, seed)
        t = tensors[pk.T[name]]
        per_value = 0.75 if cfg.six else 1.0
        got_v = np.zeros(values.size, dtype=np.uint8)
        got_s = np.zeros(scales.size, dtype=np.uint8)
        pk.hip_engine.check(lib.he_checkpoint_read(eng._h, int(t.offset + first * per_value), got_v.size,
                                                   ctypes.c_void_p(got_v.ctypes.data)))
        pk.hip_engine.check(lib.he_checkpoint_read(eng._h, int(t.scales + first // 32 * 4), got_s.size,
                                                   ctypes.c_void_p(got_s.ctypes.data)))
        assert np.array_equal(got_v, values), (name, layer, r0)
        assert np.array_equal(got_s, scales), (name, layer, r0)


def full_depth(fields, theta, prompt_len, decode, seed, samples):
    """every layer, the device-made checkpoint: its sampled tensors equal the host's synthesis; the prompt through
    forwardMany (MFMA GEMM passes of 512) equals it one token at a time (the GEMV), cache bits; then replayed greedy
    steps equal eager steps (he_forward and the host's argmax), tokens, last logits and cache bits"""
    pk = package()
    cfg = ol.config(**fields)
    tensors, size = ol.places(cfg)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, theta)
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=prompt_len)]
    fed = [1] + prompt[:-1]
    steps = prompt_len + decode
    many = pk.open_synthetic(cfg, tensors, size, 0, cos, sin, max_block=prompt_len)
    check_synthesis(many, cfg, tensors, 0, samples)
    one = pk.open_synthetic(cfg, tensors, size, 0, cos, sin, max_block=1)
    many.forwardMany(fed, 0)
    for pos, tok in enumerate(fed):
        one.forward(tok, pos, False)
    a, b = many.keysAndValues(0, prompt_len), one.keysAndValues(0, prompt_len)
    assert same_bits(a["keys"], b["keys"]) and same_bits(a["values"], b["values"]), "prompt cache"
    del a, b
    replayed, token, pos = [], prompt[-1], prompt_len
    while pos < steps:
        ids = many.generateMany(token, pos, [], 0, min(64, steps - pos), 0.0, 0.9, 1.0, [], [])
        replayed += ids
        token, pos = ids[-1], pos + len(ids)
    eager, token = [], prompt[-1]
    for pos in range(prompt_len, steps):
        one.forward(token, pos, True)
        token = int(np.argmax(one.logits()))
        eager.append(token)
    assert replayed == eager
    assert same_bits(many.logits(), one.logits())
    a, b = many.keysAndValues(prompt_len, decode), one.keysAndValues(prompt_len, decode)
    assert same_bits(a["keys"], b["keys"]) and same_bits(a["values"], b["values"]), "decode cache"
    many.release()
    one.release()


def test_llama3_8b_full_depth_prompt_blocks_and_replayed_steps():
    """all 32 layers of the Llama-3-8B shape: a 2048-token prompt, 256 greedy steps"""
    full_depth(LLAMA3_8B, THETA["llama3-8b"], 2048, 256, seed=31,
               samples=[("wq", 0, 0, 64), ("wq", 31, 4032, 64), ("w2", 0, 0, 16), ("w2", 31, 4080, 16),
                        ("wcls", 0, 0, 256), ("wcls", 0, 128000, 256), ("token_embedding_table", 0, 77, 8)])


def test_qwen25_7b_int6_full_depth_prompt_blocks_and_replayed_steps():
    """all 28 layers of the Qwen2.5-7B shape in int6: a 1024-token prompt, 256 greedy steps"""
    full_depth(QWEN25_7B_INT6, THETA["qwen25-7b-int6"], 1024, 256, seed=32,
               samples=[("wq", 0, 0, 64), ("wq", 27, 3520, 64), ("w2", 0, 0, 16), ("w2", 27, 3568, 16),
                        ("wcls", 0, 151808, 256)])
