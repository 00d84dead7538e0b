"""The engine (include/pyodide_llm_hip.h he_*) against the oracle's run() on the same checkpoint bytes: logits and
the KV cache to the bit at every position, prompt blocks equal to one token at a time, the device-made checkpoint
equal to the host-made one, and greedy generation token-identical, on models of the reference's shapes."""
import numpy as np
import pytest

import oracle_lib as ol
from paths import package

pytestmark = pytest.mark.gpu

MODELS = {
    "tiny_gqa": (dict(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2, head_size=16, vocab_size=320,
                      seq_len=48, shared_classifier=1), 10000.0),
    "tiny_qwen_int6": (dict(dim=128, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=1, head_size=32,
                            vocab_size=288, seq_len=48, shared_classifier=0, six=1, qkv_bias=1), 1000000.0),
    "stories15m": (dict(dim=288, hidden_dim=768, n_layers=6, n_heads=6, n_kv_heads=6, head_size=48, vocab_size=32000,
                        seq_len=256, shared_classifier=1), 10000.0),
}


def build(name, **extra):
    fields, theta = MODELS[name]
    cfg = ol.config(**{**fields, **extra})
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=7)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, theta)
    return cfg, tensors, ck, cos, sin, size


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("name", sorted(MODELS))
@pytest.mark.parametrize("relaxed", [1, 0])
@pytest.mark.parametrize("half_kv", [0, 1])
def test_forward_logits_and_cache_bits(name, relaxed, half_kv):
    cfg, tensors, ck, cos, sin, _ = build(name, relaxed=relaxed, half_kv=half_kv)
    pk = package()
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    rng = np.random.default_rng(5)
    tokens = rng.integers(0, cfg.vocab_size, size=12)
    for pos, tok in enumerate(tokens):
        ref.run([int(tok)], pos, True)
        eng.forward(int(tok), pos, True)
        assert same_bits(eng.logits(), ref.logits()), pos
    k_ref, v_ref = ref.kv(0, len(tokens))
    kv = eng.keysAndValues(0, len(tokens))
    assert same_bits(kv["keys"], k_ref.reshape(-1)) and same_bits(kv["values"], v_ref.reshape(-1))
    eng.release()


def test_kv_read_keeps_an_infinite_half_infinite():
    """keysAndValues() of a float16 cache reads an infinity (a value past 65520) as infinity, as public/forward.js:
    593-597 halfToFloat does, and the oracle's cache bits; attention reads it as 65536 (kernels/kernel.ts:383-392),
    and the logits are the oracle's"""
    cfg, tensors, ck, cos, sin, _ = build("tiny_qwen_int6", half_kv=1)
    at = tensors[package().T["bv"]].offset
    ck[at:at + 4] = np.frombuffer(np.float32(1e5).tobytes(), dtype=np.uint8)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=8)
    ref.run([1, 17, 3], 0, True)
    eng.forwardMany([1, 17], 0)
    eng.forward(3, 2, True)
    assert same_bits(eng.logits(), ref.logits())
    kv, (k, v) = eng.keysAndValues(0, 3), ref.kv(0, 3)
    assert np.all(np.isposinf(kv["values"].reshape(v.shape)[0, :, 0]))
    assert same_bits(kv["keys"], k.reshape(-1)) and same_bits(kv["values"], v.reshape(-1))
    eng.release()


@pytest.mark.parametrize("name", ["tiny_gqa", "stories15m"])
def test_prompt_blocks_equal_one_at_a_time(name):
    cfg, tensors, ck, cos, sin, _ = build(name)
    pk = package()
    rng = np.random.default_rng(6)
    tokens = [int(t) for t in rng.integers(0, cfg.vocab_size, size=40)]
    one = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    for pos, tok in enumerate(tokens):
        one.forward(tok, pos, pos == len(tokens) - 1)
    many = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    many.forwardMany(tokens[:-1], 0)
    many.forward(tokens[-1], len(tokens) - 1, True)
    assert same_bits(one.logits(), many.logits())
    a, b = one.keysAndValues(0, len(tokens)), many.keysAndValues(0, len(tokens))
    assert same_bits(a["keys"], b["keys"]) and same_bits(a["values"], b["values"])


def test_profiled_prompt_times_every_kind_and_keeps_the_bits():
    """he_profile_forward_many runs the prompt chunk as forwardMany does (the cache gets the oracle's bits) and reports
    the prompt's matmuls as GEMM launches"""
    cfg, tensors, ck, cos, sin, _ = build("stories15m")
    pk = package()
    tokens = [int(t) for t in np.random.default_rng(8).integers(0, cfg.vocab_size, size=40)]
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    prof = eng.profileMany(tokens, 0)
    assert prof["gemm"][2] == cfg.n_layers * 4 and prof["gemm"][0] > 0  # q/k/v, wo, w1/w3, w2 a layer
    assert prof["gemv"][2] == 0 and prof["attention"][2] >= cfg.n_layers and prof["argmax"][2] == 0
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    ref.run(tokens, 0, False)
    k, v = ref.kv(0, len(tokens))
    kv = eng.keysAndValues(0, len(tokens))
    assert same_bits(kv["keys"], k.reshape(-1)) and same_bits(kv["values"], v.reshape(-1))
    with pytest.raises(pk.HipError):
        eng.profileMany(tokens * 2, 0)  # more than the prompt block
    eng.release()


@pytest.mark.parametrize("name", sorted(MODELS))
def test_device_checkpoint_equals_host_checkpoint(name):
    cfg, tensors, ck, cos, sin, size = build(name)
    pk = package()
    eng = pk.open_synthetic(cfg, tensors, size, 7, cos, sin, max_block=8)
    import ctypes
    out = np.zeros(size, dtype=np.uint8)
    pk.hip_engine.check(pk.library().he_checkpoint_read(eng._h, 0, size, ctypes.c_void_p(out.ctypes.data)))
    assert np.array_equal(out, ck)


def test_greedy_generation_matches_the_oracle():
    """stories15M shape: a 32-token prompt through forwardMany, then 128 greedy tokens (stop tokens off)"""
    cfg, tensors, ck, cos, sin, _ = build("stories15m", half_kv=1)
    rng = np.random.default_rng(2)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=32)]
    steps = 32 + 128
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    want, want_logits = ref.generate(prompt, steps)
    pk = package()
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany([1] + prompt[:-1], 0)
    got, token, pos = [], prompt[-1], len(prompt)
    while pos < steps:
        ids = eng.generateMany(token, pos, [], 0, min(16, steps - pos), 0.0, 0.9, 1.0, [], [])
        got += ids
        token, pos = ids[-1], pos + len(ids)
    assert got == [int(t) for t in want]
    assert same_bits(eng.logits(), want_logits)


@pytest.mark.parametrize("fill_kib", ["0", "16", "3072"])
def test_l2_fills_change_no_bits(fill_kib, monkeypatch):
    """the rmsnorm launches' L2 fills ahead of the q/k/v, w1/w3 and classifier GEMVs only read: none, a part of the
    first GEMV blocks (16 KiB an XCD) or all of them give the oracle's tokens and logits, replayed steps included"""
    monkeypatch.setenv("PYODIDE_LLM_HIP_L2FETCH", fill_kib)
    cfg, tensors, ck, cos, sin, _ = build("stories15m", half_kv=1)
    rng = np.random.default_rng(3)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=8)]
    steps = 8 + 24
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    want, want_logits = ref.generate(prompt, steps)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany([1] + prompt[:-1], 0)
    got, token, pos = [], prompt[-1], len(prompt)
    while pos < steps:
        ids = eng.generateMany(token, pos, [], 0, min(16, steps - pos), 0.0, 0.9, 1.0, [], [])
        got += ids
        token, pos = ids[-1], pos + len(ids)
    assert got == [int(t) for t in want]
    assert same_bits(eng.logits(), want_logits)
    eng.release()


@pytest.mark.parametrize("half_kv", [0, 1])
def test_long_context_crosses_attention_chunks(half_kv):
    """positions past 512 and 1024 (the value kernel's chunks) and every count % 4, against the oracle to the bit"""
    fields, theta = MODELS["tiny_gqa"]
    cfg = ol.config(**{**fields, "seq_len": 1200, "half_kv": half_kv})
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=9)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, theta)
    rng = np.random.default_rng(11)
    tokens = [int(t) for t in rng.integers(0, cfg.vocab_size, size=1100)]
    pk = package()
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=1100)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=1100)
    eng.forwardMany(tokens[:1090], 0)
    ref.run(tokens[:1090], 0, False)
    for pos in range(1090, 1100):
        eng.forward(tokens[pos], pos, True)
        ref.run([tokens[pos]], pos, True)
        assert same_bits(eng.logits(), ref.logits()), pos
    a, (k, v) = eng.keysAndValues(0, 1100), ref.kv(0, 1100)
    assert same_bits(a["keys"], k.reshape(-1)) and same_bits(a["values"], v.reshape(-1))


LONG = {
    # head size 128, four query heads a kv head (the 8B's grouping): 15 chunks of 256 positions, past the producers'
    # two chunks in registers
    "hs128_mul4": (dict(dim=512, hidden_dim=256, n_layers=1, n_heads=4, n_kv_heads=1, head_size=128, vocab_size=320,
                        seq_len=3700, shared_classifier=1), 3600),
    # past 4096 positions: more than 1024 four-position blocks a sum, where the decode kernel's ordered sums run
    # from LDS instead of registers
    "hs128_mul4_4600": (dict(dim=512, hidden_dim=256, n_layers=1, n_heads=4, n_kv_heads=1, head_size=128,
                             vocab_size=320, seq_len=4700, shared_classifier=1), 4600),
    # eight query heads a kv head past 2048 positions, heads of 16 (a block takes 16 columns)
    "mul8_hs16": (dict(dim=256, hidden_dim=128, n_layers=1, n_heads=16, n_kv_heads=2, head_size=16,
                       vocab_size=320, seq_len=2200, shared_classifier=1), 2100),
}


@pytest.mark.parametrize("name", sorted(LONG))
@pytest.mark.parametrize("half_kv", [0, 1])
@pytest.mark.parametrize("attend", ["fused", "split"])
def test_long_decode_attention(name, half_kv, attend, monkeypatch):
    """decode steps after a long prompt, every count % 4, against the oracle to the bit: through the fused decode
    kernel, and through the separate softmax and weighted-value kernels that contexts past its LDS take
    (PYODIDE_LLM_HIP_ATTEND=split sends every decode step there)"""
    monkeypatch.setenv("PYODIDE_LLM_HIP_ATTEND", attend)
    fields, prompt = LONG[name]
    cfg = ol.config(**{**fields, "half_kv": half_kv})
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=9)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, 10000.0)
    tokens = [int(t) for t in np.random.default_rng(12).integers(0, cfg.vocab_size, size=prompt + 8)]
    pk = package()
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=512)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=prompt)
    eng.forwardMany(tokens[:prompt], 0)
    ref.run(tokens[:prompt], 0, False)
    for pos in range(prompt, prompt + 8):
        eng.forward(tokens[pos], pos, True)
        ref.run([tokens[pos]], pos, True)
        assert same_bits(eng.logits(), ref.logits()), pos
    eng.release()


PROMPT_HEADS = {
    # every head size the prompt kernels take, with 1, 2, 4 and 8 query heads a kv head: the score kernel's 32- or
    # 16-dimension chunks and its token rows a block (64 / heads a kv head), the weighted-value kernel's 32- or
    # 16-column tiles
    "hs16_mul8": dict(dim=256, hidden_dim=64, n_heads=16, n_kv_heads=2, head_size=16),
    "hs48_mul1": dict(dim=96, hidden_dim=64, n_heads=2, n_kv_heads=2, head_size=48),
    "hs64_mul2": dict(dim=128, hidden_dim=64, n_heads=2, n_kv_heads=1, head_size=64),
    "hs96_mul2": dict(dim=192, hidden_dim=64, n_heads=2, n_kv_heads=1, head_size=96),
    "hs128_mul4": dict(dim=256, hidden_dim=64, n_heads=4, n_kv_heads=1, head_size=128),
    "hs256_mul2": dict(dim=512, hidden_dim=64, n_heads=4, n_kv_heads=2, head_size=256),
}


@pytest.mark.parametrize("name", sorted(PROMPT_HEADS))
@pytest.mark.parametrize("half_kv", [0, 1])
def test_prompt_kernels_every_head_size(name, half_kv):
    """prompt blocks of more than 8 tokens (the score, softmax and weighted-value kernels of many tokens a launch),
    a second block starting past the first's 64-position tiles and ragged ends, then decode steps: the cache (the
    second layer's keys and values carry every prompt token's first-layer attention) and the logits against the
    oracle to the bit"""
    cfg = ol.config(**{**PROMPT_HEADS[name], "n_layers": 2, "vocab_size": 320, "seq_len": 200,
                       "shared_classifier": 1, "half_kv": half_kv})
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=13)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, 10000.0)
    tokens = [int(t) for t in np.random.default_rng(14).integers(0, cfg.vocab_size, size=175)]
    pk = package()
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=100)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=100)
    for at, end in ((0, 93), (93, 171)):
        eng.forwardMany(tokens[at:end], at)
        ref.run(tokens[at:end], at, False)
    kv, (k, v) = eng.keysAndValues(0, 171), ref.kv(0, 171)
    assert same_bits(kv["keys"], k.reshape(-1)) and same_bits(kv["values"], v.reshape(-1))
    for pos in range(171, 175):
        eng.forward(tokens[pos], pos, True)
        ref.run([tokens[pos]], pos, True)
        assert same_bits(eng.logits(), ref.logits()), pos
    eng.release()


@pytest.mark.parametrize("name", ["hs16_mul8", "hs256_mul2"])
def test_prompt_pass_in_attention_pieces(name):
    """a 1090-token prompt: a pass of 1024 tokens whose attention runs as two pieces of 512 that reuse the score rows,
    then a pass of 66; the cache and the decode steps after it against the oracle to the bit"""
    cfg = ol.config(**{**PROMPT_HEADS[name], "n_layers": 2, "vocab_size": 320, "seq_len": 1200,
                       "shared_classifier": 1})
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=15)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, 10000.0)
    tokens = [int(t) for t in np.random.default_rng(16).integers(0, cfg.vocab_size, size=1094)]
    pk = package()
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=1100)
    assert eng.promptBlock == 1100
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=1100)
    eng.forwardMany(tokens[:1090], 0)
    ref.run(tokens[:1090], 0, False)
    kv, (k, v) = eng.keysAndValues(0, 1090), ref.kv(0, 1090)
    assert same_bits(kv["keys"], k.reshape(-1)) and same_bits(kv["values"], v.reshape(-1))
    for pos in range(1090, 1094):
        eng.forward(tokens[pos], pos, True)
        ref.run([tokens[pos]], pos, True)
        assert same_bits(eng.logits(), ref.logits()), pos
    eng.release()


@pytest.mark.parametrize("piece", [3, 5, 8])
def test_prompt_in_small_pieces_equals_one_at_a_time(piece):
    """prompt pieces of up to 8 tokens run the decode attention with several tokens a launch"""
    cfg, tensors, ck, cos, sin, _ = build("tiny_qwen_int6")
    pk = package()
    rng = np.random.default_rng(8)
    tokens = [int(t) for t in rng.integers(0, cfg.vocab_size, size=41)]
    one = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    for pos, tok in enumerate(tokens):
        one.forward(tok, pos, pos == len(tokens) - 1)
    many = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    for at in range(0, len(tokens) - 1, piece):
        many.forwardMany(tokens[at:min(at + piece, len(tokens) - 1)], at)
    many.forward(tokens[-1], len(tokens) - 1, True)
    assert same_bits(one.logits(), many.logits())
    a, b = one.keysAndValues(0, len(tokens)), many.keysAndValues(0, len(tokens))
    assert same_bits(a["keys"], b["keys"]) and same_bits(a["values"], b["values"])


@pytest.mark.parametrize("name", sorted(MODELS))
def test_replayed_steps_with_stops_and_eager_steps_between(name):
    """generateMany's replayed decode steps (one captured step graph): a stop token ends a call at the right step with
    that step's logits; eager steps between calls; a later call without stops runs its steps back to back. Every token
    and the logits of every call's last step against the oracle's greedy steps, to the bit."""
    cfg, tensors, ck, cos, sin, _ = build(name)
    rng = np.random.default_rng(4)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=20)]
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    ref.run(prompt[:-1], 0, False)
    want, logits = [], []
    tok, pos = prompt[-1], len(prompt) - 1
    for _ in range(26):
        ref.run([tok], pos, True)
        lg = ref.logits()
        tok, pos = int(np.argmax(lg)), pos + 1
        want.append(tok)
        logits.append(lg)
    pk = package()
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany(prompt[:-1], 0)
    p0 = len(prompt) - 1
    # a stop token: the first call ends at the step that produced it (want[6] may also appear earlier)
    stop = want[6]
    first = want.index(stop)
    ids = eng.generateMany(prompt[-1], p0, [], 0, 12, 0.0, 0.9, 1.0, [], [stop])
    assert ids == want[:first + 1]
    assert same_bits(eng.logits(), logits[first])
    n = len(ids)
    # an eager step, then replayed steps without stops, twice
    eng.forward(ids[-1], p0 + n, True)
    assert same_bits(eng.logits(), logits[n])
    done = n + 1
    for count in (7, 16 - n):
        got = eng.generateMany(want[done - 1], p0 + done, [], 0, count, 0.0, 0.9, 1.0, [], [])
        assert got == want[done:done + count]
        assert same_bits(eng.logits(), logits[done + count - 1])
        done += count
    eng.release()


@pytest.mark.parametrize("name", sorted(MODELS))
@pytest.mark.parametrize("temperature, topp, penalty", [(0.8, 1.0, 1.1), (0.0, 0.9, 1.3)])
def test_replayed_draws_with_stop_tokens(name, temperature, topp, penalty):
    """generateMany's replayed steps with a stop token, a draw and a penalty (the call's settings, the round's random
    numbers and the penalty's window in device memory): a call ends at the step that took the stop token, with that
    step's (penalized) logits, though the round's later replays ran; the next calls go on from there, one of them over
    more steps than a stop-token round (16), so that the window and the random numbers cross rounds. Tokens and logits
    against the oracle's steps to the bit."""
    from steps import oracle_steps
    cfg, tensors, ck, cos, sin, _ = build(name)
    rng = np.random.default_rng(int(100 * temperature + 10 * penalty))
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=10)]
    total = min(46, cfg.seq_len - len(prompt))
    randoms = list(rng.random(total)) if temperature > 0.0 else [0.0] * total
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    ref.run([1] + prompt[:-1], 0, False)
    history = [1] + prompt
    want, want_logits = oracle_steps(ref, list(history), len(prompt), total, temperature, topp, penalty, randoms)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany([1] + prompt[:-1], 0)
    stop = want[13]
    first = want.index(stop)
    unseen = [t for t in range(cfg.vocab_size) if t not in want][:3]
    done, pos = 0, len(prompt)
    for count, stops in ((30, [stop] + unseen), (6, []), (total - first - 7, unseen)):
        r = randoms[done:done + count] if temperature > 0.0 else []
        got = eng.generateMany(history[-1], pos, history[-64:], len(history), count, temperature, topp, penalty, r,
                               stops)
        n = first + 1 if done == 0 else count
        assert got == want[done:done + n], (done, count)
        assert same_bits(eng.logits(), want_logits[done + n - 1])
        history += got
        done, pos = done + n, pos + n
    assert done == total
    eng.release()
    ref.close()


def nucleus_size(logits, temperature, topp):
    """how many tokens the nucleus sort takes (float64 NumPy: the cases here lie far from the device's 8192)"""
    if not 0 < topp < 1:
        return 0
    best = float(logits.max())
    kept = logits[logits >= best - temperature * 16.118095].astype(np.float64)
    p = np.exp((kept - best) / temperature)
    return int((p >= min((1 - topp) / max(p.size - 1, 1) * p.sum(), p.max())).sum())


@pytest.mark.parametrize("name", sorted(MODELS))
@pytest.mark.parametrize("temperature, topp, penalty", [(0.8, 0.9, 1.3), (1.0, 1.0, 1.0), (0.0, 0.9, 1.5),
                                                        (0.5, 0.6, 0.8)])
def test_sampled_generation_matches_the_oracle(name, temperature, topp, penalty):
    """generate() with a temperature, top-p and a repetition penalty (public/llama2_numpy.py:1565-1640): the steps
    generateMany takes against the oracle's forward pass, or_penalize over the latest 64 of the history and or_sample
    with the same random numbers, token for token; a step the engine declines (a nucleus larger than it sorts) is the
    caller's: forward() and the oracle's draw, as the reference's CPU step takes it"""
    cfg, tensors, ck, cos, sin, _ = build(name)
    rng = np.random.default_rng(int(10 * temperature + 100 * topp + 1000 * penalty))
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=12)]
    steps = min(12 + 40, cfg.seq_len)
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    ref.run([1] + prompt[:-1], 0, False)
    eng = package().open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany([1] + prompt[:-1], 0)
    history = [1] + prompt
    token, pos, declined = prompt[-1], len(prompt), 0

    def oracle_step(u):
        ref.run([token], pos, True)
        lg = ref.logits()
        if penalty != 1.0:
            lg = ol.penalize(lg, set(history[-64:]), penalty)
        if temperature == 0.0:
            return int(np.argmax(lg)), lg
        return ol.sample(lg, temperature, topp, u), lg

    while pos < steps:
        count = min(8, steps - pos)
        randoms = list(rng.random(count)) if temperature != 0.0 else []
        got = eng.generateMany(token, pos, history[-64:], len(history), count, temperature, topp, penalty, randoms,
                               [])
        got = got or []
        for i, t in enumerate(got):
            want, _ = oracle_step(randoms[i] if randoms else 0.0)
            assert t == want, (pos, i)
            history.append(t)
            token, pos = t, pos + 1
        if len(got) < count:
            # declined: the caller's step, through forward() and the oracle's draw
            want, lg = oracle_step(randoms[len(got)])
            assert nucleus_size(lg, temperature, topp) > 8192
            eng.forward(token, pos, True)
            assert same_bits(ol.penalize(eng.logits(), set(history[-64:]), penalty) if penalty != 1.0
                             else eng.logits(), lg)
            history.append(want)
            token, pos = want, pos + 1
            declined += 1
    assert pos == steps
    if cfg.vocab_size < 8192:
        assert declined == 0
    eng.release()


@pytest.mark.parametrize("name", ["tiny_gqa", "tiny_qwen_int6"])
def test_prompt_attention_with_subnormal_products(name):
    """the prompt attention's products on the matrix core (v_mfma_f32_32x32x1_2b_f32 for q.k, v_mfma_f32_16x16x1_4b_f32
    for p.v, each with a zero accumulator) must give every product's float32 bits, subnormals kept: wq and wk scaled so
    that q . k's products lie near 1e-39, wv so that the values (and p . v) are subnormal; a 40-token prompt through
    forwardMany (the prompt kernels) and one more step with logits, cache and logits against the oracle to the bit"""
    cfg, tensors, ck, cos, sin, _ = build(name)
    pk = package()
    ol.sharpen(cfg, tensors, ck, 1.5e-19)  # wq, wk: q and k near 3e-20
    t = tensors[pk.T["wv"]]
    n = cfg.n_layers * cfg.n_kv_heads * cfg.head_size * (cfg.dim // 32)
    scales = np.frombuffer(ck[t.scales:t.scales + 4 * n].tobytes(), dtype=np.float32) * np.float32(5e-39)
    ck[t.scales:t.scales + 4 * n] = np.frombuffer(scales.astype(np.float32).tobytes(), dtype=np.uint8)
    for bias, factor in (("bq", 1.5e-19), ("bk", 1.5e-19), ("bv", 5e-39)):  # Qwen2's q/k/v biases alike
        b = tensors[pk.T[bias]]
        if b.offset:
            m = ol.vector_length(cfg, bias)
            v = np.frombuffer(ck[b.offset:b.offset + 4 * m].tobytes(), dtype=np.float32) * np.float32(factor)
            ck[b.offset:b.offset + 4 * m] = np.frombuffer(v.astype(np.float32).tobytes(), dtype=np.uint8)
    rng = np.random.default_rng(31)
    tokens = [int(x) for x in rng.integers(0, cfg.vocab_size, size=41)]
    ref = ol.Model(cfg, tensors, ck, cos, sin, max_block=64)
    ref.run(tokens[:-1], 0, False)
    ref.run([tokens[-1]], 40, True)
    eng = pk.open_config(cfg, tensors, ck, cos, sin, max_block=64)
    eng.forwardMany(tokens[:-1], 0)
    eng.forward(tokens[-1], 40, True)
    keys, values = ref.kv(0, 41)
    kv = eng.keysAndValues(0, 41)
    assert same_bits(kv["keys"], keys.reshape(-1)), "keys"
    assert same_bits(kv["values"], values.reshape(-1)), "values"
    assert same_bits(eng.logits(), ref.logits())
    # the case is the one meant: many q . k-sized products (k . k of one head) and many values are subnormal
    tiny = np.finfo(np.float32).tiny
    k0 = keys[0].reshape(41, cfg.n_kv_heads, cfg.head_size)[:, 0, :]
    prods = (k0[:, None, :] * k0[None, :, :]).astype(np.float32)
    assert np.mean((prods != 0) & (np.abs(prods) < tiny)) > 0.2
    assert np.mean((values != 0) & (np.abs(values) < tiny)) > 0.5
    eng.release()
    ref.close()
