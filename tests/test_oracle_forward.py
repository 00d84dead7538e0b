"""The oracle's run() (public/forward.js:1011-1090) on tiny synthetic models: the checkpoint bytes the golden script
fed the reference, the reference NumPy forward's logits within the int8 line (tests/test_quantize.py:81-90: the int8
path quantizes activations, NumPy does not), and blocks equal to one token at a time to the bit
(tests/forward-check.mjs:438-452)."""
import hashlib
import os

import numpy as np
import pytest

import oracle_lib as ol
from paths import GOLDEN_DIR
from tiny import TINY, sharp_checkpoint

NF = np.load(os.path.join(GOLDEN_DIR, "numpy_forward.npz"))
SHARP = np.load(os.path.join(GOLDEN_DIR, "numpy_forward_sharp.npz"))


def build(name, **extra):
    fields, theta = TINY[name]
    cfg = ol.config(**{**fields, **extra})
    tensors, size = ol.places(cfg)
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=7)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, theta)
    return cfg, tensors, ck, cos, sin


@pytest.mark.parametrize("name", sorted(TINY))
def test_checkpoint_is_the_golden_one(name):
    _, _, ck, _, _ = build(name)
    assert np.array_equal(np.frombuffer(hashlib.sha256(ck.tobytes()).digest(), dtype=np.uint8), NF[f"sha256_{name}"])


@pytest.mark.parametrize("name", sorted(TINY))
@pytest.mark.parametrize("relaxed", [1, 0])
def test_logits_follow_the_reference_numpy_forward(name, relaxed):
    cfg, tensors, ck, cos, sin = build(name, relaxed=relaxed)
    model = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    want = NF[f"logits_{name}"]
    for pos, tok in enumerate(NF["tokens"]):
        model.run([tok], pos, True)
        got = model.logits().astype(np.float64)
        expected = want[pos].astype(np.float64)
        assert np.abs(got - expected).max() / np.abs(expected).max() < 0.1
        assert np.corrcoef(got, expected)[0, 1] > 0.99


@pytest.mark.parametrize("name", sorted(TINY))
@pytest.mark.parametrize("relaxed", [1, 0])
def test_logits_follow_the_reference_numpy_forward_where_attention_is_sharp(name, relaxed):
    """the reference NumPy forward on checkpoints whose attention leans on a few keys (q / k scales x5, norm weights
    and biases varied) over 24 positions: the int8 line holds (worst relative error 0.036 measured, correlation
    0.9995), while an oracle whose RoPE turns the other way misses it on every model (0.08 to 0.7, correlation 0.81 to
    0.995), as an attention or RoPE mistake would"""
    cfg, tensors, ck, cos, sin, tokens = sharp_checkpoint(name, relaxed=relaxed)
    assert np.array_equal(np.frombuffer(hashlib.sha256(ck.tobytes()).digest(), dtype=np.uint8), SHARP[f"sha256_{name}"])
    assert tokens == list(SHARP[f"tokens_{name}"])
    model = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    want = SHARP[f"logits_{name}"]
    for pos, tok in enumerate(tokens):
        model.run([tok], pos, True)
        got = model.logits().astype(np.float64)
        expected = want[pos].astype(np.float64)
        assert np.abs(got - expected).max() / np.abs(expected).max() < 0.06, pos
        assert np.corrcoef(got, expected)[0, 1] > 0.999, pos


@pytest.mark.parametrize("name", sorted(TINY))
@pytest.mark.parametrize("half_kv", [0, 1])
def test_blocks_equal_one_at_a_time(name, half_kv):
    cfg, tensors, ck, cos, sin = build(name, half_kv=half_kv)
    tokens = [1, 17, 3, 99, 5, 6, 7, 250, 9, 10, 11]
    one = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    for pos, tok in enumerate(tokens):
        one.run([tok], pos, pos == len(tokens) - 1)
    many = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    many.run(tokens[:3], 0, False)
    many.run(tokens[3:10], 3, False)
    many.run(tokens[10:], 10, True)
    assert np.array_equal(one.logits().view(np.uint32), many.logits().view(np.uint32))
    k1, v1 = one.kv(0, len(tokens))
    k2, v2 = many.kv(0, len(tokens))
    assert np.array_equal(k1.view(np.uint32), k2.view(np.uint32)) and np.array_equal(v1.view(np.uint32), v2.view(np.uint32))


def test_generate_is_greedy_over_forward():
    cfg, tensors, ck, cos, sin = build("tiny_gqa_int8")
    model = ol.Model(cfg, tensors, ck, cos, sin, max_block=4)
    prompt = [5, 6, 7, 8, 9]
    out, last = model.generate(prompt, steps=12)
    assert out.size == 12 - len(prompt)
    step = ol.Model(cfg, tensors, ck, cos, sin, max_block=4)
    fed = [1] + prompt[:-1]
    for pos, tok in enumerate(fed):
        step.run([tok], pos, False)
    token = prompt[-1]
    for pos in range(len(prompt), 12):
        step.run([token], pos, True)
        token = int(np.argmax(step.logits()))
        assert token == out[pos - len(prompt)]
    assert np.array_equal(step.logits(), last)


def overflowing_value_bias(name="tiny_qwen_int6"):
    """a float16-cache model whose layer-0 value bias of channel 0 is 1e5: that value rounds to infinity in the cache
    (kernels/kernel.ts:570-599 to_f16 gives infinity from 65520 on)"""
    from paths import package
    cfg, tensors, ck, cos, sin = build(name, half_kv=1)
    at = tensors[package().T["bv"]].offset
    ck[at:at + 4] = np.frombuffer(np.float32(1e5).tobytes(), dtype=np.uint8)
    return cfg, tensors, ck, cos, sin


def test_keys_and_values_keep_an_infinite_half_infinite():
    """public/forward.js:593-597 halfToFloat, which keysAndValues() reads a float16 cache with: a cached infinity
    stays infinite (the kernels' half() reads it as 65536 inside attention; the logits stay finite)"""
    cfg, tensors, ck, cos, sin = overflowing_value_bias()
    model = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    model.run([1, 17, 3], 0, True)
    keys, values = model.kv(0, 3)
    assert np.all(np.isposinf(values[0, :, 0]))
    assert np.all(np.isfinite(values[0, :, 1:])) and np.all(np.isfinite(values[1:])) and np.all(np.isfinite(keys))
    assert np.all(np.isfinite(model.logits()))
