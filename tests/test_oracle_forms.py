"""The oracle's other forms (GPT-2, GPT-NeoX, Qwen3's head norms, the outlier channels), pinned by what the reference
itself says of them: the tensor layout its llama2_convert.layout()/tensor_bytes() gives (tests/golden/layouts.json),
its NumPy forward's logits on tiny models of every form within the int8 line (tests/golden/numpy_forms.npz,
tests/test_quantize.py:81-90), float64 expectations of layernorm and gelu, the order of add_columns by a case that
only the reference's order gets right, and blocks equal to one token at a time (tests/forward-check.mjs:438-452)."""
import hashlib
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as ol
from forms import FORM_TINY, form_checkpoint, form_model
from paths import GOLDEN_DIR, package

NF = np.load(os.path.join(GOLDEN_DIR, "numpy_forms.npz"))
with open(os.path.join(GOLDEN_DIR, "layouts.json")) as f:
    LAYOUTS = json.load(f)
ARCH = {"llama": 0, "gpt2": 1, "neox": 2}


def layout_config(entry):
    dim, hidden, layers, heads, kv_heads, vocab, seq_len = entry["header"]
    form = entry["form"]
    head_size = form.get("head_dim") or dim // heads
    return ol.config(dim=dim, hidden_dim=hidden, n_layers=layers, n_heads=heads, n_kv_heads=kv_heads,
                     head_size=head_size, vocab_size=abs(vocab), seq_len=seq_len, shared_classifier=int(vocab > 0),
                     six=int(entry["dtype"] == "int6"), qkv_bias=int(bool(form.get("bias"))),
                     qk_norm=int(bool(form.get("qk_norm"))), arch=ARCH[form.get("arch", "llama")])


@pytest.mark.parametrize("name", sorted(LAYOUTS))
@pytest.mark.parametrize("places", ["oracle", "package"])
def test_places_follow_the_reference_layout(name, places):
    """every tensor where layout() puts it, in its order, with tensor_bytes() between them, and the file's size"""
    entry = LAYOUTS[name]
    cfg = layout_config(entry)
    tensors, size = ol.places(cfg) if places == "oracle" else package().places(cfg)
    assert size == entry["size"]
    T = package().T
    mine = sorted({tensors[i].offset for name_, i in T.items() if tensors[i].offset
                   and not (name_ == "wcls" and cfg.shared_classifier)})
    theirs = [e["offset"] for e in entry["layout"] if e["bytes"]]
    assert mine == theirs
    # a matrix's scales follow its values (int8: one byte a value; int6: 24 bytes a group)
    for e in entry["layout"]:
        if e["matrix"] and e["bytes"]:
            i = next(i for i in T.values() if tensors[i].offset == e["offset"])
            count = math.prod(e["shape"])
            assert tensors[i].scales == e["offset"] + (count * 3 // 4 if cfg.six else count)


@pytest.mark.parametrize("name", sorted(FORM_TINY))
def test_checkpoint_is_the_golden_one(name):
    _, _, ck = form_checkpoint(name)
    assert np.array_equal(np.frombuffer(hashlib.sha256(ck.tobytes()).digest(), dtype=np.uint8), NF[f"sha256_{name}"])


def max_error(model):
    worst = 0.0
    for pos, tok in enumerate(NF["tokens"]):
        model.run([tok], pos, True)
        got = model.logits().astype(np.float64)
        expected = NF[f"logits_{model.name}"][pos].astype(np.float64)
        assert np.corrcoef(got, expected)[0, 1] > 0.99, pos
        worst = max(worst, np.abs(got - expected).max() / np.abs(expected).max())
    return worst


@pytest.mark.parametrize("name", sorted(FORM_TINY))
@pytest.mark.parametrize("relaxed", [1, 0])
def test_logits_follow_the_reference_numpy_forward(name, relaxed):
    cfg, tensors, ck, cos, sin, _ = form_model(name, relaxed=relaxed)
    model = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    model.name = name
    assert max_error(model) < 0.1


def test_outlier_channels_are_found_and_bring_the_logits_closer():
    """the final norm's outliers (public/llama2_numpy.py:807-813): multiplied apart in float32 (public/forward.js:
    1084-1089), the int8 logits come closer to the float forward's than with every channel quantized"""
    name = "tiny_llama_outliers_int8"
    cfg, tensors, ck, cos, sin, channels = form_model(name)
    assert {3, 17, 40, 71} <= set(channels) and len(channels) == 8
    apart = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    apart.name = name
    plain_cfg = form_model(name, outliers=False)[0]
    plain = ol.Model(plain_cfg, tensors, ck, cos, sin, max_block=8)
    plain.name = name
    assert max_error(apart) < 0.7 * max_error(plain)


@pytest.mark.parametrize("name", sorted(FORM_TINY))
@pytest.mark.parametrize("half_kv", [0, 1])
def test_blocks_equal_one_at_a_time(name, half_kv):
    cfg, tensors, ck, cos, sin, _ = form_model(name, half_kv=half_kv)
    tokens = [1, 17, 3, 99, 5, 6, 7, 250, 9, 10, 11]
    one = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    for pos, tok in enumerate(tokens):
        one.run([tok], pos, pos == len(tokens) - 1)
    many = ol.Model(cfg, tensors, ck, cos, sin, max_block=8)
    many.run(tokens[:3], 0, False)
    many.run(tokens[3:10], 3, False)
    many.run(tokens[10:], 10, True)
    assert np.array_equal(one.logits().view(np.uint32), many.logits().view(np.uint32))


@pytest.mark.parametrize("n", [768, 1023, 6])
def test_layernorm_is_the_float64_one_within_a_few_ulp(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3 + 1.5).astype(np.float32)
    w = (1 + 0.3 * rng.standard_normal(n)).astype(np.float32)
    b = (0.2 * rng.standard_normal(n)).astype(np.float32)
    out = np.zeros(n, dtype=np.float32)
    ol.load().or_layernorm(ol.ptr(out), ol.ptr(x), ol.ptr(w), ol.ptr(b), n)
    x64 = x.astype(np.float64)
    mean = x64.mean()
    want = w * ((x64 - mean) / np.sqrt(((x64 - mean) ** 2).mean() + 1e-5)) + b
    assert np.abs(out - want).max() < 1e-5 * (np.abs(want).max() + 1)
    # a dropped bias, a weight on the wrong side of the mean or the variance of x instead of x - mean all fail this
    assert np.abs(out - want).max() < 0.01 * np.abs(b).max()


def test_gelu_is_the_float64_one_within_a_few_ulp():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(1000) * 3, [0.0, -0.0, 20.0, -20.0, 60.0, -60.0]]).astype(np.float32)
    b = (0.1 * rng.standard_normal(x.size)).astype(np.float32)
    out = np.zeros(x.size, dtype=np.float32)
    ol.load().or_gelu(ol.ptr(out), ol.ptr(x), ol.ptr(b), x.size)
    v = x.astype(np.float64) + b
    # 0.5 v (1 + tanh(z)) = v / (1 + exp(-2 z)), the form without tanh's cancellation far left; exp is clamped at
    # 88 as vexp clamps it (kernels/kernel.ts:32-45)
    z = math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)
    want = v / (1 + np.exp(np.minimum(-2 * z, 88.0)))
    # float32's rounding of 2z moves exp(2z) by |2z| ulps: the bound grows with it
    assert (np.abs(out - want) <= 4e-7 * (2 + np.abs(2 * z)) * np.abs(want)).all()


def test_add_columns_adds_in_channel_order():
    """y + a0 r0 + a1 r1 + a2 r2 in that order: 1e8 + 1 - 1e8 is 0 in float32 (any other order gives 1); small
    integers give the exact sum"""
    n = 5
    y = np.zeros(n, dtype=np.float32)
    rows = np.ones((3, n), dtype=np.float32)
    a = np.array([1e8, 1.0, -1e8], dtype=np.float32)
    ol.load().or_add_columns(ol.ptr(y), ol.ptr(rows), ol.ptr(a), 3, n)
    assert (y == 0).all()
    rng = np.random.default_rng(2)
    y = rng.integers(-50, 50, size=300).astype(np.float32)
    rows = rng.integers(-9, 9, size=(4, 300)).astype(np.float32)
    a = np.array([3, -2, 7, 1], dtype=np.float32)
    want = y.astype(np.float64) + a.astype(np.float64) @ rows.astype(np.float64)
    ol.load().or_add_columns(ol.ptr(y), ol.ptr(rows), ol.ptr(a), 4, 300)
    assert np.array_equal(y, want)
