"""The oracle's weight formats and checkpoint placement against the reference's own outputs (golden vectors written by
tests/golden/make_golden.py from public/llama2_convert.py and public/llama2_numpy.py) and the layout closed forms of
the reference's tests."""
import json
import os

import numpy as np
import pytest

import oracle_lib as ol
from paths import GOLDEN_DIR, package

G = np.load(os.path.join(GOLDEN_DIR, "quantizers.npz"))


@pytest.mark.parametrize("k", [96, 48, 40])
def test_quantize_matches_the_reference_quantize(k):
    """public/llama2_convert.py:125-130 quantize(): the int8 values and float32 scales to the bit (groups of 32, 16
    and 8 by group_size, a group of zeros, a group with one large value)"""
    q, s = ol.quantize(G[f"q8_x_{k}"])
    assert np.array_equal(q.reshape(-1), G[f"q8_values_{k}"].reshape(-1))
    assert np.array_equal(s.view(np.uint32), G[f"q8_scales_{k}"].view(np.uint32))


def test_quantize6_and_pack6_match_the_reference():
    """public/llama2_numpy.py:678-702: quantize6's int8 (4v) and scale/4, pack6's 24 bytes a group"""
    q, s = ol.quantize6(G["q6_x"])
    assert np.array_equal(q.reshape(-1), G["q6_ints"].reshape(-1))
    assert np.array_equal(s.view(np.uint32), G["q6_scales"].view(np.uint32))
    assert np.array_equal(ol.pack6(q), G["q6_packed"])


def test_unpack6_matches_the_reference_and_the_kernel_closed_form():
    """unpack6 (public/llama2_numpy.py:687-692) golden bytes, and the byte-by-byte form of tests/forward-check.mjs:
    44-49 over every value of the bytes each position reads"""
    assert np.array_equal(ol.unpack6(G["six_raw"]), G["six_values"])
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, size=(256, 24), dtype=np.uint8)
    for j in range(24):
        raw[:, j] = np.arange(256, dtype=np.uint8)  # every byte value at every place
    got = ol.unpack6(raw)
    for g in range(raw.shape[0]):
        for j in range(32):
            low = raw[g, j] & 15 if j < 16 else raw[g, j - 16] >> 4
            top = (raw[g, 16 + j % 8] >> (2 * (j // 8))) & 3
            want = np.int8(np.uint8(((int(low) | (int(top) << 4)) << 2) & 255).view(np.int8))
            assert got[g, j] == want


def test_pack6_layout_closed_form():
    """tests/test_int6.py:16-26: the low four bits of j and j+16 in byte j, the top two bits in bytes 16..23"""
    rng = np.random.default_rng(1)
    values = (rng.integers(-32, 32, size=(5, 64)) * 4).astype(np.int8)
    packed = ol.pack6(values)
    assert packed.shape == (10, 24)
    assert np.array_equal(ol.unpack6(packed).reshape(values.shape), values)
    six = np.arange(-32, 0, dtype=np.int8)
    bits = six.view(np.uint8) & 63
    p = ol.pack6(six * 4)
    assert p[0, 0] == (bits[0] & 15) | ((bits[16] & 15) << 4)
    assert p[0, 16] == sum(((int(bits[k]) >> 4) & 3) << s for k, s in ((0, 0), (8, 2), (16, 4), (24, 6)))


PLANS = json.load(open(os.path.join(GOLDEN_DIR, "plans.json")))
NAMES = {"token_embedding_table": 0, "rms_att_weight": 1, "wq": 2, "wk": 3, "wv": 4, "wo": 5, "rms_ffn_weight": 6,
         "w1": 7, "w2": 8, "w3": 9, "rms_final_weight": 10, "wcls": 11, "bq": 12, "bk": 13, "bv": 14}


def plan_config(entry):
    dim, hidden, layers, heads, kv_heads, vocab, seq = entry["header"]
    return ol.config(dim=dim, hidden_dim=hidden, n_layers=layers, n_heads=heads, n_kv_heads=kv_heads,
                     head_size=dim // heads, vocab_size=abs(vocab), seq_len=seq, shared_classifier=int(vocab > 0),
                     six=int(entry["dtype"] == "int6"), qkv_bias=int(bool(entry["form"].get("bias"))))


@pytest.mark.parametrize("name", sorted(PLANS))
def test_places_match_the_reference_external_tensors(name):
    """public/llama2_numpy.py:751-795 Places/external_tensors: every tensor's offset (and scales) to the byte, and the
    file size of public/llama2_convert.py:114-122 checkpoint_size"""
    entry = PLANS[name]
    cfg = plan_config(entry)
    tensors, size = ol.places(cfg)
    assert size == entry["size"]
    for tname, plan in entry["tensors"].items():
        if tname in ("freq_cis_real", "freq_cis_imag"):
            continue
        i = NAMES[tname]
        assert tensors[i].offset == plan["offset"], tname
        assert tensors[i].scales == plan["scales"], tname
    if cfg.shared_classifier:
        assert tensors[NAMES["wcls"]].offset == tensors[0].offset


RT = np.load(os.path.join(GOLDEN_DIR, "rope_tables.npz"))


@pytest.mark.parametrize("tag", ["256_48_10000", "256_64_10000", "512_128_500000", "512_128_1000000"])
def test_rope_tables_against_the_reference(tag):
    """public/llama2_numpy.py:484-542 rope_tables() cast to float32: the C float64 cos/sin agree to the bit but for a
    rare last-place difference of the float64 libm (the reference itself holds them only to 1e-6,
    tests/test_quantize.py:54-59); the engine takes whatever tables the caller gives it"""
    seq, hs, theta = (int(v) for v in tag.split("_"))
    cos, sin = ol.rope_tables(seq, hs, float(theta))
    for got, want in ((cos, RT[f"cos_{tag}"]), (sin, RT[f"sin_{tag}"])):
        ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
        assert ulps.max() <= 1
        assert (ulps == 0).mean() > 0.999


def test_synthetic_values_are_standardised_and_deterministic():
    """the generator's moments (mean 0, sd sigma) and its bits from one call to the next"""
    x = ol.synth(1 << 20, seed=5, stream=2, sigma=0.02)
    assert abs(float(x.mean())) < 1e-4 and abs(float(x.std()) - 0.02) < 2e-4
    assert np.array_equal(x[:1000], ol.synth(1000, seed=5, stream=2, sigma=0.02))
    assert np.array_equal(x[500:700], ol.synth(200, seed=5, stream=2, sigma=0.02, first=500))
    assert not np.array_equal(x[:1000], ol.synth(1000, seed=5, stream=3, sigma=0.02))


def test_package_config_structs_match_the_header():
    """the ctypes structs of the package are the layout of include/pyodide_llm_hip.h"""
    import ctypes
    pk = package()
    layout = np.zeros(6, dtype=np.int64)
    ol.load().or_abi_layout(ol.ptr(layout))
    assert ctypes.sizeof(pk.HeConfig) == layout[0]
    assert (pk.HeConfig.rms_norm_eps.offset, pk.HeConfig.arch.offset, pk.HeConfig.outliers.offset) == tuple(layout[1:4])
    assert ctypes.sizeof(pk.HeTensor) == layout[4]
    assert len(pk.TENSORS) == layout[5]


@pytest.mark.parametrize("name", sorted(PLANS))
def test_package_places_equal_the_reference_plans(name):
    """the package's own Places (what bench.py and synthetic engines use) against external_tensors()"""
    entry = PLANS[name]
    cfg = plan_config(entry)
    tensors, size = package().places(cfg)
    assert size == entry["size"]
    for tname, plan in entry["tensors"].items():
        if tname in ("freq_cis_real", "freq_cis_imag"):
            continue
        assert (tensors[NAMES[tname]].offset, tensors[NAMES[tname]].scales) == (plan["offset"], plan["scales"])


@pytest.mark.parametrize("tag", ["256_48_10000", "512_128_500000"])
def test_package_rope_tables_equal_the_reference(tag):
    """NumPy float64 cos/sin cast to float32, as llama2_numpy computes them"""
    seq, hs, theta = (int(v) for v in tag.split("_"))
    cos, sin = package().rope_tables(seq, hs, float(theta))
    assert np.array_equal(cos, RT[f"cos_{tag}"]) and np.array_equal(sin, RT[f"sin_{tag}"])
