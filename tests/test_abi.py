"""The drop-in boundary without a GPU: the built library loads and exports every entry point include/*.h declares,
and the package's plan conversion refuses the forms the engine does not run (as public/forward.js throws)."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

from paths import REPO, package


def declared():
    names = []
    for header in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(he_[a-z_]+|hk_[a-z_]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_engine_and_kernel_entry_points():
    names = declared()
    for name in ("he_open", "he_forward", "he_forward_many", "he_generate_many", "he_logits", "he_kv_read",
                 "he_close", "hk_matmul", "hk_quantize_x", "hk_group_sums", "hk_penalize", "hk_sample"):
        assert name in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(package().hip_engine.LIBRARY)
    for name in declared():
        assert hasattr(lib, name), name


def test_plan_conversion_takes_the_reference_plan_and_refuses_other_forms():
    pk = package()
    tensors = {name: {"kind": "int8", "offset": 28 + i * 1000, "shape": [1], "group": 32, "scales": 28 + i * 1000 + 500}
               for i, name in enumerate(("token_embedding_table", "wq", "wk", "wv", "wo", "w1", "w2", "w3"))}
    for i, name in enumerate(("rms_att_weight", "rms_ffn_weight", "rms_final_weight")):
        tensors[name] = {"kind": "f32", "offset": 50000 + i * 100, "shape": [1], "group": 0, "scales": 0}
    plan = {"arch": "llama", "dim": 64, "hidden_dim": 128, "n_layers": 2, "n_heads": 4, "n_kv_heads": 2,
            "head_size": 16, "vocab_size": 320, "seq_len": 32, "rotary": 0, "parallel_residual": False,
            "kv_start": 256, "rms_norm_eps": 1e-5, "shared_classifier": True, "int8": True, "relaxed": True,
            "tensors": tensors, "derived": {}, "outliers": [], "half_kv": True, "form": {}}
    cfg, t = pk.plan_to_config(plan)
    # a grouped-query model keeps float32 keys and values unless told otherwise (public/forward.js:762)
    assert (cfg.dim, cfg.n_kv_heads, cfg.relaxed, cfg.half_kv, cfg.six, cfg.qkv_bias) == (64, 2, 1, 0, 0, 0)
    assert pk.plan_to_config(plan, half_keys=True)[0].half_kv == 1
    assert pk.plan_to_config({**plan, "n_kv_heads": 4})[0].half_kv == 1
    assert t[pk.T["wcls"]].offset == tensors["token_embedding_table"]["offset"]
    for change in ({"arch": "qwen35"}, {"int8": False}, {"rotary": 8}, {"outliers": list(range(9))}):
        with pytest.raises(pk.HipError):
            pk.plan_to_config({**plan, **change})
    # the other forms: outliers, Qwen3's head norms, GPT-2 (its positions), GPT-NeoX (partial rotary, parallel)
    c, _ = pk.plan_to_config({**plan, "outliers": [40, 3]})
    assert (c.n_outliers, list(c.outliers)[:2]) == (2, [3, 40])
    norms = {name: {"kind": "f32", "offset": 60000 + i * 100, "shape": [2, 16], "group": 0, "scales": 0}
             for i, name in enumerate(("q_norm", "k_norm"))}
    assert pk.plan_to_config({**plan, "tensors": {**tensors, **norms}})[0].qk_norm == 1
    assert pk.plan_to_config({**plan, "parallel_residual": True})[0].parallel_residual == 0  # llama: not read
    with pytest.raises(KeyError):
        pk.plan_to_config({**plan, "arch": "gpt2"})  # a GPT-2 plan places its positions
    gpt2 = {**tensors, "positions": dict(tensors["wq"], offset=70000, scales=70500)}
    c, t = pk.plan_to_config({**plan, "arch": "gpt2", "tensors": gpt2, "rotary": 8})
    assert (c.arch, c.rotary, t[pk.T["positions"]].offset) == (1, 0, 70000)
    c, _ = pk.plan_to_config({**plan, "arch": "neox", "rotary": 8, "parallel_residual": True})
    assert (c.arch, c.rotary, c.parallel_residual) == (2, 8, 1)


def test_open_refuses_a_context_past_the_attention_kernels():
    """a (token, head)'s exponentials are summed in order from one block's LDS (160 KiB): he_open refuses a seq_len
    past what that holds (40704 positions) before it touches the device"""
    pk = package()
    lib = pk.library()
    cfg = pk.config(dim=64, hidden_dim=128, n_layers=1, n_heads=4, n_kv_heads=4, head_size=16, vocab_size=64,
                    seq_len=40708, shared_classifier=1)
    tables = np.zeros(16, dtype=np.float32)
    p = ctypes.c_void_p(tables.ctypes.data)
    h = ctypes.c_void_p()
    rc = lib.he_open(ctypes.byref(cfg), pk.TensorArray(), p, 16, p, p, 1, ctypes.byref(h))
    assert rc == pk.hip_engine.HE_E_ARG and not h.value
    assert b"seq_len is longer than the attention kernels take (40704 positions)" in lib.he_last_error()
