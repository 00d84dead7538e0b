"""Writes the golden fixtures of tests/golden/ from the reference's own Python (run in the build container only).

The fixtures pin the functions of the path that no closed form or known-answer test of the reference pins on its
own: the bits of quantize() (public/llama2_convert.py:125-130), quantize6()/pack6()/unpack6()
(public/llama2_numpy.py:678-702), rope_tables() (public/llama2_numpy.py:484-542, the float32 tables a caller hands the
engine), external_tensors() (public/llama2_numpy.py:778-795, where every tensor of a checkpoint is), layout() and
tensor_bytes() of the GPT-2, GPT-NeoX and Qwen3 forms (public/llama2_convert.py:32-83,105-118), and the NumPy
forward's logits on tiny int8/int6 models of every form (public/llama2_numpy.py:1310-1383; the float reference the
int8 path is held to within a line, tests/test_quantize.py:81-90). Inputs are seeded; outputs are stored as NumPy arrays (no pickles)
and JSON. The reference is read from /root/reference/public; it does not travel with the fixtures.

    python tests/golden/make_golden.py [group ...]   (default: every group of GROUPS)
"""
import ctypes
import hashlib
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, "/root/reference/public")

import llama2_convert  # noqa: E402
import llama2_numpy  # noqa: E402

sys.path.insert(0, os.path.join(REPO, "tests"))
import oracle_lib  # noqa: E402
from forms import FORM_TINY, form_checkpoint  # noqa: E402
from tiny import TINY, sharp_checkpoint  # noqa: E402


def save(name, **arrays):
    np.savez(os.path.join(HERE, name), **arrays)


def quantizers():
    rng = np.random.default_rng(20261201)
    out = {}
    for k in (96, 48, 40):  # group 32, 16 and 8 (group_size)
        x = (rng.standard_normal((12, k)) * 0.02).astype(np.float32)
        x[0, :] = 0.0  # a group of zeros: scale 0, inverse 0
        x[1, 3] = 0.5  # a group whose largest value stands out
        values, scales = llama2_convert.quantize(x)
        out[f"q8_x_{k}"], out[f"q8_values_{k}"], out[f"q8_scales_{k}"] = x, values, scales
    x = rng.standard_normal((6, 64)).astype(np.float32)
    x[0, :32] = 0.0
    ints, scales = llama2_numpy.quantize6(x)
    out["q6_x"], out["q6_ints"], out["q6_scales"], out["q6_packed"] = x, ints, scales, llama2_numpy.pack6(ints)
    raw = rng.integers(0, 256, size=(64, 24), dtype=np.uint8)
    out["six_raw"], out["six_values"] = raw, llama2_numpy.unpack6(raw)
    save("quantizers.npz", **out)


def ropes():
    out = {}
    for seq, hs, theta in ((256, 48, 10000.0), (256, 64, 10000.0), (512, 128, 500000.0), (512, 128, 1000000.0)):
        cos, sin = llama2_numpy.rope_tables(seq, hs, theta)
        tag = f"{seq}_{hs}_{int(theta)}"
        out[f"cos_{tag}"], out[f"sin_{tag}"] = cos.astype(np.float32), sin.astype(np.float32)
    save("rope_tables.npz", **out)


CONFIGS = {
    # name: (header, dtype, form)
    "stories15m_int8": ((288, 768, 6, 6, 6, 32000, 256), "int8", None),
    "llm150m_int8": ((512, 2048, 12, 8, 8, 99487, 1024), "int8", None),
    "llama3_8b_int8": ((4096, 14336, 32, 32, 8, -128256, 4096), "int8", None),
    "qwen25_7b_int6": ((3584, 18944, 28, 28, 4, -152064, 2048), "int6", {"bias": True}),
    "tiny_gqa_int8": ((64, 128, 2, 4, 2, 320, 32), "int8", None),
}


def plans():
    out = {}
    for name, (header, dtype, form) in CONFIGS.items():
        tensors = llama2_numpy.external_tensors(header, dtype, form)
        size = llama2_convert.checkpoint_size(header, dtype, form)
        out[name] = {"header": list(header), "dtype": dtype, "form": form or {}, "size": int(size),
                     "tensors": tensors}
    with open(os.path.join(HERE, "plans.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


FORMS = {
    # name: (header, dtype, form) of the other forms (public/llama2_convert.py:32-83)
    "gpt2_int8": ((64, 128, 2, 4, 4, 320, 32), "int8", {"arch": "gpt2"}),
    "gpt2_int6_own_cls": ((64, 96, 2, 2, 2, -256, 32), "int6", {"arch": "gpt2"}),
    "neox_int8": ((64, 128, 2, 4, 4, -320, 32), "int8", {"arch": "neox"}),
    "qwen3_int8": ((64, 96, 2, 4, 2, -288, 32), "int8", {"qk_norm": True, "head_dim": 32}),
    "qwen3_bias_int6": ((64, 96, 2, 4, 1, 288, 32), "int6", {"bias": True, "qk_norm": True}),
}


def layouts():
    """llama2_convert.layout() of every form: shape, whether a matrix, and the offset and bytes tensor_bytes() gives
    each tensor in file order (the RoPE tables of an int8 file take none)"""
    out = {}
    for name, (header, dtype, form) in FORMS.items():
        offset, entries = 28, []
        for shape, is_matrix in llama2_convert.layout(*header, **form):
            size = llama2_convert.tensor_bytes(shape, is_matrix, dtype)
            entries.append({"shape": list(shape), "matrix": is_matrix, "offset": offset, "bytes": int(size)})
            offset += size
        out[name] = {"header": list(header), "dtype": dtype, "form": form, "layout": entries,
                     "size": int(llama2_convert.checkpoint_size(header, dtype, form))}
    with open(os.path.join(HERE, "layouts.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


def tokenizer_bytes(vocab):
    """llama2.c's tokenizer.bin (tests/conftest.py:172-176): the pieces are placeholders, never decoded here."""
    pieces = [(0.0, b"<unk>"), (0.0, b"<s>"), (0.0, b"</s>")] + [(0.0, b"<p%d>" % i) for i in range(3, vocab)]
    out = [struct.pack("<i", max(len(p) for _, p in pieces))]
    out += [struct.pack("<fi", s, len(p)) + p for s, p in pieces]
    return b"".join(out)


TOKENS = [1, 5, 9, 3, 7, 200, 11, 4]


def forwards():
    out = {}
    for name, (fields, theta) in TINY.items():
        cfg = oracle_lib.config(**fields)
        tensors, size = oracle_lib.places(cfg)
        ck = oracle_lib.synth_checkpoint(cfg, tensors, size, seed=7)
        dtype = "int6" if fields["six"] else "int8"
        model = llama2_numpy.Llama(bytes(ck), tokenizer_bytes(fields["vocab_size"]), dtype=dtype, rope_theta=theta,
                                   bias=bool(fields["qkv_bias"]))
        logits = np.stack([model.forward(tok, pos).astype(np.float32) for pos, tok in enumerate(TOKENS)])
        out[f"logits_{name}"] = logits
        out[f"sha256_{name}"] = np.frombuffer(hashlib.sha256(bytes(ck)).digest(), dtype=np.uint8)
    out["tokens"] = np.array(TOKENS, dtype=np.int32)
    save("numpy_forward.npz", **out)


def sharp_forwards():
    """the NumPy forward's logits on the TINY models with attention that leans on a few keys (sharp_checkpoint)"""
    out = {}
    for name, (fields, theta) in TINY.items():
        _, _, ck, _, _, tokens = sharp_checkpoint(name)
        dtype = "int6" if fields["six"] else "int8"
        model = llama2_numpy.Llama(bytes(ck), tokenizer_bytes(fields["vocab_size"]), dtype=dtype, rope_theta=theta,
                                   bias=bool(fields["qkv_bias"]))
        out[f"logits_{name}"] = np.stack([model.forward(tok, pos).astype(np.float32) for pos, tok in enumerate(tokens)])
        out[f"tokens_{name}"] = np.array(tokens, dtype=np.int32)
        out[f"sha256_{name}"] = np.frombuffer(hashlib.sha256(bytes(ck)).digest(), dtype=np.uint8)
    save("numpy_forward_sharp.npz", **out)


def form_forwards():
    out = {}
    for name, (fields, theta, keywords) in FORM_TINY.items():
        cfg, _, ck = form_checkpoint(name)
        dtype = "int6" if fields["six"] else "int8"
        model = llama2_numpy.Llama(bytes(ck), tokenizer_bytes(fields["vocab_size"]), dtype=dtype, rope_theta=theta,
                                   **keywords)
        logits = np.stack([model.forward(tok, pos).astype(np.float32) for pos, tok in enumerate(TOKENS)])
        out[f"logits_{name}"] = logits
        out[f"sha256_{name}"] = np.frombuffer(hashlib.sha256(bytes(ck)).digest(), dtype=np.uint8)
    out["tokens"] = np.array(TOKENS, dtype=np.int32)
    save("numpy_forms.npz", **out)


GROUPS = {"quantizers": quantizers, "ropes": ropes, "plans": plans, "forwards": forwards, "layouts": layouts,
          "form_forwards": form_forwards, "sharp_forwards": sharp_forwards}

if __name__ == "__main__":
    oracle_lib.load()
    for group in sys.argv[1:] or list(GROUPS):
        GROUPS[group]()
    print("golden fixtures written to", HERE)
