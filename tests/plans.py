"""Plans as Llama.external_forward hands them to forward.js (public/llama2_numpy.py:1261-1270), made from an engine
config and its tensor places, for the hosts' tests."""
import numpy as np

NAMES = ("token_embedding_table", "rms_att_weight", "wq", "wk", "wv", "wo", "rms_ffn_weight", "w1", "w2", "w3",
         "rms_final_weight", "wcls", "bq", "bk", "bv")


def shapes(cfg):
    L, d, h, v = cfg.n_layers, cfg.dim, cfg.hidden_dim, cfg.vocab_size
    q, kv = cfg.n_heads * cfg.head_size, cfg.n_kv_heads * cfg.head_size
    return {"token_embedding_table": ([v, d], True), "rms_att_weight": ([L, d], False), "wq": ([L, q, d], True),
            "wk": ([L, kv, d], True), "wv": ([L, kv, d], True), "wo": ([L, d, q], True),
            "rms_ffn_weight": ([L, d], False), "w1": ([L, h, d], True), "w2": ([L, d, h], True),
            "w3": ([L, h, d], True), "rms_final_weight": ([d], False), "wcls": ([v, d], True),
            "bq": ([L, q], False), "bk": ([L, kv], False), "bv": ([L, kv], False)}


def plan_of(cfg, tensors, theta=10000.0):
    """the plan dict (without derived: the RoPE tables go beside it)"""
    six = bool(cfg.six)
    out = {}
    for i, name in enumerate(NAMES):
        if name == "wcls" and cfg.shared_classifier:
            continue
        if name in ("bq", "bk", "bv") and not cfg.qkv_bias:
            continue
        shape, matrix = shapes(cfg)[name]
        t = tensors[i]
        if matrix:
            out[name] = {"kind": "int6" if six else "int8", "offset": int(t.offset), "shape": shape, "group": 32,
                         "scales": int(t.scales)}
        else:
            out[name] = {"kind": "f32", "offset": int(t.offset), "shape": shape, "group": 0, "scales": 0}
    return {"arch": "llama", "dim": cfg.dim, "hidden_dim": cfg.hidden_dim, "n_layers": cfg.n_layers,
            "n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads, "head_size": cfg.head_size,
            "vocab_size": cfg.vocab_size, "seq_len": cfg.seq_len, "rotary": 0, "parallel_residual": False,
            "kv_start": 256, "rms_norm_eps": float(np.float32(cfg.rms_norm_eps)),
            "shared_classifier": bool(cfg.shared_classifier), "int8": True, "relaxed": bool(cfg.relaxed),
            "tensors": out, "outliers": [], "half_kv": bool(cfg.half_kv), "form": {}}
