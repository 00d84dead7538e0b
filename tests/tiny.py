"""The tiny Llama-form models whose NumPy-forward logits tests/golden/numpy_forward.npz and numpy_forward_sharp.npz
hold: their engine configs and RoPE theta, and the sensitive variant of their checkpoints."""
import numpy as np

import oracle_lib

TINY = {
    # name: (he_config fields, rope theta)
    "tiny_gqa_int8": (dict(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2, head_size=16, vocab_size=320,
                           seq_len=32, shared_classifier=1, six=0, qkv_bias=0), 10000.0),
    "tiny_mha_own_cls_int8": (dict(dim=96, hidden_dim=160, n_layers=2, n_heads=3, n_kv_heads=3, head_size=32,
                                   vocab_size=256, seq_len=32, shared_classifier=0, six=0, qkv_bias=0), 10000.0),
    "tiny_qwen_int6": (dict(dim=64, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=1, head_size=16, vocab_size=288,
                            seq_len=32, shared_classifier=0, six=1, qkv_bias=1), 1000000.0),
}
SHARP_TOKENS = 24
SHARP_FACTOR = 5.0


def sharp_checkpoint(name, **extra):
    """(config, places, checkpoint bytes, RoPE tables, tokens) of a TINY model made sensitive to attention and RoPE:
    its norm weights and biases varied, its q / k scales times SHARP_FACTOR (attention leans on a few keys), and
    SHARP_TOKENS positions to feed"""
    fields, theta = TINY[name]
    cfg = oracle_lib.config(**{**fields, **extra})
    tensors, size = oracle_lib.places(cfg)
    ck = oracle_lib.synth_checkpoint(cfg, tensors, size, seed=7)
    oracle_lib.vary_vectors(cfg, tensors, ck, seed=13)
    oracle_lib.sharpen(cfg, tensors, ck, SHARP_FACTOR)
    cos, sin = oracle_lib.rope_tables(cfg.seq_len, cfg.head_size, theta)
    rng = np.random.default_rng(99)
    tokens = [1] + [int(t) for t in rng.integers(3, cfg.vocab_size, size=SHARP_TOKENS - 1)]
    return cfg, tensors, ck, cos, sin, tokens
