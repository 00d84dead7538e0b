"""The tiny models of the other forms (GPT-2, GPT-NeoX, Qwen3, a final norm with outlier channels) whose NumPy-forward
logits tests/golden/numpy_forms.npz holds: their engine configs, RoPE theta, the Llama() keywords the golden script
gave the reference, and their checkpoint bytes (synthetic, vectors varied, outlier channels set)."""
import numpy as np

import oracle_lib

FORM_TINY = {
    # name: (he_config fields, rope theta, Llama() keywords) of the other forms, their vectors varied (vary_vectors)
    "tiny_gpt2_int8": (dict(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=4, head_size=16, vocab_size=320,
                            seq_len=32, shared_classifier=1, six=0, arch=1), 10000.0, dict(arch="gpt2")),
    "tiny_neox_parallel_int8": (dict(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=4, head_size=16,
                                     vocab_size=320, seq_len=32, shared_classifier=0, six=0, arch=2, rotary=8,
                                     parallel_residual=1), 10000.0,
                                dict(arch="neox", rotary=8, parallel_residual=True)),
    "tiny_neox_int6": (dict(dim=64, hidden_dim=96, n_layers=2, n_heads=2, n_kv_heads=2, head_size=32, vocab_size=256,
                            seq_len=32, shared_classifier=1, six=1, arch=2, rotary=16), 10000.0,
                       dict(arch="neox", rotary=16)),
    "tiny_qwen3_int8": (dict(dim=64, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=2, head_size=32, vocab_size=288,
                             seq_len=32, shared_classifier=0, six=0, qk_norm=1, rms_norm_eps=1e-6), 1000000.0,
                        dict(qk_norm=True, head_dim=32, rms_norm_eps=1e-6)),
    "tiny_qwen3_bias_int6": (dict(dim=64, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=1, head_size=32,
                                  vocab_size=288, seq_len=32, shared_classifier=1, six=1, qkv_bias=1, qk_norm=1),
                             1000000.0, dict(bias=True, qk_norm=True, head_dim=32)),
    # a final norm with outlier channels (public/llama2_numpy.py:807-813 finds them; the int8 path multiplies them
    # apart, NumPy's float forward has nothing to do)
    "tiny_llama_outliers_int8": (dict(dim=96, hidden_dim=160, n_layers=2, n_heads=3, n_kv_heads=3, head_size=32,
                                      vocab_size=256, seq_len=32, shared_classifier=0, six=0), 10000.0, dict()),
}
OUTLIERS = {"tiny_llama_outliers_int8": {3: 9.0, 17: -7.5, 40: 8.0, 71: 6.5}}


def form_checkpoint(name):
    """(config, places, checkpoint bytes) of a FORM_TINY model: synthetic, its vectors varied, its outlier channels set"""
    fields = FORM_TINY[name][0]
    cfg = oracle_lib.config(**fields)
    tensors, size = oracle_lib.places(cfg)
    ck = oracle_lib.vary_vectors(cfg, tensors, oracle_lib.synth_checkpoint(cfg, tensors, size, seed=7), seed=11)
    final = tensors[oracle_lib.package().T["rms_final_weight"]].offset
    for channel, value in OUTLIERS.get(name, {}).items():
        ck[final + 4 * channel:final + 4 * channel + 4] = np.frombuffer(np.float32(value).tobytes(), dtype=np.uint8)
    return cfg, tensors, ck


def form_model(name, outliers=True, **extra):
    """(config with the outlier channels the reference finds, places, checkpoint, RoPE tables, channels)"""
    cfg, tensors, ck = form_checkpoint(name)
    fields, theta, _ = FORM_TINY[name]
    pk = oracle_lib.package()
    final = np.frombuffer(ck.tobytes(), dtype=np.float32, count=cfg.dim, offset=tensors[pk.T["rms_final_weight"]].offset)
    channels = oracle_lib.outlier_channels(final) if outliers else []
    cfg = oracle_lib.config(**{**fields, **extra, "outliers": channels})
    cos, sin = pk.rope_tables(cfg.seq_len, cfg.head_size, theta, cfg.rotary if cfg.arch == 2 else 0)
    return cfg, tensors, ck, cos, sin, channels
