"""ctypes over oracle/liboracle.so — TEST INFRASTRUCTURE (the parity reference and the CPU baseline), never the product."""
import ctypes
import os

import numpy as np

from paths import ORACLE_DIR, package

LIB = os.path.join(ORACLE_DIR, "liboracle.so")
_lib = None
P, I32, I64, U64, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built (make -C oracle)")
        pk = package()
        lib = ctypes.CDLL(LIB)
        cfgp, tp = ctypes.POINTER(pk.HeConfig), ctypes.POINTER(pk.HeTensor)
        sig = {
            "or_mix64": (U64, [U64]),
            "or_synth_factor": (F, [ctypes.c_double]),
            "or_synth_value": (F, [U64, I32, U64, F]),
            "or_synth_fill": (None, [P, U64, U64, I32, U64, ctypes.c_double]),
            "or_group_size": (I32, [I32]),
            "or_quantize": (None, [P, P, P, I64, I32]),
            "or_quantize6": (None, [P, P, P, I64]),
            "or_pack6": (None, [P, P, I64]),
            "or_unpack6": (None, [P, P, I64]),
            "or_quantize_x": (None, [P, P, P, I32, I32]),
            "or_matmul_q8r": (None, [P, P, P, P, P, I32, I32, I32]),
            "or_matmul_q8": (None, [P, P, P, P, P, I32, I32, I32]),
            "or_matmul_q6r": (None, [P, P, P, P, P, I32, I32, I32]),
            "or_matmul_q6": (None, [P, P, P, P, P, I32, I32, I32]),
            "or_group_sums": (None, [P, P, P, I32, I32, I32, I32]),
            "or_matmul": (None, [P, P, P, P, P, I32, I32, I32, I32, I32]),
            "or_rmsnorm": (None, [P, P, P, I32, F]),
            "or_rope": (None, [P, P, P, I32, I32, I32]),
            "or_attention": (None, [P, P, P, P, P, I32, I32, I32, I32, I32, I32, I32]),
            "or_to_f16": (None, [P, P, I32]),
            "or_from_f16": (None, [P, P, I32]),
            "or_fexp": (F, [F]),
            "or_vexp": (None, [P, I32]),
            "or_swiglu": (None, [P, P, P, I32]),
            "or_layernorm": (None, [P, P, P, P, I32]),
            "or_gelu": (None, [P, P, P, I32]),
            "or_add_columns": (None, [P, P, P, I32, I32]),
            "or_add": (None, [P, P, I32]),
            "or_argmax": (I32, [P, I32]),
            "or_penalize": (None, [P, P, I32, F]),
            "or_sample": (I32, [P, I32, F, F, ctypes.c_double, P, P, P]),
            "or_places": (I64, [cfgp, tp]),
            "or_synth_checkpoint": (None, [cfgp, tp, P, I64, U64]),
            "or_rope_tables": (None, [P, P, I32, I32, ctypes.c_double]),
            "or_model_open": (P, [cfgp, tp, P, P, P, I32]),
            "or_model_run": (I32, [P, P, I32, I32, I32]),
            "or_model_logits": (P, [P]),
            "or_model_kv": (None, [P, I32, I32, P, P]),
            "or_model_close": (None, [P]),
            "or_generate": (I32, [P, P, I32, I32, I32, P, P]),
            "or_abi_layout": (None, [P]),
            "or_set_threads": (None, [I32]),
            "or_get_threads": (I32, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    return _lib


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def config(**fields):
    return package().config(**fields)


def places(cfg):
    t = package().TensorArray()
    size = load().or_places(ctypes.byref(cfg), t)
    return t, int(size)


def synth_checkpoint(cfg, tensors, size, seed=0):
    out = np.zeros(size, dtype=np.uint8)
    load().or_synth_checkpoint(ctypes.byref(cfg), tensors, ptr(out), size, seed)
    return out


def rope_tables(seq_len, hs, theta):
    cos = np.zeros((seq_len, hs // 2), dtype=np.float32)
    sin = np.zeros_like(cos)
    load().or_rope_tables(ptr(cos), ptr(sin), seq_len, hs, theta)
    return cos, sin


def synth(n, seed, stream, sigma, first=0):
    out = np.zeros(n, dtype=np.float32)
    load().or_synth_fill(ptr(out), n, seed, stream, first, sigma)
    return out


def quantize(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    group = load().or_group_size(k)
    q = np.zeros(x.shape, dtype=np.int8)
    s = np.zeros(x.size // group, dtype=np.float32)
    load().or_quantize(ptr(q), ptr(s), ptr(x), x.size, group)
    return q, s


def quantize6(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.shape, dtype=np.int8)
    s = np.zeros(x.size // 32, dtype=np.float32)
    load().or_quantize6(ptr(q), ptr(s), ptr(x), x.size // 32)
    return q, s


def pack6(q):
    q = np.ascontiguousarray(q, dtype=np.int8)
    out = np.zeros((q.size // 32, 24), dtype=np.uint8)
    load().or_pack6(ptr(out), ptr(q), q.size // 32)
    return out


def unpack6(raw):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros((raw.size // 24, 32), dtype=np.int8)
    load().or_unpack6(ptr(out), ptr(raw), raw.size // 24)
    return out


def quantize_x(x, bias):
    """rows of x ([m][n] or [n]) -> (int8 [m][n], scales [m][n/32])"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.reshape(-1, x.shape[-1])
    n = rows.shape[1]
    q = np.zeros(rows.shape, dtype=np.int8)
    s = np.zeros((rows.shape[0], n // 32), dtype=np.float32)
    for i in range(rows.shape[0]):
        load().or_quantize_x(ptr(q[i]), ptr(s[i]), ptr(rows[i]), n, bias)
    return q.reshape(x.shape), s.reshape(x.shape[:-1] + (n // 32,))


def matmul(xq, xs, w, ws, rows, k, bias, six):
    """y [m][rows] of the oracle's matmul_q8r / q8 / q6r / q6"""
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, k)
    xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1, k // 32)
    m = xq.shape[0]
    y = np.zeros((m, rows), dtype=np.float32)
    w = np.ascontiguousarray(w)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    load().or_matmul(ptr(y), ptr(xq), ptr(xs), ptr(w), ptr(ws), m, rows, k, bias, six)
    return y


def group_sums(xq, w, rows, k, bias, six):
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, k)
    per = (k // 32) * (1 if bias else 4)
    out = np.zeros((xq.shape[0], rows, per), dtype=np.int32)
    w = np.ascontiguousarray(w)
    for t in range(xq.shape[0]):
        load().or_group_sums(ptr(out[t]), ptr(xq[t]), ptr(w), rows, k, bias, six)
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    load().or_rmsnorm(ptr(out), ptr(x), ptr(np.ascontiguousarray(w, dtype=np.float32)), x.size, eps)
    return out


def fexp(x):
    return load().or_fexp(float(x))


def vexp(x):
    x = np.array(x, dtype=np.float32)
    load().or_vexp(ptr(x), x.size)
    return x


def to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size, dtype=np.uint16)
    load().or_to_f16(ptr(out), ptr(x), x.size)
    return out


def from_f16(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.zeros(h.size, dtype=np.float32)
    load().or_from_f16(ptr(out), ptr(h), h.size)
    return out


def attention(q, kc, vc, pos, nh, nkv, hs, half=False):
    """one token's attention at position pos over the cache rows 0..pos"""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc)
    vc = np.ascontiguousarray(vc)
    out = np.zeros(nh * hs, dtype=np.float32)
    att = np.zeros(nh * (pos + 1), dtype=np.float32)
    load().or_attention(ptr(out), ptr(q), ptr(kc), ptr(vc), ptr(att), pos, nh, nkv, hs, 0, nh, int(half))
    return out


class Model:
    """or_model: the reference's run() on the host"""

    def __init__(self, cfg, tensors, checkpoint, cos, sin, max_block=64):
        self.cfg = cfg
        self._ck = np.ascontiguousarray(checkpoint, dtype=np.uint8)
        self._cos = np.ascontiguousarray(cos, dtype=np.float32)
        self._sin = np.ascontiguousarray(sin, dtype=np.float32)
        self.max_block = max_block
        self._h = load().or_model_open(ctypes.byref(cfg), tensors, ptr(self._ck), ptr(self._cos), ptr(self._sin),
                                       max_block)

    def run(self, tokens, pos0, need_logits):
        ids = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        code = load().or_model_run(self._h, ptr(ids), ids.size, pos0, int(need_logits))
        if code:
            raise RuntimeError("or_model_run refused the call")

    def logits(self):
        p = load().or_model_logits(self._h)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)),
                                     shape=(self.cfg.vocab_size,)).copy()

    def kv(self, start, count):
        kv_dim = self.cfg.n_kv_heads * self.cfg.head_size
        keys = np.zeros((self.cfg.n_layers, count, kv_dim), dtype=np.float32)
        values = np.zeros_like(keys)
        load().or_model_kv(self._h, start, count, ptr(keys), ptr(values))
        return keys, values

    def generate(self, prompt, steps, block=None):
        prompt = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        out = np.zeros(max(steps, 1), dtype=np.int32)
        logits = np.zeros(self.cfg.vocab_size, dtype=np.float32)
        n = load().or_generate(self._h, ptr(prompt), prompt.size, steps, block or self.max_block, ptr(out),
                               ptr(logits))
        if n < 0:
            raise RuntimeError("or_generate refused the call")
        return out[:n], logits

    def close(self):
        if self._h:
            load().or_model_close(self._h)
            self._h = None

    def __del__(self):
        self.close()


def penalize(logits, tokens, penalty):
    """kernels/kernel.ts:705-719 on a float32 copy"""
    out = np.ascontiguousarray(np.asarray(logits, dtype=np.float32)).copy()
    t = np.ascontiguousarray(np.asarray(list(tokens), dtype=np.int32))
    load().or_penalize(ptr(out), ptr(t), t.size, float(penalty))
    return out


def sample(logits, temperature, topp, random):
    """kernels/kernel.ts:803-868: the token drawn for one random number in [0, 1), -1 for logits that are not finite"""
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    probs = np.zeros(x.size, dtype=np.float32)
    index = np.zeros(x.size, dtype=np.int32)
    order = np.zeros(x.size, dtype=np.int32)
    return int(load().or_sample(ptr(x), x.size, float(temperature), float(topp), float(random), ptr(probs),
                                ptr(index), ptr(order)))


NORM_WEIGHTS = ("rms_att_weight", "rms_ffn_weight", "rms_final_weight", "q_norm", "k_norm")
BIASES = ("bq", "bk", "bv", "ln_att_bias", "ln_ffn_bias", "ln_final_bias", "bo", "b1", "b2")


def vector_length(cfg, name):
    """the float32 count of a vector tensor of the checkpoint"""
    L, dim, hidden, hs = cfg.n_layers, cfg.dim, cfg.hidden_dim, cfg.head_size
    qdim, kvdim = cfg.n_heads * hs, cfg.n_kv_heads * hs
    return {"rms_att_weight": L * dim, "rms_ffn_weight": L * dim, "rms_final_weight": dim, "q_norm": L * hs,
            "k_norm": L * hs, "bq": L * qdim, "bk": L * kvdim, "bv": L * kvdim, "ln_att_bias": L * dim,
            "ln_ffn_bias": L * dim, "ln_final_bias": dim, "bo": L * dim, "b1": L * hidden, "b2": L * dim}[name]


def vary_vectors(cfg, tensors, ck, seed):
    """in place: the checkpoint's norm weights 1 + 0.25 N(0, 1) and its biases 0.2 N(0, 1) (NumPy's default_rng(seed)),
    so that a dropped or misplaced weight or bias shows in the logits"""
    rng = np.random.default_rng(seed)
    T = package().T
    for name in NORM_WEIGHTS + BIASES:
        t = tensors[T[name]]
        if t.offset == 0:
            continue  # not in this form
        n = vector_length(cfg, name)
        values = (1.0 + 0.25 * rng.standard_normal(n)) if name in NORM_WEIGHTS else 0.2 * rng.standard_normal(n)
        ck[t.offset:t.offset + 4 * n] = np.frombuffer(values.astype(np.float32).tobytes(), dtype=np.uint8)
    return ck


def sharpen(cfg, tensors, ck, factor):
    """in place: the scales of every layer's wq and wk times factor (their int8 / int6 values kept), so that q . k /
    sqrt(head_size) spans a few units and each position's attention leans on a few keys: where attention is near
    uniform (N(0, 0.02) weights), a rotation turned the wrong way or a misplaced pair hardly moves the logits"""
    T = package().T
    for name, rows in (("wq", cfg.n_heads * cfg.head_size), ("wk", cfg.n_kv_heads * cfg.head_size)):
        t = tensors[T[name]]
        n = cfg.n_layers * rows * (cfg.dim // 32)
        scales = np.frombuffer(ck[t.scales:t.scales + 4 * n].tobytes(), dtype=np.float32) * np.float32(factor)
        ck[t.scales:t.scales + 4 * n] = np.frombuffer(scales.astype(np.float32).tobytes(), dtype=np.uint8)
    return ck


def outlier_channels(weight, count=8, ratio=4.0):
    """public/llama2_numpy.py:807-813: the count channels with the largest |final-norm weight|, in order, or none where
    the largest is below ratio times the median"""
    size = np.abs(np.asarray(weight, dtype=np.float32))
    if size.max() < ratio * np.median(size):
        return []
    return sorted(int(c) for c in np.argsort(-size, kind="stable")[:count])
