"""The Python side of the MI355X forward engine: ctypes over libpyodide_llm_hip.so (include/pyodide_llm_hip.h).

It offers what public/forward.js offers its Python caller (public/llama2_numpy.py:1248-1298 external_forward):
`external(checkpoint)` returns an object with `size`, `read(offset, length)` and `start(plan)`; `start` takes the plan
dict Llama.external_forward builds (public/llama2_numpy.py:1261-1270) and returns an engine with `backend`, `bind`,
`forward`, `forwardMany`, `promptBlock`, `tokenBlock`, `generateMany`, `logits`, `keysAndValues`, `memoryBytes` and
`release` (public/forward.js:1676-1955). So `llama2_numpy.Llama(None, tokenizer, dtype="int8", external=external(ck))`
runs its forward passes here. The engine never falls back to the CPU: without the built library it raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libpyodide_llm_hip.so")

# include/pyodide_llm_hip.h HE_T_*: the tensors the forward reads, by their plan names (public/llama2_numpy.py
# TENSOR_NAMES)
TENSORS = ("token_embedding_table", "rms_att_weight", "wq", "wk", "wv", "wo", "rms_ffn_weight", "w1", "w2", "w3",
           "rms_final_weight", "wcls", "bq", "bk", "bv", "q_norm", "k_norm", "positions", "ln_att_bias", "ln_ffn_bias",
           "ln_final_bias", "bo", "b1", "b2")
ARCHS = {"llama": 0, "gpt2": 1, "neox": 2}  # include/pyodide_llm_hip.h HE_ARCH_*
OUTLIERS_MOST = 8  # HE_OUTLIERS_MOST (public/llama2_numpy.py:561 OUTLIER_CHANNELS)
T = {name: i for i, name in enumerate(TENSORS)}
HE_OK, HE_E_ARG, HE_E_HIP, HE_E_STATE, HE_E_NOTFINITE = 0, -1, -2, -3, -4
KINDS = ("gemv", "gemm", "attention", "norm", "elementwise", "argmax")  # include/pyodide_llm_hip.h HE_K_*
NOT_FINITE = ("The model computed logits that are not finite numbers (NaN or infinity), so no token can be drawn: "
              "its weights are broken or its numbers overflowed.")  # public/llama2_numpy.py:548


class HeConfig(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in (
        "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_size", "vocab_size", "seq_len",
        "shared_classifier", "six", "qkv_bias", "relaxed", "half_kv")] + [("rms_norm_eps", ctypes.c_float)] + [
        (name, ctypes.c_int32) for name in ("arch", "rotary", "parallel_residual", "qk_norm", "n_outliers")] + [
        ("outliers", ctypes.c_int32 * OUTLIERS_MOST)]


class HeTensor(ctypes.Structure):
    _fields_ = [("offset", ctypes.c_int64), ("scales", ctypes.c_int64)]


TensorArray = HeTensor * len(TENSORS)


def config(**fields):
    """an HeConfig from keyword fields; relaxed defaults to 1 (bias 64, the reference's default path), eps 1e-5;
    outliers takes a list of channels"""
    c = HeConfig()
    c.relaxed = 1
    c.rms_norm_eps = 1e-5
    for key, value in fields.items():
        if key == "outliers":
            c.n_outliers = len(value)
            for i, channel in enumerate(value):
                c.outliers[i] = int(channel)
        elif key == "arch" and isinstance(value, str):
            c.arch = ARCHS[value]
        else:
            setattr(c, key, value)
    if c.head_size == 0 and c.n_heads:
        c.head_size = c.dim // c.n_heads
    return c


class HipError(RuntimeError):
    """a failed engine call, with the message of he_last_error()"""


_lib = None


def library():
    """libpyodide_llm_hip.so, loaded once; a missing library is an error, never a quiet fallback"""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise HipError(f"{LIBRARY} is not built: run __graft_entry__.build() (hipcc for gfx950) first")
        lib = ctypes.CDLL(LIBRARY)
        P, I32, I64, U64, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float
        sig = {
            "he_last_error": (ctypes.c_char_p, []),
            "he_open": (I32, [ctypes.POINTER(HeConfig), ctypes.POINTER(HeTensor), P, U64, P, P, I32,
                              ctypes.POINTER(P)]),
            "he_open_synthetic": (I32, [ctypes.POINTER(HeConfig), ctypes.POINTER(HeTensor), U64, U64, P, P, I32,
                                        ctypes.POINTER(P)]),
            "he_forward": (I32, [P, I32, I32, I32, P]),
            "he_forward_many": (I32, [P, P, I32, I32]),
            "he_generate_many": (I32, [P, I32, I32, P, I32, I32, I32, F, F, F, P, I32, P, I32, P, P]),
            "he_logits": (I32, [P, P]),
            "he_kv_read": (I32, [P, I32, I32, P, P]),
            "he_checkpoint_read": (I32, [P, U64, U64, P]),
            "he_prompt_block": (I32, [P]),
            "he_device_bytes": (U64, [P]),
            "he_close": (I32, [P]),
            "he_profile_forward": (I32, [P, I32, I32, I32, P, P, P]),
            "he_profile_forward_many": (I32, [P, P, I32, I32, P, P, P]),
            "he_profile_matmul": (I32, [P, I32, I32, P, P, P]),
            "hk_quantize_x": (I32, [P, P, P, I32, I32, I32, P]),
            "hk_matmul": (I32, [P, P, P, P, P, I32, I32, I32, I32, I32, P]),
            "hk_group_sums": (I32, [P, P, P, I32, I32, I32, I32, I32, I32, P]),
            "hk_penalize": (I32, [P, I32, P, I32, F, P]),
            "hk_ordered_sum": (I32, [P, I32, I32, P, P, P]),
            "hk_sample": (I32, [P, I32, F, F, ctypes.c_double, P, P]),
            "hk_sample_static": (I32, [P, I32, F, F, ctypes.c_double, P, P]),
            "hk_read_ceiling": (I32, [P, ctypes.c_int64, I32, P, P, P]),
            "hk_read_floor": (I32, [P, ctypes.c_int64, ctypes.c_int64, I32, P, P]),
            "hk_valu_ceiling": (I32, [I32, F, F, F, P, P, P, P]),
            "hk_mfma_ceiling": (I32, [I32, I32, I32, I32, P, P, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        del I64
        _lib = lib
    return _lib


def check(code):
    if code != HE_OK:
        message = library().he_last_error().decode()
        if code == HE_E_NOTFINITE:
            raise ValueError(NOT_FINITE)
        raise HipError(f"engine call failed ({code}): {message}")
    return code


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def plan_to_config(plan, half_keys=None):
    """he_config and he_tensor[] from a plan dict (public/llama2_numpy.py:1261-1270): the llama form (with Qwen2's
    biases and Qwen3's head norms where the tensors are there), gpt2 and neox (public/forward.js:636); forms the engine
    does not take are refused by name, as public/forward.js refuses what its kernels cannot run. Keys and values are
    float16 where the plan allows it and every head has its own (or half_keys says so): public/forward.js:762"""
    arch = plan.get("arch", "llama")
    if arch not in ARCHS:
        raise HipError(f"the engine runs the llama, gpt2 and neox forms, not {arch}")
    if not plan.get("int8"):
        raise HipError("the engine multiplies int8/int6 matrices only (plan.int8)")
    tensors = plan["tensors"]
    layer_norm = arch != "llama"
    names = ("wq", "wk", "wv", "wo", "w1", "w2", "token_embedding_table") + (() if layer_norm else ("w3",)) + (
        ("positions",) if arch == "gpt2" else ())
    kinds = {tensors[name]["kind"] for name in names}
    if not kinds <= {"int8", "int6"} or len(kinds) != 1:
        raise HipError(f"the engine takes int8 or int6 matrices, not {sorted(kinds)}")
    six = kinds == {"int6"}
    rotary = int(plan.get("rotary") or 0)
    if arch == "llama" and rotary and rotary != plan["head_size"]:
        raise HipError("partial rotary embeddings belong to the neox form")
    outliers = sorted(int(channel) for channel in (plan.get("outliers") or []))
    if len(outliers) > OUTLIERS_MOST:
        raise HipError(f"at most {OUTLIERS_MOST} outlier channels")
    c = config(dim=plan["dim"], hidden_dim=plan["hidden_dim"], n_layers=plan["n_layers"], n_heads=plan["n_heads"],
               n_kv_heads=plan["n_kv_heads"], head_size=plan["head_size"], vocab_size=plan["vocab_size"],
               seq_len=plan["seq_len"], shared_classifier=int(bool(plan["shared_classifier"])), six=int(six),
               qkv_bias=int("bq" in tensors), relaxed=int(bool(plan.get("relaxed", True))),
               half_kv=int(bool(plan.get("half_kv", False)) and (
                   bool(half_keys) if half_keys is not None else plan["n_kv_heads"] >= plan["n_heads"])),
               rms_norm_eps=float(plan.get("rms_norm_eps", 1e-5)), arch=ARCHS[arch],
               rotary=rotary if arch == "neox" else 0,
               parallel_residual=int(layer_norm and bool(plan.get("parallel_residual"))),
               qk_norm=int("q_norm" in tensors and "k_norm" in tensors), outliers=outliers)
    t = TensorArray()
    for name, i in T.items():
        if name == "wcls" and c.shared_classifier:
            src = tensors["token_embedding_table"]
        elif name in tensors:
            src = tensors[name]
        else:
            continue
        t[i].offset, t[i].scales = int(src["offset"]), int(src.get("scales") or 0)
    return c, t


class Engine:
    """the object public/forward.js createForward returns, for int8/int6 checkpoints of the llama (Qwen2, Qwen3), gpt2
    and neox forms"""

    backend = "MI355X HIP kernels (gfx950)"

    def __init__(self, handle, cfg):
        self._h, self.config = handle, cfg
        self._bound = None
        self._logits = np.zeros(cfg.vocab_size, dtype=np.float32)
        self.backend = f"MI355X HIP kernels (gfx950), {'int6' if cfg.six else 'int8'}" + (
            ", relaxed order" if cfg.relaxed else "")

    # -- public/forward.js:1901-1912
    def bind(self, array):
        if array.dtype != np.float32 or not array.flags.c_contiguous or array.size != self.config.vocab_size:
            raise TypeError("bind() takes a contiguous float32 array of vocab_size logits")
        self._bound = array

    def forward(self, token, pos, need_logits=True):
        out = self._bound if self._bound is not None else self._logits
        check(library().he_forward(self._h, int(token), int(pos), int(bool(need_logits)),
                                   _ptr(out) if need_logits else None))
        if need_logits and out is not self._logits:
            self._logits[:] = out

    def forwardMany(self, tokens, pos):
        ids = np.ascontiguousarray(np.asarray(list(tokens), dtype=np.int32))
        block = self.promptBlock
        for at in range(0, ids.size, block):
            piece = np.ascontiguousarray(ids[at:at + block])
            check(library().he_forward_many(self._h, _ptr(piece), int(piece.size), int(pos) + at))

    @property
    def promptBlock(self):
        return int(library().he_prompt_block(self._h))

    @property
    def tokenBlock(self):
        """steps a generateMany() call takes (greedy decoding on the device)"""
        return 16

    def generateMany(self, token, pos, history, length, count, temperature, topp, penalty, randoms, stops):
        """public/forward.js:1831-1890: the ids of up to count steps (a stop token last), each the forward pass, the
        repetition penalty over the latest 64 of history and the ids chosen (where penalty != 1), and greedy argmax
        (temperature 0) or a draw with randoms[i] (kernels/kernel.ts:803-868); None where the engine does not take the
        first step (its nucleus holds more tokens than the device sorts: the caller takes it) or where a largest logit
        is not finite (the caller's own step then stops on NOT_FINITE, public/forward.js:1866-1880)"""
        if count < 1:
            return None
        past = np.ascontiguousarray(np.asarray(list(history), dtype=np.int32))
        draws = np.ascontiguousarray(np.asarray(list(randoms), dtype=np.float64))
        if temperature != 0.0 and draws.size < count:
            return None
        stop = np.ascontiguousarray(np.asarray(list(stops), dtype=np.int32))
        ids = np.zeros(int(count), dtype=np.int32)
        n = ctypes.c_int32(0)
        code = library().he_generate_many(self._h, int(token), int(pos), _ptr(past), int(past.size), int(length),
                                          int(count), float(temperature), float(topp), float(penalty), _ptr(draws),
                                          int(draws.size), _ptr(stop), int(stop.size), _ptr(ids), ctypes.byref(n))
        if code == HE_E_NOTFINITE:
            return None
        check(code)
        if n.value == 0:
            return None
        if self._bound is not None:
            check(library().he_logits(self._h, _ptr(self._bound)))
        return [int(i) for i in ids[:n.value]]

    def logits(self):
        check(library().he_logits(self._h, _ptr(self._logits)))
        return self._logits

    def keysAndValues(self, start, count):
        c = self.config
        kv_dim = c.n_kv_heads * c.head_size
        keys = np.zeros((c.n_layers, count, kv_dim), dtype=np.float32)
        values = np.zeros_like(keys)
        check(library().he_kv_read(self._h, int(start), int(count), _ptr(keys), _ptr(values)))
        return {"keys": keys.reshape(-1), "values": values.reshape(-1)}

    def profile(self, token, pos, need_logits=True):
        """one forward step timed by kind of kernel: {kind: (ms, algorithmic bytes, launches)}"""
        ms = np.zeros(len(KINDS), dtype=np.float64)
        nbytes = np.zeros(len(KINDS), dtype=np.float64)
        launches = np.zeros(len(KINDS), dtype=np.int32)
        check(library().he_profile_forward(self._h, int(token), int(pos), int(bool(need_logits)), _ptr(ms),
                                           _ptr(nbytes), _ptr(launches)))
        return {k: (float(ms[i]), float(nbytes[i]), int(launches[i])) for i, k in enumerate(KINDS)}

    def profileMany(self, tokens, pos):
        """one prompt chunk (forwardMany of at most promptBlock tokens) timed by kind of kernel: {kind: (ms,
        algorithmic bytes, launches)}"""
        ms = np.zeros(len(KINDS), dtype=np.float64)
        nbytes = np.zeros(len(KINDS), dtype=np.float64)
        launches = np.zeros(len(KINDS), dtype=np.int32)
        ids = np.ascontiguousarray(tokens, dtype=np.int32)
        check(library().he_profile_forward_many(self._h, _ptr(ids), len(ids), int(pos), _ptr(ms), _ptr(nbytes),
                                                _ptr(launches)))
        return {k: (float(ms[i]), float(nbytes[i]), int(launches[i])) for i, k in enumerate(KINDS)}

    MATMULS ={"all": -1, "qkv": 0, "wo": 1, "w13": 2, "w2": 3, "classifier": 4}

    def profile_matmul(self, which="all", rounds=4):
        """the decode matmuls of `which` (every layer) timed back to back: (ms a pass, algorithmic bytes a pass,
        launches a pass)"""
        ms, nbytes, launches = ctypes.c_double(), ctypes.c_double(), ctypes.c_int32()
        check(library().he_profile_matmul(self._h, self.MATMULS[which], int(rounds), ctypes.byref(ms),
                                          ctypes.byref(nbytes), ctypes.byref(launches)))
        return ms.value, nbytes.value, launches.value

    def memoryBytes(self):
        return int(library().he_device_bytes(self._h))

    def release(self):
        if self._h:
            check(library().he_close(self._h))
            self._h = None
        self._bound = None
        return True

    # the thread controls of public/forward.js:1677-1760 have nothing to do on one GPU
    def setThreads(self, n):
        return 1

    def newGeneration(self):
        pass

    @property
    def threads(self):
        return 1

    def stopThreads(self):
        pass

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


def group_size(row_length):
    """public/llama2_convert.py:25-29"""
    size = 32
    while row_length % size:
        size //= 2
    return size


def places(cfg):
    """public/llama2_numpy.py:751-775 Places.take over the tensor order of the form (public/llama2_convert.py:32-83:
    Llama's, then Qwen2's biases and Qwen3's head norms; GPT-2's and GPT-NeoX's own order) of an int8 or int6
    checkpoint (which leaves the RoPE tables out): (HeTensor array, file size)"""
    t = TensorArray()
    offset = 28
    L, dim, hidden, vocab = cfg.n_layers, cfg.dim, cfg.hidden_dim, cfg.vocab_size
    qdim, kvdim = cfg.n_heads * cfg.head_size, cfg.n_kv_heads * cfg.head_size

    def matrix(name, count, last):
        nonlocal offset
        stored = count * 3 // 4 if cfg.six else count
        t[T[name]].offset, t[T[name]].scales = offset, offset + stored
        offset += stored + 4 * (count // group_size(last))

    def vector(name, count):
        nonlocal offset
        t[T[name]].offset, t[T[name]].scales = offset, 0
        offset += 4 * count

    def classifier():
        if cfg.shared_classifier:
            t[T["wcls"]].offset, t[T["wcls"]].scales = t[0].offset, t[0].scales
        else:
            matrix("wcls", vocab * dim, dim)

    if cfg.arch in (ARCHS["gpt2"], ARCHS["neox"]):  # llama2_numpy.py:1203-1240 gpt2_tensors
        matrix("token_embedding_table", vocab * dim, dim)
        if cfg.arch == ARCHS["gpt2"]:
            matrix("positions", cfg.seq_len * dim, dim)
        vector("rms_att_weight", L * dim)
        vector("ln_att_bias", L * dim)
        matrix("wq", L * dim * dim, dim)
        matrix("wk", L * kvdim * dim, dim)
        matrix("wv", L * kvdim * dim, dim)
        vector("bq", L * dim)
        vector("bk", L * kvdim)
        vector("bv", L * kvdim)
        matrix("wo", L * dim * dim, dim)
        vector("bo", L * dim)
        vector("rms_ffn_weight", L * dim)
        vector("ln_ffn_bias", L * dim)
        matrix("w1", L * hidden * dim, dim)
        vector("b1", L * hidden)
        matrix("w2", L * dim * hidden, hidden)
        vector("b2", L * dim)
        vector("rms_final_weight", dim)
        vector("ln_final_bias", dim)
        classifier()
        return t, offset
    matrix("token_embedding_table", vocab * dim, dim)
    vector("rms_att_weight", L * dim)
    matrix("wq", L * qdim * dim, dim)
    matrix("wk", L * kvdim * dim, dim)
    matrix("wv", L * kvdim * dim, dim)
    matrix("wo", L * dim * qdim, qdim)
    vector("rms_ffn_weight", L * dim)
    matrix("w1", L * hidden * dim, dim)
    matrix("w2", L * dim * hidden, hidden)
    matrix("w3", L * hidden * dim, dim)
    vector("rms_final_weight", dim)
    classifier()
    if cfg.qkv_bias:
        vector("bq", L * qdim)
        vector("bk", L * kvdim)
        vector("bv", L * kvdim)
    if cfg.qk_norm:
        vector("q_norm", L * cfg.head_size)
        vector("k_norm", L * cfg.head_size)
    return t, offset


def rope_tables(seq_len, head_size, theta, rotary=0):
    """public/llama2_numpy.py:484-542 rope_tables() without scaling, as float32 (:1177-1179): what a caller hands the
    engine as plan.derived. rotary (GPT-NeoX): the tables of the first `rotary` values of a head in the first
    rotary / 2 columns, zeros past them (:1235-1240)"""
    width = rotary if 0 < rotary < head_size else head_size
    freq = 1.0 / theta ** (np.arange(0, width, 2, dtype=np.float64) / width)
    angles = np.arange(seq_len, dtype=np.float64)[:, None] * freq
    cos = np.zeros((seq_len, head_size // 2), dtype=np.float32)
    sin = np.zeros_like(cos)
    cos[:, :width // 2], sin[:, :width // 2] = np.cos(angles), np.sin(angles)
    return cos, sin


def start(plan, checkpoint, max_block=2048):
    """public/forward.js:571-590 start(plan) over checkpoint bytes (any buffer) that hold the file"""
    c, t = plan_to_config(plan)
    buf = np.frombuffer(checkpoint, dtype=np.uint8)
    derived = plan.get("derived") or {}
    if "freq_cis_real" not in derived:
        raise HipError("the plan carries no RoPE tables (plan.derived.freq_cis_real/imag)")
    cos = np.frombuffer(bytes(derived["freq_cis_real"]), dtype=np.float32)
    sin = np.frombuffer(bytes(derived["freq_cis_imag"]), dtype=np.float32)
    if cos.size != c.seq_len * (c.head_size // 2) or sin.size != cos.size:
        raise HipError("the RoPE tables are not [seq_len][head_size / 2]")
    h = ctypes.c_void_p()
    check(library().he_open(ctypes.byref(c), t, _ptr(buf), buf.size, _ptr(cos), _ptr(sin), int(max_block),
                            ctypes.byref(h)))
    return Engine(h, c)


def open_config(cfg, tensors, checkpoint, rope_cos, rope_sin, max_block=2048):
    """an engine from an HeConfig, an HeTensor array and the checkpoint bytes"""
    buf = np.frombuffer(checkpoint, dtype=np.uint8)
    cos = np.ascontiguousarray(rope_cos, dtype=np.float32)
    sin = np.ascontiguousarray(rope_sin, dtype=np.float32)
    h = ctypes.c_void_p()
    check(library().he_open(ctypes.byref(cfg), tensors, _ptr(buf), buf.size, _ptr(cos), _ptr(sin), int(max_block),
                            ctypes.byref(h)))
    return Engine(h, cfg)


def open_synthetic(cfg, tensors, size, seed, rope_cos, rope_sin, max_block=2048):
    """an engine whose checkpoint is made on the device from seed (he_open_synthetic)"""
    cos = np.ascontiguousarray(rope_cos, dtype=np.float32)
    sin = np.ascontiguousarray(rope_sin, dtype=np.float32)
    h = ctypes.c_void_p()
    check(library().he_open_synthetic(ctypes.byref(cfg), tensors, int(size), int(seed), _ptr(cos), _ptr(sin),
                                      int(max_block), ctypes.byref(h)))
    return Engine(h, cfg)


class External:
    """public/forward.js:571-590 external(): the checkpoint's bytes, read(offset, length), start(plan)"""

    def __init__(self, checkpoint, max_block=2048):
        self._bytes = checkpoint
        self.size = len(checkpoint)
        self.max_block = max_block
        self.engine = None

    def read(self, offset, length):
        return bytes(memoryview(self._bytes)[offset:offset + length])

    def start(self, plan):
        self.engine = start(plan, self._bytes, self.max_block)
        return self.engine


def external(checkpoint, max_block=2048):
    return External(checkpoint, max_block)
