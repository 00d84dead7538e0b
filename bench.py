#!/usr/bin/env python3
"""The headline measurement: greedy decode of a Llama-3-8B-shaped int8 model at batch 1 on one MI355X, after a
2048-token prompt prefill, through the engine's C ABI (include/pyodide_llm_hip.h).

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--model llama3-8b] [--only] [--no-cpu] [--no-node]

A step is one decode token: the forward pass of the token fed at its position over the growing KV cache, the
classifier, and the greedy choice on the device. Weights are synthetic (N(0, 0.02) by a counter-based generator made
on the device, quantized by the reference's quantize() rules into the quantize.py layout); the prompt is random ids.
Printed: one JSON line with decode tok/s as `value`, the decode GEMV's HBM GB/s against the 8 TB/s roofline (the
algorithmic bytes of every matmul launch of a decode step over their HIP-event-timed duration), the prompt's GEMM
against the int8 MFMA peak and the ceilings measured in the same run (kernels/ceilings.ts on the device), the same
decode timed through the JavaScript host (Node over forward_hip.mjs), the oracle's decode rate on the host's cores as
the CPU baseline, and a record of each other model shape (150M, stories15M, Qwen2.5-7B int6) unless --only.
"""
import argparse
import ctypes
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "tests"))

from paths import package  # noqa: E402

METRIC = "decode tok/s + GEMV HBM GB/s (8B-shape int8, batch 1); prefill tok/s"
HBM_PEAK_GBS = 8000.0
I8_MFMA_PEAK_TOPS = 5000.0  # MI355X dense int8
PROFILED_STEPS = 8
# HBM bytes of one pass of the decode matmuls (every layer's, and the classifier's), from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE runs of this script, each counter scaled by what it reads on HIP's device-to-device copy of 1 GiB
# (FETCH_SIZE read half the bytes copied: x2; WRITE_SIZE all of them: x1). The profile summary names the commands.
TRAFFIC = {
    "llama3-8b": {"bytes_per_pass": round((2 * (32 * (13900 + 9304 + 64600 + 32500) + 288700)
                                           + (32 * (48.63 + 16 + 112 + 32) + 502.3)) * 1024),
                  "source": "profiles/decode_gemv_llama3-8b.md"},
    "qwen25-7b-int6": {"bytes_per_pass": round((2 * (28 * (7180.9 + 5583.0 + 58119.9 + 29261.5) + 232951.8)
                                                + (28 * (32.1 + 14 + 148.1 + 28) + 594.6)) * 1024),
                       "source": "profiles/decode_gemv6_qwen25-7b-int6.md"},
}

MODELS = {
    # Llama-3-8B shape (hidden 4096, 32 layers, 32 q / 8 kv heads of 128, SwiGLU 14336, vocab 128256, theta 5e5):
    # GQA, so its cache is float32 as the reference keeps a grouped-query model's on CPU (public/forward.js:762)
    "llama3-8b": dict(cfg=dict(dim=4096, hidden_dim=14336, n_layers=32, n_heads=32, n_kv_heads=8, head_size=128,
                               vocab_size=128256, seq_len=4096, shared_classifier=0, half_kv=0),
                      theta=500000.0, prompt=2048, decode=256),
    "llm150m": dict(cfg=dict(dim=512, hidden_dim=2048, n_layers=12, n_heads=8, n_kv_heads=8, head_size=64,
                             vocab_size=99487, seq_len=1024, shared_classifier=1, half_kv=1),
                    theta=10000.0, prompt=512, decode=256),
    "stories15m": dict(cfg=dict(dim=288, hidden_dim=768, n_layers=6, n_heads=6, n_kv_heads=6, head_size=48,
                                vocab_size=32000, seq_len=256, shared_classifier=1, half_kv=1),
                       theta=10000.0, prompt=32, decode=128),
    "qwen25-7b-int6": dict(cfg=dict(dim=3584, hidden_dim=18944, n_layers=28, n_heads=28, n_kv_heads=4, head_size=128,
                                    vocab_size=152064, seq_len=2048, shared_classifier=0, six=1, qkv_bias=1,
                                    half_kv=0, rms_norm_eps=1e-6),
                           theta=1000000.0, prompt=1024, decode=256),
}
OTHERS = ("llm150m", "stories15m", "qwen25-7b-int6")


def hip_sync():
    lib = ctypes.CDLL("libamdhip64.so")
    code = lib.hipDeviceSynchronize()
    if code != 0:
        raise RuntimeError(f"hipDeviceSynchronize failed ({code})")


def copy_calibration(nbytes=1 << 30, reps=4):
    """a plain device-to-device copy of known size (HIP's own copy kernel), for scaling the FETCH_SIZE / WRITE_SIZE
    counters of a profiled run to bytes: each copy reads and writes nbytes"""
    lib = ctypes.CDLL("libamdhip64.so")
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    for buf in (src, dst):
        if lib.hipMalloc(ctypes.byref(buf), ctypes.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMalloc failed")
    if lib.hipMemset(src, 1, ctypes.c_size_t(nbytes)) != 0:
        raise RuntimeError("hipMemset failed")
    for _ in range(reps):
        if lib.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3) != 0:  # hipMemcpyDeviceToDevice
            raise RuntimeError("hipMemcpy failed")
    hip_sync()
    for buf in (src, dst):
        lib.hipFree(buf)
    print(json.dumps({"copy_bytes": nbytes, "copies": reps}))


def read_ceiling(pk, floors=(), nbytes=4 << 30, passes=4):
    """the HBM read bandwidth a plain streaming kernel reaches on this GPU (hk_read_ceiling, the device form of the
    reference's kernels/ceilings.ts read()): 4 GiB (more than the 256 MB MALL holds), the fastest of its launch shapes,
    GB/s of one pass; and for each size in `floors` the same kernel's cold read of that many bytes (hk_read_floor:
    launches back to back, each on the next window of the 4 GiB), mean µs a launch"""
    lib = ctypes.CDLL("libamdhip64.so")
    buf = ctypes.c_void_p()
    if lib.hipMalloc(ctypes.byref(buf), ctypes.c_size_t(nbytes)) != 0:
        raise RuntimeError("hipMalloc failed")
    us = {}
    try:
        if lib.hipMemset(buf, 1, ctypes.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMemset failed")
        checksum, ms = ctypes.c_int32(0), ctypes.c_double(0.0)
        pk.hip_engine.check(pk.library().hk_read_ceiling(buf, nbytes, passes, ctypes.byref(checksum), ctypes.byref(ms),
                                                         None))
        for size in floors:
            got = ctypes.c_double(0.0)
            pk.hip_engine.check(pk.library().hk_read_floor(buf, nbytes, size - size % 64, 32, ctypes.byref(got), None))
            us[size] = got.value
    finally:
        hip_sync()
        lib.hipFree(buf)
    return nbytes / (ms.value * 1e-3) / 1e9, us


def valu_ceiling(pk, passes=65536):
    """ceilings.ts fma(passes, 1, 0.9999, 1e-7) in every lane of a launch that fills the device: float32 multiply +
    add pairs a second, each rounded (no FMA, no packed FP32)"""
    result, ms, pairs = ctypes.c_float(0), ctypes.c_double(0), ctypes.c_double(0)
    pk.hip_engine.check(pk.library().hk_valu_ceiling(passes, 1.0, 0.9999, 1e-7, ctypes.byref(result), ctypes.byref(ms),
                                                     ctypes.byref(pairs), None))
    return pairs.value / (ms.value * 1e-3), result.value


def mfma_ceiling(pk, passes=16384):
    """v_mfma_i32_32x32x32_i8 from registers in a launch that fills the device: int operations a second"""
    checksum, ms, ops = ctypes.c_int32(0), ctypes.c_double(0), ctypes.c_double(0)
    pk.hip_engine.check(pk.library().hk_mfma_ceiling(passes, 3, 5, 0x81, ctypes.byref(checksum), ctypes.byref(ms),
                                                     ctypes.byref(ops), None))
    return ops.value / (ms.value * 1e-3)


def host_cpu():
    """the host's CPU model and the logical CPUs this process may run on"""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "logical_cpus_available": len(os.sched_getaffinity(0))}


def cpu_baseline(pk, spec, prompt_len, tokens, seconds=15.0):
    """the oracle (oracle/liboracle.so, the reference's arithmetic restated in C) on the host's cores, on a bounded
    sample of the same workload: the whole model (every layer, the classifier, the greedy choice) decoding the
    measured run's tokens at its positions, from the prompt's end (the cache before it left at zero: attention reads
    that many positions, the same arithmetic), until `tokens` steps or `seconds` have passed"""
    import oracle_lib as ol
    fields = dict(spec["cfg"])
    fields.update(seq_len=prompt_len + tokens + 1)
    cfg = pk.config(**fields)
    tensors, size = ol.places(cfg)
    made = time.perf_counter()
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=0)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, spec["theta"])
    model = ol.Model(cfg, tensors, ck, cos, sin, max_block=1)
    made = time.perf_counter() - made
    pos, token, done = prompt_len, 1, 0
    model.run([token], pos, True)  # the first step (page-ins) untimed
    token, pos = int(np.argmax(model.logits())), pos + 1
    begin = time.perf_counter()
    while done < tokens and (time.perf_counter() - begin < seconds or done < 2):
        model.run([token], pos, True)
        token = int(np.argmax(model.logits()))
        pos, done = pos + 1, done + 1
    spent = time.perf_counter() - begin
    model.close()
    del ck
    return {"value": round(done / spent, 4), "unit": "tok/s", "cores": int(ol.load().or_get_threads()),
            "kind": "port", "host": host_cpu(),
            "sample": (f"oracle greedy decode (C restatement of the reference's WASM path, OpenMP) of the whole model "
                       f"({cfg.n_layers} layers and the classifier), {done} tokens at positions {prompt_len + 1}-"
                       f"{pos - 1} (a cache of zeros before them) in {spent:.1f} s; checkpoint made on the host in "
                       f"{made:.1f} s")}


def layer_weights(cfg):
    """the weights of one layer's matrices"""
    q, kv = cfg.n_heads * cfg.head_size, cfg.n_kv_heads * cfg.head_size
    return cfg.dim * (q + 2 * kv) + q * cfg.dim + 3 * cfg.dim * cfg.hidden_dim


def node_decode(pk, name, spec, cfg, tensors, size, prompt, warmup, steps):
    """the same decode through the JavaScript host: Node runs pyodide-llm_amd/decode_bench.mjs on an engine made from
    the same seed, and its ids must equal this process's"""
    from plans import plan_of
    node = shutil.which("node")
    addon = os.path.join(HERE, "pyodide-llm_amd", "hip_engine.node")
    if node is None or not os.path.exists(addon):
        return None
    cos, sin = pk.rope_tables(cfg.seq_len, cfg.head_size, spec["theta"])
    with tempfile.TemporaryDirectory() as tmp:
        np.asarray(cos, np.float32).tofile(os.path.join(tmp, "cos.bin"))
        np.asarray(sin, np.float32).tofile(os.path.join(tmp, "sin.bin"))
        job = {"plan": plan_of(cfg, tensors), "size": int(size), "seed": 0, "prompt": prompt, "warmup": warmup,
               "steps": steps, "promptBlock": len(prompt)}
        with open(os.path.join(tmp, "job.json"), "w") as f:
            json.dump(job, f)
        print(f"node host: {name}", file=sys.stderr, flush=True)
        proc = subprocess.run([node, os.path.join(HERE, "pyodide-llm_amd", "decode_bench.mjs"),
                               os.path.join(tmp, "job.json")], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                              text=True, timeout=300)
    if proc.returncode != 0:
        raise RuntimeError("node decode failed:\n" + proc.stderr[-3000:])
    return json.loads(proc.stdout.strip().splitlines()[-1])


def measure(pk, name, steps=None, warmup=8, prompt_len=None, detail=False, cpu=True, node=False):
    """one model shape: open (synthetic), prompt, timed greedy decode; the decode matmuls' GB/s; with detail the
    per-kind profile of decode steps and of the prompt, each kind of matrix on its own, the Node host's run"""
    spec = MODELS[name]
    steps = steps if steps is not None else spec["decode"]
    prompt_len = prompt_len if prompt_len is not None else spec["prompt"]
    cfg = pk.config(**spec["cfg"])
    if prompt_len + warmup + steps + PROFILED_STEPS + 1 > cfg.seq_len:
        raise SystemExit("the prompt and the steps do not fit the context")
    tensors, size = pk.places(cfg)
    cos, sin = pk.rope_tables(cfg.seq_len, cfg.head_size, spec["theta"])
    print(f"model: {name}", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    eng = pk.open_synthetic(cfg, tensors, size, 0, cos, sin, max_block=prompt_len)
    setup_s = time.perf_counter() - t0
    rng = np.random.default_rng(2)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, size=prompt_len)]

    # the prompt: [BOS] + prompt[:-1] through forwardMany (public/llama2_numpy.py:1586-1606)
    fed = [1] + prompt[:-1]
    hip_sync()
    t0 = time.perf_counter()
    eng.forwardMany(fed, 0)
    hip_sync()
    prefill_s = time.perf_counter() - t0

    token, pos = prompt[-1], prompt_len
    block = eng.tokenBlock
    ids = []

    def decode(n, stops):
        # greedy steps as generate() asks for them, stop_tokens=(BOS,) by default (public/llama2_numpy.py:989); a
        # stop token returned early only makes the next call start from it (the timed steps go on)
        nonlocal token, pos
        done = 0
        while done < n:
            got = eng.generateMany(token, pos, [], 0, min(block, n - done), 0.0, 0.9, 1.0, [], stops)
            ids.extend(got)
            token, pos, done = got[-1], pos + len(got), done + len(got)

    decode(warmup, [1])
    hip_sync()
    start = (token, pos, len(ids))
    t0 = time.perf_counter()
    decode(steps, [1])
    hip_sync()
    decode_s = time.perf_counter() - t0
    rec = {"model": name, "dtype": "int6" if cfg.six else "int8", "kv_cache": "f16" if cfg.half_kv else "f32",
           "prompt_tokens": prompt_len, "decode_tokens": steps, "warmup": warmup,
           "tok_s": steps / decode_s, "ms_per_step": 1e3 * decode_s / steps, "prefill_tok_s": prompt_len / prefill_s,
           "setup_s": setup_s}
    if detail:
        # the same steps from the same position again without stop tokens (the cache rows get the same bits), then
        # sampled steps (the draw and the penalty on the device, the caller's random numbers) from there too
        end = (token, pos, list(ids))
        token, pos = start[0], start[1]
        t0 = time.perf_counter()
        decode(steps, [])
        hip_sync()
        rec["no_stops_tok_s"] = steps / (time.perf_counter() - t0)
        assert ids[start[2] + steps:] == end[2][start[2]:], "the steps without stop tokens chose other tokens"
        del ids[start[2] + steps:]
        rec["sampled"] = {}
        for temperature, topp, penalty in ((0.8, 1.0, 1.1), (0.8, 0.9, 1.1)):
            token, pos = start[0], start[1]
            history = ([1] + prompt + ids[:start[2]])[-64:]
            r = np.random.default_rng(3)
            done, declined = 0, False
            t0 = time.perf_counter()
            while done < steps:
                count = min(block, steps - done)
                got = eng.generateMany(token, pos, history[-64:], len(history), count, temperature, topp, penalty,
                                       list(r.random(count)), [1])
                if not got:
                    declined = True  # the caller's own step would follow (its nucleus is larger than the device sorts)
                    break
                history += got
                token, pos, done = got[-1], pos + len(got), done + len(got)
            hip_sync()
            elapsed = time.perf_counter() - t0
            rec["sampled"][f"t{temperature}_p{topp}_r{penalty}"] = {
                "temperature": temperature, "topp": topp, "penalty": penalty, "stops": [1], "steps": done,
                "tok_s": round(done / elapsed, 3) if done else None, "declined": declined}
        token, pos = end[0], end[1]

    # the roofline's kernel: every decode matmul of a step (m = 1, the engine's weights, every layer, the classifier)
    # back to back between one HIP event pair on the engine's stream, 4 passes
    gemv_ms, gemv_bytes, gemv_launches = eng.profile_matmul("all", rounds=4)
    rec["gemv"] = {"ms_per_pass": gemv_ms, "bytes_per_pass": gemv_bytes, "launches_per_pass": gemv_launches,
                   "gb_s": gemv_bytes / (gemv_ms * 1e-3) / 1e9}
    # the weights a decode step streams at the measured step rate
    rec["effective_gb_s"] = gemv_bytes * rec["tok_s"] / 1e9
    # the whole step against HBM: every matmul's bytes and the cache rows the attention reads (keys and values of
    # every position up to the step's, at the timed steps' mean position)
    kv_bytes = 2.0 * cfg.n_layers * (prompt_len + warmup + steps / 2.0 + 1) * cfg.n_kv_heads * cfg.head_size * \
        (2 if cfg.half_kv else 4)
    step_bytes = gemv_bytes + kv_bytes
    rec["step_roofline"] = {"bound": "hbm", "bytes_per_step": round(step_bytes), "kv_bytes_per_step": round(kv_bytes),
                            "achieved": round(step_bytes * rec["tok_s"] / 1e9, 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(step_bytes * rec["tok_s"] / 1e9 / HBM_PEAK_GBS, 4),
                            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1)}
    if detail:
        # decode steps timed kernel by kind (a HIP event pair around every launch on the engine's stream), at the
        # positions the run reached
        prof = {}
        for i in range(PROFILED_STEPS):
            for kind, (ms, nbytes, launches) in eng.profile(token, pos + i, True).items():
                acc = prof.setdefault(kind, [0.0, 0.0, 0])
                acc[0] += ms / PROFILED_STEPS
                acc[1] += nbytes / PROFILED_STEPS
                acc[2] += launches / PROFILED_STEPS
        rec["profile_ms"] = {k: round(v[0], 4) for k, v in prof.items()}
        rec["profiled_step_ms"] = round(sum(v[0] for v in prof.values()), 4)
        by_matrix = {}
        for which in ("qkv", "wo", "w13", "w2", "classifier"):
            ms, nbytes, launches = eng.profile_matmul(which, rounds=2)
            by_matrix[which] = {"us_per_launch": round(1e3 * ms / launches, 2),
                                "bytes_per_launch": round(nbytes / launches),
                                "gb_s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        rec["gemv_by_matrix"] = by_matrix
        # the prompt again (the same tokens at the same positions: the cache gets the same bits), every launch timed
        pprof = eng.profileMany(fed, 0)
        rec["prefill_profile_ms"] = {k: round(v[0], 3) for k, v in pprof.items()}
        rec["prefill_gemm"] = {"ms": pprof["gemm"][0], "launches": pprof["gemm"][2],
                               "int_ops": 2.0 * prompt_len * cfg.n_layers * layer_weights(cfg)}
    eng.release()
    if node:
        got = node_decode(pk, name, spec, cfg, tensors, size, prompt, warmup, steps)
        if got is not None:
            rec["node_host"] = {"tok_s": round(got["decode_tok_s"], 3), "ms_per_step": round(got["ms_per_step"], 4),
                                "prefill_tok_s": round(got["prefill_tok_s"], 2),
                                "ids_equal": got["ids"] == [int(t) for t in ids]}
    if cpu:
        rec["cpu_baseline"] = cpu_baseline(pk, spec, prompt_len, steps, seconds=15.0 if detail else 10.0)
    return rec


def brief(rec):
    """the record of another model shape in the JSON line"""
    out = {"value": round(rec["tok_s"], 3), "unit": "tok/s", "dtype": rec["dtype"], "kv_cache": rec["kv_cache"],
           "workload": f"{rec['model']}-shape {rec['dtype']} greedy decode at batch 1 after a "
                       f"{rec['prompt_tokens']}-token prefill",
           "decode_tokens": rec["decode_tokens"], "ms_per_step": round(rec["ms_per_step"], 4),
           "prefill_tok_s": round(rec["prefill_tok_s"], 2),
           "gemv_gb_s": round(rec["gemv"]["gb_s"], 1),
           "effective_gb_s": round(rec["effective_gb_s"], 1),
           "weights_bytes_per_step": round(rec["gemv"]["bytes_per_pass"])}
    if rec["dtype"] == "int6":
        # the fused 6-bit loader: 0.75 B a weight and 4 B of scale a group of 32, 0.875 B a weight
        out["roofline"] = {"bound": "hbm", "achieved": round(rec["gemv"]["gb_s"], 1), "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": round(rec["gemv"]["gb_s"] / HBM_PEAK_GBS, 4),
                           "kernel": "decode GEMV on int6 rows (every matmul of a decode step, m = 1, back to back)",
                           "bytes_per_weight": 0.875,
                           "launches_per_pass": int(rec["gemv"]["launches_per_pass"]),
                           "us_per_launch": round(1e3 * rec["gemv"]["ms_per_pass"] / rec["gemv"]["launches_per_pass"], 3)}
        traffic = TRAFFIC.get(rec["model"])
        if traffic:
            out["roofline"]["traffic"] = round(traffic["bytes_per_pass"] / rec["gemv"]["launches_per_pass"])
            out["roofline"]["traffic_source"] = traffic["source"]
    else:
        out["note"] = ("the weights fit the 256 MB MALL: effective_gb_s is the step's matmul bytes at the decode rate "
                       "(cache-resident, not an HBM figure)")
    if "cpu_baseline" in rec:
        out["cpu_baseline"] = rec["cpu_baseline"]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="decode steps timed (default: the model's 256/128)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--model", default="llama3-8b", choices=sorted(MODELS))
    ap.add_argument("--prompt", type=int, default=None)
    ap.add_argument("--only", action="store_true", help="only the named model (no records of the other shapes)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the oracle's CPU baselines")
    ap.add_argument("--no-node", action="store_true", help="skip the decode through the JavaScript host")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 4 device copies of 1 GiB (the reference kernel for scaling HBM counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: every box here has one, and this engine has no multi-GPU path "
              f"(asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    pk = package()
    rec = measure(pk, args.model, args.steps, args.warmup, args.prompt, detail=True, cpu=not args.no_cpu,
                  node=not args.no_node)
    print("ceilings", file=sys.stderr, flush=True)
    by_matrix = rec["gemv_by_matrix"]
    ceiling_gbs, floor_us = read_ceiling(pk, [m["bytes_per_launch"] for m in by_matrix.values()])
    for m in by_matrix.values():
        # one cold read of the matrix's bytes by the plain streaming kernel: the launch's ramp and first loads'
        # latency included, which a small matrix cannot hide
        m["stream_floor_us"] = round(floor_us[m["bytes_per_launch"]], 2)
        m["frac_of_stream_floor"] = round(floor_us[m["bytes_per_launch"]] / m["us_per_launch"], 3)
    pairs_s, _ = valu_ceiling(pk)
    mfma_ops_s = mfma_ceiling(pk)
    rec["step_roofline"]["read_ceiling_gb_s"] = round(ceiling_gbs, 1)
    rec["step_roofline"]["frac_of_read_ceiling"] = round(rec["step_roofline"]["achieved"] / ceiling_gbs, 4)
    others = {}
    if not args.only:
        for name in OTHERS:
            if name != args.model:
                others[name] = brief(measure(pk, name, warmup=args.warmup, cpu=not args.no_cpu))

    gemv = rec["gemv"]
    gemv_gbs = gemv["gb_s"]
    traffic = TRAFFIC.get(args.model)
    gemm = rec["prefill_gemm"]
    gemm_tops = gemm["int_ops"] / (gemm["ms"] * 1e-3) / 1e12
    # the exact order's float32 work after each int32 group sum: 4 VALU operations (the scale product, the
    # conversion, the multiply, the add to the chain) for the group's 32 multiply-adds (64 int operations) of a
    # (row, token): at the measured multiply + add rate (2 operations a pair), 16 int operations an operation
    valu_ops_s = 2.0 * pairs_s
    exact_cap_tops = valu_ops_s * 16 / 1e12
    cfg_name = args.model
    out = {
        "metric": METRIC,
        "value": round(rec["tok_s"], 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": rec["decode_tokens"],
        "warmup": args.warmup,
        "ms_per_step": round(rec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": rec["dtype"],
        "data": "synthetic (random-init weights N(0,0.02) quantized by the reference's rules; random prompt ids)",
        "config": {"workload": f"{cfg_name}-shape {rec['dtype']} greedy decode at batch 1 after a "
                               f"{rec['prompt_tokens']}-token prefill, stop token BOS as generate() asks",
                   "model": cfg_name, "prompt_tokens": rec["prompt_tokens"], "decode_tokens": rec["decode_tokens"],
                   "kv_cache": rec["kv_cache"], "order": "exact (the reference's float32 order)"},
        "prefill_tok_s": round(rec["prefill_tok_s"], 2),
        "no_stops_tok_s": round(rec["no_stops_tok_s"], 3),
        "sampled": rec["sampled"],
        "gemv_hbm_gb_s": round(gemv_gbs, 1),
        "effective_gb_s": round(rec["effective_gb_s"], 1),
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
                     "traffic": round(traffic["bytes_per_pass"] / gemv["launches_per_pass"]) if traffic else None,
                     "kernel": "decode GEMV (every matmul of a decode step, m = 1, back to back)",
                     "launches_per_pass": int(gemv["launches_per_pass"]),
                     "algorithmic_bytes_per_launch": round(gemv["bytes_per_pass"] / gemv["launches_per_pass"]),
                     "us_per_launch": round(1e3 * gemv["ms_per_pass"] / gemv["launches_per_pass"], 3),
                     "traffic_source": traffic["source"] if traffic else None,
                     "read_ceiling_gb_s": round(ceiling_gbs, 1),
                     "frac_of_read_ceiling": round(gemv_gbs / ceiling_gbs, 4)},
        "prefill_roofline": {"bound": "mfma", "kernel": "prompt GEMM (gemm_kernel, every matmul of the prompt)",
                             "achieved": round(gemm_tops, 1), "peak": I8_MFMA_PEAK_TOPS, "unit": "TOP/s",
                             "frac": round(gemm_tops / I8_MFMA_PEAK_TOPS, 4),
                             "gemm_ms": round(gemm["ms"], 3), "int_ops": gemm["int_ops"],
                             "mfma_ceiling_top_s": round(mfma_ops_s / 1e12, 1),
                             "frac_of_mfma_ceiling": round(gemm_tops * 1e12 / mfma_ops_s, 4),
                             "exact_order_cap_top_s": round(exact_cap_tops, 1),
                             "frac_of_exact_order_cap": round(gemm_tops / exact_cap_tops, 4)},
        "ceilings": {"read_gb_s": round(ceiling_gbs, 1),
                     "valu_mul_add_pairs_t_s": round(pairs_s / 1e12, 3),
                     "valu_f32_ops_t_s": round(valu_ops_s / 1e12, 2),
                     "mfma_i8_top_s": round(mfma_ops_s / 1e12, 1),
                     "source": "hk_read_ceiling, hk_valu_ceiling, hk_mfma_ceiling (kernels/ceilings.ts on the device)"},
        "step_roofline": rec["step_roofline"],
        "gemv_by_matrix": rec["gemv_by_matrix"],
        "profile_ms": rec["profile_ms"],
        "profiled_step_ms": rec["profiled_step_ms"],
        "prefill_profile_ms": rec["prefill_profile_ms"],
        "setup_s": round(rec["setup_s"], 2),
        "node_host": rec.get("node_host"),
        "cpu_baseline": rec.get("cpu_baseline"),
        "other_shapes": others,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
