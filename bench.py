#!/usr/bin/env python3
"""The headline measurement: greedy decode of a Llama-3-8B-shaped int8 model at batch 1 on one MI355X, after a
2048-token prompt prefill, through the engine's C ABI (include/pyodide_llm_hip.h).

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--model llama3-8b] [--no-cpu]

A step is one decode token: the forward pass of the token fed at its position over the growing KV cache, the
classifier, and the greedy choice on the device. Weights are synthetic (N(0, 0.02) by a counter-based generator made
on the device, quantized by the reference's quantize() rules into the quantize.py layout); the prompt is random ids.
Printed: one JSON line with decode tok/s as `value`, prefill tok/s, the decode GEMV's HBM GB/s against the 8 TB/s
roofline (the algorithmic bytes of every matmul launch of one profiled decode step over their HIP-event-timed
duration), and the oracle's decode rate on the host's cores as the CPU baseline.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "tests"))

from paths import package  # noqa: E402

METRIC = "decode tok/s + GEMV HBM GB/s (8B-shape int8, batch 1); prefill tok/s"
HBM_PEAK_GBS = 8000.0
PROFILED_STEPS = 8
# HBM bytes of one pass of the decode matmuls (every layer's, and the classifier's), from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE runs of this script, each counter scaled by what it reads on HIP's device-to-device copy of 1 GiB
# (FETCH_SIZE read half the bytes copied: x2; WRITE_SIZE all of them: x1). The profile summary names the commands.
TRAFFIC = {
    "llama3-8b": {"bytes_per_pass": round((2 * (32 * (13893.9 + 9339.0 + 64598.4 + 32465.7) + 288662.5)
                                           + (32 * (48.6 + 32 + 112 + 32) + 502.3)) * 1024),
                  "source": "profiles/decode_gemv_llama3-8b.md"},
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


def read_ceiling(pk, nbytes=4 << 30, passes=4):
    """the HBM read bandwidth a plain streaming kernel reaches on this GPU (hk_read_ceiling, the device form of the
    reference's kernels/ceilings.ts read()): 4 GiB (more than the 256 MB MALL holds) read 4 times after a memset,
    GB/s of one pass. A practical figure, not a bound: the decode GEMV's access pattern reads its largest matrices a
    little faster."""
    lib = ctypes.CDLL("libamdhip64.so")
    buf = ctypes.c_void_p()
    if lib.hipMalloc(ctypes.byref(buf), ctypes.c_size_t(nbytes)) != 0:
        raise RuntimeError("hipMalloc failed")
    try:
        if lib.hipMemset(buf, 1, ctypes.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMemset failed")
        checksum, ms = ctypes.c_int32(0), ctypes.c_double(0.0)
        pk.hip_engine.check(pk.library().hk_read_ceiling(buf, nbytes, passes, ctypes.byref(checksum), ctypes.byref(ms),
                                                         None))
    finally:
        hip_sync()
        lib.hipFree(buf)
    return nbytes / (ms.value * 1e-3) / 1e9


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


def cpu_baseline(pk, spec, seconds=20.0):
    """the oracle (oracle/liboracle.so, the reference's arithmetic restated in C) on the host's cores, on a bounded
    sample of the same workload: the model's widths with 2 of its layers and its classifier, a few decode tokens,
    scaled to all layers"""
    import oracle_lib as ol
    fields = dict(spec["cfg"])
    layers = fields["n_layers"]
    sample_layers = min(2, layers)
    fields.update(n_layers=sample_layers, seq_len=64)
    cfg = pk.config(**fields)
    tensors, size = ol.places(cfg)
    made = time.perf_counter()
    ck = ol.synth_checkpoint(cfg, tensors, size, seed=0)
    cos, sin = ol.rope_tables(cfg.seq_len, cfg.head_size, spec["theta"])
    model = ol.Model(cfg, tensors, ck, cos, sin, max_block=1)
    made = time.perf_counter() - made
    t_layers, t_full, pos, token = [], [], 0, 1
    begin = time.perf_counter()
    while pos < 48 and (time.perf_counter() - begin < seconds or pos < 4):
        t0 = time.perf_counter()
        model.run([token], pos, False)
        t1 = time.perf_counter()
        model.run([token], pos + 1, True)
        t2 = time.perf_counter()
        t_layers.append(t1 - t0)
        t_full.append(t2 - t1)
        token = int(np.argmax(model.logits()))
        pos += 2
    tl, tf = float(np.median(t_layers)), float(np.median(t_full))
    per_token = tl * layers / sample_layers + (tf - tl)
    model.close()
    return {"value": 1.0 / per_token, "unit": "tok/s", "cores": int(ol.load().or_get_threads()), "kind": "port",
            "host": host_cpu(),
            "sample": (f"oracle decode (C restatement of the reference's WASM path, OpenMP) at the model's widths with "
                       f"{sample_layers} of {layers} layers and the classifier, {len(t_layers) * 2} tokens at positions "
                       f"0-{pos - 1}; per-layer time scaled to {layers} layers; short context (the measured 8B run is "
                       f"at positions past the prompt); checkpoint made in {made:.1f} s")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="decode steps timed (default: the model's 256/128)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--model", default="llama3-8b", choices=sorted(MODELS))
    ap.add_argument("--prompt", type=int, default=None)
    ap.add_argument("--no-cpu", action="store_true", help="skip the oracle's CPU baseline")
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
    spec = MODELS[args.model]
    steps = args.steps if args.steps is not None else spec["decode"]
    prompt_len = args.prompt if args.prompt is not None else spec["prompt"]
    pk = package()
    cfg = pk.config(**spec["cfg"])
    if prompt_len + args.warmup + steps + PROFILED_STEPS > cfg.seq_len:
        raise SystemExit("the prompt and the steps do not fit the context")
    tensors, size = pk.places(cfg)
    cos, sin = pk.rope_tables(cfg.seq_len, cfg.head_size, spec["theta"])
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

    def decode(n):
        nonlocal token, pos
        done = 0
        while done < n:
            ids = eng.generateMany(token, pos, [], 0, min(block, n - done), 0.0, 0.9, 1.0, [], [])
            token, pos, done = ids[-1], pos + len(ids), done + len(ids)

    decode(args.warmup)
    hip_sync()
    t0 = time.perf_counter()
    decode(steps)
    hip_sync()
    decode_s = time.perf_counter() - t0
    tok_s = steps / decode_s

    # decode steps timed kernel by kind (a HIP event pair around every launch on the engine's stream), at the
    # positions the run reached: the GEMV's achieved GB/s is the algorithmic bytes of its launches over their time
    prof = {}
    for i in range(PROFILED_STEPS):
        for kind, (ms, nbytes, launches) in eng.profile(token, pos + i, True).items():
            acc = prof.setdefault(kind, [0.0, 0.0, 0])
            acc[0] += ms / PROFILED_STEPS
            acc[1] += nbytes / PROFILED_STEPS
            acc[2] += launches / PROFILED_STEPS
    step_ms = sum(v[0] for v in prof.values())
    # the roofline's kernel: every decode matmul of a step (m = 1, the engine's weights, every layer, the classifier)
    # back to back between one HIP event pair on the engine's stream, 4 passes; then each kind of matrix alone
    gemv_ms, gemv_bytes, gemv_launches = eng.profile_matmul("all", rounds=4)
    gemv_gbs = gemv_bytes / (gemv_ms * 1e-3) / 1e9
    by_matrix = {}
    for which in ("qkv", "wo", "w13", "w2", "classifier"):
        ms, nbytes, launches = eng.profile_matmul(which, rounds=2)
        by_matrix[which] = {"us_per_launch": round(1e3 * ms / launches, 2), "bytes_per_launch": round(nbytes / launches),
                            "gb_s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    traffic = TRAFFIC.get(args.model)
    eng.release()
    ceiling_gbs = read_ceiling(pk)

    cpu = None if args.no_cpu else cpu_baseline(pk, spec)
    out = {
        "metric": METRIC,
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * decode_s / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int6" if cfg.six else "int8",
        "data": "synthetic (random-init weights N(0,0.02) quantized by the reference's rules; random prompt ids)",
        "config": {"workload": f"{args.model}-shape {'int6' if cfg.six else 'int8'} greedy decode at batch 1 after a "
                               f"{prompt_len}-token prefill",
                   "model": args.model, "prompt_tokens": prompt_len, "decode_tokens": steps,
                   "kv_cache": "f16" if cfg.half_kv else "f32", "order": "exact (the reference's float32 order)"},
        "prefill_tok_s": round(prompt_len / prefill_s, 2),
        "gemv_hbm_gb_s": round(gemv_gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
                     "traffic": round(traffic["bytes_per_pass"] / gemv_launches) if traffic else None,
                     "kernel": "decode GEMV (gemv1_kernel: every matmul of a decode step, m = 1, back to back)",
                     "launches_per_pass": int(gemv_launches),
                     "algorithmic_bytes_per_launch": round(gemv_bytes / gemv_launches),
                     "us_per_launch": round(1e3 * gemv_ms / gemv_launches, 3),
                     "traffic_source": traffic["source"] if traffic else None,
                     "read_ceiling_gb_s": round(ceiling_gbs, 1),
                     "frac_of_read_ceiling": round(gemv_gbs / ceiling_gbs, 4)},
        "gemv_by_matrix": by_matrix,
        "profile_ms": {k: round(v[0], 4) for k, v in prof.items()},
        "profiled_step_ms": round(step_ms, 4),
        "setup_s": round(setup_s, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
