"""Builds the engine for gfx950: libpyodide_llm_hip.so (the C ABI of include/pyodide_llm_hip.h, hipcc) and
hip_engine.node (the N-API addon forward_hip.mjs loads, gcc against Node's headers). In-tree, so that the built files
travel with the repository.

    python pyodide-llm_amd/build.py
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libpyodide_llm_hip.so")
ADDON = os.path.join(HERE, "hip_engine.node")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
NODE_INCLUDE = "/usr/include/node"

# every float32 multiply and add rounded on its own (no contraction into FMA), correctly rounded division and square
# root, and no packed FP32 instructions
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function"]
# the decode step's kernels first in each source's code object (function sections, ordered by the device linker)
ORDER = os.path.join(CSRC, "decode_order.txt")
ORDER_FLAGS = ["-ffunction-sections", "-Xoffload-linker", f"--symbol-ordering-file={ORDER}", "-Xoffload-linker",
               "--no-warn-symbol-ordering"]
SOURCES = ["gemv.hip", "gemm.hip", "misc.hip", "forms.hip", "attention.hip", "attention_tokens.hip", "sampling.hip",
           "ceilings.hip", "engine.cpp"]


def run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + proc.stdout)
    return proc.stdout


def compile_one(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
    run([HIPCC, *HIP_FLAGS, *ORDER_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_library():
    os.makedirs(BUILD, exist_ok=True)
    sources = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objects = list(pool.map(compile_one, sources))
    tmp = LIBRARY + ".tmp"
    run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objects])
    os.replace(tmp, LIBRARY)
    return LIBRARY


def build_addon():
    src = os.path.join(CSRC, "napi_addon.c")
    if not os.path.exists(src) or not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return None
    tmp = ADDON + ".tmp"
    run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-I", NODE_INCLUDE, "-I", os.path.join(HERE, ".."),
         "-DNAPI_VERSION=8", "-DNODE_GYP_MODULE_NAME=hip_engine", "-o", tmp, src, "-L", HERE, "-lpyodide_llm_hip", "-Wl,-rpath,$ORIGIN",
         "-Wl,--unresolved-symbols=ignore-in-object-files"])
    os.replace(tmp, ADDON)
    return ADDON


def build():
    lib = build_library()
    addon = build_addon()
    shutil.rmtree(BUILD, ignore_errors=True)
    return lib, addon


if __name__ == "__main__":
    print(build())
    sys.exit(0)
