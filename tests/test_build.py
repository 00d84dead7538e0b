"""The built library's gfx950 code objects: every kernel without scratch (private) memory. A kernel that indexes an
argument struct's array at run time, or spills, gets a private segment; the decode kernels are written so that none
does (a struct in scratch made the GEMVs three times slower). Runs on the CPU over the library build() made."""
import os
import re
import shutil
import subprocess

import pytest

from paths import package

LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def code_objects(tmp_path):
    lib = package().hip_engine.LIBRARY
    fat = tmp_path / "fatbin.bin"
    # the section copied out into a file of its own (objcopy given no output file would rewrite the library in place)
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", lib, str(fat)], check=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in the library"
    out = []
    for i, at in enumerate(starts):
        piece = tmp_path / f"bundle{i}.bin"
        piece.write_bytes(data[at:starts[i + 1] if i + 1 < len(starts) else len(data)])
        co = tmp_path / f"dev{i}.co"
        subprocess.run([f"{LLVM}/clang-offload-bundler", "--type=o", "--unbundle", f"--input={piece}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
        out.append(co)
    return out


@pytest.mark.skipif(not (os.path.exists(f"{LLVM}/clang-offload-bundler") and shutil.which("objcopy")),
                    reason="ROCm's clang-offload-bundler or objcopy missing")
def test_no_kernel_uses_scratch(tmp_path):
    kernels, scratch = 0, []
    for co in code_objects(tmp_path):
        notes = subprocess.run([f"{LLVM}/llvm-readelf", "--notes", str(co)], check=True, stdout=subprocess.PIPE,
                               text=True).stdout
        name = None
        for line in notes.splitlines():
            m = re.match(r"\s+\.name:\s+(\S+)", line)
            if m:
                name = m.group(1)
            m = re.match(r"\s+\.private_segment_fixed_size:\s+(\d+)", line)
            if m:
                kernels += 1
                if int(m.group(1)):
                    scratch.append((name, int(m.group(1))))
    assert kernels > 100
    assert not scratch, scratch


@pytest.mark.skipif(not (os.path.exists(f"{LLVM}/clang-offload-bundler") and shutil.which("objcopy")),
                    reason="ROCm's clang-offload-bundler or objcopy missing")
def test_decode_kernels_lead_their_code_objects(tmp_path):
    """every name of csrc/decode_order.txt is a kernel of the library, and in its code object those named lie first,
    in the file's order (the device linker's symbol order; a renamed kernel would otherwise drop out of it silently)"""
    order_file = os.path.join(os.path.dirname(package().hip_engine.LIBRARY), "csrc", "decode_order.txt")
    wanted = [ln.strip() for ln in open(order_file) if ln.strip() and not ln.startswith("#")]
    assert len(wanted) == len(set(wanted)) > 10
    found = set()
    for co in code_objects(tmp_path):
        syms = subprocess.run([f"{LLVM}/llvm-readelf", "-sW", str(co)], check=True, stdout=subprocess.PIPE,
                              text=True).stdout
        funcs = {}
        for line in syms.splitlines():
            f = line.split()
            if len(f) >= 8 and f[3] == "FUNC" and int(f[2]) > 0:
                funcs.setdefault(f[7], int(f[1], 16))
        by_address = [name for name, _ in sorted(funcs.items(), key=lambda kv: kv[1])]
        here = [name for name in wanted if name in funcs]
        assert by_address[:len(here)] == here, (co.name, by_address[:len(here)], here)
        found.update(here)
    assert found == set(wanted), sorted(set(wanted) - found)
