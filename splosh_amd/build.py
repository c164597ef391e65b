"""Build libsplosh_q4.so (the HIP kernels and the C ABI) in-tree for gfx950 with hipcc.

    python -m splosh_amd.build          # or splosh_amd.build.build()

Objects go to splosh_amd/_build/, the library to splosh_amd/libsplosh_q4.so. The measurement
probes of csrc/bench/ (not part of the path) go into a library of their own,
splosh_amd/libsplosh_probe.so, which only bench.py loads.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsplosh_q4.so"
SOURCES = ["api.cpp", "q4_basic.hip", "stream.hip", "lanes.hip", "decode.hip", "mma.hip", "tile.hip", "prefill.hip", "q5k.hip", "q5k_decode.hip", "operand.hip", "gguf_native.hip", "gguf_tile.hip"]
PROBE_LIB = PKG / "libsplosh_probe.so"
PROBE_SOURCES = ["bench/probe.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 instructions (v_pk_fma_f32 and the like) are disabled for every device pass: the
# compiler would otherwise form them from ordinary float code, and some of their forms have given
# wrong results on this hardware without an error.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-result",
          f"-I{ROOT / 'include'}"]


def _compile(src):
    obj = BUILD / (src.replace(".", "_").replace("/", "_") + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def _link(objs, lib):
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(lib)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed for {lib.name}:\n{res.stderr}")


def build(verbose=True):
    BUILD.mkdir(exist_ok=True)
    jobs = min(len(SOURCES) + len(PROBE_SOURCES), max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, SOURCES + PROBE_SOURCES))
    _link(objs[: len(SOURCES)], LIB)
    _link(objs[len(SOURCES):], PROBE_LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB.name}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
