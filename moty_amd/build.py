"""Build libmoty_hw_hip.so (hipcc, gfx950) in-tree.

    python -m moty_amd.build          # or __graft_entry__.build()

Every source under moty_amd/csrc is compiled for gfx950 only, with
-ffp-contract=off (the kernels write each FMA the reference performs
explicitly) and with packed-FP32 instruction selection disabled."""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmoty_hw_hip.so")
# measurement support for bench.py (launch and pure-read floors, hand-off
# latency); not part of the product library
PROBE_SRC = "floor_probe.hip"
PROBE_LIB = os.path.join(HERE, "libmoty_probe.so")
SOURCES = ["quant.hip", "gemv_q8.hip", "ffn1.hip", "gemm_q8.hip", "q4g.hip", "r4.hip", "moe.hip", "ops.hip", "gguf.hip", "api.cpp", "expert_cache.cpp"]
HEADERS = ["common.h", "kernels.h", "dev.h"]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


FLAGS = [
    "-O3", "--offload-arch=gfx950", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I" + os.path.join(ROOT, "include"),
]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj] + FLAGS
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, r.stderr))
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, r.stderr))
    os.replace(tmp, LIB)
    pobj = _compile(PROBE_SRC)
    cmd = [hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", "-o", PROBE_LIB + ".tmp", pobj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, r.stderr))
    os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    if verbose:
        print("built", LIB, "and", PROBE_LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
