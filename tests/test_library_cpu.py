"""CPU: the C-ABI library loads and exports every symbol include/moty_hw_hip.h
declares (no compute without a GPU), and the host-side error behaviour."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moty_hw_hip.h")
LIB = os.path.join(ROOT, "moty_amd", "libmoty_hw_hip.so")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(moty_hip_\w+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared()
    assert "moty_hip_matmul_q_s" in names and "moty_hip_moe_topk_dev" in names
    assert len(names) >= 20


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(l.split()[-1] for l in out.splitlines() if " T " in l)
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_python_binding_covers_header():
    import moty_amd
    assert set(declared()) == set(moty_amd.SIGNATURES)
    L = moty_amd.lib()
    assert L.moty_hip_kernel_tier() == b"gfx950-mfma-i8/gfx950-f32"


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_no_device_reports_error_not_abort():
    import torch
    if torch.cuda.is_available():
        pytest.skip("has a GPU")
    import moty_amd
    rc = moty_amd.lib().moty_hip_init(0)
    assert rc != 0
    assert moty_amd.lib().moty_hip_last_error()


def test_bench_refuses_several_gpus():
    # one GPU per box: --gpus N > 1 exits with a message before touching a device
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and not r.stdout
