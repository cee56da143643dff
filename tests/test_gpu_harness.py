"""GPU: the reference-side C binding (tests/c/mat_apply_hip.c, built by
oracle/Makefile against the reference's own objects and the HIP library):
moty_mat_apply with the HIP drop-ins first for WF_I8, WF_I4G, WF_I4, WF_F32,
WF_Q4R4, WF_Q8R4 and the reference's dispatch as the fallback, the
HwBackend matmul_i8 / matmul_i4 slots, and the MoE d1 / batch layers, each
bit for bit against the reference's CPU function, with IDOT4 on and off."""
import os
import subprocess

import pytest

from cpu_libs import cpu_has_vnni
from gpu_util import say

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "oracle", "_ref", "mat_apply_hip")


@pytest.mark.skipif(not os.path.exists(HARNESS) or not cpu_has_vnni(),
                    reason="harness not built (needs the reference tree at build time) or no AVX512-VNNI host")
@pytest.mark.parametrize("idot4", ["1", None])
def test_reference_binding(dev, idot4):
    say("mat_apply_hip harness IDOT4=%s" % idot4)
    env = dict(os.environ)
    env.pop("IDOT4", None)
    env.pop("IDOT", None)
    if idot4:
        env["IDOT4"] = idot4
    r = subprocess.run([HARNESS], env=env, capture_output=True, text=True, timeout=240)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "ALL PASS" in r.stdout
