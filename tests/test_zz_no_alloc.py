"""GPU: the no-allocation MoE entry point (moty_hip_moe_topk_noalloc_dev,
fixed device scratch) against the allocating one (moty_hip_moe_topk_dev),
bit for bit, through the C-ABI: two calls in a row, the second smaller, so
the fixed array's leftover contents from the first call must not matter."""
import ctypes as C

import numpy as np
import pytest
import torch

from cpu_libs import fast_moe_weights, randn
from gpu_util import same_bits, say, to_dev, to_np

pytestmark = pytest.mark.gpu


def call(lib, fn, view, x, out, idx, w, cnt):
    import moty_amd
    v = moty_amd.MotyHipMoe.from_buffer_copy(view)
    v.idx_out, v.w_out, v.counts_out = idx.data_ptr(), w.data_ptr(), cnt.data_ptr()
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return getattr(lib, fn)(C.byref(v), C.c_void_p(x.data_ptr()), x.shape[0], C.c_void_p(out.data_ptr()), st)


@pytest.mark.parametrize("order,norm", [(1, 1), (0, 0)])
def test_noalloc_moe_matches_allocating_entry(dev, order, norm):
    import moty_amd
    from moty_amd.ops import MoeLayer
    lib = moty_amd.lib()
    E, K, I, D = 64, 8, 1024, 2048
    say("noalloc moe", order, norm)
    ex = {k: to_dev(v) for k, v in fast_moe_weights(E, I, D, seed=70).items()}
    Wr = to_dev(randn(71, (E, D), 0.02))
    L = MoeLayer(Wr, ex["G"], ex["GS"], ex["U"], ex["US"], ex["Dn"], ex["DS"], K, norm_topk=norm, order=order)
    for T in (256, 37):  # the second call is smaller
        x = to_dev(randn(72 + T, (T, D)))
        res = []
        for fn in ("moty_hip_moe_topk_noalloc_dev", "moty_hip_moe_topk_dev"):
            out = torch.full((T, D), float("nan"), device=dev)
            idx = torch.full((T, K), -1, dtype=torch.int32, device=dev)
            w = torch.full((T, K), float("nan"), device=dev)
            cnt = torch.full((E,), -1, dtype=torch.int32, device=dev)
            assert call(lib, fn, L.view, x, out, idx, w, cnt) == 0, lib.moty_hip_last_error()
            res.append([to_np(t) for t in (out, idx, w, cnt)])
        for a, b in zip(*res):
            assert same_bits(a, b)


def test_noalloc_rejects_oversized(dev):
    import moty_amd
    from moty_amd.ops import MoeLayer
    lib = moty_amd.lib()
    E, K, I, D = 8, 8, 1024, 2048
    ex = {k: to_dev(v) for k, v in fast_moe_weights(E, I, D, seed=80).items()}
    Wr = to_dev(randn(81, (E, D), 0.02))
    L = MoeLayer(Wr, ex["G"], ex["GS"], ex["U"], ex["US"], ex["Dn"], ex["DS"], K)
    T = 2048  # 16384 pairs: about 200 MiB of scratch
    x = torch.zeros((T, D), device=dev)
    out = torch.zeros((T, D), device=dev)
    idx = torch.zeros((T, K), dtype=torch.int32, device=dev)
    w = torch.zeros((T, K), device=dev)
    cnt = torch.zeros(E, dtype=torch.int32, device=dev)
    rc = call(lib, "moty_hip_moe_topk_noalloc_dev", L.view, x, out, idx, w, cnt)
    assert rc == moty_amd.EINVAL
    assert b"fixed" in lib.moty_hip_last_error()
