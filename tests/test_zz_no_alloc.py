"""GPU: the no-allocation MoE entry point (moty_hip_moe_topk_noalloc_dev,
fixed device scratch) against the allocating one (moty_hip_moe_topk_dev),
bit for bit, through the C-ABI: two calls in a row, the second smaller, so
the fixed array's leftover contents from the first call must not matter;
sequential calls on two streams; calls captured into a HIP graph (where an
allocation, an arena resize or a device synchronisation would fail the
capture) and replayed; and the set-up rule (moty_hip_init first)."""
import threading
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


def bufs(dev, T, D, K, E):
    return (torch.full((T, D), float("nan"), device=dev), torch.full((T, K), -1, dtype=torch.int32, device=dev),
            torch.full((T, K), float("nan"), device=dev), torch.full((E,), -1, dtype=torch.int32, device=dev))


def layer(E, K, I, D, seed, norm=1, order=1):
    from moty_amd.ops import MoeLayer
    ex = {k: to_dev(v) for k, v in fast_moe_weights(E, I, D, seed=seed).items()}
    Wr = to_dev(randn(seed + 1, (E, D), 0.02))
    return MoeLayer(Wr, ex["G"], ex["GS"], ex["U"], ex["US"], ex["Dn"], ex["DS"], K, norm_topk=norm, order=order)


@pytest.mark.parametrize("order,norm", [(1, 1), (0, 0)])
def test_noalloc_moe_matches_allocating_entry(dev, order, norm):
    import moty_amd
    from moty_amd.ops import MoeLayer
    lib = moty_amd.lib()
    assert lib.moty_hip_init(0) == 0, lib.moty_hip_last_error()
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
    assert lib.moty_hip_init(0) == 0, lib.moty_hip_last_error()
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


def test_noalloc_two_streams_in_sequence(dev):
    # call 1 on stream A (large), call 2 on stream B (small) right after it,
    # no host synchronisation between: B must wait for A's use of the array
    import moty_amd
    lib = moty_amd.lib()
    assert lib.moty_hip_init(0) == 0, lib.moty_hip_last_error()
    E, K, I, D = 64, 8, 1024, 2048
    say("noalloc two streams")
    L = layer(E, K, I, D, 90)
    xa, xb = to_dev(randn(91, (256, D))), to_dev(randn(92, (40, D)))
    want = []
    for x in (xa, xb):
        b = bufs(dev, x.shape[0], D, K, E)
        assert call(lib, "moty_hip_moe_topk_dev", L.view, x, *b) == 0, lib.moty_hip_last_error()
        want.append([to_np(t) for t in b])
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ba, bb = bufs(dev, 256, D, K, E), bufs(dev, 40, D, K, E)
    torch.cuda.synchronize()
    with torch.cuda.stream(sa):
        assert call(lib, "moty_hip_moe_topk_noalloc_dev", L.view, xa, *ba) == 0, lib.moty_hip_last_error()
    with torch.cuda.stream(sb):
        assert call(lib, "moty_hip_moe_topk_noalloc_dev", L.view, xb, *bb) == 0, lib.moty_hip_last_error()
    torch.cuda.synchronize()
    for got, exp in zip((ba, bb), want):
        for a, b in zip([to_np(t) for t in got], exp):
            assert same_bits(a, b)


def test_noalloc_under_graph_capture(dev):
    # captured into a graph (no allocation or synchronisation may happen in
    # the call), replayed several times with eager work between the
    # replays; every replay must equal the allocating entry's result
    import moty_amd
    lib = moty_amd.lib()
    assert lib.moty_hip_init(0) == 0, lib.moty_hip_last_error()
    E, K, I, D = 64, 8, 1024, 2048
    T = 64
    say("noalloc graph capture")
    L = layer(E, K, I, D, 95, norm=0, order=0)
    x = to_dev(randn(96, (T, D)))
    ref = bufs(dev, T, D, K, E)
    assert call(lib, "moty_hip_moe_topk_dev", L.view, x, *ref) == 0, lib.moty_hip_last_error()
    want = [to_np(t) for t in ref]
    got = bufs(dev, T, D, K, E)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            rc = call(lib, "moty_hip_moe_topk_noalloc_dev", L.view, x, *got)
    assert rc == 0, lib.moty_hip_last_error()
    for rep in range(4):
        for t in got:
            t.fill_(-7)
        # eager use of the same fixed array between replays (a different shape)
        xo = to_dev(randn(97 + rep, (33, D)))
        assert call(lib, "moty_hip_moe_topk_noalloc_dev", L.view, xo, *bufs(dev, 33, D, K, E)) == 0
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip([to_np(t) for t in got], want):
            assert same_bits(a, b), "replay %d" % rep


def test_noalloc_needs_init_on_the_thread(dev):
    # a thread that never called moty_hip_init gets EINVAL, not a silent
    # set-up that allocates
    import moty_amd
    lib = moty_amd.lib()
    E, K, I, D = 8, 2, 128, 256
    L = layer(E, K, I, D, 98)
    x = to_dev(randn(99, (4, D)))
    b = bufs(dev, 4, D, K, E)
    res = {}

    def run():
        res["rc"] = call(lib, "moty_hip_moe_topk_noalloc_dev", L.view, x, *b)
        res["msg"] = lib.moty_hip_last_error()

    th = threading.Thread(target=run)
    th.start()
    th.join()
    assert res["rc"] == moty_amd.EINVAL
    assert b"moty_hip_init" in res["msg"]
