"""GPU: the device expert cache (runtime/moecache.c on HBM slots) and the MoE
layer over it.  Bookkeeping (slot of every expert, heat/recency/clock,
hits/misses, the loads issued) against the oracle's restatement driven with
the reference's expert_get sequence; layer outputs bit-exact against the
oracle's uncached layer, with caches small enough to force evictions inside
a call (several GEMM passes) and across calls."""
import ctypes as C

import numpy as np
import pytest
import torch

from cpu_libs import OCache, o_matmul_q_s, o_moe, o_quantize_rows, randn
from gpu_util import mismatch, same_bits, say, to_dev, to_np

pytestmark = pytest.mark.gpu


def q8(seed, shape):
    w = randn(seed, shape, 0.02)
    q, s = o_quantize_rows(w.reshape(-1, shape[-1]))
    return q.reshape(shape), s.reshape(shape[:-1])


def experts(E, I, D, seed=10):
    G, GS = q8(seed, (E, I, D))
    U, US = q8(seed + 1, (E, I, D))
    Dn, DS = q8(seed + 2, (E, D, I))
    return dict(G=G, GS=GS, U=U, US=US, Dn=Dn, DS=DS)


class Loader:
    """LoadExpertFn over host-resident stacked experts; records each call."""

    def __init__(self, ex, layer=3):
        from moty_amd import LOAD_EXPERT_FN
        self.ex, self.layer = ex, layer
        self.calls, self.errors = [], []
        self.fn = LOAD_EXPERT_FN(self._load)

    def _load(self, ctx, layer, eid, slot, inter, hidden):
        try:
            s = slot.contents
            assert s.eid == eid and layer == self.layer
            ex = self.ex
            assert (inter, hidden) == ex["G"].shape[1:]
            for dst, key in ((s.g, "G"), (s.u, "U"), (s.d, "Dn"), (s.gs, "GS"), (s.us, "US"), (s.ds, "DS")):
                a = np.ascontiguousarray(ex[key][eid])
                C.memmove(dst, a.ctypes.data, a.nbytes)
            self.calls.append(eid)
        except Exception as e:  # a callback cannot raise through C
            self.errors.append(repr(e))


class Cache:
    def __init__(self, cap, E):
        from moty_amd import lib
        self.L, self.cap, self.E = lib(), cap, E
        self.p = C.c_void_p()
        assert self.L.moty_hip_expert_cache_init(C.byref(self.p), cap, E) == 0

    def free(self):
        assert self.L.moty_hip_expert_cache_free(self.p) == 0

    def state(self):
        n = C.c_int()
        eids = np.empty(max(self.cap, 1), np.int32)
        heat = np.zeros(max(self.E, 1), np.uint32)
        last = np.zeros(max(self.E, 1), np.uint32)
        clock = C.c_uint32()
        hits, misses = C.c_longlong(), C.c_longlong()
        P = lambda a: C.c_void_p(a.ctypes.data)
        assert self.L.moty_hip_expert_cache_stats(self.p, C.byref(n), P(eids), P(heat), P(last), C.byref(clock),
                                                  C.byref(hits), C.byref(misses)) == 0
        return (n.value, tuple(eids[:n.value].tolist()), tuple(heat[:self.E].tolist()),
                tuple(last[:self.E].tolist()), clock.value, hits.value, misses.value)


def oracle_key(o):
    st = o.state()
    return (st.n, tuple(st.eids[:st.n]), tuple(st.heat), tuple(st.last), st.clock, st.hits, st.misses)


def get_sequence(idx, E, order):
    if order == "batch":  # nn/moe.c:186-203: ascending id, once per active expert
        return [e for e in range(E) if (idx == e).any()]
    return [int(e) for e in idx.reshape(-1)]  # engines/olmoe.c:230-233: per token, top-k order


def run_layer(cache, loader, Wr_d, K, norm, order, x, E, I, D, stream=True):
    from moty_amd import MotyHipMoe, ORDER_EXPERT, ORDER_TOPK, lib
    S = x.shape[0]
    m = MotyHipMoe()
    m.router = C.c_void_p(Wr_d.data_ptr())
    m.E, m.K, m.I, m.D = E, K, I, D
    m.norm_topk = norm
    m.combine_order = ORDER_EXPERT if order == "batch" else ORDER_TOPK
    idx = torch.empty((S, K), dtype=torch.int32, device="cuda:0")
    m.idx_out = C.c_void_p(idx.data_ptr())
    xd = to_dev(x)
    y = torch.empty((S, D), device="cuda:0")
    rc = lib().moty_hip_moe_topk_cached_dev(C.byref(m), cache.p, None, loader.layer, loader.fn,
                                            C.c_void_p(xd.data_ptr()), S, C.c_void_p(y.data_ptr()),
                                            C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib().moty_hip_last_error()
    return to_np(y), to_np(idx)


@pytest.mark.parametrize("E,K,I,D,S,cap", [(16, 4, 64, 128, 24, 16), (16, 4, 64, 128, 24, 5), (64, 8, 256, 512, 32, 64),
                                           (64, 8, 256, 512, 32, 12), (8, 2, 32, 64, 9, 1), (32, 8, 64, 96, 40, 8),
                                           (16, 4, 96, 128, 200, 3)])
@pytest.mark.parametrize("order", ["batch", "olmoe"])
def test_cached_layer(dev, E, K, I, D, S, cap, order):
    say("moe cached", E, K, I, D, S, cap, order)
    ex = experts(E, I, D)
    Wr = randn(1, (E, D), 0.02)
    norm = 1 if order == "batch" else 0
    cache, oc, loader = Cache(cap, E), OCache(cap, E), Loader(ex)
    expect_loads = []
    try:
        Wr_d = to_dev(Wr)
        for call in range(3):  # state carries across calls
            x = randn(20 + call, (S, D))
            y, idx = run_layer(cache, loader, Wr_d, K, norm, order, x, E, I, D)
            y2, idx2, _ = o_moe(x, Wr, ex, K, order, norm=norm)
            assert (idx == idx2).all()
            assert same_bits(y, y2), mismatch(y, y2)
            for e in get_sequence(idx2, E, order):
                _, loaded = oc.get(e)
                if loaded:
                    expect_loads.append(e)
            assert cache.state() == oracle_key(oc), "call %d" % call
        assert not loader.errors, loader.errors
        assert loader.calls == expect_loads
    finally:
        cache.free()


def test_cached_layer_host(dev):
    # the host-pointer drop-in: x/out/router on the host
    from moty_amd import MotyHipMoe, ORDER_EXPERT, lib
    say("moe cached host")
    E, K, I, D, S, cap = 16, 4, 64, 128, 30, 6
    ex = experts(E, I, D, seed=40)
    Wr = randn(2, (E, D), 0.02)
    x = randn(3, (S, D))
    cache, loader = Cache(cap, E), Loader(ex)
    try:
        m = MotyHipMoe()
        m.router = C.c_void_p(Wr.ctypes.data)
        m.E, m.K, m.I, m.D = E, K, I, D
        m.norm_topk, m.combine_order = 1, ORDER_EXPERT
        idx = np.empty((S, K), np.int32)
        m.idx_out = C.c_void_p(idx.ctypes.data)
        y = np.empty((S, D), np.float32)
        assert lib().moty_hip_moe_topk_cached(C.byref(m), cache.p, None, loader.layer, loader.fn,
                                              C.c_void_p(x.ctypes.data), S, C.c_void_p(y.ctypes.data)) == 0
        y2, idx2, _ = o_moe(x, Wr, ex, K, "batch")
        assert (idx == idx2).all() and same_bits(y, y2)
        assert not loader.errors
    finally:
        cache.free()


def test_get_pin_standalone(dev):
    # expert_get / expert_pin return device slots holding the expert: checked
    # through a matmul over the slot's gate rows and down rows
    from moty_amd import MotyHipExpertSlot, lib, ops
    say("expert get/pin")
    E, I, D, cap = 24, 64, 96, 5
    ex = experts(E, I, D, seed=50)
    cache, oc, loader = Cache(cap, E), OCache(cap, E), Loader(ex)
    g = np.random.default_rng(4)
    x = randn(5, (3, D))
    xi = randn(6, (3, I))
    try:
        for step in range(120):
            e = int(g.integers(0, E)) if g.random() > 0.3 else int(g.integers(0, 4))
            pin = g.random() < 0.05
            sp = C.POINTER(MotyHipExpertSlot)()
            fn = lib().moty_hip_expert_pin if pin else lib().moty_hip_expert_get
            assert fn(cache.p, None, loader.layer, e, loader.fn, I, D, C.byref(sp)) == 0
            (oc.pin if pin else oc.get)(e)
            assert cache.state() == oracle_key(oc), step
            s = sp.contents
            assert s.eid == e
            if step % 10 == 0:
                y = torch.empty((3, I), device="cuda:0")
                rc = lib().moty_hip_matmul_q_s_dev(C.c_void_p(y.data_ptr()), C.c_void_p(to_dev(x).data_ptr()),
                                                   C.c_void_p(s.g), C.c_void_p(s.gs), 3, D, I,
                                                   C.c_void_p(torch.cuda.current_stream().cuda_stream))
                assert rc == 0
                assert same_bits(to_np(y), o_matmul_q_s(x, ex["G"][e], ex["GS"][e]))
                y = torch.empty((3, D), device="cuda:0")
                rc = lib().moty_hip_matmul_q_s_dev(C.c_void_p(y.data_ptr()), C.c_void_p(to_dev(xi).data_ptr()),
                                                   C.c_void_p(s.d), C.c_void_p(s.ds), 3, I, D,
                                                   C.c_void_p(torch.cuda.current_stream().cuda_stream))
                assert rc == 0
                assert same_bits(to_np(y), o_matmul_q_s(xi, ex["Dn"][e], ex["DS"][e]))
        assert not loader.errors
        logits = randn(7, (E,))
        a = logits.copy()
        lib().moty_hip_moe_route_bias(C.c_void_p(a.ctypes.data), cache.p, 0.5)
        assert same_bits(a, oc.route_bias(logits, 0.5))
    finally:
        cache.free()


def test_cache_errors(dev):
    from moty_amd import MotyHipExpertSlot, lib
    E, I, D = 8, 32, 64
    ex = experts(E, I, D, seed=60)
    cache, loader = Cache(2, E), Loader(ex)
    sp = C.POINTER(MotyHipExpertSlot)()
    try:
        assert lib().moty_hip_expert_get(cache.p, None, 3, E, loader.fn, I, D, C.byref(sp)) == 1  # eid out of range
        assert lib().moty_hip_expert_get(cache.p, None, 3, 1, loader.fn, I, D, C.byref(sp)) == 0
        assert lib().moty_hip_expert_get(cache.p, None, 3, 2, loader.fn, I * 2, D, C.byref(sp)) == 1  # other shape
    finally:
        cache.free()
