"""CPU: the expert-cache bookkeeping oracle (LFRU slots, pins, hit/miss
counters, route bias) against the reference's own runtime/moecache.c
(compiled into oracle/_ref) on random get/pin sequences, and the closed-form
behaviour of runtime/moe.h's contract: no eviction when cap >= n_experts,
pinned experts never evicted while an unpinned one is resident."""
import numpy as np
import pytest

from cpu_libs import OCache, RefCache, ref

needs_ref = pytest.mark.skipif(ref(True) is None, reason="oracle/_ref not built or no AVX512-VNNI host")


def drive(caches, ops_):
    for op, eid in ops_:
        outs = [getattr(c, op)(eid) for c in caches]
        assert all(o == outs[0] for o in outs), (op, eid, outs)
        states = [c.state().key() for c in caches]
        assert all(s == states[0] for s in states), (op, eid)


def random_ops(seed, E, n, pin_rate=0.03, hot=None):
    g = np.random.default_rng(seed)
    ops_ = []
    for _ in range(n):
        if hot is not None and g.random() < 0.6:
            e = int(g.choice(hot))
        else:
            e = int(g.integers(0, E))
        ops_.append(("pin" if g.random() < pin_rate else "get", e))
    return ops_


@needs_ref
@pytest.mark.parametrize("cap,E,seed", [(1, 8, 0), (4, 16, 1), (8, 64, 2), (20, 64, 3), (64, 64, 4), (100, 64, 5),
                                        (24, 128, 6)])
def test_against_ref(cap, E, seed):
    hot = list(range(0, E, max(1, E // 8)))
    drive([OCache(cap, E), RefCache(ref(True), cap, E)], random_ops(seed, E, 3000, hot=hot))


@needs_ref
def test_against_ref_no_heat():
    # n_experts = 0: no heat tracking, the reference's LRU-by-fill stand-in
    drive([OCache(5, 0), RefCache(ref(True), 5, 0)], [("get", int(e)) for e in
                                                      np.random.default_rng(9).integers(0, 30, 500)])


@needs_ref
def test_against_ref_all_pinned():
    # every resident pinned: get still evicts slot 0, pin takes slot 0
    ops_ = [("pin", e) for e in range(4)] + [("get", 7), ("get", 8), ("pin", 9), ("get", 1), ("get", 10)]
    drive([OCache(4, 16), RefCache(ref(True), 4, 16)], ops_)


@needs_ref
def test_clock_wrap_recency():
    # recency = 255 - age, floored at 0: long runs push old experts to 0
    ops_ = [("get", e % 3) for e in range(600)] + [("get", 5), ("get", 6), ("get", 0), ("get", 7)]
    drive([OCache(3, 8), RefCache(ref(True), 3, 8)], ops_)


@needs_ref
def test_route_bias_against_ref():
    o, r = OCache(6, 32), RefCache(ref(True), 6, 32)
    drive([o, r], random_ops(11, 32, 200, pin_rate=0.1))
    logits = np.random.default_rng(3).standard_normal(32).astype(np.float32)
    a, b = o.route_bias(logits, 0.75), r.route_bias(logits, 0.75)
    assert (a.view(np.uint32) == b.view(np.uint32)).all()
    assert (o.route_bias(logits, 0.0) == logits).all()


def test_resident_when_cap_covers_experts():
    c = OCache(64, 64)
    for e in np.random.default_rng(0).integers(0, 64, 2000):
        c.get(int(e))
    st = c.state()
    assert st.misses == len(set(st.eids[:st.n])) == st.n  # each expert loaded once, never evicted
    assert st.hits + st.misses == 2000


def test_pinned_survive():
    c = OCache(8, 64)
    for e in (3, 9):
        c.pin(e)
    g = np.random.default_rng(1)
    for e in g.integers(10, 64, 1000):
        c.get(int(e))
        st = c.state()
        assert 3 in st.eids[:st.n] and 9 in st.eids[:st.n]


def test_victim_is_least_score():
    # brute force: after filling, each miss evicts the unpinned resident of
    # least (heat << 8 | recency), first slot on ties
    c = OCache(5, 40)
    g = np.random.default_rng(2)
    heat, last, clock = [0] * 40, [0] * 40, 0
    slots = []
    for e in g.integers(0, 40, 800):
        e = int(e)
        heat[e] += 1
        last[e] = clock
        clock += 1
        if e in slots:
            exp = slots.index(e)
        elif len(slots) < 5:
            slots.append(e)
            exp = len(slots) - 1
        else:
            def score(x):
                age = (clock - last[x]) & 0xFFFFFFFF
                return (heat[x] << 8) | (255 - age if age < 255 else 0)
            sc = [score(x) for x in slots]
            exp = sc.index(min(sc))
            slots[exp] = e
        s, _ = c.get(e)
        assert s == exp
