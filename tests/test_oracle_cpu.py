"""CPU: the oracle restatement against the compiled reference (oracle/_ref),
closed forms, brute force and the reference's own test properties
(c/tests/simd_tests.c, kernels_tests.c, qwen_tests.c, moe_tests.c)."""
import ctypes as C

import numpy as np
import pytest

from cpu_libs import (o_matmul_f32, o_matmul_i4g, o_matmul_q8_acc, o_matmul_q_s, o_moe, o_pack_int4_grouped,
                      o_qrow, o_quantize_rows, o_route, oracle, ptr, randn, ref, rng)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else a.dtype)


needs_ref = pytest.mark.skipif(ref(True) is None, reason="oracle/_ref not built or no AVX512-VNNI host")


# ---- a1 qrow_i8: reconstruction bound (simd_tests.c:127-145) and _ref ----
@pytest.mark.parametrize("n", [1, 7, 64, 1000, 4096])
def test_qrow_bound(n):
    x = randn(n, (4, n)) * 3
    q, sx = o_qrow(x)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    err = np.abs(x.astype(np.float64) - sx[:, None].astype(np.float64) * q)
    assert np.all(err <= sx[:, None] * 0.5 * (1 + 1e-5))


def test_qrow_zero_row_clamps():
    q, sx = o_qrow(np.zeros((1, 32), np.float32))
    assert sx[0] == np.float32(1e-12) and not q.any()


@needs_ref
def test_qrow_matches_ref():
    r = ref(True)
    for n in [1, 33, 1024, 3072]:
        x = randn(n + 1, n) * 5
        q1, s1 = o_qrow(x[None])
        q2 = np.empty(n, np.int8)
        s2 = r.ref_qrow_i8(ptr(x), ptr(q2), n)
        assert np.float32(s2) == s1[0] and (q1[0] == q2).all()


# ---- a2 dot_i8i8: exact vs int64 (simd_tests.c:22-44), w = -128 rep ----
@needs_ref
def test_dot_i8i8_exact():
    r = ref(True)
    g = rng(5)
    for n in list(range(1, 258, 17)) + [4096]:
        for rep in range(3):
            w = g.integers(-128, 128, n, dtype=np.int8) if rep else np.full(n, -128, np.int8)
            x = g.integers(-127, 128, n, dtype=np.int8)
            exact = int(np.dot(w.astype(np.int64), x.astype(np.int64)))
            assert oracle().o_dot_i8i8(ptr(w), ptr(x), n) == exact
            assert r.ref_dot_i8i8(ptr(w), ptr(x), n) == exact


# ---- a4 / a6 quantizers ----
@needs_ref
@pytest.mark.parametrize("O,I", [(7, 33), (64, 1024), (16, 3072)])
def test_quantize_rows_matches_ref(O, I):
    w = randn(O * I, (O, I), 0.02)
    q, s = o_quantize_rows(w)
    q2 = np.empty_like(q)
    s2 = np.empty_like(s)
    ref(True).ref_quantize_rows(ptr(w), ptr(q2), ptr(s2), O, I, 8)
    assert (q == q2).all() and (bits(s) == bits(s2)).all()


@needs_ref
@pytest.mark.parametrize("O,I,gs", [(5, 31, 16), (8, 100, 32), (64, 4096, 32)])
def test_pack_int4_grouped_matches_ref(O, I, gs):
    w = randn(O + I, (O, I), 0.02)
    q4, s = o_pack_int4_grouped(w, gs)
    q42 = np.empty_like(q4)
    s2 = np.empty_like(s)
    ref(True).ref_pack_int4_grouped(ptr(w), ptr(q42), ptr(s2), O, I, gs)
    assert (q4 == q42).all() and (bits(s) == bits(s2)).all()


def test_pack_int4_grouped_roundtrip():
    # qwen_tests.c:137-170: |w - s*(n-8)| <= s/2 inside the clip range
    O, I = 8, 256
    w = randn(3, (O, I), 0.02)
    q4, s = o_pack_int4_grouped(w, 32)
    n = np.zeros((O, I), np.int32)
    n[:, 0::2] = q4 & 15
    n[:, 1::2] = q4 >> 4
    deq = (n - 8) * np.repeat(s, 32, axis=1)
    assert np.all(np.abs(w - deq) <= np.repeat(s, 32, axis=1) * 0.5 * (1 + 1e-5) + 1e-9)


# ---- a3 matmul_q_s ----
@needs_ref
@pytest.mark.parametrize("S,I,O", [(1, 1024, 96), (4, 48, 24), (8, 3072, 32), (3, 17, 5)])
def test_matmul_q_s_matches_ref(S, I, O):
    w = randn(1, (O, I), 0.02)
    q, s = o_quantize_rows(w)
    x = randn(2, (S, I))
    y = o_matmul_q_s(x, q, s)
    y2 = np.empty_like(y)
    ref(True).ref_matmul_q_s(ptr(y2), ptr(x), ptr(q), ptr(s), S, I, O)
    assert (bits(y) == bits(y2)).all()


def test_matmul_q_s_batch_invariance():
    # qwen_tests.c:96-110: S rows == S single calls, memcmp
    w = randn(4, (24, 96), 0.02)
    q, s = o_quantize_rows(w)
    x = randn(5, (4, 96))
    y = o_matmul_q_s(x, q, s)
    for i in range(4):
        assert (bits(o_matmul_q_s(x[i:i + 1], q, s)) == bits(y[i:i + 1])).all()


def test_q8_acc_brute_force():
    g = rng(9)
    xq = g.integers(-127, 128, (3, 200), dtype=np.int8)
    q = g.integers(-128, 128, (7, 200), dtype=np.int8)
    acc = o_matmul_q8_acc(xq, q)
    assert (acc == xq.astype(np.int64) @ q.astype(np.int64).T).all()


def test_matmul_q_close_to_f32():
    # qwen_tests.c:82-93: matmul_q vs f32 matmul, |d| < 0.05 at O=24 I=32
    w = rng(6).uniform(-1, 1, (24, 32)).astype(np.float32)
    x = rng(7).uniform(-1, 1, (1, 32)).astype(np.float32)
    q, s = o_quantize_rows(w)
    assert np.abs(o_matmul_q_s(x, q, s) - x @ w.T).max() < 0.05


# ---- a7/a8 grouped int4 ----
@needs_ref
@pytest.mark.parametrize("I", [64, 1024, 4096, 12288])
def test_i4g_idot4_matches_ref(I):
    w = randn(I, (32, I), 0.02)
    q4, s = o_pack_int4_grouped(w)
    x = randn(I + 1, (3, I))
    y = o_matmul_i4g(x, q4, s, True)
    y2 = np.empty_like(y)
    ref(True).ref_matmul_i4_grouped_s(ptr(y2), ptr(x), ptr(q4), ptr(s), 3, I, 32, 32)
    assert (bits(y) == bits(y2)).all()


@needs_ref
@pytest.mark.parametrize("I", [32, 96, 1024, 4096])
def test_i4g_f32_matches_ref(I):
    w = randn(I, (32, I), 0.02)
    q4, s = o_pack_int4_grouped(w)
    x = randn(I + 1, (3, I))
    y = o_matmul_i4g(x, q4, s, False)
    y2 = np.empty_like(y)
    ref(False).ref_matmul_i4_grouped_s(ptr(y2), ptr(x), ptr(q4), ptr(s), 3, I, 32, 32)
    assert (bits(y) == bits(y2)).all()


@pytest.mark.parametrize("I", [128, 256, 1024, 2048, 1792])
def test_i4g_vs_double_dequant(I):
    # kernels_tests.c:30-64: rel 5e-3*(1+|ref|) against a double dequant reference
    w = randn(I, (8, I), 0.02)
    q4, s = o_pack_int4_grouped(w)
    x = randn(I + 7, (1, I))
    n = np.zeros((8, I), np.int64)
    n[:, 0::2] = q4 & 15
    n[:, 1::2] = q4 >> 4
    deq = (n - 8) * np.repeat(s.astype(np.float64), 32, axis=1)
    xi, sx = o_qrow(x)
    for idot4 in (True, False):
        # the IDOT4 path computes with the int8 activations, as the reference test does
        xv = xi.astype(np.float64) * np.float64(sx[0]) if idot4 else x.astype(np.float64)
        refv = xv @ deq.T
        y = o_matmul_i4g(x, q4, s, idot4)
        assert np.all(np.abs(y - refv) <= 5e-3 * (1 + np.abs(refv)))


def test_i4g_batch_invariance():
    # kernels_tests.c:88-114: S=8 == 8 x S=1
    w = randn(2, (16, 256), 0.02)
    q4, s = o_pack_int4_grouped(w)
    x = randn(3, (8, 256))
    for idot4 in (True, False):
        y = o_matmul_i4g(x, q4, s, idot4)
        for i in range(8):
            assert (bits(o_matmul_i4g(x[i:i + 1], q4, s, idot4)) == bits(y[i:i + 1])).all()


# ---- a10 router dot_f32 ----
@needs_ref
def test_dot_f32_matches_ref():
    r = ref(True)
    for n in [1, 15, 16, 17, 31, 32, 33, 48, 100, 2047, 2048, 2049]:
        a, b = randn(n, n), randn(n + 1, n)
        assert np.float32(oracle().o_dot_f32(ptr(a), ptr(b), n)) == np.float32(r.ref_dot_f32(ptr(a), ptr(b), n))
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        assert abs(oracle().o_dot_f32(ptr(a), ptr(b), n) - exact) <= 1e-5 * (np.abs(a * b).sum() + 1e-30)


@needs_ref
def test_matmul_f32_matches_ref():
    W = randn(3, (64, 2048), 0.02)
    x = randn(4, (8, 2048))
    y = o_matmul_f32(x, W)
    y2 = np.empty_like(y)
    ref(True).ref_matmul(ptr(y2), ptr(x), ptr(W), 8, 2048, 64)
    assert (bits(y) == bits(y2)).all()


# ---- expf / silu / softmax / topk ----
def test_expf_restatement_sampled():
    # every 2^32/2^24-th pattern plus the edges; the full sweep is test_expf_exhaustive
    o = oracle()
    for lo in range(0, 1 << 32, 1 << 28):
        assert o.o_expf_check_range(lo, lo + (1 << 20)) == 0
    edges = [0x42b17217, 0x42b17218, 0xc2cff1b4, 0xc2cff1b5, 0xc2aeac50, 0x7f800000, 0xff800000, 0, 0x80000000, 1]
    for e in edges:
        assert o.o_expf_check_range(e, e + 1) == 0


@pytest.mark.slow
def test_expf_exhaustive():
    assert oracle().o_expf_check_range(0, 1 << 32) == 0


@needs_ref
def test_silu_softmax_topk_match_ref():
    r = ref(True)
    g = randn(1, 5000) * 4
    u = randn(2, 5000)
    g1, g2 = g.copy(), g.copy()
    oracle().o_silu_mul(ptr(g1), ptr(u), 5000)
    r.ref_silu_mul(ptr(g2), ptr(u), 5000)
    assert (bits(g1) == bits(g2)).all()
    for E in (8, 64, 128):
        x = randn(E, E) * 3
        a, b = x.copy(), x.copy()
        oracle().o_softmax(ptr(a), E)
        r.ref_softmax(ptr(b), E)
        assert (bits(a) == bits(b)).all()


def naive_topk(p, K, norm):
    idx, w = [], []
    for _ in range(K):
        best, bv = -1, np.float32(-1e30)
        for e in range(len(p)):
            if e not in idx and p[e] > bv:
                best, bv = e, p[e]
        idx.append(best)
        w.append(bv)
    w = np.array(w, np.float32)
    if norm:
        sm = np.float32(0)
        for v in w:
            sm = np.float32(sm + v)
        if sm > 0:
            w = (w / sm).astype(np.float32)
    return np.array(idx), w


def test_topk_vs_naive():
    # moe_tests.c:15-39: 200 random cases E <= 41, K <= 8, norm on/off, with ties
    g = rng(11)
    for case in range(200):
        E = int(g.integers(1, 42))
        K = int(g.integers(1, min(8, E) + 1))
        p = g.integers(0, 6, E).astype(np.float32) / 5  # many ties
        norm = case % 2
        idx = np.empty(K, np.int32)
        w = np.empty(K, np.float32)
        oracle().o_topk(ptr(p), E, K, ptr(idx), ptr(w), norm)
        ni, nw = naive_topk(p, K, norm)
        assert (idx == ni).all() and (bits(w) == bits(nw)).all()


# ---- a13 MoE ----
def moe_weights(E, I, D, seed=3):
    ex = {}
    for nm, sh, sd in [("G", (E, I, D), seed), ("U", (E, I, D), seed + 1), ("Dn", (E, D, I), seed + 2)]:
        w = randn(sd, sh, 0.02)
        q, s = o_quantize_rows(w.reshape(-1, sh[2]))
        ex[nm] = q.reshape(sh)
        ex[{"G": "GS", "U": "US", "Dn": "DS"}[nm]] = s.reshape(sh[0], sh[1])
    return ex


@needs_ref
def test_moe_matches_ref():
    E, K, I, D, S = 16, 4, 128, 256, 24
    Wr = randn(1, (E, D), 0.02)
    x = randn(2, (S, D))
    ex = moe_weights(E, I, D)
    args = [ptr(ex[k]) for k in ("G", "GS", "U", "US", "Dn", "DS")]
    out, idx, w = o_moe(x, Wr, ex, K, "batch")
    o2 = np.empty_like(out)
    ref(True).ref_moe_batch(ptr(o2), ptr(x), S, ptr(Wr), *args, E, K, I, D)
    assert (bits(out) == bits(o2)).all()
    for norm in (0, 1):
        out, idx, w = o_moe(x, Wr, ex, K, "olmoe", norm=norm)
        o2 = np.empty_like(out)
        i2 = np.empty_like(idx)
        ref(True).ref_moe_olmoe(ptr(o2), ptr(x), S, ptr(Wr), *args, E, K, I, D, norm, ptr(i2))
        assert (bits(out) == bits(o2)).all() and (idx == i2).all()


def test_moe_orders_agree_to_rounding():
    E, K, I, D, S = 8, 2, 64, 64, 5
    Wr = randn(1, (E, D), 0.02)
    x = randn(2, (S, D))
    ex = moe_weights(E, I, D)
    a, ia, _ = o_moe(x, Wr, ex, K, "batch")
    b, ib, _ = o_moe(x, Wr, ex, K, "olmoe", norm=1)
    assert (ia == ib).all()
    assert np.allclose(a, b, rtol=1e-5, atol=1e-7)


def test_route_bias_moves_argmax():
    # moe_tests.c route-bias case: a bias on one expert makes it the top choice
    E, D = 16, 64
    Wr = randn(1, (E, D), 0.02)
    x = randn(2, (4, D))
    bias = np.zeros(E, np.float32)
    bias[5] = 100.0
    idx, _, _ = o_route(x, Wr, 2, 1, bias)
    assert (idx[:, 0] == 5).all()


@needs_ref
@pytest.mark.parametrize("E,K,I,D", [(16, 4, 128, 256), (64, 8, 1024, 2048), (128, 8, 768, 2048), (8, 8, 32, 64)])
def test_moe_d1_matches_ref(E, K, I, D):
    # moty_nn_moe_topk_d1 (nn/moe.c:33-153) is the olmoe order with the
    # routing always normalised: the oracle's olmoe layer at norm = 1
    from cpu_libs import fast_moe_weights
    ex = fast_moe_weights(E, I, D, seed=E + I)
    Wr = randn(E + 1, (E, D), 0.02)
    for seed in (3, 4):
        x = randn(seed, (1, D))
        out, idx, w = o_moe(x, Wr, ex, K, "olmoe", norm=1)
        o2 = np.empty_like(out)
        ref(True).ref_moe_d1(ptr(o2), ptr(x), ptr(Wr), *[ptr(ex[k]) for k in ("G", "GS", "U", "US", "Dn", "DS")],
                             E, K, I, D)
        assert (bits(out) == bits(o2)).all()


@needs_ref
@pytest.mark.parametrize("skewed", [False, True])
def test_moe_batch_matches_ref_at_c5(skewed):
    # the C5 workload (Qwen3-30B-A3B MoE: T = 1072, E = 128, top-8, I = 768,
    # D = 2048) through moe_batch_core (nn/moe.c:159-205): every output row
    from cpu_libs import fast_moe_weights, skew_inputs
    E, K, I, D, T = 128, 8, 768, 2048, 1072
    ex = fast_moe_weights(E, I, D, seed=50)
    Wr = randn(51, (E, D), 0.02)
    x = randn(52, (T, D))
    hot = np.arange(0, 128, 16)
    if skewed:
        x, Wr = skew_inputs(x, Wr, hot)
    out, idx, w = o_moe(x, Wr, ex, K, "batch")
    o2 = np.empty_like(out)
    ref(True).ref_moe_batch(ptr(o2), ptr(x), T, ptr(Wr), *[ptr(ex[k]) for k in ("G", "GS", "U", "US", "Dn", "DS")],
                            E, K, I, D)
    assert (bits(out) == bits(o2)).all()
    cnt = np.bincount(idx.ravel(), minlength=E)
    if skewed:
        assert cnt[hot].sum() > 0.5 * cnt.sum()


# ---- per-row int4 (WF_I4): the HwBackend.matmul_i4 slot ----
@needs_ref
@pytest.mark.parametrize("O,I", [(37, 64), (5, 33), (64, 4096), (9, 1)])
def test_pack_int4_matches_ref(O, I):
    from cpu_libs import o_pack_int4
    w = randn(O + I, (O, I), 0.02)
    w[0] = 0.0  # the 1e-8 clamp
    q4, s = o_pack_int4(w)
    q2 = np.empty_like(q4)
    s2 = np.empty_like(s)
    ref(True).moty_pack_int4(ptr(w), ptr(q2), ptr(s2), O, I)
    assert (q4 == q2).all() and (bits(s) == bits(s2)).all()


@needs_ref
@pytest.mark.parametrize("S,I,O", [(1, 4096, 64), (5, 1024, 33), (3, 96, 17), (2, 64, 8)])
@pytest.mark.parametrize("idot4", [True, False])
def test_matmul_i4_matches_ref(S, I, O, idot4):
    # the reference latches IDOT4 per process: _ref (IDOT4=1) and _ref_f32
    from cpu_libs import o_matmul_i4, o_pack_int4
    q4, s = o_pack_int4(randn(O + 2 * I, (O, I), 0.02))
    x = randn(S + I, (S, I))
    y = o_matmul_i4(x, q4, s, idot4)
    y2 = np.empty_like(y)
    ref(idot4).moty_matmul_i4_s(ptr(y2), ptr(x), ptr(q4), ptr(s), S, I, O)
    assert (bits(y) == bits(y2)).all()


def test_matmul_i4_idot4_brute_force():
    # the integer dot against an int64 brute force, and the f32 path against
    # a double-precision dequantized sum
    from cpu_libs import o_matmul_i4, o_pack_int4, o_qrow
    S, I, O = 3, 320, 11
    q4, s = o_pack_int4(randn(5, (O, I), 0.02))
    x = randn(6, (S, I))
    n = np.empty((O, I), np.int64)
    n[:, 0::2] = (q4 & 15).astype(np.int64) - 8
    n[:, 1::2] = (q4 >> 4).astype(np.int64) - 8
    xq, sx = o_qrow(x)
    d = xq.astype(np.int64) @ n.T
    y = o_matmul_i4(x, q4, s, True)
    y2 = (s[None, :] * sx[:, None]).astype(np.float32) * d.astype(np.float32)
    assert (bits(y) == bits(y2.astype(np.float32))).all()
    yf = o_matmul_i4(x, q4, s, False)
    yd = (x.astype(np.float64) @ n.T.astype(np.float64)) * s.astype(np.float64)[None, :]
    assert np.allclose(yf, yd, rtol=1e-5, atol=1e-5 * np.abs(yd).max())
