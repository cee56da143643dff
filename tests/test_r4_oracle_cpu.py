"""CPU: the Q4R4 / Q8R4 oracle (f16 group scales, 4-row blocks, group-32
int8 activations) against the compiled reference (oracle/_ref), and the
reference's own properties from c/tests/q4r4_tests.c."""
import ctypes as C

import numpy as np
import pytest

from cpu_libs import (o_matmul_r4, o_pack_r4, o_quant_g32, oracle, ptr, randn, ref, ref_matmul_r4, ref_pack_r4,
                      f32)

needs_ref = pytest.mark.skipif(ref(True) is None, reason="oracle/_ref not built or no AVX512-VNNI host")


def f16_all():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_f16_roundtrip_every_finite_half():
    # q4r4_tests.c:25-38: every finite half survives f16 -> f32 -> f16
    o = oracle()
    for h in f16_all():
        if ((int(h) >> 10) & 0x1f) == 0x1f:
            continue
        f = o.o_f16_to_f32(int(h))
        b = o.o_f32_to_f16(f)
        assert b == h or (f == 0.0 and (b & 0x7fff) == 0), hex(h)
    assert o.o_f32_to_f16(1.0) == 0x3c00 and o.o_f32_to_f16(65504.0) == 0x7bff
    assert o.o_f32_to_f16(1e6) == 0x7c00
    assert o.o_f32_to_f16(1.00048828125) == 0x3c00 and o.o_f32_to_f16(1.00146484375) == 0x3c02


def test_f16_to_f32_matches_numpy():
    # IEEE binary16 decoding is fixed by the standard: numpy's float16 is a
    # second, independent decoder (every half, subnormals and inf/nan incl.)
    o = oracle()
    for h in f16_all()[::7].tolist() + [0x0001, 0x03ff, 0x0400, 0x7bff, 0x7c00, 0xfc00, 0x8001]:
        a = np.float32(o.o_f16_to_f32(h))
        b = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        assert (np.isnan(a) and np.isnan(b)) or a.view(np.uint32) == b.view(np.uint32), hex(h)


def test_f32_to_f16_matches_numpy_rounding():
    # numpy's float32 -> float16 cast rounds to nearest even (IEEE); NaN
    # payloads aside the reference's encoder must agree on every input
    o = oracle()
    rs = np.random.default_rng(5)
    xs = np.concatenate([rs.standard_normal(3000).astype(np.float32) * 10.0 ** rs.integers(-9, 6, 3000),
                         np.array([6.1e-5, 6.0e-8, 5.9e-8, 2.98e-8, 65519.0, 65520.0, -0.0, 0.0], np.float32)])
    for x in xs.astype(np.float32):
        a = o.o_f32_to_f16(float(x))
        with np.errstate(over="ignore"):
            b = int(np.array([x], np.float32).astype(np.float16).view(np.uint16)[0])
        assert a == b, (x, hex(a), hex(b))


@needs_ref
def test_f16_conversions_match_ref():
    o, r = oracle(), ref(True)
    for h in f16_all()[::3]:
        a, b = np.float32(o.o_f16_to_f32(int(h))), np.float32(r.moty_hw_f16_to_f32(int(h)))
        assert (np.isnan(a) and np.isnan(b)) or a.view(np.uint32) == b.view(np.uint32)
    for x in (randn(11, 2000) * np.float32(1e3)).astype(np.float32):
        assert o.o_f32_to_f16(float(x)) == r.moty_f32_to_f16(float(x))


def test_quant_g32_properties():
    # q4r4_tests.c:41-59: sum of codes, |q| <= 127, the group max maps to 127,
    # an all-zero group gets s = 1e-30 and zero codes
    I = 32 * 37
    x = randn(2, (1, I)) * 3
    x[0, ::53] *= 13
    x[0, 64:96] = 0
    xq, xs, xm = o_quant_g32(x)
    g = xq.reshape(-1, 32).astype(np.int32)
    assert (g.sum(1) == xm[0]).all() and np.abs(g).max() <= 127
    amax = np.abs(g).max(1)
    assert amax[2] == 0 and xs[0, 2] == np.float32(1e-30)
    assert (np.delete(amax, 2) == 127).all()
    err = np.abs(x.reshape(-1, 32).astype(np.float64) - xs[0][:, None].astype(np.float64) * g)
    assert (err <= xs[0][:, None] * 0.5 * (1 + 1e-5)).all()


@needs_ref
def test_quant_g32_matches_ref():
    r = ref(True)
    for I in (32, 96, 1024, 4096):
        x = randn(I + 3, (1, I)) * 4
        x[0, :32] = 0
        a = o_quant_g32(x)
        q = np.empty(I, np.int8); s = np.empty(I // 32, np.float32); m = np.empty(I // 32, np.int32)
        r.moty_hw_quant_g32(ptr(f32(x[0])), I, ptr(q), ptr(s), ptr(m))
        assert (a[0][0] == q).all() and (a[1][0].view(np.uint32) == s.view(np.uint32)).all() and (a[2][0] == m).all()


@pytest.mark.parametrize("q8", [False, True])
def test_pack_r4_noclip(q8):
    # q4r4_tests.c:63-89 / 211-230: codes in range, the group max exact, every
    # weight within half a step, the step the finest that clips neither sign;
    # the missing rows of the last block are code 8 (0x88) / 0 with scale 0
    O, I = 3, 96
    w = randn(7, (O, I)) * 0.5
    w[0, 5], w[1, 40], w[2, 70], w[2, 71] = 2.0, -3.0, 0.9, -0.8
    q, d = o_pack_r4(w, q8)
    o = oracle()
    nb, lo, hi = I // 32, (128.0 if q8 else 8.0), (127.0 if q8 else 7.0)
    for g in range(nb):
        for r in range(4):
            dd = o.o_f16_to_f32(int(d[g * 4 + r]))
            if r == 3:
                assert dd == 0.0
                blk = q[g * (128 if q8 else 64) + r * (32 if q8 else 16):][:32 if q8 else 16]
                assert (blk == (0 if q8 else 0x88)).all()
                continue
            if q8:
                c = q[g * 128 + r * 32:][:32].astype(np.int32)
            else:
                b = q[g * 64 + r * 16:][:16].astype(np.int32)
                c = np.concatenate([b & 15, b >> 4]) - 8
            wg = w[r, g * 32:(g + 1) * 32].astype(np.float64)
            assert (np.abs(c * dd - wg) <= 0.5 * abs(dd) * 1.001 + 1e-7).all()
            mx = wg[np.argmax(np.abs(wg))]
            opp = np.abs(wg[(wg > 0) != (mx > 0)]).max(initial=0.0)
            dm = max(abs(mx) / lo, opp / hi)
            assert abs(abs(dd) - dm) <= dm * 1e-3 and (dd < 0) == (mx > 0)


@needs_ref
@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("O,I", [(64, 96), (37, 64), (38, 128), (5, 4096)])
def test_pack_r4_matches_ref(q8, O, I):
    w = randn(O * 7 + I, (O, I)) * 0.02
    w[0, :32] = 0  # an all-zero group: scale 0, inverse 0
    q1, d1 = o_pack_r4(w, q8)
    q2, d2 = ref_pack_r4(ref(True), w, q8)
    assert (q1.view(np.uint8) == q2.view(np.uint8)).all() and (d1 == d2).all()


@needs_ref
@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("O,I,S", [(64, 96, 1), (37, 64, 1), (38, 128, 7), (20, 64, 37), (12, 4800, 6),
                                   (16, 1024, 4), (24, 512, 3), (8, 64, 33)])
def test_matmul_r4_matches_ref(q8, O, I, S):
    # the reference's driver: 4-token tiles, per-token tails, > 1 32-token tile
    w = randn(O + I, (O, I)) * 0.02
    x = randn(S + 2 * I, (S, I))
    x[:, ::31] *= 8
    q, d = o_pack_r4(w, q8)
    y1 = o_matmul_r4(x, q, d, O, q8)
    y2 = ref_matmul_r4(ref(True), x, q, d, O, q8)
    assert (y1.view(np.uint32) == y2.view(np.uint32)).all()


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("O,I,S", [(64, 96, 1), (37, 64, 1), (38, 128, 7), (20, 64, 37)])
def test_matmul_r4_vs_double_dequant(q8, O, I, S):
    # q4r4_tests.c:155-194 / 274-306: worst relative error <= 1e-6 of the
    # magnitude sum against a double dequantized reference
    w = randn(O + I + 1, (O, I))
    x = randn(S + I + 2, (S, I))
    x[:, ::31] *= 8
    q, d = o_pack_r4(w, q8)
    y = o_matmul_r4(x, q, d, O, q8).astype(np.float64)
    xq, xs, _ = o_quant_g32(x)
    o = oracle()
    nb = I // 32
    dd = np.array([o.o_f16_to_f32(int(v)) for v in d], np.float64).reshape(-1, nb, 4)
    if q8:
        c = q.reshape(-1, nb, 4, 32).astype(np.float64)
    else:
        b = q.reshape(-1, nb, 4, 16).astype(np.int32)
        c = (np.concatenate([b & 15, b >> 4], axis=3) - 8).astype(np.float64)
    worst = 0.0
    for t in range(S):
        xg = xq[t].reshape(nb, 32).astype(np.float64)
        for o_ in range(O):
            bb, r = o_ // 4, o_ % 4
            f = dd[bb, :, r] * xs[t]
            a = (f[:, None] * c[bb, :, r] * xg).sum()
            mag = (np.abs(f)[:, None] * (128 if q8 else 8) * np.abs(xg)).sum()
            worst = max(worst, abs(y[t, o_] - a) / (mag + 1e-30))
    assert worst <= 1e-6
