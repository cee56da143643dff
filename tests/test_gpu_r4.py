"""GPU: Q4R4 / Q8R4 (f16 group scales, 4-row blocks, group-32 int8
activations) against the oracle, bit for bit: packers, the activation
quantizer, the decode GEMV (S <= 4) and the MFMA GEMM (4-token tile form for
t < 4*floor(S/4), per-token form after), the host drop-in."""
import ctypes as C

import numpy as np
import pytest
import torch

from cpu_libs import o_matmul_r4, o_pack_r4, o_quant_g32, randn
from gpu_util import mismatch, same_bits, say, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(dev):
    from moty_amd import ops as o
    return o


def dev_r4(q, d):
    return to_dev(q), to_dev(d.view(np.int16))


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("O,I,scale", [(64, 96, 0.02), (37, 64, 1.0), (5, 4096, 0.02), (9, 32, 1e-6),
                                       (16, 1024, 3e-9), (3, 128, 1e5)])
def test_pack_r4(ops, q8, O, I, scale):
    # tiny and huge weights drive the f16 scales into subnormals and overflow
    say("pack_r4", q8, O, I, scale)
    w = randn(O * 3 + I, (O, I)) * np.float32(scale)
    w[0, :32] = 0  # an all-zero group: scale 0
    if O > 2:
        w[1, 5] = -3 * abs(w[1]).max()  # a negative group max
    q, d = ops.pack_r4(to_dev(w), q8)
    q2, d2 = o_pack_r4(w, q8)
    assert same_bits(to_np(q).view(np.uint8), q2.view(np.uint8))
    assert same_bits(to_np(d).view(np.uint16), d2)


@pytest.mark.parametrize("S,I", [(1, 32), (3, 96), (7, 1024), (2, 4096), (1, 16384)])
def test_quant_g32(ops, S, I):
    say("quant_g32", S, I)
    x = randn(S * I, (S, I)) * 3
    x[0, :32] = 0
    x[-1, -5] = 1e-30
    xq, xs, xm = ops.quant_g32(to_dev(x))
    a, b, c = o_quant_g32(x)
    assert same_bits(to_np(xq), a) and same_bits(to_np(xs), b) and same_bits(to_np(xm), c)


CASES = [(64, 96, 1), (37, 64, 1), (38, 128, 7), (20, 64, 37), (12, 4800, 6), (16, 1024, 4), (24, 512, 3),
         (8, 64, 33), (1000, 1024, 1), (3072, 1024, 1), (1024, 3072, 1), (1024, 4096, 2), (256, 8192, 1),
         (100, 12288, 1), (192, 4096, 64), (130, 1024, 130), (4096, 1024, 5), (2048, 2048, 4), (64, 4096, 3),
         (1, 32, 1), (7, 32, 9), (64, 16384, 1), (64, 8192, 2), (300, 12288, 1), (40, 8192, 1),
         (256, 3040, 1), (520, 7200, 2), (6000, 2048, 1), (4100, 1056, 3),
         # GEMM grids past 256 tiles (four 32 x 32 waves), ragged and whole token tiles
         (8192, 512, 130), (17000, 256, 64)]


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("O,I,S", CASES)
def test_matmul_r4(ops, q8, O, I, S):
    say("matmul_r4", q8, O, I, S)
    w = randn(O + I, (O, I)) * 0.02
    x = randn(S + 2 * I, (S, I))
    x[:, ::31] *= 8
    q, d = o_pack_r4(w, q8)
    qd, dd = dev_r4(q, d)
    y = to_np(ops.matmul_r4(to_dev(x), qd, dd, O, q8))
    y2 = o_matmul_r4(x, q, d, O, q8)
    assert same_bits(y, y2), mismatch(y, y2)


@pytest.mark.parametrize("q8", [False, True])
def test_matmul_r4_extremes(ops, q8):
    # codes at the ends of their range against activations at +-127 (the
    # int16-lane worst cases of c/tests/q4r4_tests.c), a zero-scale group
    O, I, S = 8, 256, 6
    w = randn(5, (O, I))
    w[0] = np.where(np.arange(I) % 2, 1.0, -1.0)  # codes at -8 / +7 (Q8: -128 / +127)
    w[1] = 1.0
    w[2, :32] = 0
    x = randn(6, (S, I))
    x[0] = np.where(np.arange(I) % 2, 1.0, -1.0)
    x[1] = 1.0
    x[2] = -1.0
    q, d = o_pack_r4(w, q8)
    qd, dd = dev_r4(q, d)
    y = to_np(ops.matmul_r4(to_dev(x), qd, dd, O, q8))
    assert same_bits(y, o_matmul_r4(x, q, d, O, q8))


@pytest.mark.parametrize("q8", [False, True])
def test_matmul_r4_device_packed(ops, q8):
    # weights packed on the device feed the matmul directly
    O, I, S = 96, 2048, 9
    w = randn(3, (O, I)) * 0.02
    x = randn(4, (S, I))
    qd, dd = ops.pack_r4(to_dev(w), q8)
    y = to_np(ops.matmul_r4(to_dev(x), qd, dd, O, q8))
    q, d = o_pack_r4(w, q8)
    assert same_bits(y, o_matmul_r4(x, q, d, O, q8))


@pytest.mark.parametrize("q8", [False, True])
def test_matmul_r4_host_dropin(ops, q8):
    # moty_hip_matmul_q4r4_s / q8r4_s on host pointers, weights cached by pointer
    import moty_amd
    lib = moty_amd.lib()
    O, I = 52, 320
    w = randn(9, (O, I)) * 0.02
    q, d = o_pack_r4(w, q8)
    fn = lib.moty_hip_matmul_q8r4_s if q8 else lib.moty_hip_matmul_q4r4_s
    for S in (1, 5, 11):
        x = randn(10 + S, (S, I))
        y = np.empty((S, O), np.float32)
        rc = fn(C.c_void_p(y.ctypes.data), C.c_void_p(x.ctypes.data), C.c_void_p(q.ctypes.data),
                C.c_void_p(d.ctypes.data), S, I, O)
        assert rc == 0, lib.moty_hip_last_error()
        assert same_bits(y, o_matmul_r4(x, q, d, O, q8))
    # both arrays are cached by address: a later array at the same address
    # must not find these
    assert lib.moty_hip_weight_forget(C.c_void_p(q.ctypes.data)) == 0
    assert lib.moty_hip_weight_forget(C.c_void_p(d.ctypes.data)) == 0


def o_silu(g, u):
    from cpu_libs import oracle, ptr
    g = np.ascontiguousarray(g, np.float32).copy()
    u = np.ascontiguousarray(u, np.float32)  # held: ptr() does not keep a temporary alive
    oracle().o_silu_mul(ptr(g), ptr(u), g.size)
    return g


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("D,I", [(1024, 3072), (4096, 1024), (96, 40), (2048, 5632), (8192, 256)])
def test_gate_up_silu_r4(ops, q8, D, I):
    # one pass over the row-fused [gate; up] matrix (moty_mat_fuse_rows)
    # (Q8R4 at D = 8192: past the fused GEMV's register budget, the entry
    # point takes the plain R4 GEMV over all 2I rows then SiLU -- same bits)
    say("gate_up_silu_r4", q8, D, I)
    gu = randn(D + I, (2 * I, D)) * 0.02
    x = randn(D + 1, (1, D))
    q, d = o_pack_r4(gu, q8)
    qd, dd = dev_r4(q, d)
    h = to_np(ops.gate_up_silu_r4(to_dev(x), qd, dd, I, q8))
    y = o_matmul_r4(x, q, d, 2 * I, q8)
    h2 = o_silu(y[:, :I], y[:, I:])
    assert same_bits(h, h2), mismatch(h, h2)


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("S,D,I", [(1, 1024, 3072), (2, 256, 512), (5, 512, 256), (33, 256, 1024), (1, 4096, 1024),
                                   (68, 256, 1056), (7, 512, 160), (3, 256, 96), (1, 8192, 256)])
def test_dense_ffn_r4(ops, q8, S, D, I):
    # moty_nn_dense_ffn with the fused gate_up (nn/ffn.c:26-41)
    say("dense_ffn_r4", q8, S, D, I)
    gu = randn(S + D, (2 * I, D)) * 0.02
    dn = randn(S + I, (D, I)) * 0.02
    x = randn(S + 7, (S, D))
    q, d = o_pack_r4(gu, q8)
    q2, d2 = o_pack_r4(dn, q8)
    qd, dd = dev_r4(q, d)
    q2d, d2d = dev_r4(q2, d2)
    out = to_np(ops.dense_ffn_r4(to_dev(x), qd, dd, q2d, d2d, I, q8))
    y = o_matmul_r4(x, q, d, 2 * I, q8)
    h = o_silu(y[:, :I], y[:, I:])
    ref = o_matmul_r4(h, q2, d2, D, q8)
    assert same_bits(out, ref), mismatch(out, ref)
