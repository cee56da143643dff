"""GPU: the host-pointer drop-ins (the entry points the reference's own
callers would bind: moty_matmul_q_s, moty_matmul_i4_grouped_s, moty_matmul,
the HwBackend matmul_i8 slot, the MoE layer) bit for bit against the oracle,
through the C-ABI, and the weight cache behind them: keyed by host address,
re-uploaded when a different buffer takes a freed address or after
moty_hip_weight_forget."""
import ctypes as C

import numpy as np
import pytest

from cpu_libs import o_matmul_f32, o_matmul_i4g, o_matmul_q_s, o_moe, o_pack_int4_grouped, o_quantize_rows, randn
from gpu_util import mismatch, same_bits, say

pytestmark = pytest.mark.gpu


def P(a):
    return C.c_void_p(a.ctypes.data)


@pytest.fixture(scope="module")
def lib(dev):
    import moty_amd
    return moty_amd.lib()


def forget(lib, *arrays):
    for a in arrays:
        assert lib.moty_hip_weight_forget(P(a)) == 0


@pytest.mark.parametrize("S,I,O", [(1, 1024, 3072), (5, 96, 40), (33, 256, 130), (1, 4096, 1000), (70, 128, 33)])
def test_matmul_q_s_host(lib, S, I, O):
    say("dropin q_s", S, I, O)
    q, s = o_quantize_rows(randn(1 + I, (O, I), 0.02))
    x = randn(2 + S, (S, I))
    y = np.empty((S, O), np.float32)
    try:
        assert lib.moty_hip_matmul_q_s(P(y), P(x), P(q), P(s), S, I, O) == 0, lib.moty_hip_last_error()
        y2 = o_matmul_q_s(x, q, s)
        assert same_bits(y, y2), mismatch(y, y2)
        # the HwBackend slot returns nothing and fills y the same way
        y3 = np.full((S, O), np.nan, np.float32)
        lib.moty_hip_hw_matmul_i8(P(y3), P(x), P(q), P(s), S, I, O)
        assert same_bits(y3, y2)
    finally:
        forget(lib, q, s)


@pytest.fixture(scope="module")
def idot4_env(lib):
    """The library reads IDOT4 from the process environment at its first
    host-pointer grouped-int4 call (as nn/matmul.c:171 does).  The C
    environment, not os.environ, is what it sees -- the compiled reference's
    ref_init sets IDOT4 with setenv when test modules are collected -- so
    read it there and make that first call now, latching the same value."""
    libc = C.CDLL(None)
    libc.getenv.restype, libc.getenv.argtypes = C.c_char_p, [C.c_char_p]
    libc.atoi.restype, libc.atoi.argtypes = C.c_int, [C.c_char_p]
    v = libc.getenv(b"IDOT4")
    on = v is not None and libc.atoi(v) != 0
    x = np.zeros((1, 64), np.float32)
    q4 = np.zeros((1, 32), np.uint8)
    s = np.ones((1, 2), np.float32)
    y = np.empty((1, 1), np.float32)
    try:
        assert lib.moty_hip_matmul_i4_grouped_s(P(y), P(x), P(q4), P(s), 1, 64, 1, 32) == 0
    finally:
        forget(lib, q4, s)
    return on


@pytest.mark.parametrize("S,I,O", [(1, 1024, 512), (3, 256, 70), (17, 2048, 96), (1, 4096, 64)])
def test_matmul_i4_grouped_s_host(lib, idot4_env, S, I, O):
    idot4 = idot4_env and I % 64 == 0 and I <= 16384
    say("dropin i4g", S, I, O, idot4)
    q4, s = o_pack_int4_grouped(randn(3 + I, (O, I), 0.02), 32)
    x = randn(4 + S, (S, I))
    y = np.empty((S, O), np.float32)
    try:
        assert lib.moty_hip_matmul_i4_grouped_s(P(y), P(x), P(q4), P(s), S, I, O, 32) == 0, lib.moty_hip_last_error()
        y2 = o_matmul_i4g(x, q4, s, idot4)
        assert same_bits(y, y2), mismatch(y, y2)
    finally:
        forget(lib, q4, s)


@pytest.mark.parametrize("S,I,O", [(1, 2048, 64), (9, 256, 128), (40, 96, 8)])
def test_matmul_f32_host(lib, S, I, O):
    say("dropin f32", S, I, O)
    W = randn(5 + I, (O, I), 0.02)
    x = randn(6 + S, (S, I))
    y = np.empty((S, O), np.float32)
    try:
        assert lib.moty_hip_matmul(P(y), P(x), P(W), S, I, O) == 0, lib.moty_hip_last_error()
        y2 = o_matmul_f32(x, W)
        assert same_bits(y, y2), mismatch(y, y2)
    finally:
        forget(lib, W)


@pytest.mark.parametrize("order", ["batch", "olmoe"])
@pytest.mark.parametrize("E,K,I,D,S", [(16, 4, 64, 128, 24), (8, 2, 96, 64, 1), (32, 8, 128, 256, 70)])
def test_moe_topk_host(lib, order, E, K, I, D, S):
    from moty_amd import MotyHipMoe, ORDER_EXPERT, ORDER_TOPK
    say("dropin moe", order, E, K, I, D, S)
    ex = {}
    for key, sk, shape, seed in (("G", "GS", (E, I, D), 7), ("U", "US", (E, I, D), 8), ("Dn", "DS", (E, D, I), 9)):
        q, s = o_quantize_rows(randn(seed, shape, 0.02).reshape(-1, shape[-1]))
        ex[key], ex[sk] = q.reshape(shape), s.reshape(shape[:-1])
    Wr = randn(10, (E, D), 0.02)
    bias = randn(11, (E,), 0.01)
    x = randn(12, (S, D))
    norm = 1 if order == "batch" else 0
    m = MotyHipMoe()
    m.router, m.logit_bias = P(Wr), P(bias)
    m.g, m.u, m.d = P(ex["G"]), P(ex["U"]), P(ex["Dn"])
    m.gs, m.us, m.ds = P(ex["GS"]), P(ex["US"]), P(ex["DS"])
    m.E, m.K, m.I, m.D = E, K, I, D
    m.norm_topk = norm
    m.combine_order = ORDER_EXPERT if order == "batch" else ORDER_TOPK
    idx = np.empty((S, K), np.int32)
    w = np.empty((S, K), np.float32)
    cnt = np.empty(E, np.int32)
    m.idx_out, m.w_out, m.counts_out = P(idx), P(w), P(cnt)
    y = np.empty((S, D), np.float32)
    try:
        assert lib.moty_hip_moe_topk(C.byref(m), P(x), S, P(y)) == 0, lib.moty_hip_last_error()
        y2, idx2, w2 = o_moe(x, Wr, ex, K, order, norm=norm, bias=bias)
        assert (idx == idx2).all()
        assert same_bits(w, w2)
        assert (cnt == np.bincount(idx2.ravel(), minlength=E)).all()
        assert same_bits(y, y2), mismatch(y, y2)
    finally:
        forget(lib, Wr, bias, *ex.values())


def test_weight_cache_address_reuse(lib):
    # a buffer rewritten at a cached address (what a freed and reallocated
    # weight looks like) is uploaded afresh; weight_forget drops the copy
    S, I, O = 3, 256, 48
    x = randn(20, (S, I))
    q, s = o_quantize_rows(randn(21, (O, I), 0.02))
    qb, sb = q.copy(), s.copy()
    y = np.empty((S, O), np.float32)
    try:
        assert lib.moty_hip_matmul_q_s(P(y), P(x), P(qb), P(sb), S, I, O) == 0
        assert same_bits(y, o_matmul_q_s(x, q, s))
        q2, s2 = o_quantize_rows(randn(22, (O, I), 0.02))
        qb[...] = q2  # whole new content at the same addresses
        sb[...] = s2
        assert lib.moty_hip_matmul_q_s(P(y), P(x), P(qb), P(sb), S, I, O) == 0
        assert same_bits(y, o_matmul_q_s(x, q2, s2))
        forget(lib, qb, sb)
        qb[O // 2, I // 2] ^= 1  # a one-byte rewrite, announced by the forget above
        assert lib.moty_hip_matmul_q_s(P(y), P(x), P(qb), P(sb), S, I, O) == 0
        assert same_bits(y, o_matmul_q_s(x, qb, sb))
    finally:
        forget(lib, qb, sb)


def test_dropin_bad_arguments(lib):
    y = np.empty(4, np.float32)
    x = np.empty(4, np.float32)
    q = np.empty(4, np.int8)
    s = np.empty(1, np.float32)
    assert lib.moty_hip_matmul_q_s(P(y), P(x), P(q), P(s), -1, 4, 1) != 0
    assert lib.moty_hip_matmul_q_s(None, P(x), P(q), P(s), 1, 4, 1) != 0
    assert lib.moty_hip_matmul(P(y), P(x), None, 1, 4, 1) != 0
    assert lib.moty_hip_matmul_i4_grouped_s(P(y), P(x), P(q), P(s), 1, 4, 1, 0) != 0
    # empty problems succeed without touching anything
    assert lib.moty_hip_matmul_q_s(P(y), P(x), P(q), P(s), 0, 4, 1) == 0
    assert lib.moty_hip_matmul_q_s(P(y), P(x), P(q), P(s), 1, 4, 0) == 0


def test_hw_slot_failure_poisons_y_and_errors_clear(lib):
    # the void HwBackend.matmul_i8 slot cannot return a code: an unsupported
    # shape (I % 16 != 0) leaves every y a NaN and a message; the next call
    # that succeeds clears the message
    S, I, O = 2, 40, 8
    q, s = o_quantize_rows(randn(30, (O, I), 0.02))
    x = randn(31, (S, I))
    y = np.zeros((S, O), np.float32)
    try:
        lib.moty_hip_hw_matmul_i8(P(y), P(x), P(q), P(s), S, I, O)
        assert np.isnan(y).all()
        assert lib.moty_hip_last_error()
        I2 = 64
        q2, s2 = o_quantize_rows(randn(32, (O, I2), 0.02))
        x2 = randn(33, (S, I2))
        y2 = np.empty((S, O), np.float32)
        lib.moty_hip_hw_matmul_i8(P(y2), P(x2), P(q2), P(s2), S, I2, O)
        assert lib.moty_hip_last_error() == b""
        assert same_bits(y2, o_matmul_q_s(x2, q2, s2))
    finally:
        forget(lib, q, s)


def test_scratch_shared_across_streams(lib):
    # sequential _dev calls on two streams share the device scratch: the
    # second call is ordered behind the first (a long GEMM on stream A, then
    # a different GEMM on stream B that reuses the same activation scratch)
    import torch
    from moty_amd import ops
    from gpu_util import to_dev, to_np
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    S, I, O = 512, 4096, 8192
    q, s = o_quantize_rows(randn(40, (O, I), 0.02))
    x1 = randn(41, (S, I))
    x2 = randn(42, (S, I)) * 3
    qd, sd, x1d, x2d = to_dev(q), to_dev(s), to_dev(x1), to_dev(x2)
    r1, r2 = o_matmul_q_s(x1, q, s), o_matmul_q_s(x2, q, s)
    torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(a):
            y1 = ops.matmul_q_s(x1d, qd, sd)
        with torch.cuda.stream(b):
            y2 = ops.matmul_q_s(x2d, qd, sd)
        torch.cuda.synchronize()
        assert same_bits(to_np(y1), r1)
        assert same_bits(to_np(y2), r2)


def test_hw_matmul_i4_slot(lib, idot4_env):
    # HwBackend.matmul_i4 (hw/hw_backend.h:59-60): moty_matmul_i4_s with the
    # process's IDOT4, through the host-pointer path; an unsupported width
    # (I % 16 != 0) leaves NaNs and a message
    from cpu_libs import o_matmul_i4, o_pack_int4
    S, I, O = 3, 256, 40
    q4, s = o_pack_int4(randn(50, (O, I), 0.02))
    x = randn(51, (S, I))
    y = np.full((S, O), np.nan, np.float32)
    try:
        assert lib.moty_hip_matmul_i4_s(P(y), P(x), P(q4), P(s), S, I, O) == 0, lib.moty_hip_last_error()
        y2 = o_matmul_i4(x, q4, s, bool(idot4_env))
        assert same_bits(y, y2), mismatch(y, y2)
        y3 = np.zeros((S, O), np.float32)
        lib.moty_hip_hw_matmul_i4(P(y3), P(x), P(q4), P(s), S, I, O)
        assert same_bits(y3, y2)
        q5, s5 = o_pack_int4(randn(52, (O, 40), 0.02))
        y4 = np.zeros((S, O), np.float32)
        lib.moty_hip_hw_matmul_i4(P(y4), P(randn(53, (S, 40))), P(q5), P(s5), S, 40, O)
        assert np.isnan(y4).all() and lib.moty_hip_last_error()
    finally:
        forget(lib, q4, s)
