"""GPU parity at BASELINE.json's workload sizes, on the exact call chains
bench.py times: every output row, routing and count against the oracle,
bit-exact.  Launch-shape choices (MoE M-tile size, GEMV variant, GEMM
tiling, KS split) switch at exactly these sizes, so the small-shape tests
elsewhere do not cover them.

Workloads:
  C2  Qwen3-0.6B projections at M = 512: qrow_i8 once per input, then the
      pre-quantized Q8 GEMM (q/k/v/gate/up row-fused N = 10240, o, down)
  C3  8B-dense FFN, D = 4096, I = 12288, M = 1 and M = 256, grouped int4
      (IDOT4) and Q4R4
  C4  OLMoE MoE layer, T = 256, E = 64, top-8, olmoe order, norm 0: all rows
  C5  Qwen3-30B-A3B MoE layer, T = 1072, E = 128, top-8, batch order,
      uniform and skewed (+2.0 logit bias on 8 hot experts): all rows
  d1  moty_nn_moe_topk_d1 (nn/moe.c:33-153): S = 1, top-k order, norm 1

Weights are drawn directly as codes and scales (cpu_libs.fast_q8): the
quantizers are tested on their own elsewhere, and workload-sized stacks
then take seconds to make."""
import ctypes as C

import numpy as np
import pytest
import torch

from cpu_libs import (f32, fast_moe_weights, fast_q8, o_matmul_i4g, o_matmul_q_s, o_matmul_r4, o_moe, oracle,
                      ptr, r4_sizes, randn, rng)
from gpu_util import mismatch, same_bits, say, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(dev):
    import moty_amd
    moty_amd.lib()
    from moty_amd import ops
    return ops


def o_silu(g, u):
    g = f32(g).copy()
    u = f32(u)
    oracle().o_silu_mul(ptr(g), ptr(u), g.size)
    return g


def moe_layer(ops, Wr, ex, K, norm, order, bias=None):
    from moty_amd.ops import MoeLayer
    d = {k: to_dev(v) for k, v in ex.items()}
    return MoeLayer(to_dev(Wr), d["G"], d["GS"], d["U"], d["US"], d["Dn"], d["DS"], K, norm_topk=norm, order=order,
                    logit_bias=None if bias is None else to_dev(bias))


def check_moe(ops, L, x, Wr, ex, K, order, norm, bias=None):
    E = Wr.shape[0]
    y, idx, w, cnt = L(to_dev(x), want_routing=True)
    y2, idx2, w2 = o_moe(x, Wr, ex, K, order, norm=norm, bias=bias)
    assert (to_np(idx) == idx2).all(), "routing ids differ"
    assert same_bits(to_np(w), w2), "routing weights differ"
    c = to_np(cnt)
    assert (c == np.bincount(idx2.ravel(), minlength=E)).all(), "expert counts differ"
    assert same_bits(to_np(y), y2), mismatch(to_np(y), y2)
    return c


# ---------------- C4 / C5 MoE layers ----------------
def test_c4_olmoe_all_rows(ops):
    E, K, I, D, T = 64, 8, 1024, 2048, 256
    say("C4", E, K, I, D, T)
    from moty_amd import ORDER_TOPK
    ex = fast_moe_weights(E, I, D, seed=40)
    Wr = randn(41, (E, D), 0.02)
    x = randn(42, (T, D))
    L = moe_layer(ops, Wr, ex, K, 0, ORDER_TOPK)
    check_moe(ops, L, x, Wr, ex, K, "olmoe", 0)


@pytest.mark.parametrize("skewed", [False, True])
def test_c5_batch_all_rows(ops, skewed):
    E, K, I, D, T = 128, 8, 768, 2048, 1072
    say("C5", "skewed" if skewed else "uniform", E, K, I, D, T)
    from moty_amd import ORDER_EXPERT
    ex = fast_moe_weights(E, I, D, seed=50)
    Wr = randn(51, (E, D), 0.02)
    x = randn(52, (T, D))
    bias = None
    hot = np.arange(0, 128, 16)
    if skewed:
        bias = np.zeros(E, np.float32)
        bias[hot] = 2.0
    L = moe_layer(ops, Wr, ex, K, 1, ORDER_EXPERT, bias)
    c = check_moe(ops, L, x, Wr, ex, K, "batch", 1, bias)
    if skewed:  # the hot experts take most pairs: 128-slot tiles, several per expert
        assert c[hot].sum() > 0.5 * c.sum() and c.max() > 256


@pytest.mark.parametrize("E,K,I,D", [(64, 8, 1024, 2048), (128, 8, 768, 2048), (16, 4, 128, 256), (8, 8, 64, 96)])
def test_moe_d1(ops, E, K, I, D):
    # S = 1, top-k combine order, routing normalised: moty_nn_moe_topk_d1
    say("d1", E, K, I, D)
    from moty_amd import ORDER_TOPK
    ex = fast_moe_weights(E, I, D, seed=60 + E)
    Wr = randn(61, (E, D), 0.02)
    L = moe_layer(ops, Wr, ex, K, 1, ORDER_TOPK)
    for seed in (62, 63):
        check_moe(ops, L, randn(seed, (1, D)), Wr, ex, K, "olmoe", 1)


# ---------------- C2 prefill projections ----------------
@pytest.mark.parametrize("I,O", [(1024, 10240), (2048, 1024), (3072, 1024)])
def test_c2_preq_chain(ops, I, O):
    # bench.py's C2 step: moty_hip_qrow_i8_dev once per input, then
    # moty_hip_matmul_q8_preq_dev; the pair equals matmul_q_s
    M = 512
    say("C2", M, I, O)
    q, s = fast_q8(70 + I, (O, I))
    x = randn(71 + I, (M, I))
    xq, sx, _ = ops.qrow_i8(to_dev(x))
    y = to_np(ops.matmul_q8_preq(xq, sx, to_dev(q), to_dev(s)))
    y2 = o_matmul_q_s(x, q, s)
    assert same_bits(y, y2), mismatch(y, y2)


# ---------------- C3 8B-dense FFN, grouped int4 ----------------
def fast_q4(seed, O, I):
    g = rng(seed)
    q4 = np.frombuffer(g.bytes(O * I // 2), np.uint8).reshape(O, I // 2).copy()
    s = g.uniform(1e-3, 3e-3, (O, I // 32)).astype(np.float32)
    return q4, s


@pytest.fixture(scope="module")
def c3_weights():
    D, I = 4096, 12288
    return D, I, fast_q4(80, I, D), fast_q4(81, I, D), fast_q4(82, D, I)


def test_c3_i4g_decode(ops, c3_weights):
    # M = 1: fused gate/up + SiLU GEMV, then the down GEMV (bench.py C3 M1)
    D, I, (gq, gs), (uq, us), (dq, ds) = c3_weights
    say("C3 i4g M=1")
    x = randn(83, (1, D))
    h = ops.gate_up_silu_i4g(to_dev(x), to_dev(gq), to_dev(gs), to_dev(uq), to_dev(us))
    y = to_np(ops.matmul_i4_grouped_s(h, to_dev(dq), to_dev(ds), 32, True))
    h2 = o_silu(o_matmul_i4g(x, gq, gs, True), o_matmul_i4g(x, uq, us, True))
    assert same_bits(to_np(h), h2), mismatch(to_np(h), h2)
    y2 = o_matmul_i4g(h2, dq, ds, True)
    assert same_bits(y, y2), mismatch(y, y2)


def test_c3_i4g_prefill(ops, c3_weights):
    # M = 256: gate GEMM, up GEMM, silu_mul, down GEMM (bench.py C3 M256)
    D, I, (gq, gs), (uq, us), (dq, ds) = c3_weights
    M = 256
    say("C3 i4g M=256")
    x = randn(84, (M, D))
    xd = to_dev(x)
    g = ops.matmul_i4_grouped_s(xd, to_dev(gq), to_dev(gs), 32, True)
    u = ops.matmul_i4_grouped_s(xd, to_dev(uq), to_dev(us), 32, True)
    g2 = o_matmul_i4g(x, gq, gs, True)
    u2 = o_matmul_i4g(x, uq, us, True)
    assert same_bits(to_np(g), g2), mismatch(to_np(g), g2)
    assert same_bits(to_np(u), u2), mismatch(to_np(u), u2)
    ops.silu_mul(g, u)
    h2 = o_silu(g2, u2)
    assert same_bits(to_np(g), h2)
    y = to_np(ops.matmul_i4_grouped_s(g, to_dev(dq), to_dev(ds), 32, True))
    y2 = o_matmul_i4g(h2, dq, ds, True)
    assert same_bits(y, y2), mismatch(y, y2)


@pytest.mark.parametrize("M", [1, 256])
def test_c3_i4g_exact_f32_ffn(ops, c3_weights, M):
    # the reference's default grouped-int4 path (IDOT4 unset: f32
    # activations, nn/matmul.c:199-253) through the FFN entry bench.py times
    # (moty_hip_dense_ffn_i4g_dev, idot4 = 0) at the full C3 shapes.  Every
    # output row depends only on its own input row, so at M = 256 the oracle
    # (scalar C) checks a spread of rows of the full-size run.
    D, I, (gq, gs), (uq, us), (dq, ds) = c3_weights
    say("C3 i4g exact f32 M=%d" % M)
    x = randn(85 + M, (M, D))
    out = to_np(ops.dense_ffn_i4g(to_dev(x), to_dev(gq), to_dev(gs), to_dev(uq), to_dev(us), to_dev(dq),
                                  to_dev(ds), idot4=False))
    rows = [0] if M == 1 else [0, 1, 37, 128, 200, 255]
    xs = x[rows]
    h2 = o_silu(o_matmul_i4g(xs, gq, gs, False), o_matmul_i4g(xs, uq, us, False))
    y2 = o_matmul_i4g(h2, dq, ds, False)
    assert same_bits(out[rows], y2), mismatch(out[rows], y2)


# ---------------- C3 shapes in Q4R4 ----------------
def fast_r4(seed, O, I):
    g = rng(seed)
    nq, nd = r4_sizes(O, I, False)
    q = np.frombuffer(g.bytes(nq), np.uint8).copy()
    d = g.uniform(1e-3, 3e-3, nd).astype(np.float16).view(np.uint16).copy()
    return q, d


@pytest.fixture(scope="module")
def c3_r4_weights():
    D, I = 4096, 12288
    return D, I, fast_r4(90, 2 * I, D), fast_r4(91, D, I)


@pytest.mark.parametrize("M", [1, 256])
def test_c3_r4_ffn(ops, c3_r4_weights, M):
    # moty_hip_dense_ffn_q4r4_dev over the row-fused gate_up (bench.py C3 Q4R4)
    D, I, (q, d), (q2, d2) = c3_r4_weights
    say("C3 q4r4 ffn M=%d" % M)
    x = randn(92 + M, (M, D))
    dv = lambda a: to_dev(a.view(np.int16) if a.dtype == np.uint16 else a)
    out = to_np(ops.dense_ffn_r4(to_dev(x), dv(q), dv(d), dv(q2), dv(d2), I))
    y = o_matmul_r4(x, q, d, 2 * I)
    h = o_silu(y[:, :I], y[:, I:])
    ref = o_matmul_r4(h, q2, d2, D)
    assert same_bits(out, ref), mismatch(out, ref)


@pytest.mark.parametrize("M", [256, 1])
def test_c3_i4g_dense_ffn(ops, c3_weights, M):
    # moty_hip_dense_ffn_i4g_dev (bench.py C3): gate and up in one pass with
    # the SiLU epilogue, then down
    D, I, (gq, gs), (uq, us), (dq, ds) = c3_weights
    say("C3 i4g dense ffn M=%d" % M)
    x = randn(85 + M, (M, D))
    y = to_np(ops.dense_ffn_i4g(to_dev(x), to_dev(gq), to_dev(gs), to_dev(uq), to_dev(us), to_dev(dq), to_dev(ds)))
    h = o_silu(o_matmul_i4g(x, gq, gs, True), o_matmul_i4g(x, uq, us, True))
    y2 = o_matmul_i4g(h, dq, ds, True)
    assert same_bits(y, y2), mismatch(y, y2)


def test_moe_refuses_unaligned(ops):
    # the MoE kernels move x, out, the router and the expert rows in 16-byte
    # units: a 4-byte-aligned activation view is refused, never read
    import moty_amd
    E, K, I, D = 8, 2, 64, 96
    say("moe unaligned")
    ex = fast_moe_weights(E, I, D, seed=90)
    Wr = randn(91, (E, D), 0.02)
    L = moe_layer(ops, Wr, ex, K, 1, moty_amd.ORDER_EXPERT)
    buf = torch.zeros(2 * D + 1, dtype=torch.float32, device="cuda")
    xv = buf[1:].view(2, D)
    xv.copy_(to_dev(randn(92, (2, D))))
    with pytest.raises(moty_amd.MotyHipError, match="16-byte aligned"):
        L(xv)
