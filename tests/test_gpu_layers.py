"""GPU parity for the layer-level paths: the dense Q8 SwiGLU FFN and the MoE
layer (router, grouping, grouped GEMMs, combine) against the oracle."""
import numpy as np
import pytest
import torch

from cpu_libs import o_dense_ffn_q8, o_moe, o_quantize_rows, o_route, randn
from gpu_util import mismatch, same_bits, say, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(dev):
    from moty_amd import ops
    return ops


def q8(seed, shape):
    w = randn(seed, shape, 0.02)
    q, s = o_quantize_rows(w.reshape(-1, shape[-1]))
    return q.reshape(shape), s.reshape(shape[:-1])


@pytest.mark.parametrize("S,D,I", [(1, 1024, 3072), (4, 1024, 3072), (9, 256, 512), (1, 64, 32), (1, 2048, 6144),
                                   (1, 4096, 2048), (1, 3088, 2800),
                                   (1, 4096, 1024), (1, 1040, 2000), (1, 4096, 4096)])
def test_dense_ffn_q8(ops, S, D, I):
    say("dense_ffn", S, D, I)
    G, GS = q8(1, (I, D))
    U, US = q8(2, (I, D))
    Dn, DS = q8(3, (D, I))
    x = randn(4, (S, D))
    y = to_np(ops.dense_ffn_q8(to_dev(x), to_dev(G), to_dev(GS), to_dev(U), to_dev(US), to_dev(Dn), to_dev(DS)))
    y2 = o_dense_ffn_q8(x, G, GS, U, US, Dn, DS)
    assert same_bits(y, y2), mismatch(y, y2)


def test_dense_ffn_decode_repeated_and_graph(ops):
    # many back-to-back launches, eager and replayed from a HIP graph (with
    # eager work between replays), all give the oracle's bits
    say("ffn repeated")
    D, I = 1024, 3072
    G, GS = q8(1, (I, D))
    U, US = q8(2, (I, D))
    Dn, DS = q8(3, (D, I))
    xs = [randn(40 + k, (1, D)) for k in range(4)]
    ref = [o_dense_ffn_q8(x, G, GS, U, US, Dn, DS) for x in xs]
    w = [to_dev(a) for a in (G, GS, U, US, Dn, DS)]
    xd = [to_dev(x) for x in xs]
    outs = [torch.empty((1, D), device="cuda:0") for _ in xs]
    for _ in range(25):
        for x, o in zip(xd, outs):
            ops.dense_ffn_q8(x, *w, out=o)
    for o, r in zip(outs, ref):
        assert same_bits(to_np(o), r)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g):
            for x, o in zip(xd, outs):
                ops.dense_ffn_q8(x, *w, out=o)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(5):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert same_bits(to_np(o), r), "replay %d" % rep


@pytest.mark.parametrize("D,I", [(1024, 3072), (1024, 1024), (2048, 4096), (2048, 2048), (1024, 4096)])
def test_dense_ffn_q8_one_launch(ops, D, I):
    # the one-launch decode FFN (workgroups exchanging h through device
    # memory) against the oracle: several calls in a row on rotating inputs
    # (the per-workgroup call counters advance), then graph replays with
    # eager calls between them; no bounded wait may run out
    say("ffn one-launch", D, I)
    G, GS = q8(11, (I, D))
    U, US = q8(12, (I, D))
    Dn, DS = q8(13, (D, I))
    xs = [randn(50 + k, (1, D)) * (k + 1) for k in range(3)]
    xs.append(np.zeros((1, D), np.float32))  # all-zero h: the 1e-12 scale floor
    ref = [o_dense_ffn_q8(x, G, GS, U, US, Dn, DS) for x in xs]
    w = [to_dev(a) for a in (G, GS, U, US, Dn, DS)]
    xd = [to_dev(x) for x in xs]
    outs = [torch.empty((1, D), device="cuda:0") for _ in xs]
    ops.set_ffn1(1)
    try:
        assert ops.wait_errors() == 0
        for _ in range(6):
            for x, o in zip(xd, outs):
                ops.dense_ffn_q8(x, *w, out=o)
        for o, r in zip(outs, ref):
            assert same_bits(to_np(o), r), mismatch(to_np(o), r)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g):
                for x, o in zip(xd, outs):
                    ops.dense_ffn_q8(x, *w, out=o)
        torch.cuda.current_stream().wait_stream(s)
        for rep in range(4):
            for o in outs:
                o.zero_()
            g.replay()
            ops.dense_ffn_q8(xd[0], *w, out=outs[0])
            torch.cuda.synchronize()
            for o, r in zip(outs, ref):
                assert same_bits(to_np(o), r), "replay %d" % rep
        assert ops.wait_errors() == 0
    finally:
        ops.set_ffn1(0)


def moe_weights(E, I, D, seed=10):
    G, GS = q8(seed, (E, I, D))
    U, US = q8(seed + 1, (E, I, D))
    Dn, DS = q8(seed + 2, (E, D, I))
    return dict(G=G, GS=GS, U=U, US=US, Dn=Dn, DS=DS)


def layer(ops, Wr, ex, K, norm, order, bias=None):
    from moty_amd.ops import MoeLayer
    d = {k: to_dev(v) for k, v in ex.items()}
    return MoeLayer(to_dev(Wr), d["G"], d["GS"], d["U"], d["US"], d["Dn"], d["DS"], K, norm_topk=norm, order=order,
                    logit_bias=None if bias is None else to_dev(bias))


@pytest.mark.parametrize("E,K,I,D,S", [(16, 4, 128, 256, 24), (8, 2, 64, 64, 1), (64, 8, 1024, 2048, 32),
                                       (128, 8, 768, 2048, 20), (5, 5, 32, 32, 7), (8, 2, 64, 128, 300),
                                       (6, 2, 96, 160, 50), (16, 4, 96, 128, 400), (32, 8, 64, 96, 257)])
@pytest.mark.parametrize("order", ["batch", "olmoe"])
def test_moe_layer(ops, E, K, I, D, S, order):
    say("moe", E, K, I, D, S, order)
    Wr = randn(1, (E, D), 0.02)
    x = randn(2, (S, D))
    ex = moe_weights(E, I, D)
    norm = 1 if order == "batch" else 0
    from moty_amd import ORDER_EXPERT, ORDER_TOPK
    L = layer(ops, Wr, ex, K, norm, ORDER_EXPERT if order == "batch" else ORDER_TOPK)
    y, idx, w, cnt = L(to_dev(x), want_routing=True)
    y2, idx2, w2 = o_moe(x, Wr, ex, K, order, norm=norm)
    assert (to_np(idx) == idx2).all()
    assert same_bits(to_np(w), w2)
    assert (to_np(cnt) == np.bincount(idx2.ravel(), minlength=E)).all()
    assert same_bits(to_np(y), y2), mismatch(to_np(y), y2)


@pytest.mark.parametrize("order", ["batch", "olmoe"])
def test_moe_routing_ties(ops, order):
    # duplicated router rows give exactly equal logits and probabilities:
    # the greedy top-k must take the lower expert id first (strict '>')
    E, K, I, D, S = 16, 5, 32, 64, 33
    Wr = randn(7, (E // 2, D), 0.02)
    Wr = np.repeat(Wr, 2, axis=0)
    x = randn(8, (S, D))
    ex = moe_weights(E, I, D, seed=30)
    from moty_amd import ORDER_EXPERT, ORDER_TOPK
    norm = 1 if order == "batch" else 0
    L = layer(ops, Wr, ex, K, norm, ORDER_EXPERT if order == "batch" else ORDER_TOPK)
    y, idx, w, cnt = L(to_dev(x), want_routing=True)
    y2, idx2, w2 = o_moe(x, Wr, ex, K, order, norm=norm)
    assert (to_np(idx) == idx2).all() and same_bits(to_np(w), w2)
    assert same_bits(to_np(y), y2)


@pytest.mark.parametrize("E,K,D,S", [(40, 6, 96, 9), (100, 8, 160, 33), (200, 8, 96, 17), (256, 16, 4160, 5),
                                     (72, 64, 128, 3), (129, 8, 64, 1), (64, 8, 128, 1030), (16, 4, 96, 1025),
                                     (32, 4, 16384, 3)])
def test_moe_routing_expert_counts(ops, E, K, D, S):
    # expert counts off the router's tiles (8 / 32 experts per workgroup),
    # the 256-expert configuration, rows past the register-held int8-row path
    # (D > 4096, up to 16384), K = 64, and few experts past 1024 tokens (the
    # large tile)
    say("moe routing", E, K, D, S)
    Wr = randn(11, (E, D), 0.02)
    x = randn(12, (S, D))
    ex = moe_weights(E, 32, D, seed=13)
    from moty_amd import ORDER_EXPERT
    L = layer(ops, Wr, ex, K, 1, ORDER_EXPERT)
    y, idx, w, cnt = L(to_dev(x), want_routing=True)
    y2, idx2, w2 = o_moe(x, Wr, ex, K, "batch", norm=1)
    assert (to_np(idx) == idx2).all()
    assert same_bits(to_np(w), w2)
    assert same_bits(to_np(y), y2), mismatch(to_np(y), y2)


@pytest.mark.parametrize("S", [40, 400])
def test_moe_skewed_bias(ops, S):
    # +2.0 on 8 hot experts' logits (the skewed continuous-batch variant);
    # S = 400 takes 128-slot M-tiles, hot experts spanning several
    E, K, I, D = 32, 4, 64, 128
    Wr = randn(5, (E, D), 0.02)
    x = randn(6, (S, D))
    ex = moe_weights(E, I, D, seed=20)
    bias = np.zeros(E, np.float32)
    bias[[1, 3, 5, 7, 11, 13, 17, 19]] = 2.0
    from moty_amd import ORDER_EXPERT
    L = layer(ops, Wr, ex, K, 1, ORDER_EXPERT, bias)
    y, idx, w, cnt = L(to_dev(x), want_routing=True)
    y2, idx2, w2 = o_moe(x, Wr, ex, K, "batch", bias=bias)
    assert (to_np(idx) == idx2).all()
    assert same_bits(to_np(y), y2), mismatch(to_np(y), y2)
    c = to_np(cnt)
    assert c[[1, 3, 5, 7, 11, 13, 17, 19]].sum() > c.sum() * 0.5


def test_moe_olmoe_full_routing_and_sampled_rows(ops):
    # C4 at T=256: routing for every token against the oracle, outputs of a
    # sample of tokens (tokens are independent rows of the layer)
    E, K, I, D, T = 64, 8, 1024, 2048, 256
    Wr = randn(100, (E, D), 0.02)
    x = randn(101, (T, D))
    ex = moe_weights(E, I, D, seed=102)
    from moty_amd import ORDER_TOPK
    L = layer(ops, Wr, ex, K, 0, ORDER_TOPK)
    y, idx, w, cnt = L(to_dev(x), want_routing=True)
    idx2, w2, _ = o_route(x, Wr, K, 0)
    assert (to_np(idx) == idx2).all() and same_bits(to_np(w), w2)
    sample = np.array([0, 1, 77, 128, 200, 255])
    y2, _, _ = o_moe(x[sample], Wr, ex, K, "olmoe", norm=0)
    assert same_bits(to_np(y)[sample], y2)
    # determinism across calls (slot order inside experts is atomic-order)
    y3 = L(to_dev(x))
    assert same_bits(to_np(y), to_np(y3))
