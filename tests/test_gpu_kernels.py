"""GPU parity: every HIP kernel against the oracle on the same seeded inputs,
bit-exact (int8 activations, int32 accumulators, f32 outputs)."""
import numpy as np
import pytest
import torch

from cpu_libs import (o_matmul_f32, o_matmul_i4g, o_matmul_q_s, o_pack_int4_grouped, o_qrow, o_quantize_rows,
                      oracle, ptr, randn, rng)
from gpu_util import mismatch, same_bits, say, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(dev):
    import moty_amd
    moty_amd.lib()
    from moty_amd import ops
    return ops


def test_expf_matches_oracle(ops):
    say("expf sweep")
    # strided sweep over all bit patterns plus dense blocks where silu/softmax live
    pats = np.concatenate([
        np.arange(0, 1 << 32, 4093, dtype=np.uint64).astype(np.uint32),
        np.arange(0x3f000000, 0x3f000000 + (1 << 21), dtype=np.uint32),
        np.arange(0xc0000000, 0xc0000000 + (1 << 21), dtype=np.uint32),
        np.array([0x42b17217, 0x42b17218, 0xc2cff1b4, 0xc2cff1b5, 0xc2aeac50, 0xc2b00000, 0xc2c80000,
                  0x7f800000, 0xff800000, 0, 0x80000000, 1], dtype=np.uint32)])
    x = pats.view(np.float32)
    x = x[~np.isnan(x)]
    y = to_np(ops.expf(to_dev(x)))
    o = oracle()
    ref = np.array([o.o_expf(float(v)) for v in x[:20000]], np.float32)
    assert same_bits(y[:20000], ref), mismatch(y[:20000], ref)
    ref_all = np.exp(x.astype(np.float64)).astype(np.float32)
    # the restated algorithm is within 1 ulp of the correctly rounded value everywhere
    fin = np.isfinite(ref_all) & (ref_all > 1e-37)
    ulp = np.abs(y[fin].view(np.int32).astype(np.int64) - ref_all[fin].view(np.int32).astype(np.int64))
    assert ulp.max() <= 1


def test_expf_full_against_oracle_blocks(ops):
    # 2^24 consecutive patterns in each of 4 blocks, checked against the
    # oracle's libm-identical expf via the oracle's own range check
    o = oracle()
    for lo in (0x3e800000, 0x40000000, 0xbf000000, 0xc1000000):
        say("expf block", hex(lo))
        pats = np.arange(lo, lo + (1 << 22), dtype=np.uint64).astype(np.uint32)
        y = to_np(ops.expf(to_dev(pats.view(np.float32))))
        ref = np.empty_like(y)
        xs = pats.view(np.float32)
        ref = np.frompyfunc(lambda v: o.o_expf(float(v)), 1, 1)(xs[::97]).astype(np.float32)
        assert same_bits(y[::97], ref)


@pytest.mark.parametrize("S,I", [(1, 1024), (3, 3072), (7, 100), (2, 16384)])
def test_qrow_i8(ops, S, I):
    say("qrow", S, I)
    x = randn(S * I, (S, I)) * 3
    x[0, :5] = [0.0, -0.0, 1e-30, 5.5, -5.5]
    q, sx, xg = ops.qrow_i8(to_dev(x), group_sums=(I % 32 == 0))
    q2, sx2 = o_qrow(x)
    assert same_bits(to_np(sx), sx2) and same_bits(to_np(q), q2)
    if xg is not None:
        assert (to_np(xg) == q2.reshape(S, -1, 32).astype(np.int32).sum(-1)).all()


@pytest.mark.parametrize("jobs", [[(512, 1024), (512, 2048), (512, 3072)], [(1, 16)], [(0, 64), (5, 4096)],
                                  [(3, 48), (7, 2000), (9, 3072), (130, 1008)]])
def test_qrow_i8_multi(ops, jobs):
    """Several row sets in one launch, each against the oracle's qrow_i8."""
    say("qrow multi", jobs)
    xs = [randn(S * I + j, (S, I)) * 3 for j, (S, I) in enumerate(jobs)]
    if xs[-1].size:
        xs[-1][0, :5] = [0.0, -0.0, 1e-30, 5.5, -5.5]
    outs = ops.qrow_i8_multi([to_dev(x) for x in xs])
    for x, (q, sx) in zip(xs, outs):
        if not x.size:
            continue
        q2, sx2 = o_qrow(x)
        assert same_bits(to_np(sx), sx2) and same_bits(to_np(q), q2)


@pytest.mark.parametrize("S,I", [(1, 1024), (5, 4096), (3, 48), (7, 2000), (9, 3072), (4, 5008), (6, 1030)])
def test_qrow_i8_rows(ops, S, I):
    """Without group sums: rows of I <= 4096 (I % 16 == 0) take the
    wave-per-row kernel, the rest the workgroup-per-row one."""
    say("qrow rows", S, I)
    x = randn(S * I + 7, (S, I)) * 3
    x[0, :3] = [0.0, 1e-30, -5.5]
    q, sx, _ = ops.qrow_i8(to_dev(x), group_sums=False)
    q2, sx2 = o_qrow(x)
    assert same_bits(to_np(sx), sx2) and same_bits(to_np(q), q2)


def test_qrow_zero_row(ops):
    q, sx, _ = ops.qrow_i8(torch.zeros((2, 64), device="cuda:0"))
    assert (to_np(sx) == np.float32(1e-12)).all() and not to_np(q).any()


# I % 4 == 0 and I <= 16384: one pass in registers (1, 2, 4, 8 or 16 float4
# per thread); other rows: the two-pass kernel.  A zero row takes s = 1e-8.
@pytest.mark.parametrize("O,I", [(64, 1024), (7, 33), (3, 3072), (5, 16384), (2, 20000), (9, 4100), (4, 12),
                                 (3, 8190)])
@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_rows(ops, O, I, bits):
    say("quantize_rows", O, I, bits)
    w = randn(O + I, (O, I), 0.02)
    w[0, :5] = [0.0, 1e-30, -0.07, 0.07, 0.035]
    if O > 2:
        w[1] = 0.0
    q, s = ops.quantize_rows(to_dev(w), bits)
    q2, s2 = o_quantize_rows(w, bits)
    assert same_bits(to_np(q), q2) and same_bits(to_np(s), s2)


def test_weight_packers_unaligned(ops):
    # weights that are only 4-byte aligned take the element-wise kernels: same bits
    O, I = 6, 256
    say("packers unaligned")
    w = randn(O + 5 * I, (O, I), 0.02)
    buf = torch.zeros(O * I + 1, dtype=torch.float32, device="cuda")
    wv = buf[1:].view(O, I)
    wv.copy_(to_dev(w))
    q, s = ops.quantize_rows(wv)
    q2, s2 = o_quantize_rows(w)
    assert same_bits(to_np(q), q2) and same_bits(to_np(s), s2)
    q4, s4 = ops.pack_int4_grouped(wv, 32)
    q42, s42 = o_pack_int4_grouped(w, 32)
    assert same_bits(to_np(q4), q42) and same_bits(to_np(s4), s42)


# gs = 32 with I % 32 == 0: one workgroup per 256 consecutive groups staged
# through LDS (full and ragged last workgroup); other shapes: one thread per group
@pytest.mark.parametrize("O,I,gs", [(64, 4096, 32), (5, 31, 16), (8, 100, 32), (300, 1024, 32), (3, 96, 32),
                                    (1, 32, 32), (7, 12288, 32), (4, 64, 16)])
def test_pack_int4_grouped(ops, O, I, gs):
    say("pack_i4g", O, I, gs)
    w = randn(O * 7 + I, (O, I), 0.02)
    w[0, :gs] = 0.0  # an all-zero group: s = 1e-8
    q4, s = ops.pack_int4_grouped(to_dev(w), gs)
    q42, s2 = o_pack_int4_grouped(w, gs)
    assert same_bits(to_np(q4), q42) and same_bits(to_np(s), s2)


Q8_CASES = [(1, 1024, 3072), (1, 3072, 1024), (1, 3072, 2000), (1, 4096, 1500), (1, 4096, 2100), (2, 1024, 100), (3, 48, 24), (4, 2048, 1024),
            (1, 16384, 64), (5, 1024, 256), (8, 3072, 96), (64, 1024, 1024), (512, 1024, 2048),
            (130, 2048, 200), (33, 16, 17), (1024, 1024, 4096), (256, 1040, 8192), (200, 3072, 1000),
            # K % 128 == 0 past the GEMV: the DMA-staged GEMM, one-block and ragged tiles
            (70, 128, 33), (9, 256, 1), (130, 384, 65), (600, 4096, 100), (5, 128, 7),
            # few tiles: K split over four wave groups (K blocks 4, 5, 16)
            (17, 512, 50), (40, 640, 96), (130, 2048, 200),
            # S = 1 past 16 MiB of weights: the shared-activation GEMV, full and ragged
            (1, 4096, 4096), (1, 3088, 5500), (1, 1040, 16200),
            # ... with 4096 or more waves of two rows: 8-wave workgroups
            (1, 4096, 8200)]


@pytest.mark.parametrize("S,I,O", Q8_CASES)
def test_matmul_q_s(ops, S, I, O):
    say("matmul_q_s", S, I, O)
    w = randn(O + 3 * I, (O, I), 0.02)
    q, s = o_quantize_rows(w)
    x = randn(S + I, (S, I))
    y = to_np(ops.matmul_q_s(to_dev(x), to_dev(q), to_dev(s)))
    y2 = o_matmul_q_s(x, q, s)
    assert same_bits(y, y2), mismatch(y, y2)


def test_matmul_q8_extremes(ops):
    # w = -128 everywhere and activations at +-127 (simd_tests.c rep 0)
    S, I, O = 9, 4096, 40
    q = np.full((O, I), -128, np.int8)
    s = np.full(O, 0.01, np.float32)
    x = np.where(rng(1).integers(0, 2, (S, I)) > 0, 1.0, -1.0).astype(np.float32)
    for SS in (1, S):
        y = to_np(ops.matmul_q_s(to_dev(x[:SS]), to_dev(q), to_dev(s)))
        assert same_bits(y, o_matmul_q_s(x[:SS], q, s))


@pytest.mark.parametrize("S,I,O", [(1, 4096, 256), (2, 1024, 64), (4, 12288, 128), (1, 64, 5),
                                   (256, 4096, 192), (37, 1024, 100), (5, 128, 64), (1, 12288, 100),
                                   (9, 192, 40), (70, 64, 33), (65, 12288, 70),
                                   (1, 8192, 77), (1, 16384, 40), (1, 2048, 1000), (130, 1088, 200), (64, 12288, 64),
                                   (250, 1024, 4100)])
def test_i4g_idot4(ops, S, I, O):
    say("i4g idot4", S, I, O)
    w = randn(O + I, (O, I), 0.02)
    q4, s = o_pack_int4_grouped(w)
    x = randn(S + 2 * I, (S, I))
    y = to_np(ops.matmul_i4_grouped_s(to_dev(x), to_dev(q4), to_dev(s), 32, True))
    y2 = o_matmul_i4g(x, q4, s, True)
    assert same_bits(y, y2), mismatch(y, y2)


@pytest.mark.parametrize("D,I", [(4096, 300), (64, 17), (8192, 64), (12288, 40), (16384, 33), (2048, 513)])
def test_gate_up_silu_i4g(ops, D, I):
    say("gate_up_silu_i4g", D, I)
    G = randn(D + 1, (I, D), 0.02)
    U = randn(D + 2, (I, D), 0.02)
    gq, gs = o_pack_int4_grouped(G)
    uq, us = o_pack_int4_grouped(U)
    x = randn(D + 3, (1, D))
    h = to_np(ops.gate_up_silu_i4g(to_dev(x), to_dev(gq), to_dev(gs), to_dev(uq), to_dev(us)))
    g = o_matmul_i4g(x, gq, gs, True)
    u = o_matmul_i4g(x, uq, us, True)
    oracle().o_silu_mul(ptr(g), ptr(u), g.size)
    assert same_bits(h, g), mismatch(h, g)


@pytest.mark.parametrize("S,I,O", [(1, 4096, 256), (3, 96, 40), (16, 1024, 64),
                                   # one token: the GEMV form (1..8 chunks of 64 groups, partial
                                   # chunks, ragged rows; past 12288 more than 64 KiB of LDS), and
                                   # past its 16384 bound the fallback
                                   (1, 12288, 100), (1, 8192, 77), (1, 96, 40), (1, 2080, 300), (1, 16384, 20),
                                   (1, 14336, 300), (2, 16384, 64), (1, 16416, 10),
                                   (1, 64, 1000),
                                   # 2..24 tokens: the GEMV per token; more: the tiled GEMM (64 x 64
                                   # tiles, ragged in tokens and rows; I % 64 != 0 falls back)
                                   (4, 2048, 100), (65, 4096, 130), (256, 1088, 70), (7, 128, 33),
                                   (24, 1024, 96), (25, 1024, 96), (40, 128, 33), (5, 96, 40)])
def test_i4g_f32(ops, S, I, O):
    say("i4g f32", S, I, O)
    w = randn(O + I, (O, I), 0.02)
    q4, s = o_pack_int4_grouped(w)
    x = randn(S + 2 * I, (S, I))
    y = to_np(ops.matmul_i4_grouped_s(to_dev(x), to_dev(q4), to_dev(s), 32, False))
    y2 = o_matmul_i4g(x, q4, s, False)
    assert same_bits(y, y2), mismatch(y, y2)


@pytest.mark.parametrize("S,I,O", [(8, 2048, 64), (3, 33, 5), (2, 16, 3), (1, 100, 7), (5, 2049, 128)])
def test_matmul_f32(ops, S, I, O):
    say("matmul_f32", S, I, O)
    W = randn(I, (O, I), 0.02)
    x = randn(I + 1, (S, I))
    y = to_np(ops.matmul(to_dev(x), to_dev(W)))
    assert same_bits(y, o_matmul_f32(x, W))


def test_silu_and_softmax(ops):
    say("silu/softmax")
    g = randn(1, 100000) * 6
    g[:6] = [0.0, -0.0, 100.0, -100.0, -90.0, 89.0]
    u = randn(2, 100000)
    gd = to_dev(g)
    ops.silu_mul(gd, to_dev(u))
    g2 = g.copy()
    oracle().o_silu_mul(ptr(g2), ptr(u), g.size)
    assert same_bits(to_np(gd), g2)
    for E in (8, 64, 128, 300):
        x = randn(E, (4, E)) * 3
        xd = to_dev(x)
        ops.softmax_rows(xd)
        x2 = x.copy()
        for r in range(4):
            oracle().o_softmax(ptr(x2[r]), E)
        assert same_bits(to_np(xd), x2)


@pytest.mark.parametrize("idot4", [True, False])
@pytest.mark.parametrize("S,D,I", [(37, 256, 384), (5, 128, 128), (4, 256, 128), (1, 128, 64), (130, 1024, 640),
                                   (70, 192, 320), (3, 4096, 96), (300, 512, 1280),
                                   # 64 x 192 gate/up tiles, ragged in tokens and rows
                                   (130, 256, 12416),
                                   # one token through the exact-f32 fused gate/up GEMV
                                   (1, 4096, 1056), (1, 96, 8192), (1, 12288, 2080),
                                   # rows past 12288 (more than 64 KiB of x in LDS), and 2-4
                                   # tokens through the per-token GEMV
                                   (1, 1024, 14336), (1, 16384, 96), (3, 1024, 2048), (4, 14336, 64)])
def test_dense_ffn_i4g(ops, idot4, S, D, I):
    # nn/ffn.c:26-55 over grouped-int4 Mats: the fused gate/up f16 pass
    # (S > 4, D and I multiples of 128), the int8 GEMM fallback (other
    # multiples of 64), the GEMVs (S <= 4) and the exact f32 path
    say("dense_ffn_i4g", idot4, S, D, I)
    gq, gs = o_pack_int4_grouped(randn(S + D, (I, D), 0.02))
    uq, us = o_pack_int4_grouped(randn(S + D + 1, (I, D), 0.02))
    dq, ds = o_pack_int4_grouped(randn(S + I, (D, I), 0.02))
    x = randn(S + 3, (S, D))
    y = to_np(ops.dense_ffn_i4g(to_dev(x), to_dev(gq), to_dev(gs), to_dev(uq), to_dev(us), to_dev(dq), to_dev(ds),
                                idot4))
    # the reference picks the IDOT4 path per matrix: row length % 64 == 0
    g = o_matmul_i4g(x, gq, gs, idot4 and D % 64 == 0)
    u = o_matmul_i4g(x, uq, us, idot4 and D % 64 == 0)
    oracle().o_silu_mul(ptr(g), ptr(u), g.size)
    y2 = o_matmul_i4g(g, dq, ds, idot4 and I % 64 == 0)
    assert same_bits(y, y2), mismatch(y, y2)


@pytest.mark.parametrize("O,I", [(37, 64), (5, 33), (300, 4096), (9, 1)])
def test_pack_int4(ops, O, I):
    # per-row int4 (WF_I4), nn/quant.c:34-55
    from cpu_libs import o_pack_int4
    say("pack_int4", O, I)
    w = randn(O + I, (O, I), 0.02)
    w[0] = 0.0
    q4, s = ops.pack_int4(to_dev(w))
    q2, s2 = o_pack_int4(w)
    assert same_bits(to_np(q4), q2) and same_bits(to_np(s), s2)


@pytest.mark.parametrize("idot4", [True, False])
@pytest.mark.parametrize("S,I,O", [(1, 4096, 256), (3, 1024, 100), (4, 96, 17), (37, 2048, 300), (512, 1024, 1024),
                                   (9, 16, 5), (2, 2048, 20000), (6, 4096, 12288)])
def test_matmul_i4_s(ops, idot4, S, I, O):
    # moty_matmul_i4_s (nn/matmul.c:75-145): the integer dot straight from
    # the nibbles (IDOT4) or the AVX2-order exact f32 path; the last two
    # shapes are large-O weights (no int8 copy of them is made)
    from cpu_libs import o_matmul_i4, o_pack_int4
    say("matmul_i4_s", idot4, S, I, O)
    q4, s = o_pack_int4(randn(O + 2 * I, (O, I), 0.02))
    x = randn(S + I, (S, I))
    y = to_np(ops.matmul_i4_s(to_dev(x), to_dev(q4), to_dev(s), idot4))
    y2 = o_matmul_i4(x, q4, s, idot4)
    assert same_bits(y, y2), mismatch(y, y2)


@pytest.mark.parametrize("idot4", [True, False])
def test_matmul_i4_s_misaligned(ops, idot4):
    # the kernels read 8 nibble bytes per load: a weight view that is not
    # 8-byte aligned is refused with an error, never read out of line
    import torch
    from cpu_libs import o_pack_int4
    S, I, O = 2, 256, 8
    say("matmul_i4_s misaligned", idot4)
    q4, s = o_pack_int4(randn(O + 2 * I, (O, I), 0.02))
    buf = torch.zeros(O * I // 2 + 1, dtype=torch.uint8, device="cuda")
    qv = buf[1:].view(O, I // 2)
    qv.copy_(to_dev(q4))
    import moty_amd
    with pytest.raises(moty_amd.MotyHipError, match="aligned"):
        ops.matmul_i4_s(to_dev(randn(S + I, (S, I))), qv, to_dev(s), idot4)


@pytest.mark.parametrize("case", ["denormal", "large", "huge", "inf"])
@pytest.mark.parametrize("S", [1, 3])
def test_i4g_f32_activation_extremes(ops, S, case):
    # the one-token GEMV holds x as 16 x (nibbles as (n - 8) / 16) while
    # every |x| < 2^123, else x as it is: both must give the reference's bits,
    # with denormal, large (2^122), huge (2^126: the fallback) and infinite
    # activations
    I, O = 2048, 96
    say("i4g f32 extremes", S, case)
    q4, s = o_pack_int4_grouped(randn(O + I, (O, I), 0.02))
    x = randn(S + 11 * I, (S, I))
    if case == "denormal":
        x[:, ::3] *= np.float32(1e-40)
    elif case == "large":
        x[:, 5] = np.float32(2.0 ** 122)
    elif case == "huge":
        x[:, 7] = np.float32(2.0 ** 126)
        x[:, 9] = np.float32(-3e38)
    else:
        x[:, 3] = np.float32(np.inf)
    y = to_np(ops.matmul_i4_grouped_s(to_dev(x), to_dev(q4), to_dev(s), 32, False))
    y2 = o_matmul_i4g(x, q4, s, False)
    # NaNs (inf * 0 and inf - inf) compare as NaNs: the host and the GPU
    # make default NaNs with different sign bits
    nan = np.isnan(y2)
    assert (np.isnan(y) == nan).all()
    assert same_bits(np.where(nan, 0, y).astype(np.float32), np.where(nan, 0, y2).astype(np.float32)), mismatch(y, y2)


@pytest.mark.parametrize("S", [1, 9])
def test_i4g_f32_unaligned_activations(ops, S):
    # the exact-f32 GEMV / tiled GEMM read x in 16-byte units: an activation
    # view that is only 4-byte aligned takes the lane-per-output kernel, same bits
    I, O = 1024, 72
    say("i4g f32 unaligned x", S)
    q4, s = o_pack_int4_grouped(randn(O + I, (O, I), 0.02))
    x = randn(S + 5 * I, (S, I))
    buf = torch.zeros(S * I + 1, dtype=torch.float32, device="cuda")
    xv = buf[1:].view(S, I)
    xv.copy_(to_dev(x))
    y = to_np(ops.matmul_i4_grouped_s(xv, to_dev(q4), to_dev(s), 32, False))
    y2 = o_matmul_i4g(x, q4, s, False)
    assert same_bits(y, y2), mismatch(y, y2)


def test_qrow_i8_multi_refuses(ops):
    # job counts outside 1..4, rows past 4096 elements or not a multiple of
    # 16, and unaligned rows are refused with an error, never run
    import ctypes as C
    import moty_amd
    say("qrow multi refuses")
    x = torch.zeros((2, 4112), dtype=torch.float32, device="cuda")
    with pytest.raises(moty_amd.MotyHipError, match="4096"):
        ops.qrow_i8_multi([x])
    with pytest.raises(moty_amd.MotyHipError, match="4096"):
        ops.qrow_i8_multi([torch.zeros((2, 40), dtype=torch.float32, device="cuda")])
    buf = torch.zeros(2 * 64 + 1, dtype=torch.float32, device="cuda")
    with pytest.raises(moty_amd.MotyHipError, match="aligned"):
        ops.qrow_i8_multi([buf[1:].view(2, 64)])
    with pytest.raises(moty_amd.MotyHipError, match="bad arguments"):
        ops.qrow_i8_multi([torch.zeros((1, 64), dtype=torch.float32, device="cuda")] * 5)
    lib = moty_amd.lib()
    z = (C.c_void_p * 1)()
    n = (C.c_int * 1)(1)
    assert lib.moty_hip_qrow_i8_multi_dev(0, z, z, z, n, n, None) != 0


def test_q8_refuses_unaligned_weights(ops):
    # the Q8 GEMV/GEMM read weight rows in 16-byte units: a weight view one
    # byte off is refused with an error, never read out of line
    import moty_amd
    I, O = 1024, 64
    say("q8 unaligned weights")
    q, s = o_quantize_rows(randn(O + I, (O, I), 0.02))
    buf = torch.zeros(O * I + 1, dtype=torch.int8, device="cuda")
    qv = buf[1:].view(O, I)
    qv.copy_(to_dev(q))
    for S in (1, 8):
        with pytest.raises(moty_amd.MotyHipError, match="16-byte aligned"):
            ops.matmul_q_s(to_dev(randn(S + I, (S, I))), qv, to_dev(s))
