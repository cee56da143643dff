"""GPU: GGUF block formats on the device (io/gguf.h) against the oracle, bit
for bit: the five block dequantisers, the lossless Q4_0 -> grouped-int4
repack, unaligned sources, partial last workgroups, the host drop-ins, and
the load_mat_bits chains (dequant -> quantize_rows / pack_int4_grouped)."""
import ctypes as C

import numpy as np
import pytest
import torch

from cpu_libs import (GG_BLOCK, GG_Q4_0, GG_Q4_K, GG_Q8_0, gg_blocks, o_gguf_dequant, o_gguf_repack_q4_0,
                      o_pack_int4_grouped, o_quantize_rows, ptr)
from gpu_util import same_bits, say, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(dev):
    from moty_amd import ops as o
    return o


def nan_same(a, b):
    """bit-equal, except that NaNs need only be NaN in both"""
    a, b = np.asarray(a), np.asarray(b)
    n = np.isnan(a)
    return bool((n == np.isnan(b)).all()) and same_bits(np.where(n, 0, a), np.where(n, 0, b))


# block counts: one partial workgroup, exactly one, several with a partial tail
@pytest.mark.parametrize("dtype", sorted(GG_BLOCK))
@pytest.mark.parametrize("nblk", [1, 7, 32, 256, 1000, 4099])
def test_gguf_dequant(ops, dtype, nblk):
    say("gguf_dequant", dtype, nblk)
    E, B = GG_BLOCK[dtype]
    raw = gg_blocks(nblk * 7 + dtype, dtype, nblk)
    y = ops.gguf_dequant(dtype, to_dev(raw), nblk * E)
    assert same_bits(to_np(y), o_gguf_dequant(dtype, raw, nblk * E))


@pytest.mark.parametrize("dtype", sorted(GG_BLOCK))
def test_gguf_dequant_nonfinite_scales(ops, dtype):
    # raw f16 fields include Inf / NaN / subnormal halves
    say("gguf_dequant nonfinite", dtype)
    E, B = GG_BLOCK[dtype]
    raw = gg_blocks(dtype + 100, dtype, 2048, finite=False)
    y = ops.gguf_dequant(dtype, to_dev(raw), 2048 * E)
    assert nan_same(to_np(y), o_gguf_dequant(dtype, raw, 2048 * E))


@pytest.mark.parametrize("dtype", sorted(GG_BLOCK))
@pytest.mark.parametrize("off", [1, 2, 6])
def test_gguf_dequant_unaligned_source(ops, dtype, off):
    # a tensor's data at an odd offset of a mapped file: byte-staged path
    say("gguf_dequant unaligned", dtype, off)
    E, B = GG_BLOCK[dtype]
    nblk = 300
    raw = gg_blocks(dtype + 7 * off, dtype, nblk)
    buf = torch.zeros(nblk * B + 64, dtype=torch.uint8, device="cuda:0")
    buf[off:off + nblk * B] = to_dev(raw)
    y = ops.gguf_dequant(dtype, buf[off:off + nblk * B], nblk * E)
    assert same_bits(to_np(y), o_gguf_dequant(dtype, raw, nblk * E))


@pytest.mark.parametrize("O,I", [(1, 32), (3, 64), (17, 96), (64, 4096), (300, 1024), (1, 32 * 300)])
def test_gguf_repack_q4_0(ops, O, I):
    say("gguf_repack_q4_0", O, I)
    raw = gg_blocks(O + I, GG_Q4_0, O * I // 32, finite=False)
    q4, qs = ops.gguf_repack_q4_0(to_dev(raw), O, I)
    eq4, eqs = o_gguf_repack_q4_0(raw, O, I)
    assert same_bits(to_np(q4).reshape(-1), eq4)
    assert same_bits(to_np(qs).reshape(-1), eqs)  # scales widened bit-exactly, NaN payloads included


def test_gguf_repack_q4_0_unaligned(ops):
    say("gguf_repack_q4_0 unaligned")
    O, I = 40, 256
    raw = gg_blocks(5, GG_Q4_0, O * I // 32)
    buf = torch.zeros(raw.size + 32, dtype=torch.uint8, device="cuda:0")
    buf[3:3 + raw.size] = to_dev(raw)
    q4, qs = ops.gguf_repack_q4_0(buf[3:3 + raw.size], O, I)
    eq4, eqs = o_gguf_repack_q4_0(raw, O, I)
    assert same_bits(to_np(q4).reshape(-1), eq4) and same_bits(to_np(qs).reshape(-1), eqs)


def test_gguf_q8_0_to_i8_chain(ops):
    # load_mat_bits QBITS=8 on a Q8_0 tensor: dequant to f32, quantize_rows
    say("gguf Q8_0 -> WF_I8")
    O, I = 96, 512
    raw = gg_blocks(11, GG_Q8_0, O * I // 32)
    w = ops.gguf_dequant(GG_Q8_0, to_dev(raw), O * I).view(O, I)
    q, s = ops.quantize_rows(w, 8)
    eq, es = o_quantize_rows(o_gguf_dequant(GG_Q8_0, raw, O * I).reshape(O, I), 8)
    assert same_bits(to_np(q), eq) and same_bits(to_np(s), es)


def test_gguf_q4_k_to_i4g_chain(ops):
    # load_mat_bits QBITS=4 QGROUP=32 on a Q4_K tensor: dequant, pack_int4_grouped
    say("gguf Q4_K -> WF_I4G")
    O, I = 64, 1024
    raw = gg_blocks(12, GG_Q4_K, O * I // 256)
    w = ops.gguf_dequant(GG_Q4_K, to_dev(raw), O * I).view(O, I)
    q4, s = ops.pack_int4_grouped(w, 32)
    eq4, es = o_pack_int4_grouped(o_gguf_dequant(GG_Q4_K, raw, O * I).reshape(O, I), 32)
    assert same_bits(to_np(q4).reshape(-1), eq4.reshape(-1)) and same_bits(to_np(s).reshape(-1), es.reshape(-1))


def test_gguf_host_dropins(dev):
    from moty_amd import lib
    say("gguf host drop-ins")
    L = lib()
    for dtype, (E, B) in sorted(GG_BLOCK.items()):
        raw = gg_blocks(dtype * 3, dtype, 77)
        out = np.empty(77 * E, np.float32)
        assert L.moty_hip_gguf_dequant(dtype, ptr(raw), 77 * E, ptr(out)) == 0
        assert same_bits(out, o_gguf_dequant(dtype, raw, 77 * E))
    O, I = 9, 160
    raw = gg_blocks(4, GG_Q4_0, O * I // 32)
    q4 = np.empty(O * I // 2, np.uint8)
    qs = np.empty(O * I // 32, np.float32)
    assert L.moty_hip_gguf_repack_q4_0(ptr(raw), ptr(q4), ptr(qs), O, I) == 0
    eq4, eqs = o_gguf_repack_q4_0(raw, O, I)
    assert same_bits(q4, eq4) and same_bits(qs, eqs)


def test_gguf_errors(dev):
    from moty_amd import lib
    L = lib()
    raw = torch.zeros(1024, dtype=torch.uint8, device="cuda:0")
    out = torch.zeros(1024, dtype=torch.float32, device="cuda:0")
    p = lambda t: C.c_void_p(t.data_ptr())
    assert L.moty_hip_gguf_dequant_dev(3, p(raw), 32, p(out), None) == 4   # not a block type
    assert L.moty_hip_gguf_dequant_dev(4, p(raw), 48, p(out), None) == 1   # not whole blocks
    assert L.moty_hip_gguf_repack_q4_0_dev(p(raw), p(raw), p(out), 2, 48, None) == 1
    assert L.moty_hip_gguf_dequant_dev(4, p(raw), 0, p(out), None) == 0
