"""CPU: the GGUF block-format oracle (o_gguf_dequant, o_gguf_repack_q4_0)
pinned against the compiled reference (io/gguf.h built into oracle/_ref),
the known-answer blocks of c/tests/headers_tests.c:131-211 and
c/tests/qwen_tests.c:799-847, and blocks built by encoders written from the
format description (the inverse of the decoders), so a transposed field or a
wrong bit position fails."""
import numpy as np
import pytest

from cpu_libs import (GG_BLOCK, GG_Q4_0, GG_Q4_K, GG_Q5_K, GG_Q6_K, GG_Q8_0, gg_blocks, o_gguf_dequant,
                      o_gguf_repack_q4_0, oracle, ptr, ref, ref_gguf_dequant, ref_gguf_repack_q4_0)

needs_ref = pytest.mark.skipif(ref(True) is None, reason="oracle/_ref not built or no AVX512-VNNI host")

F16_ONE, F16_HALF, F16_TWO = 0x3C00, 0x3800, 0x4000


def nan_same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    n = np.isnan(a)
    return bool((n == np.isnan(b)).all()) and bool((np.where(n, 0, a).view(np.uint32) ==
                                                    np.where(n, 0, b).view(np.uint32)).all())


def put16(buf, off, h):
    buf[off] = h & 0xFF
    buf[off + 1] = h >> 8


# ---------------- against the compiled reference ----------------
@needs_ref
@pytest.mark.parametrize("dtype", sorted(GG_BLOCK))
@pytest.mark.parametrize("finite", [True, False])
def test_dequant_matches_ref(dtype, finite):
    E, _ = GG_BLOCK[dtype]
    raw = gg_blocks(dtype * 5 + finite, dtype, 3000, finite=finite)
    a = o_gguf_dequant(dtype, raw, 3000 * E)
    b = ref_gguf_dequant(ref(True), dtype, raw, 3000 * E)
    assert nan_same(a, b)


@needs_ref
@pytest.mark.parametrize("O,I", [(1, 32), (7, 96), (64, 1024)])
def test_repack_matches_ref(O, I):
    raw = gg_blocks(O * I, GG_Q4_0, O * I // 32, finite=False)
    a4, as_ = o_gguf_repack_q4_0(raw, O, I)
    b4, bs = ref_gguf_repack_q4_0(ref(True), raw, O, I)
    assert (a4 == b4).all() and (as_.view(np.uint32) == bs.view(np.uint32)).all()


@needs_ref
@pytest.mark.parametrize("dtype", [GG_Q4_K, GG_Q5_K])
def test_kquant_product_is_exact(dtype):
    # sc*q - mn: d*sc is an f16 mantissa (11 bits) times a 6-bit integer and q
    # has at most 5 bits, so sc*q is exact in f32 and the result does not
    # depend on whether a compiler fuses the multiply-subtract: the unfused
    # form equals the reference bit for bit
    E, B = GG_BLOCK[dtype]
    nblk = 2000
    raw = gg_blocks(77 + dtype, dtype, nblk, finite=False)
    r = ref_gguf_dequant(ref(True), dtype, raw, nblk * E)
    blk = raw.reshape(nblk, B)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(-1)
    sc, mn = k4_unpack(blk[:, 4:16])
    q = kquant_codes(blk, dtype == GG_Q5_K)  # [nblk, 256]
    with np.errstate(all="ignore"):
        scf = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
        mnf = (dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
        sub = np.arange(256) // 32
        unfused = (scf[:, sub] * q.astype(np.float32)).astype(np.float32) - mnf[:, sub]
    assert nan_same(unfused.reshape(-1), r)


# ---------------- format encoders (inverse of the decoders) ----------------
def k4_pack(sc, mn):
    """12 scale bytes holding 6-bit (scale, min) for 8 sub-blocks."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return s


def k4_unpack(s):
    """[n, 12] scale bytes -> ([n, 8] scales, [n, 8] mins), by bit positions."""
    s = s.astype(np.int64)
    sc = np.zeros((s.shape[0], 8), np.int64)
    mn = np.zeros_like(sc)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        mn[:, j] = s[:, j + 4] & 63
        sc[:, j + 4] = (s[:, j + 8] & 15) + 16 * (s[:, j] >> 6)
        mn[:, j + 4] = (s[:, j + 8] >> 4) + 16 * (s[:, j + 4] >> 6)
    return sc, mn


def kquant_codes(blk, q5):
    """[n, B] Q4_K / Q5_K blocks -> [n, 256] unsigned codes."""
    ql = blk[:, 48:176] if q5 else blk[:, 16:144]
    q = np.zeros((blk.shape[0], 256), np.int64)
    for e in range(256):
        c, h, l = e // 64, (e // 32) % 2, e % 32
        v = (ql[:, 32 * c + l] >> (4 * h)) & 15
        if q5:
            v = v + 16 * ((blk[:, 16 + l] >> (2 * c + h)) & 1)
        q[:, e] = v
    return q


def enc_kquant(d16, dmin16, sc, mn, q, q5):
    B = 176 if q5 else 144
    b = np.zeros(B, np.uint8)
    put16(b, 0, d16)
    put16(b, 2, dmin16)
    b[4:16] = k4_pack(sc, mn)
    ql = b[48:176] if q5 else b[16:144]
    for e in range(256):
        c, h, l = e // 64, (e // 32) % 2, e % 32
        ql[32 * c + l] |= (q[e] & 15) << (4 * h)
        if q5 and q[e] >= 16:
            b[16 + l] |= 1 << (2 * c + h)
    return b


def enc_q6k(d16, sc, q):
    b = np.zeros(210, np.uint8)
    for e in range(256):
        n, r, l = e // 128, (e // 32) % 4, e % 32
        b[64 * n + l + 32 * (r & 1)] |= (q[e] & 15) << (4 * (r >> 1))
        b[128 + 32 * n + l] |= (q[e] >> 4) << (2 * r)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    put16(b, 208, d16)
    return b


def enc_q4_0(d16, v):
    b = np.zeros(18, np.uint8)
    put16(b, 0, d16)
    for i in range(16):
        b[2 + i] = v[i] | (v[i + 16] << 4)
    return b


@pytest.mark.parametrize("q5", [False, True])
def test_kquant_encoded_blocks(q5):
    g = np.random.default_rng(5 + q5)
    for _ in range(20):
        sc = g.integers(0, 64, 8)
        mn = g.integers(0, 64, 8)
        q = g.integers(0, 32 if q5 else 16, 256)
        raw = enc_kquant(F16_ONE, F16_HALF, sc, mn, q, q5)
        y = o_gguf_dequant(GG_Q5_K if q5 else GG_Q4_K, raw, 256)
        sub = np.arange(256) // 32
        # d = 1, dmin = 0.5, integer codes: every step exact
        assert (y == sc[sub] * q - 0.5 * mn[sub]).all()
        assert (k4_unpack(raw[None, 4:16])[0][0] == sc).all()


def test_q6k_encoded_blocks():
    g = np.random.default_rng(6)
    for _ in range(20):
        sc = g.integers(-128, 128, 16)
        q = g.integers(0, 64, 256)
        y = o_gguf_dequant(GG_Q6_K, enc_q6k(F16_TWO, sc, q), 256)
        e = np.arange(256)
        si = 8 * (e // 128) + (e % 32) // 16 + 2 * ((e // 32) % 4)
        assert (y == 2.0 * sc[si] * (q - 32)).all()


def test_q4_0_q8_0_encoded_blocks():
    g = np.random.default_rng(7)
    for _ in range(20):
        v = g.integers(0, 16, 32)
        y = o_gguf_dequant(GG_Q4_0, enc_q4_0(F16_HALF, v), 32)
        assert (y == 0.5 * (v - 8)).all()
        q = g.integers(-128, 128, 32)
        b = np.zeros(34, np.uint8)
        put16(b, 0, 0xC400)  # -4.0
        b[2:] = q.astype(np.int8).view(np.uint8)
        assert (o_gguf_dequant(GG_Q8_0, b, 32) == -4.0 * q).all()


# ---------------- the reference's known-answer tests ----------------
def test_headers_q80_q40_known_answers():
    # headers_tests.c:131-157
    b8 = np.zeros(34, np.uint8)
    put16(b8, 0, F16_TWO)
    b8[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    assert (o_gguf_dequant(GG_Q8_0, b8, 32) == 2.0 * (np.arange(32) - 16)).all()
    b4 = np.zeros(18, np.uint8)
    put16(b4, 0, F16_HALF)
    i = np.arange(16)
    b4[2:] = (i & 15) | (((15 - i) & 15) << 4)
    out = o_gguf_dequant(GG_Q4_0, b4, 32)
    assert (out[:16] == 0.5 * (i - 8)).all() and (out[16:] == 0.5 * ((15 - i) - 8)).all()
    q4, qs = o_gguf_repack_q4_0(b4, 1, 32)
    assert qs[0] == 0.5
    k = np.arange(32)
    v = np.where(k & 1, q4[k >> 1] >> 4, q4[k >> 1] & 15).astype(np.int64) - 8
    assert (qs[0] * v == out).all()


def test_headers_kquant_known_answers():
    # headers_tests.c:159-211: hand-built superblocks
    b = np.zeros(210, np.uint8)
    put16(b, 0, F16_ONE)
    put16(b, 2, F16_HALF)
    b[4:16] = np.arange(12) + 1
    b[16:144] = (np.arange(128) * 7) & 0xFF
    y = o_gguf_dequant(GG_Q4_K, b[:144], 256)
    sc, mn = k4_unpack(b[None, 4:16])
    q = kquant_codes(b[None, :144], False)[0]
    sub = np.arange(256) // 32
    assert (y == sc[0][sub] * q - 0.5 * mn[0][sub]).all()

    b = np.zeros(210, np.uint8)
    put16(b, 0, F16_ONE)
    put16(b, 2, F16_HALF)
    b[4:16] = 13 - np.arange(12)
    b[16:48] = (np.arange(32) * 11) & 0xFF
    b[48:176] = 255 - np.arange(128)
    y = o_gguf_dequant(GG_Q5_K, b[:176], 256)
    sc, mn = k4_unpack(b[None, 4:16])
    q = kquant_codes(b[None, :176], True)[0]
    assert (y == sc[0][sub] * q - 0.5 * mn[0][sub]).all()

    b = np.zeros(210, np.uint8)
    b[:128] = (np.arange(128) * 3) & 0xFF
    b[128:192] = (np.arange(64) * 5) & 0xFF
    b[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    put16(b, 208, F16_ONE)
    y = o_gguf_dequant(GG_Q6_K, b, 256)
    ql, qh, s6 = b[:128].astype(np.int64), b[128:192].astype(np.int64), b[192:208].view(np.int8)
    for n in range(2):
        for l in range(32):
            isc = 8 * n + l // 16
            q1 = (ql[64 * n + l] & 15) | ((qh[32 * n + l] & 3) << 4)
            q2 = (ql[64 * n + l + 32] & 15) | (((qh[32 * n + l] >> 2) & 3) << 4)
            q3 = (ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)
            q4_ = (ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)
            base = 128 * n + l
            assert y[base] == s6[isc] * (q1 - 32) and y[base + 32] == s6[isc + 2] * (q2 - 32)
            assert y[base + 64] == s6[isc + 4] * (q3 - 32) and y[base + 96] == s6[isc + 6] * (q4_ - 32)


def xorshift64_bytes(seed, n):
    s = seed
    out = []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        out.append(s & 0xFF)
    return out


def test_qwen_q4_0_load_blocks():
    # qwen_tests.c:799-847: O=4, I=64 Q4_0 blocks, scales alternating 1.0 /
    # 0.5, nibbles from the test's xorshift64 (seed 4242); the repack is
    # lossless: dequantizing the grouped int4 equals the Q4_0 dequant
    O, I = 4, 64
    nb = O * I // 32
    bytes_ = xorshift64_bytes(4242, nb * 16)
    raw = np.zeros(nb * 18, np.uint8)
    for b in range(nb):
        put16(raw, b * 18, (F16_ONE, F16_HALF)[b & 1])
        raw[b * 18 + 2:b * 18 + 18] = bytes_[b * 16:(b + 1) * 16]
    q4, qs = o_gguf_repack_q4_0(raw, O, I)
    deq = o_gguf_dequant(GG_Q4_0, raw, O * I)
    k = np.arange(O * I)
    v = np.where(k & 1, q4[k >> 1] >> 4, q4[k >> 1] & 15).astype(np.int64) - 8
    assert (np.repeat(qs, 32) * v == deq).all()
    assert (qs == np.tile([1.0, 0.5], nb // 2)).all()


def test_block_table():
    o = oracle()
    import ctypes as C
    e, b = C.c_int(), C.c_int()
    for dt, (E, B) in GG_BLOCK.items():
        assert o.o_gguf_block(dt, C.byref(e), C.byref(b)) == 1 and (e.value, b.value) == (E, B)
    assert o.o_gguf_block(3, C.byref(e), C.byref(b)) == 0
    assert o.o_gguf_dequant(9, ptr(np.zeros(256, np.uint8)), 256, ptr(np.zeros(256, np.float32))) == -1
