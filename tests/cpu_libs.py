"""ctypes loaders for the CPU checkers: the oracle restatement
(oracle/liboracle.so) and the compiled reference (oracle/_ref/*.so).

Test infrastructure only; the product library is loaded by moty_amd."""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libmotyref.so")
REF_F32_SO = os.path.join(ROOT, "oracle", "_ref", "libmotyref_f32.so")

P = C.c_void_p
I32 = C.c_int
I64 = C.c_int64
F32 = C.c_float


def ptr(a):
    """Address of a numpy array; the pointer object keeps the array alive, so
    a temporary (e.g. ptr(f32(x)) after a conversion) outlives the call."""
    if a is None:
        return None
    p = C.c_void_p(a.ctypes.data)
    p._keep = a
    return p


_SIGS = {
    "o_qrow_i8": (F32, [P, P, I32]),
    "o_dot_i8i8": (C.c_int32, [P, P, I32]),
    "o_quantize_rows": (None, [P, P, P, I32, I32, I32]),
    "o_pack_int4_grouped": (None, [P, P, P, I32, I32, I32]),
    "o_matmul_q_s": (None, [P, P, P, P, I32, I32, I32]),
    "o_matmul_q8_preq": (None, [P, P, P, P, P, P, I32, I32, I32]),
    "o_dot_i4g8p": (F32, [P, P, P, P, I32]),
    "o_pack_int4": (None, [P, P, P, I32, I32]),
    "o_matmul_i4_idot4": (None, [P, P, P, P, I32, I32, I32]),
    "o_matmul_i4_f32": (None, [P, P, P, P, I32, I32, I32]),
    "moty_pack_int4": (None, [P, P, P, I32, I32]),
    "moty_matmul_i4_s": (None, [P, P, P, P, I32, I32, I32]),
    "o_matmul_i4g_idot4": (None, [P, P, P, P, I32, I32, I32]),
    "o_matmul_i4g_f32": (None, [P, P, P, P, I32, I32, I32]),
    "o_dot_f32": (F32, [P, P, I32]),
    "o_matmul_f32": (None, [P, P, P, I32, I32, I32]),
    "o_expf": (F32, [F32]),
    "o_expf_table": (None, [P]),
    "o_expf_check_range": (I64, [C.c_uint64, C.c_uint64]),
    "o_silu_mul": (None, [P, P, I64]),
    "o_softmax": (None, [P, I32]),
    "o_topk": (None, [P, I32, I32, P, P, I32]),
    "o_route": (None, [P, P, P, I32, I32, I32, I32, I32, P, P, P]),
    "o_moe_olmoe": (None, [P, P, I32, P, P, P, P, P, P, P, P, I32, I32, I32, I32, I32, P, P]),
    "o_moe_batch": (None, [P, P, I32, P, P, P, P, P, P, P, P, I32, I32, I32, I32, P, P]),
    "o_dense_ffn_q8": (None, [P, P, I32, P, P, P, P, P, P, I32, I32]),
    "o_f16_to_f32": (F32, [C.c_uint16]),
    "o_f32_to_f16": (C.c_uint16, [F32]),
    "o_quant_g32": (None, [P, I32, P, P, P]),
    "o_pack_q4r4": (None, [P, I32, I32, P, P]),
    "o_pack_q8r4": (None, [P, I32, I32, P, P]),
    "o_matmul_q4r4": (None, [P, P, P, P, I32, I32, I32]),
    "o_matmul_q8r4": (None, [P, P, P, P, I32, I32, I32]),
    "o_gguf_block": (I32, [I32, P, P]),
    "o_gguf_repack_q4_0": (None, [P, P, P, I64, I64]),
    "o_gguf_dequant": (I32, [I32, P, I64, P]),
    "ref_gguf_repack_q4_0": (None, [P, P, P, I64, I64]),
    "ref_gguf_dequant": (None, [I32, P, I64, P]),
    "o_ecache_new": (P, [I32, I32]),
    "o_ecache_free": (None, [P]),
    "o_ecache_get": (I32, [P, I32, P]),
    "o_ecache_pin": (I32, [P, I32]),
    "o_ecache_state": (None, [P, P, P, P, P, P, P, P]),
    "o_ecache_route_bias": (None, [P, P, F32]),
    # the reference's own R4 symbols (nn/quant.c, hw/hw_q4r4.h, nn/matmul.c)
    "moty_hw_f16_to_f32": (F32, [C.c_uint16]),
    "moty_f32_to_f16": (C.c_uint16, [F32]),
    "moty_hw_quant_g32": (None, [P, I32, P, P, P]),
    "moty_pack_q4r4_block": (None, [P, I32, I32, P, P]),
    "moty_pack_q8r4_block": (None, [P, I32, I32, P, P]),
    "moty_matmul_q4r4_s": (None, [P, P, P, P, I32, I32, I32]),
    "moty_matmul_q8r4_s": (None, [P, P, P, P, I32, I32, I32]),
    "ref_init": (None, [I32]),
    "ref_tier": (C.c_char_p, []),
    "ref_qrow_i8": (F32, [P, P, I32]),
    "ref_dot_i8i8": (C.c_int32, [P, P, I32]),
    "ref_dot_f32": (F32, [P, P, I32]),
    "ref_dot_i4g8p": (F32, [P, P, P, P, I32]),
    "ref_quantize_rows": (None, [P, P, P, I32, I32, I32]),
    "ref_pack_int4_grouped": (None, [P, P, P, I32, I32, I32]),
    "ref_matmul_q_s": (None, [P, P, P, P, I32, I32, I32]),
    "ref_matmul_i4_grouped_s": (None, [P, P, P, P, I32, I32, I32, I32]),
    "ref_matmul": (None, [P, P, P, I32, I32, I32]),
    "ref_silu_mul": (None, [P, P, I64]),
    "ref_softmax": (None, [P, I32]),
    "ref_expf": (F32, [F32]),
    "ref_topk": (None, [P, I32, I32, P, P, I32]),
    "ref_moe_batch": (None, [P, P, I32, P, P, P, P, P, P, P, I32, I32, I32, I32]),
    "ref_moe_batch_cap": (None, [P, P, I32, P, P, P, P, P, P, P, I32, I32, I32, I32, I32]),
    "ref_moe_d1": (None, [P, P, P, P, P, P, P, P, P, I32, I32, I32, I32]),
    "ref_moe_olmoe": (None, [P, P, I32, P, P, P, P, P, P, P, I32, I32, I32, I32, I32, P]),
}


def _bind(lib):
    for name, (res, args) in _SIGS.items():
        if hasattr(lib, name):
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
    return lib


_cache = {}


def oracle():
    if "o" not in _cache:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle/liboracle.so is not built (run __graft_entry__.build())")
        _cache["o"] = _bind(C.CDLL(ORACLE_SO))
    return _cache["o"]


def cpu_has_vnni():
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return "avx512_vnni" in flags and "avx512bw" in flags
    except OSError:
        return False


def ref(idot4=True):
    """The compiled reference; None when it is not built or the host lacks
    the AVX512-VNNI tier it was compiled for."""
    key = "r4" if idot4 else "r32"
    if key not in _cache:
        path = REF_SO if idot4 else REF_F32_SO
        if not os.path.exists(path) or not cpu_has_vnni():
            _cache[key] = None
        else:
            lib = _bind(C.CDLL(path))
            lib.ref_init(1 if idot4 else 0)
            _cache[key] = lib
    return _cache[key]


# ---- numpy-level helpers over the oracle ----
def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def o_quantize_rows(w, bits=8):
    O, I = w.shape
    q = np.empty((O, I), np.int8)
    s = np.empty(O, np.float32)
    oracle().o_quantize_rows(ptr(f32(w)), ptr(q), ptr(s), O, I, bits)
    return q, s


def o_pack_int4_grouped(w, gs=32):
    O, I = w.shape
    ng = (I + gs - 1) // gs
    q4 = np.empty((O, (I + 1) // 2), np.uint8)
    s = np.empty((O, ng), np.float32)
    oracle().o_pack_int4_grouped(ptr(f32(w)), ptr(q4), ptr(s), O, I, gs)
    return q4, s


def o_qrow(x):
    x = f32(x)
    S, I = x.shape
    q = np.empty((S, I), np.int8)
    sx = np.empty(S, np.float32)
    for s in range(S):
        sx[s] = oracle().o_qrow_i8(C.c_void_p(x.ctypes.data + s * I * 4), C.c_void_p(q.ctypes.data + s * I), I)
    return q, sx


def o_matmul_q_s(x, q, scale):
    x = f32(x)
    S, I = x.shape
    O = q.shape[0]
    y = np.empty((S, O), np.float32)
    oracle().o_matmul_q_s(ptr(y), ptr(x), ptr(q), ptr(scale), S, I, O)
    return y


def o_matmul_q8_acc(xq, q):
    S, I = xq.shape
    O = q.shape[0]
    acc = np.empty((S, O), np.int32)
    sx = np.ones(S, np.float32)
    sc = np.ones(O, np.float32)
    oracle().o_matmul_q8_preq(None, ptr(xq), ptr(sx), ptr(q), ptr(sc), ptr(acc), S, I, O)
    return acc


def o_matmul_i4g(x, q4, scale, idot4=True):
    x = f32(x)
    S, I = x.shape
    O = q4.shape[0]
    y = np.empty((S, O), np.float32)
    fn = oracle().o_matmul_i4g_idot4 if idot4 else oracle().o_matmul_i4g_f32
    fn(ptr(y), ptr(x), ptr(q4), ptr(scale), S, I, O)
    return y


def o_pack_int4(w):
    O, I = w.shape
    q4 = np.empty((O, (I + 1) // 2), np.uint8)
    s = np.empty(O, np.float32)
    oracle().o_pack_int4(ptr(f32(w)), ptr(q4), ptr(s), O, I)
    return q4, s


def o_matmul_i4(x, q4, scale, idot4=True):
    x = f32(x)
    S, I = x.shape
    O = q4.shape[0]
    y = np.empty((S, O), np.float32)
    (oracle().o_matmul_i4_idot4 if idot4 else oracle().o_matmul_i4_f32)(ptr(y), ptr(x), ptr(q4), ptr(scale), S, I, O)
    return y


def o_matmul_f32(x, W):
    x = f32(x)
    S, I = x.shape
    O = W.shape[0]
    y = np.empty((S, O), np.float32)
    oracle().o_matmul_f32(ptr(y), ptr(x), ptr(f32(W)), S, I, O)
    return y


def o_route(x, Wr, K, norm, bias=None):
    x = f32(x)
    S, D = x.shape
    E = Wr.shape[0]
    idx = np.empty((S, K), np.int32)
    w = np.empty((S, K), np.float32)
    probs = np.empty((S, E), np.float32)
    oracle().o_route(ptr(x), ptr(f32(Wr)), ptr(None if bias is None else f32(bias)), S, D, E, K, norm,
                     ptr(idx), ptr(w), ptr(probs))
    return idx, w, probs


def o_moe(x, Wr, ex, K, order="batch", norm=1, bias=None):
    """ex = dict(G,GS,U,US,Dn,DS) stacked expert weights."""
    x = f32(x)
    S, D = x.shape
    E = Wr.shape[0]
    I = ex["G"].shape[1]
    out = np.empty((S, D), np.float32)
    idx = np.empty((S, K), np.int32)
    w = np.empty((S, K), np.float32)
    args = [ptr(ex[k]) for k in ("G", "GS", "U", "US", "Dn", "DS")]
    b = ptr(None if bias is None else f32(bias))
    if order == "batch":
        oracle().o_moe_batch(ptr(out), ptr(x), S, ptr(f32(Wr)), b, *args, E, K, I, D, ptr(idx), ptr(w))
    else:
        oracle().o_moe_olmoe(ptr(out), ptr(x), S, ptr(f32(Wr)), b, *args, E, K, I, D, norm, ptr(idx), ptr(w))
    return out, idx, w


def o_dense_ffn_q8(x, G, GS, U, US, Dn, DS):
    x = f32(x)
    S, D = x.shape
    I = G.shape[0]
    out = np.empty((S, D), np.float32)
    oracle().o_dense_ffn_q8(ptr(out), ptr(x), S, ptr(G), ptr(GS), ptr(U), ptr(US), ptr(Dn), ptr(DS), D, I)
    return out


def rng(seed):
    return np.random.default_rng(seed)


def randn(seed, shape, std=1.0):
    return (rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


# ---- R4 formats (Q4R4 / Q8R4) ----
def r4_sizes(O, I, q8):
    O4, nb = (O + 3) // 4, I // 32
    return O4 * nb * (128 if q8 else 64), O4 * nb * 4


def o_quant_g32(x):
    x = f32(x)
    S, I = x.shape
    xq = np.empty((S, I), np.int8)
    xs = np.empty((S, I // 32), np.float32)
    xm = np.empty((S, I // 32), np.int32)
    for t in range(S):
        oracle().o_quant_g32(C.c_void_p(x.ctypes.data + t * I * 4), I, C.c_void_p(xq.ctypes.data + t * I),
                             C.c_void_p(xs.ctypes.data + t * (I // 32) * 4), C.c_void_p(xm.ctypes.data + t * (I // 32) * 4))
    return xq, xs, xm


def o_pack_r4(w, q8=False):
    """(codes uint8/int8 flat, f16 scales uint16 flat) in the R4 layout."""
    w = f32(w)
    O, I = w.shape
    nq, nd = r4_sizes(O, I, q8)
    q = np.empty(nq, np.int8 if q8 else np.uint8)
    d = np.empty(nd, np.uint16)
    (oracle().o_pack_q8r4 if q8 else oracle().o_pack_q4r4)(ptr(w), O, I, ptr(q), ptr(d))
    return q, d


def o_matmul_r4(x, q, d, O, q8=False):
    x = f32(x)
    S, I = x.shape
    y = np.empty((S, O), np.float32)
    (oracle().o_matmul_q8r4 if q8 else oracle().o_matmul_q4r4)(ptr(y), ptr(x), ptr(q), ptr(d), S, I, O)
    return y


def ref_pack_r4(r, w, q8=False):
    """The reference's block packer over every 4-row block."""
    w = f32(w)
    O, I = w.shape
    nq, nd = r4_sizes(O, I, q8)
    q = np.empty(nq, np.int8 if q8 else np.uint8)
    d = np.empty(nd, np.uint16)
    nb, gb = I // 32, (128 if q8 else 64)
    fn = r.moty_pack_q8r4_block if q8 else r.moty_pack_q4r4_block
    for b in range((O + 3) // 4):
        fn(C.c_void_p(w.ctypes.data + b * 4 * I * 4), min(4, O - 4 * b), I,
           C.c_void_p(q.ctypes.data + b * nb * gb), C.c_void_p(d.ctypes.data + b * nb * 4 * 2))
    return q, d


def ref_matmul_r4(r, x, q, d, O, q8=False):
    x = f32(x)
    S, I = x.shape
    y = np.empty((S, O), np.float32)
    (r.moty_matmul_q8r4_s if q8 else r.moty_matmul_q4r4_s)(ptr(y), ptr(x), ptr(q), ptr(d), S, I, O)
    return y


# ---- GGUF block formats (io/gguf.h) ----
GG_Q8_0, GG_Q4_0, GG_Q4_K, GG_Q5_K, GG_Q6_K = 4, 5, 6, 7, 8
GG_BLOCK = {GG_Q8_0: (32, 34), GG_Q4_0: (32, 18), GG_Q4_K: (256, 144),
            GG_Q5_K: (256, 176), GG_Q6_K: (256, 210)}
# byte offsets of the f16 fields of each block type
GG_F16 = {GG_Q8_0: (0,), GG_Q4_0: (0,), GG_Q4_K: (0, 2), GG_Q5_K: (0, 2), GG_Q6_K: (208,)}


def gg_blocks(seed, dtype, nblk, finite=True):
    """Random blocks of one GGUF type; with finite=True the f16 scale fields
    hold finite halves in [2^-14, 2)*sign, so products stay finite."""
    E, B = GG_BLOCK[dtype]
    raw = rng(seed).integers(0, 256, size=(nblk, B), dtype=np.uint8)
    if finite:
        h = rng(seed + 1).integers(0x0400, 0x4000, size=(nblk, len(GG_F16[dtype])), dtype=np.uint16)
        h |= (rng(seed + 2).integers(0, 2, size=h.shape, dtype=np.uint16) << 15)
        for j, off in enumerate(GG_F16[dtype]):
            raw[:, off] = (h[:, j] & 0xFF).astype(np.uint8)
            raw[:, off + 1] = (h[:, j] >> 8).astype(np.uint8)
    return np.ascontiguousarray(raw.reshape(-1))


def o_gguf_dequant(dtype, raw, numel):
    out = np.empty(numel, np.float32)
    assert oracle().o_gguf_dequant(dtype, ptr(raw), numel, ptr(out)) == 0
    return out


def o_gguf_repack_q4_0(raw, O, I):
    q4 = np.empty(O * I // 2, np.uint8)
    qs = np.empty(O * I // 32, np.float32)
    oracle().o_gguf_repack_q4_0(ptr(raw), ptr(q4), ptr(qs), O, I)
    return q4, qs


def ref_gguf_dequant(r, dtype, raw, numel):
    out = np.empty(numel, np.float32)
    r.ref_gguf_dequant(dtype, ptr(raw), numel, ptr(out))
    return out


def ref_gguf_repack_q4_0(r, raw, O, I):
    q4 = np.empty(O * I // 2, np.uint8)
    qs = np.empty(O * I // 32, np.float32)
    r.ref_gguf_repack_q4_0(ptr(raw), ptr(q4), ptr(qs), O, I)
    return q4, qs


# ---- expert cache bookkeeping (runtime/moecache.c) ----
class OCacheState:
    def __init__(self, n, eids, heat, last, clock, hits, misses):
        self.n, self.eids, self.heat, self.last = n, eids, heat, last
        self.clock, self.hits, self.misses = clock, hits, misses

    def key(self):
        return (self.n, tuple(self.eids[:self.n]), tuple(self.heat), tuple(self.last), self.clock, self.hits,
                self.misses)


class OCache:
    """The oracle's restatement of ExpertCache; get/pin return (slot, loaded)."""

    def __init__(self, cap, n_experts):
        self.cap, self.E = max(cap, 1), n_experts
        self.p = oracle().o_ecache_new(cap, n_experts)

    def __del__(self):
        if getattr(self, "p", None):
            oracle().o_ecache_free(self.p)

    def get(self, eid):
        ld = C.c_int(0)
        s = oracle().o_ecache_get(self.p, eid, C.byref(ld))
        return s, bool(ld.value)

    def pin(self, eid):
        return oracle().o_ecache_pin(self.p, eid), True

    def route_bias(self, logits, bias):
        logits = f32(logits).copy()
        oracle().o_ecache_route_bias(self.p, ptr(logits), bias)
        return logits

    def state(self):
        n = C.c_int()
        eids = np.empty(self.cap, np.int32)
        heat = np.zeros(max(self.E, 1), np.uint32)
        last = np.zeros(max(self.E, 1), np.uint32)
        clock = C.c_uint32()
        hits, misses = C.c_longlong(), C.c_longlong()
        oracle().o_ecache_state(self.p, C.byref(n), ptr(eids), ptr(heat), ptr(last), C.byref(clock),
                                C.byref(hits), C.byref(misses))
        return OCacheState(n.value, eids.tolist(), heat[:self.E].tolist(), last[:self.E].tolist(), clock.value,
                           hits.value, misses.value)


class _RefSlot(C.Structure):
    _fields_ = [("eid", C.c_int), ("g", P), ("u", P), ("d", P), ("gs", P), ("us", P), ("ds", P)]


class _RefCache(C.Structure):
    _fields_ = [("slots", C.POINTER(_RefSlot)), ("n", C.c_int), ("cap", C.c_int), ("heat", C.POINTER(C.c_uint32)),
                ("last", C.POINTER(C.c_uint32)), ("pinned", C.POINTER(C.c_uint8)), ("n_experts", C.c_int),
                ("clock", C.c_uint32), ("hits", C.c_longlong), ("misses", C.c_longlong)]


REF_LOAD_FN = C.CFUNCTYPE(None, P, I32, I32, C.POINTER(_RefSlot), I32, I32)


class RefCache:
    """The reference's own ExpertCache (runtime/moecache.c compiled into
    oracle/_ref), driven with a loader that records each load."""

    def __init__(self, r, cap, n_experts, inter=4, hidden=4):
        self.r, self.E, self.I, self.D = r, n_experts, inter, hidden
        self.c = _RefCache()
        self.loads = []
        self.fn = REF_LOAD_FN(lambda ctx, layer, eid, slot, i, d: self.loads.append(eid))
        r.moty_expert_cache_init.argtypes = [C.POINTER(_RefCache), I32, I32]
        r.moty_expert_cache_init.restype = None
        for nm in ("moty_expert_get", "moty_expert_pin"):
            f = getattr(r, nm)
            f.argtypes = [C.POINTER(_RefCache), P, I32, I32, REF_LOAD_FN, I32, I32]
            f.restype = C.POINTER(_RefSlot)
        r.moty_moe_route_bias.argtypes = [P, C.POINTER(_RefCache), F32]
        r.moty_moe_route_bias.restype = None
        r.moty_expert_cache_free.argtypes = [C.POINTER(_RefCache)]
        r.moty_expert_cache_free.restype = None
        r.moty_expert_cache_init(C.byref(self.c), cap, n_experts)
        self.cap = self.c.cap

    def __del__(self):
        if getattr(self, "r", None):
            self.r.moty_expert_cache_free(C.byref(self.c))

    def _slot(self, sp):
        base = C.addressof(self.c.slots.contents)
        return (C.addressof(sp.contents) - base) // C.sizeof(_RefSlot)

    def get(self, eid):
        n0 = len(self.loads)
        sp = self.r.moty_expert_get(C.byref(self.c), None, 0, eid, self.fn, self.I, self.D)
        return self._slot(sp), len(self.loads) > n0

    def pin(self, eid):
        sp = self.r.moty_expert_pin(C.byref(self.c), None, 0, eid, self.fn, self.I, self.D)
        return self._slot(sp), True

    def route_bias(self, logits, bias):
        logits = f32(logits).copy()
        self.r.moty_moe_route_bias(ptr(logits), C.byref(self.c), bias)
        return logits

    def state(self):
        c = self.c
        eids = [c.slots[i].eid for i in range(self.cap)]
        heat = [c.heat[e] for e in range(self.E)] if self.E > 0 else []
        last = [c.last[e] for e in range(self.E)] if self.E > 0 else []
        return OCacheState(c.n, eids, heat, last, c.clock, c.hits, c.misses)


def fast_q8(seed, shape):
    """Int8 codes over the full range and positive f32 row scales, drawn
    directly (no f32 weights to quantize): workload-sized expert stacks in
    seconds.  Codes include -128, which weights may hold (the dot_i8i8
    contract restricts activations only, hw/hw.h)."""
    g = rng(seed)
    n = int(np.prod(shape))
    q = np.frombuffer(g.bytes(n), dtype=np.int8).reshape(shape).copy()
    s = g.uniform(1e-4, 3e-4, size=shape[:-1]).astype(np.float32)
    return q, s


def fast_moe_weights(E, I, D, seed=10):
    ex = {}
    ex["G"], ex["GS"] = fast_q8(seed, (E, I, D))
    ex["U"], ex["US"] = fast_q8(seed + 1, (E, I, D))
    ex["Dn"], ex["DS"] = fast_q8(seed + 2, (E, D, I))
    return ex


def skew_inputs(x, Wr, hot, lift=2.0):
    """The skewed continuous batch through the plain router: feature 0 of
    every token is 1 and the hot experts' router weight on it is `lift`, so
    their logits rise by `lift` (up to one rounding) -- the +2.0 logit bias
    of the skewed C5 variant, expressed in inputs every MoE entry point
    (the reference's moe_batch included) takes."""
    x = f32(x).copy()
    Wr = f32(Wr).copy()
    x[:, 0] = 1.0
    Wr[:, 0] = 0.0
    Wr[hot, 0] = lift
    return x, Wr
