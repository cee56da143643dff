"""torch-tensor wrappers over the device entry points of libmoty_hw_hip.

Each function mirrors one reference function (same name without the moty_
prefix, same argument meaning); tensors must live on the GPU, outputs are
allocated here, and work is queued on torch's current stream."""
import ctypes as C

import torch

from . import MotyHipMoe, ORDER_EXPERT, check, lib


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(*ts):
    for t in ts:
        if t is not None and (not t.is_cuda or not t.is_contiguous()):
            raise ValueError("expected contiguous GPU tensors")


def qrow_i8(x, group_sums=False):
    """hw/hw_quant.h:9-16 over every row: returns (q int8 [S,I], sx [S], xg)."""
    _dev(x)
    S, I = x.shape
    q = torch.empty((S, I), dtype=torch.int8, device=x.device)
    sx = torch.empty(S, dtype=torch.float32, device=x.device)
    xg = torch.empty((S, I // 32), dtype=torch.int32, device=x.device) if group_sums else None
    check(lib().moty_hip_qrow_i8_dev(_p(x), _p(q), _p(sx), _p(xg), S, I, _stream()), "qrow_i8")
    return q, sx, xg


def qrow_i8_multi(xs):
    """qrow_i8 of up to four row sets in one launch: returns [(q, sx), ...]."""
    _dev(*xs)
    n = len(xs)
    outs = [(torch.empty(x.shape, dtype=torch.int8, device=x.device),
             torch.empty(x.shape[0], dtype=torch.float32, device=x.device)) for x in xs]
    arr = lambda vals: (C.c_void_p * n)(*vals)
    check(lib().moty_hip_qrow_i8_multi_dev(n, arr([x.data_ptr() for x in xs]), arr([q.data_ptr() for q, _ in outs]),
                                           arr([s.data_ptr() for _, s in outs]), (C.c_int * n)(*[x.shape[0] for x in xs]),
                                           (C.c_int * n)(*[x.shape[1] for x in xs]), _stream()), "qrow_i8_multi")
    return outs


def quantize_rows(w, bits=8):
    """nn/quant.c:12-33: (q int8 [O,I], scale [O])."""
    _dev(w)
    O, I = w.shape
    q = torch.empty((O, I), dtype=torch.int8, device=w.device)
    s = torch.empty(O, dtype=torch.float32, device=w.device)
    check(lib().moty_hip_quantize_rows_dev(_p(w), _p(q), _p(s), O, I, bits, _stream()), "quantize_rows")
    return q, s


def pack_int4_grouped(w, gs=32):
    """nn/quant.c:57-83: (q4 uint8 [O,(I+1)/2], scale [O, ceil(I/gs)])."""
    _dev(w)
    O, I = w.shape
    q4 = torch.empty((O, (I + 1) // 2), dtype=torch.uint8, device=w.device)
    s = torch.empty((O, (I + gs - 1) // gs), dtype=torch.float32, device=w.device)
    check(lib().moty_hip_pack_int4_grouped_dev(_p(w), _p(q4), _p(s), O, I, gs, _stream()), "pack_int4_grouped")
    return q4, s


def matmul_q_s(x, q, scale, out=None):
    """nn/matmul.c:51-66: y [S,O] = Q8 matmul of x [S,I]."""
    _dev(x, q, scale)
    S, I = x.shape
    O = q.shape[0]
    y = out if out is not None else torch.empty((S, O), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_matmul_q_s_dev(_p(y), _p(x), _p(q), _p(scale), S, I, O, _stream()), "matmul_q_s")
    return y


def matmul_q8_preq(xq, sx, q, scale, out=None):
    _dev(xq, sx, q, scale)
    S, I = xq.shape
    O = q.shape[0]
    y = out if out is not None else torch.empty((S, O), dtype=torch.float32, device=xq.device)
    check(lib().moty_hip_matmul_q8_preq_dev(_p(y), _p(xq), _p(sx), _p(q), _p(scale), S, I, O, _stream()),
          "matmul_q8_preq")
    return y


def pack_int4(w):
    """nn/quant.c:34-55: per-row int4 (q4 uint8 [O,(I+1)/2], scale [O])."""
    _dev(w)
    O, I = w.shape
    q4 = torch.empty((O, (I + 1) // 2), dtype=torch.uint8, device=w.device)
    s = torch.empty(O, dtype=torch.float32, device=w.device)
    check(lib().moty_hip_pack_int4_dev(_p(w), _p(q4), _p(s), O, I, _stream()), "pack_int4")
    return q4, s


def matmul_i4_s(x, q4, scale, idot4=True, out=None):
    """nn/matmul.c:75-145, per-row int4 weights."""
    _dev(x, q4, scale)
    S, I = x.shape
    O = q4.shape[0]
    y = out if out is not None else torch.empty((S, O), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_matmul_i4_s_dev(_p(y), _p(x), _p(q4), _p(scale), S, I, O, int(bool(idot4)), _stream()),
          "matmul_i4_s")
    return y


def matmul_i4_grouped_s(x, q4, scale, gs=32, idot4=True, out=None):
    """nn/matmul.c:164-197 (idot4 picks the IDOT4=1 branch)."""
    _dev(x, q4, scale)
    S, I = x.shape
    O = q4.shape[0]
    y = out if out is not None else torch.empty((S, O), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_matmul_i4_grouped_s_dev(_p(y), _p(x), _p(q4), _p(scale), S, I, O, gs, int(bool(idot4)),
                                                 _stream()), "matmul_i4_grouped_s")
    return y


def r4_sizes(O, I, q8=False):
    """Bytes of codes and number of f16 scales of an O x I R4 matrix."""
    blocks = (O + 3) // 4 * (I // 32)
    return blocks * (128 if q8 else 64), blocks * 4


def pack_r4(w, q8=False):
    """nn/quant.c:135-177 over every 4-row block of w [O, I] (f32): returns
    (codes uint8 (Q4R4) / int8 (Q8R4) flat, f16 scales as int16 flat)."""
    _dev(w)
    O, I = w.shape
    nq, nd = r4_sizes(O, I, q8)
    q = torch.empty(nq, dtype=torch.int8 if q8 else torch.uint8, device=w.device)
    d = torch.empty(nd, dtype=torch.int16, device=w.device)
    fn = lib().moty_hip_pack_q8r4_dev if q8 else lib().moty_hip_pack_q4r4_dev
    check(fn(_p(w), _p(q), _p(d), O, I, _stream()), "pack_r4")
    return q, d


def quant_g32(x):
    """hw/hw_q4r4.h:36-46 over every row: (xq int8 [S, I], xs [S, I/32], xsum int32 [S, I/32])."""
    _dev(x)
    S, I = x.shape
    xq = torch.empty((S, I), dtype=torch.int8, device=x.device)
    xs = torch.empty((S, I // 32), dtype=torch.float32, device=x.device)
    xm = torch.empty((S, I // 32), dtype=torch.int32, device=x.device)
    check(lib().moty_hip_quant_g32_dev(_p(x), _p(xq), _p(xs), _p(xm), S, I, _stream()), "quant_g32")
    return xq, xs, xm


GGUF_BLOCK = {4: (32, 34), 5: (32, 18), 6: (256, 144), 7: (256, 176), 8: (256, 210)}


def gguf_dequant(dtype, raw, numel, out=None):
    """io/gguf.h:316-326 (gguf_dequant): `numel` elements of GGUF block type
    `dtype` (4 Q8_0, 5 Q4_0, 6 Q4_K, 7 Q5_K, 8 Q6_K) from the raw uint8 block
    bytes to f32."""
    _dev(raw)
    E, B = GGUF_BLOCK.get(dtype, (0, 0))
    if E and (numel % E or raw.numel() < numel // E * B):
        raise ValueError("gguf_dequant: raw holds fewer than numel/%d blocks of %d bytes" % (E, B))
    y = out if out is not None else torch.empty(numel, dtype=torch.float32, device=raw.device)
    check(lib().moty_hip_gguf_dequant_dev(dtype, _p(raw), numel, _p(y), _stream()), "gguf_dequant")
    return y


def gguf_repack_q4_0(blocks, O, I):
    """io/gguf.h:340-357: Q4_0 blocks of an [O, I] matrix -> (q4 uint8 [O, I/2],
    scales f32 [O, I/32]), the grouped int4 layout with gs = 32."""
    _dev(blocks)
    if I % 32 or blocks.numel() < O * (I // 32) * 18:
        raise ValueError("gguf_repack_q4_0: needs I %% 32 == 0 and O*I/32 blocks of 18 bytes")
    q4 = torch.empty((O, I // 2), dtype=torch.uint8, device=blocks.device)
    qs = torch.empty((O, I // 32), dtype=torch.float32, device=blocks.device)
    check(lib().moty_hip_gguf_repack_q4_0_dev(_p(blocks), _p(q4), _p(qs), O, I, _stream()), "gguf_repack_q4_0")
    return q4, qs


def matmul_r4(x, q, d, O, q8=False, out=None):
    """moty_matmul_q4r4_s / moty_matmul_q8r4_s (nn/matmul.c:395-466): y [S, O]."""
    _dev(x, q, d)
    S, I = x.shape
    y = out if out is not None else torch.empty((S, O), dtype=torch.float32, device=x.device)
    fn = lib().moty_hip_matmul_q8r4_s_dev if q8 else lib().moty_hip_matmul_q4r4_s_dev
    check(fn(_p(y), _p(x), _p(q), _p(d), S, I, O, _stream()), "matmul_r4")
    return y


def gate_up_silu_r4(x, gu, gus, I, q8=False, out=None):
    """Decode gate/up + SiLU over a row-fused [gate; up] R4 matrix: h [1, I]."""
    _dev(x, gu, gus)
    S, D = x.shape
    h = out if out is not None else torch.empty((1, I), dtype=torch.float32, device=x.device)
    fn = lib().moty_hip_gate_up_silu_q8r4_dev if q8 else lib().moty_hip_gate_up_silu_q4r4_dev
    check(fn(_p(h), _p(x), _p(gu), _p(gus), D, I, _stream()), "gate_up_silu_r4")
    return h


def dense_ffn_r4(x, gu, gus, dn, dns, I, q8=False, out=None):
    """nn/ffn.c:26-41 with a row-fused R4 gate_up [2I, D] and down [D, I]."""
    _dev(x, gu, gus, dn, dns)
    S, D = x.shape
    y = out if out is not None else torch.empty((S, D), dtype=torch.float32, device=x.device)
    fn = lib().moty_hip_dense_ffn_q8r4_dev if q8 else lib().moty_hip_dense_ffn_q4r4_dev
    check(fn(_p(y), _p(x), S, _p(gu), _p(gus), _p(dn), _p(dns), D, I, _stream()), "dense_ffn_r4")
    return y


def matmul(x, W, out=None):
    """nn/matmul.c:15-27 (f32, dot_f32 AVX512 order)."""
    _dev(x, W)
    S, I = x.shape
    O = W.shape[0]
    y = out if out is not None else torch.empty((S, O), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_matmul_dev(_p(y), _p(x), _p(W), S, I, O, _stream()), "matmul")
    return y


def silu_mul(g, u):
    """hw/hw_ops.h:19-21, in place on g."""
    _dev(g, u)
    check(lib().moty_hip_silu_mul_dev(_p(g), _p(u), g.numel(), _stream()), "silu_mul")
    return g


def softmax_rows(x):
    """nn/norm.c:10 per row, in place."""
    _dev(x)
    S, n = x.shape
    check(lib().moty_hip_softmax_rows_dev(_p(x), S, n, _stream()), "softmax_rows")
    return x


def expf(x):
    _dev(x)
    y = torch.empty_like(x)
    check(lib().moty_hip_expf_dev(_p(x), _p(y), x.numel(), _stream()), "expf")
    return y


def dense_ffn_q8(x, gate, gs, up, us, down, ds, out=None):
    """nn/ffn.c:26-55 over Q8 weights."""
    _dev(x, gate, gs, up, us, down, ds)
    S, D = x.shape
    I = gate.shape[0]
    y = out if out is not None else torch.empty((S, D), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_dense_ffn_q8_dev(_p(y), _p(x), S, _p(gate), _p(gs), _p(up), _p(us), _p(down), _p(ds),
                                          D, I, _stream()), "dense_ffn_q8")
    return y


def dense_ffn_i4g(x, gate, gs, up, us, down, ds, idot4=True, out=None):
    """nn/ffn.c:26-55 over grouped-int4 weights (gs = 32)."""
    _dev(x, gate, gs, up, us, down, ds)
    S, D = x.shape
    I = gate.shape[0]
    y = out if out is not None else torch.empty((S, D), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_dense_ffn_i4g_dev(_p(y), _p(x), S, _p(gate), _p(gs), _p(up), _p(us), _p(down), _p(ds),
                                           D, I, int(bool(idot4)), _stream()), "dense_ffn_i4g")
    return y


def gate_up_silu_q8(x, gate, gs, up, us, out=None):
    """nn/ffn.c:28-37 for decode: h = silu(x.gate^T) * (x.up^T), one pass."""
    _dev(x, gate, gs, up, us)
    S, D = x.shape
    I = gate.shape[0]
    h = out if out is not None else torch.empty((S, I), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_gate_up_silu_q8_dev(_p(h), _p(x), S, _p(gate), _p(gs), _p(up), _p(us), D, I, _stream()),
          "gate_up_silu_q8")
    return h


def gate_up_silu_i4g(x, gate, gs, up, us, out=None):
    """Decode gate+up+SiLU over grouped-int4 weights (IDOT4), one token."""
    _dev(x, gate, gs, up, us)
    D = x.shape[-1]
    I = gate.shape[0]
    h = out if out is not None else torch.empty((1, I), dtype=torch.float32, device=x.device)
    check(lib().moty_hip_gate_up_silu_i4g_dev(_p(h), _p(x), _p(gate), _p(gs), _p(up), _p(us), D, I, _stream()),
          "gate_up_silu_i4g")
    return h


class MoeLayer:
    """Device-resident MoE layer (MotyMoeView analogue, nn/moe.h:19-33)."""

    def __init__(self, router, g, gs, u, us, d, ds, K, norm_topk=1, order=ORDER_EXPERT, logit_bias=None):
        _dev(router, g, gs, u, us, d, ds, logit_bias)
        self.keep = (router, g, gs, u, us, d, ds, logit_bias)
        E, I, D = g.shape
        self.E, self.I, self.D, self.K = E, I, D, K
        self.view = MotyHipMoe(router=router.data_ptr(), logit_bias=None if logit_bias is None else logit_bias.data_ptr(),
                               g=g.data_ptr(), u=u.data_ptr(), d=d.data_ptr(),
                               gs=gs.data_ptr(), us=us.data_ptr(), ds=ds.data_ptr(),
                               E=E, K=K, I=I, D=D, norm_topk=norm_topk, combine_order=order)

    def __call__(self, x, out=None, want_routing=False):
        _dev(x)
        S = x.shape[0]
        y = out if out is not None else torch.empty((S, self.D), dtype=torch.float32, device=x.device)
        v = MotyHipMoe.from_buffer_copy(self.view)
        idx = w = cnt = None
        if want_routing:
            idx = torch.empty((S, self.K), dtype=torch.int32, device=x.device)
            w = torch.empty((S, self.K), dtype=torch.float32, device=x.device)
            cnt = torch.empty(self.E, dtype=torch.int32, device=x.device)
            v.idx_out, v.w_out, v.counts_out = idx.data_ptr(), w.data_ptr(), cnt.data_ptr()
        check(lib().moty_hip_moe_topk_dev(C.byref(v), _p(x), S, _p(y), _stream()), "moe_topk")
        if want_routing:
            return y, idx, w, cnt
        return y


def wait_errors():
    """Calls since the last query whose bounded device wait ran out (the
    one-launch decode FFN); 0 means every output since then is valid."""
    n = C.c_int(0)
    check(lib().moty_hip_wait_errors(C.byref(n)), "wait_errors")
    return n.value


def set_ffn1(on):
    """Route the S = 1 Q8 dense FFN through its one-launch form (on) or the
    two GEMV launches (off); the results are the same bits."""
    check(lib().moty_hip_set_ffn1(int(bool(on))), "set_ffn1")
