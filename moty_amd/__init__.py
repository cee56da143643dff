"""moty_amd -- MI355X (gfx950) backend for moty's quantized-matmul and MoE
hot path.

The product is the C-ABI library libmoty_hw_hip.so (include/moty_hw_hip.h).
This package loads it with ctypes and offers thin torch-tensor wrappers named
after the reference's functions (moty_matmul_q_s -> matmul_q_s, ...).  There
is no CPU fallback: if the library is missing, `lib()` raises."""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoty_hw_hip.so")

OK, EINVAL, EHIP, ENOMEM, EUNSUP = 0, 1, 2, 3, 4
ORDER_TOPK, ORDER_EXPERT = 0, 1

P, I32, I64 = C.c_void_p, C.c_int, C.c_int64


class MotyHipMoe(C.Structure):
    _fields_ = [
        ("router", P), ("logit_bias", P),
        ("g", P), ("u", P), ("d", P),
        ("gs", P), ("us", P), ("ds", P),
        ("E", I32), ("K", I32), ("I", I32), ("D", I32),
        ("norm_topk", I32), ("combine_order", I32),
        ("idx_out", P), ("w_out", P), ("counts_out", P),
    ]


class MotyHipExpertSlot(C.Structure):
    _fields_ = [("eid", I32), ("g", P), ("u", P), ("d", P), ("gs", P), ("us", P), ("ds", P)]


# MotyHipLoadExpertFn(ctx, layer, eid, slot, inter, hidden)
LOAD_EXPERT_FN = C.CFUNCTYPE(None, P, I32, I32, C.POINTER(MotyHipExpertSlot), I32, I32)


# name -> (restype, argtypes): every symbol include/moty_hw_hip.h declares
SIGNATURES = {
    "moty_hip_init": (I32, [I32]),
    "moty_hip_shutdown": (I32, []),
    "moty_hip_last_error": (C.c_char_p, []),
    "moty_hip_kernel_tier": (C.c_char_p, []),
    "moty_hip_wait_errors": (I32, [C.POINTER(I32)]),
    "moty_hip_set_ffn1": (I32, [I32]),
    "moty_hip_matmul_q_s": (I32, [P, P, P, P, I32, I32, I32]),
    "moty_hip_matmul_i4_grouped_s": (I32, [P, P, P, P, I32, I32, I32, I32]),
    "moty_hip_matmul_q4r4_s": (I32, [P, P, P, P, I32, I32, I32]),
    "moty_hip_matmul_q8r4_s": (I32, [P, P, P, P, I32, I32, I32]),
    "moty_hip_matmul_q4r4_s_dev": (I32, [P, P, P, P, I32, I32, I32, P]),
    "moty_hip_matmul_q8r4_s_dev": (I32, [P, P, P, P, I32, I32, I32, P]),
    "moty_hip_quant_g32_dev": (I32, [P, P, P, P, I32, I32, P]),
    "moty_hip_gate_up_silu_q4r4_dev": (I32, [P, P, P, P, I32, I32, P]),
    "moty_hip_gate_up_silu_q8r4_dev": (I32, [P, P, P, P, I32, I32, P]),
    "moty_hip_dense_ffn_q4r4_dev": (I32, [P, P, I32, P, P, P, P, I32, I32, P]),
    "moty_hip_dense_ffn_q8r4_dev": (I32, [P, P, I32, P, P, P, P, I32, I32, P]),
    "moty_hip_pack_q4r4_dev": (I32, [P, P, P, I32, I32, P]),
    "moty_hip_pack_q8r4_dev": (I32, [P, P, P, I32, I32, P]),
    "moty_hip_gguf_dequant": (I32, [I32, P, I64, P]),
    "moty_hip_gguf_repack_q4_0": (I32, [P, P, P, I64, I64]),
    "moty_hip_gguf_dequant_dev": (I32, [I32, P, I64, P, P]),
    "moty_hip_gguf_repack_q4_0_dev": (I32, [P, P, P, I64, I64, P]),
    "moty_hip_expert_cache_init": (I32, [C.POINTER(P), I32, I32]),
    "moty_hip_expert_cache_free": (I32, [P]),
    "moty_hip_expert_get": (I32, [P, P, I32, I32, LOAD_EXPERT_FN, I32, I32, C.POINTER(C.POINTER(MotyHipExpertSlot))]),
    "moty_hip_expert_pin": (I32, [P, P, I32, I32, LOAD_EXPERT_FN, I32, I32, C.POINTER(C.POINTER(MotyHipExpertSlot))]),
    "moty_hip_expert_cache_stats": (I32, [P, P, P, P, P, P, P, P]),
    "moty_hip_moe_route_bias": (None, [P, P, C.c_float]),
    "moty_hip_moe_topk_cached": (I32, [C.POINTER(MotyHipMoe), P, P, I32, LOAD_EXPERT_FN, P, I32, P]),
    "moty_hip_moe_topk_cached_dev": (I32, [C.POINTER(MotyHipMoe), P, P, I32, LOAD_EXPERT_FN, P, I32, P, P]),
    "moty_hip_matmul": (I32, [P, P, P, I32, I32, I32]),
    "moty_hip_moe_topk": (I32, [C.POINTER(MotyHipMoe), P, I32, P]),
    "moty_hip_weight_forget": (I32, [P]),
    "moty_hip_hw_matmul_i8": (None, [P, P, P, P, I32, I32, I32]),
    "moty_hip_matmul_i4_s": (I32, [P, P, P, P, I32, I32, I32]),
    "moty_hip_hw_matmul_i4": (None, [P, P, P, P, I32, I32, I32]),
    "moty_hip_pack_int4_dev": (I32, [P, P, P, I32, I32, P]),
    "moty_hip_matmul_i4_s_dev": (I32, [P, P, P, P, I32, I32, I32, I32, P]),
    "moty_hip_qrow_i8_dev": (I32, [P, P, P, P, I32, I32, P]),
    "moty_hip_qrow_i8_multi_dev": (I32, [I32, P, P, P, P, P, P]),
    "moty_hip_quantize_rows_dev": (I32, [P, P, P, I32, I32, I32, P]),
    "moty_hip_pack_int4_grouped_dev": (I32, [P, P, P, I32, I32, I32, P]),
    "moty_hip_matmul_q_s_dev": (I32, [P, P, P, P, I32, I32, I32, P]),
    "moty_hip_matmul_q8_preq_dev": (I32, [P, P, P, P, P, I32, I32, I32, P]),
    "moty_hip_matmul_i4_grouped_s_dev": (I32, [P, P, P, P, I32, I32, I32, I32, I32, P]),
    "moty_hip_matmul_dev": (I32, [P, P, P, I32, I32, I32, P]),
    "moty_hip_silu_mul_dev": (I32, [P, P, I64, P]),
    "moty_hip_softmax_rows_dev": (I32, [P, I32, I32, P]),
    "moty_hip_expf_dev": (I32, [P, P, I64, P]),
    "moty_hip_gate_up_silu_q8_dev": (I32, [P, P, I32, P, P, P, P, I32, I32, P]),
    "moty_hip_gate_up_silu_i4g_dev": (I32, [P, P, P, P, P, P, I32, I32, P]),
    "moty_hip_dense_ffn_q8_dev": (I32, [P, P, I32, P, P, P, P, P, P, I32, I32, P]),
    "moty_hip_dense_ffn_i4g_dev": (I32, [P, P, I32, P, P, P, P, P, P, I32, I32, I32, P]),
    "moty_hip_moe_topk_dev": (I32, [C.POINTER(MotyHipMoe), P, I32, P, P]),
    "moty_hip_moe_topk_noalloc_dev": (I32, [C.POINTER(MotyHipMoe), P, I32, P, P]),
}

_lib = None


class MotyHipError(RuntimeError):
    pass


def lib():
    """The loaded C-ABI library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MotyHipError("libmoty_hw_hip.so is not built: run __graft_entry__.build() "
                               "or python -m moty_amd.build")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc, what=""):
    if rc != OK:
        msg = lib().moty_hip_last_error().decode(errors="replace")
        raise MotyHipError("%s failed (code %d): %s" % (what, rc, msg))


from . import ops  # noqa: E402,F401
