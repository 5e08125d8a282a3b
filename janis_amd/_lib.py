"""ctypes binding of libjanis_hip.so (the C ABI in include/janis_hip.h).

The library is the product: there is no CPU fallback. Loading fails loudly when
the shared object has not been built (python -m janis_amd.build).
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libjanis_hip.so")

# engine.DType (engine/backend.go:11-21)
F32, F16, BF16, I32, U32, U8 = range(6)
JH_OK, JH_ERR_INVALID, JH_ERR_UNSUPPORTED, JH_ERR_HIP, JH_ERR_OOM, JH_ERR_NONFINITE, JH_ERR_TIMEOUT = range(7)
JH_CHECK_INDICES, JH_CHECK_VALUES = 1, 2  # jh_set_checks flags
JH_SCALAR_MUL, JH_SCALAR_ADD = 0, 1  # jh_scalar_op
JH_OP_ADD, JH_OP_MUL, JH_OP_SILU, JH_OP_SILU_MUL = range(4)  # jh_op
JH_PRO_NONE, JH_PRO_RMSNORM, JH_PRO_SILU_MUL, JH_PRO_NORMED = range(4)  # jh_prologue
JH_EPI_STORE, JH_EPI_RESID, JH_EPI_SWIGLU, JH_EPI_RESID_NORM = range(4)  # jh_epilogue
JH_NORM_STATS = 1024

EXPORTS = [
    "jh_version", "jh_create", "jh_destroy", "jh_last_error", "jh_device_info",
    "jh_set_stream", "jh_get_stream", "jh_set_checks", "jh_sync", "jh_alloc", "jh_free",
    "jh_h2d", "jh_d2h", "jh_dequantize", "jh_quant_matmul", "jh_gather_quant_matmul",
    "jh_moe_route", "jh_moe_swiglu", "jh_rms_norm", "jh_rope", "jh_sdpa", "jh_elementwise", "jh_argmax",
    "jh_take_rows", "jh_kv_append", "jh_qk_norm_rope_append", "jh_quant_matvec_fused",
    "jh_attention_decode", "jh_rope_table", "jh_norm_prepare", "jh_copy_strided", "jh_scatter_rows",
    "jh_softmax", "jh_mean", "jh_scalar", "jh_check_finite", "jh_attention_decode_noalloc",
    "jh_qkv_attention_decode", "jh_embed_norm_prepare", "jh_set_wait_limit",
]

_lib = None


class JanisHipError(RuntimeError):
    """A non-zero status from the C ABI (the reference backends panic here)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m janis_amd.build` "
                           "(there is no CPU fallback for this backend)")
    L = ctypes.CDLL(LIB_PATH)
    c_ctx = ctypes.c_void_p
    p = ctypes.c_void_p
    i64 = ctypes.c_int64
    i = ctypes.c_int
    L.jh_version.restype = ctypes.c_char_p
    L.jh_version.argtypes = []
    L.jh_create.argtypes = [i, ctypes.POINTER(c_ctx)]
    L.jh_create.restype = i
    L.jh_destroy.argtypes = [c_ctx]
    L.jh_destroy.restype = None
    L.jh_last_error.argtypes = [c_ctx]
    L.jh_last_error.restype = ctypes.c_char_p
    L.jh_device_info.argtypes = [c_ctx, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(i)]
    L.jh_device_info.restype = i
    L.jh_set_stream.argtypes = [c_ctx, p]
    L.jh_set_stream.restype = i
    L.jh_get_stream.argtypes = [c_ctx]
    L.jh_get_stream.restype = p
    L.jh_set_checks.argtypes = [c_ctx, i]
    L.jh_set_checks.restype = i
    L.jh_set_wait_limit.argtypes = [c_ctx, ctypes.c_int64]
    L.jh_set_wait_limit.restype = i
    L.jh_sync.argtypes = [c_ctx]
    L.jh_sync.restype = i
    L.jh_alloc.argtypes = [c_ctx, ctypes.c_size_t, ctypes.POINTER(p)]
    L.jh_alloc.restype = i
    L.jh_free.argtypes = [c_ctx, p]
    L.jh_free.restype = i
    L.jh_h2d.argtypes = [c_ctx, p, p, ctypes.c_size_t]
    L.jh_h2d.restype = i
    L.jh_d2h.argtypes = [c_ctx, p, p, ctypes.c_size_t]
    L.jh_d2h.restype = i
    L.jh_dequantize.argtypes = [c_ctx, p, p, p, i, i64, i64, i, i, p, i]
    L.jh_dequantize.restype = i
    L.jh_quant_matmul.argtypes = [c_ctx, p, i, i64, p, p, p, i, i64, i64, i, i, i, p, i]
    L.jh_quant_matmul.restype = i
    L.jh_gather_quant_matmul.argtypes = [c_ctx, p, i, i64, i64, p, p, p, i, i64, i64, i64, p,
                                         i64, i, i, i, p, i]
    L.jh_gather_quant_matmul.restype = i
    f32 = ctypes.c_float
    L.jh_rms_norm.argtypes = [c_ctx, p, i, i64, i64, p, i, f32, p, i]
    L.jh_rope.argtypes = [c_ctx, p, i, i64, i64, i64, i, i, f32, f32, i64, p, p, i]
    L.jh_sdpa.argtypes = [c_ctx, p, i, p, p, i, i64, i64, i64, i64, i64, i64, i64, f32, i, p, i]
    L.jh_elementwise.argtypes = [c_ctx, i, p, i, p, i, i64, p, i]
    L.jh_argmax.argtypes = [c_ctx, p, i, i64, i64, p]
    L.jh_take_rows.argtypes = [c_ctx, p, i64, i64, p, i64, p]
    L.jh_kv_append.argtypes = [c_ctx, p, p, i, i64, i64, i64, p, p, i, i64, i64]
    L.jh_qk_norm_rope_append.argtypes = [c_ctx, p, i, i64, i64, i64, p, p, i, f32, f32, f32, i64, p, p, i, i64, p, i]
    L.jh_attention_decode.argtypes = [c_ctx, p, i, i64, i64, i64, p, p, i, f32, f32, f32, p, i64, p, p, i, i64,
                                      f32, p, i]
    L.jh_attention_decode_noalloc.argtypes = L.jh_attention_decode.argtypes
    L.jh_attention_decode_noalloc.restype = i
    L.jh_qkv_attention_decode.argtypes = [c_ctx, p, p, f32, p, p, p, i, i64, i, i, p, i, i64, i64, i64, p, p, i, f32,
                                          f32, f32, p, i64, p, p, i, i64, f32, p, i]
    L.jh_qkv_attention_decode.restype = i
    L.jh_rope_table.argtypes = [c_ctx, i, f32, f32, i64, p, p]
    L.jh_embed_norm_prepare.argtypes = [c_ctx, p, p, p, p, i, i64, i64, i, i, p, i, p, p, p, i, f32, f32, i64, p]
    L.jh_embed_norm_prepare.restype = i
    L.jh_quant_matvec_fused.argtypes = [c_ctx, i, p, i, p, i, f32, p, p, p, i, i64, i64, i, i, i, p, p, i, p, p]
    L.jh_norm_prepare.argtypes = [c_ctx, p, i, i64, p, i, p, p]
    L.jh_copy_strided.argtypes = [c_ctx, p, i, i, p, p, p, i, p]
    L.jh_scatter_rows.argtypes = [c_ctx, p, p, i64, i64, p, i64, p]
    for name in ("jh_rms_norm", "jh_rope", "jh_sdpa", "jh_elementwise", "jh_argmax", "jh_take_rows", "jh_kv_append",
                 "jh_qk_norm_rope_append", "jh_quant_matvec_fused", "jh_attention_decode", "jh_rope_table",
                 "jh_norm_prepare", "jh_copy_strided", "jh_scatter_rows"):
        getattr(L, name).restype = i
    L.jh_softmax.argtypes = [c_ctx, p, i, i64, i64, i64, p]
    L.jh_mean.argtypes = [c_ctx, p, i, i64, i64, i64, p]
    L.jh_scalar.argtypes = [c_ctx, i, p, i, i64, f32, p, i]
    L.jh_check_finite.argtypes = [c_ctx, p, i, i64, ctypes.POINTER(i64), ctypes.POINTER(i64)]
    for name in ("jh_softmax", "jh_mean", "jh_scalar", "jh_check_finite"):
        getattr(L, name).restype = i
    L.jh_moe_route.argtypes = [c_ctx, p, i, i64, i64, i64, i, p, p]
    L.jh_moe_route.restype = i
    L.jh_moe_swiglu.argtypes = [c_ctx, p, i, i64, p, p, p, p, p, p, p, p, p, i, i64, i64, i64,
                                p, p, i64, i, i, p, i]
    L.jh_moe_swiglu.restype = i
    _lib = L
    return L


def check(ctx, rc: int) -> None:
    if rc != JH_OK:
        msg = load().jh_last_error(ctx)
        raise JanisHipError(rc, msg.decode() if msg else "")
