"""ctypes binding of libalveare_q4.so (the C ABI in include/alveare_q4.h).

The library is loaded lazily and must exist: there is no CPU fallback. A
missing or unloadable library raises ``LibraryNotBuilt`` naming the build
command.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libalveare_q4.so")

ALV_OK = 0
ALV_ERR_ARG = -1
ALV_ERR_ALIGN = -2
ALV_ERR_HANDLE = -3
ALV_ERR_HIP = -4
ALV_ERR_RANGE = -5
ALV_ACT_GELU_TANH = 0
ALV_ACT_SILU = 1

# Every symbol include/alveare_q4.h declares: name -> (restype, argtypes).
_vp = ctypes.c_void_p
_i = ctypes.c_int
SIGNATURES: dict[str, tuple] = {
    "alv_last_error": (ctypes.c_char_p, []),
    "alv_version": (ctypes.c_char_p, []),
    "alv_gemv_q": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "alv_gemm_q": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "alv_ffn_register": (_i, [_vp, _vp, _vp, _i, _i, _i, ctypes.POINTER(_vp), _vp]),
    "alv_ffn_fused": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "alv_ffn_fused_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "alv_ffn_activation": (_i, [_vp, _vp, _i, _vp]),
    "alv_ffn_gate_up": (_i, [_vp, _vp, _i, _i, _vp]),
    "alv_ffn_partials": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "alv_ffn_shape": (_i, [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "alv_ffn_exec_shape": (_i, [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "alv_ffn_release": (None, [_vp]),
    "alv_dequant_q4": (_i, [_vp, _vp, _i, _i, _vp]),
    "alv_weight_register": (_i, [_vp, _i, _i, ctypes.POINTER(_vp), _vp]),
    "alv_weight_shape": (_i, [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "alv_weight_exec_shape": (_i, [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "alv_gemv": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "alv_weight_release": (None, [_vp]),
    "alv_lm_head": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _vp, _vp]),
    "alv_lm_head_bf16": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _vp, _vp, _i, _vp]),
    "alv_lm_head_bf16_addnorm": (_i, [_vp, _vp, _vp, _vp, _i, ctypes.c_float, _i, _vp, _vp, ctypes.c_float, _i, _vp,
                                      _i, ctypes.c_float, _vp, _vp, _i, _vp]),
    "alv_quantize_q4": (_i, [_vp, _i, _i, _i, _vp, _i, _i, _vp]),
    "alv_gemv_bf16": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "alv_ffn_fused_bf16": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "alv_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float, _vp]),
    "alv_qkv_post": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _i, ctypes.c_float, _vp, _i, _i, _i, _i,
                          _vp, _i, _vp, _vp, _vp, _vp]),
    "alv_attention": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float, _vp, _vp]),
    "alv_qkv_attention": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _i, ctypes.c_float, _vp, _i, _i, _i, _i,
                               _vp, _i, _vp, _vp, _vp, _i, ctypes.c_float, _vp, _vp]),
    "alv_embed": (_i, [_vp, _i, _i, _vp, ctypes.c_double, _vp, _vp]),
    "alv_add_norm": (_i, [_vp, _i, _vp, _i, _vp, _i, ctypes.c_float, _i, _vp, _i, _vp, _vp, _i, _i, _i, _i,
                          ctypes.c_float, _vp]),
    "alv_gemv_bf16_addnorm": (_i, [_vp, _vp, _vp, _vp, _i, ctypes.c_float, _i, _vp, _vp, ctypes.c_float, _vp, _vp]),
    "alv_ffn_fused_bf16_addnorm": (_i, [_vp, _vp, _vp, _vp, _i, ctypes.c_float, _i, _vp, _vp, ctypes.c_float, _vp,
                                        _vp]),
    "alv_weight_quantize": (_i, [_vp, _i, _i, _i, _i, _i, ctypes.POINTER(_vp), _vp]),
    "alv_q4_tiled_bytes": (ctypes.c_uint64, [_i, _i]),
    "alv_q4_tile": (_i, [_vp, _vp, _i, _i, _vp]),
    "alv_chain_run": (_i, [_vp, _i, _i, _vp]),
    "alv_glu": (_i, [_vp, _vp, _vp, ctypes.c_int64, _i, _vp]),
}


class ChainOp(ctypes.Structure):
    """alv_chain_op (include/alveare_q4.h)."""

    _fields_ = [("weight", ctypes.c_void_p), ("ffn", ctypes.c_void_p), ("x", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("dep", ctypes.c_int)]


class LibraryNotBuilt(RuntimeError):
    pass


class Q4Error(RuntimeError):
    """A non-zero status from the C ABI; ``code`` is the ALV_ERR_* value."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{message} (status {code})")
        self.code = code


class Q4ValueError(Q4Error, ValueError):
    pass


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryNotBuilt(
                    f"{LIB_PATH} is missing; build it with `python -m alveare_amd.build` "
                    "(hipcc, gfx950). There is no CPU fallback.")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc == ALV_OK:
        return
    msg = lib().alv_last_error().decode(errors="replace")
    cls = Q4ValueError if rc in (ALV_ERR_ARG, ALV_ERR_ALIGN, ALV_ERR_RANGE, ALV_ERR_HANDLE) else Q4Error
    raise cls(rc, f"{what}: {msg}")
