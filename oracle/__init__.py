"""CPU oracle for the Q4 decode path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``liboracle_q4.so`` (a plain-C restatement of the
reference's fp32 CPU path, ``tools/ref/gemv_q.py:4-80`` and
``runtime/py/model.py:726-806``) plus numpy-array conveniences. Only the test
suite, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this package; the product path never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_q4.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libref_bf16.so")
_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64


def build(ref: bool = False) -> None:
    """Compile the oracle (and, with ``ref``, the reference's bf16.cpp into _ref/
    and the reference's C++ runtime against this build's NpuRegistry adapter)."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)
        subprocess.run(["make", "-s", "-C", _HERE, "ref-runtime"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_bf16_from_f32": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_f32_from_bf16": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_bf16_from_f32_n": (None, [_f32p, _u16p, _i64]),
        "orc_bf16_sweep": (ctypes.c_uint64, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32)]),
        "orc_unpack_q4": (None, [_u8p, _i64, _i64, _i8p]),
        "orc_scales_q4": (None, [_u8p, _i64, _i64, _u16p]),
        "orc_dequant_q4": (None, [_u8p, _i64, _i64, _u16p]),
        "orc_gemv_q": (None, [_u8p, _f32p, _f32p, _i64, _i64, ctypes.c_int]),
        "orc_gemv_q_f64": (None, [_u8p, _f32p, _f64p, _i64, _i64, ctypes.c_int]),
        "orc_gemm_q": (None, [_u8p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int]),
        "orc_glu": (None, [_f32p, _f32p, _f32p, _i64, ctypes.c_int]),
        "orc_ffn": (None, [_u8p, _u8p, _u8p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int]),
        "orc_ffn_f64": (None, [_u8p, _u8p, _u8p, _f32p, _f64p, _i64, _i64, ctypes.c_int]),
        "orc_quantize_q4_0": (None, [_f32p, _i64, _i64, _u8p]),
        "orc_splitmix64_at": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
        "orc_synth_q4": (None, [_u8p, _i64, _i64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
        "orc_synth_uniform": (None, [_f32p, _i64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
        "orc_synth_normal": (None, [_f32p, _i64, ctypes.c_uint64]),
        "orc_time_gemv_faithful": (ctypes.c_double, [_u8p, _f32p, _f32p, _i64, _i64, ctypes.c_int, ctypes.c_int]),
        "orc_time_gemv_predequant": (ctypes.c_double, [_u8p, _f32p, _f32p, _i64, _i64, ctypes.c_int, ctypes.c_int]),
        "orc_time_ffn_faithful": (ctypes.c_double, [_u8p, _u8p, _u8p, _f32p, _f32p, _i64, _i64, ctypes.c_int, ctypes.c_int]),
        "orc_time_ffn_predequant": (ctypes.c_double, [_u8p, _u8p, _u8p, _f32p, _f32p, _i64, _i64, ctypes.c_int, ctypes.c_int]),
        "orc_max_threads": (ctypes.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def ref_lib() -> ctypes.CDLL | None:
    """The reference's bf16.cpp built into oracle/_ref, or None if not built."""
    if not os.path.exists(_REF_PATH):
        return None
    L = ctypes.CDLL(_REF_PATH)
    L.ref_bf16_from_f32.restype = ctypes.c_uint16
    L.ref_bf16_from_f32.argtypes = [ctypes.c_float]
    L.ref_f32_from_bf16.restype = ctypes.c_float
    L.ref_f32_from_bf16.argtypes = [ctypes.c_uint16]
    return L


def _p(a: np.ndarray, t):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(t)


def _threads(threads: int | None) -> int:
    return threads if threads else lib().orc_max_threads()


# ---- array helpers ----------------------------------------------------------

def bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_from_f32_n(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def bf16_round(x: np.ndarray) -> np.ndarray:
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def unpack_q4(W: np.ndarray, N: int, K: int) -> np.ndarray:
    q = np.empty((N, K), np.int8)
    lib().orc_unpack_q4(_p(W, _u8p), N, K, _p(q, _i8p))
    return q


def scales_q4(W: np.ndarray, N: int, K: int) -> np.ndarray:
    s = np.empty((N, K // 32), np.uint16)
    lib().orc_scales_q4(_p(W, _u8p), N, K, _p(s, _u16p))
    return s


def dequant_q4(W: np.ndarray, N: int, K: int) -> np.ndarray:
    """bf16 bit patterns (N, K) of the dequantized matrix."""
    out = np.empty((N, K), np.uint16)
    lib().orc_dequant_q4(_p(W, _u8p), N, K, _p(out, _u16p))
    return out


def gemv_q(W: np.ndarray, x: np.ndarray, N: int, K: int, threads: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(N, np.float32)
    lib().orc_gemv_q(_p(W, _u8p), _p(x, _f32p), _p(y, _f32p), N, K, _threads(threads))
    return y


def gemv_q_f64(W: np.ndarray, x: np.ndarray, N: int, K: int, threads: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(N, np.float64)
    lib().orc_gemv_q_f64(_p(W, _u8p), _p(x, _f32p), _p(y, _f64p), N, K, _threads(threads))
    return y


def gemm_q(W: np.ndarray, X: np.ndarray, M: int, N: int, K: int, threads: int | None = None) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty((M, N), np.float32)
    lib().orc_gemm_q(_p(W, _u8p), _p(X, _f32p), _p(Y, _f32p), M, N, K, _threads(threads))
    return Y


def glu(g: np.ndarray, u: np.ndarray, act: int = 0) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    a = np.empty_like(g)
    lib().orc_glu(_p(g, _f32p), _p(u, _f32p), _p(a, _f32p), g.size, act)
    return a


def ffn(Wg, Wu, Wd, X: np.ndarray, H: int, I: int, act: int = 0, threads: int | None = None) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    M = X.size // H
    Y = np.empty(X.shape[:-1] + (H,), np.float32) if X.ndim > 1 else np.empty(H, np.float32)
    lib().orc_ffn(_p(Wg, _u8p), _p(Wu, _u8p), _p(Wd, _u8p), _p(X, _f32p), _p(Y, _f32p),
                  M, H, I, act, _threads(threads))
    return Y


def ffn_f64(Wg, Wu, Wd, x: np.ndarray, H: int, I: int, act: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(H, np.float64)
    lib().orc_ffn_f64(_p(Wg, _u8p), _p(Wu, _u8p), _p(Wd, _u8p), _p(x, _f32p), _p(y, _f64p), H, I, act)
    return y


def quantize_q4_0(Wf: np.ndarray) -> np.ndarray:
    Wf = np.ascontiguousarray(Wf, np.float32)
    N, K = Wf.shape
    out = np.empty((N, K // 32 * 20), np.uint8)
    lib().orc_quantize_q4_0(_p(Wf, _f32p), N, K, _p(out, _u8p))
    return out


def synth_q4(N: int, K: int, seed: int, smin: float = 0.001, smax: float = 0.02) -> np.ndarray:
    W = np.empty((N, K // 32 * 20), np.uint8)
    lib().orc_synth_q4(_p(W, _u8p), N, K, seed, smin, smax)
    return W


def synth_uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    x = np.empty(n, np.float32)
    lib().orc_synth_uniform(_p(x, _f32p), n, seed, lo, hi)
    return x


def synth_normal(n: int, seed: int) -> np.ndarray:
    x = np.empty(n, np.float32)
    lib().orc_synth_normal(_p(x, _f32p), n, seed)
    return x


def seed_for(config: int, tensor: int, layer: int = 0) -> int:
    """Seed convention: 0xA1E0_0000 + 0x100*config + tensor + 0x10000*layer."""
    return 0xA1E00000 + 0x100 * config + tensor + 0x10000 * layer
