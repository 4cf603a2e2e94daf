"""The C ABI library on the CPU: it loads, exports every symbol the header
declares with the bound signatures, and rejects bad arguments with status
codes before touching the device (no compute calls here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "alveare_q4.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(alv_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from alveare_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from alveare_amd import build

        build.build()
    return _lib.lib()


def test_header_symbols_exported_and_bound(L):
    from alveare_amd import _lib

    syms = declared_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(L, s), f"{s} declared in alveare_q4.h but not exported"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(syms)
    assert L.alv_version().decode().startswith("alveare_q4")


def test_argument_errors_without_device(L):
    from alveare_amd._lib import ALV_ERR_ALIGN, ALV_ERR_ARG, ALV_ERR_HANDLE

    p = ctypes.c_void_p(4096)
    assert L.alv_gemv_q(None, p, p, 16, 64, None) == ALV_ERR_ARG
    assert b"null" in L.alv_last_error()
    assert L.alv_gemv_q(p, p, p, 16, 48, None) == ALV_ERR_ARG  # K not a multiple of 32
    assert b"K" in L.alv_last_error()
    assert L.alv_gemv_q(p, p, p, 0, 64, None) == ALV_ERR_ARG
    assert L.alv_gemv_q(ctypes.c_void_p(4098), p, p, 16, 64, None) == ALV_ERR_ALIGN
    assert L.alv_gemm_q(p, p, p, 0, 16, 64, 64, 16, None) == ALV_ERR_ARG
    assert L.alv_gemm_q(p, p, p, 2, 16, 64, 32, 16, None) == ALV_ERR_ARG  # ldx < K
    assert L.alv_dequant_q4(p, ctypes.c_void_p(4104), 16, 64, None) == ALV_ERR_ALIGN
    h = ctypes.c_void_p()
    assert L.alv_ffn_register(p, p, p, 100, 64, 0, ctypes.byref(h), None) == ALV_ERR_ARG
    assert L.alv_ffn_register(p, p, p, 64, 64, 7, ctypes.byref(h), None) == ALV_ERR_ARG
    assert L.alv_ffn_register(None, p, p, 64, 64, 0, ctypes.byref(h), None) == ALV_ERR_ARG
    assert not h.value
    assert L.alv_ffn_fused(None, p, p, 1, 64, 64, None) == ALV_ERR_HANDLE
    bogus = (ctypes.c_uint32 * 16)()
    assert L.alv_ffn_fused(ctypes.cast(bogus, ctypes.c_void_p), p, p, 1, 64, 64, None) == ALV_ERR_HANDLE
    assert L.alv_ffn_shape(None, None, None, None) == ALV_ERR_HANDLE
    assert L.alv_ffn_activation(None, p, 1, None) == ALV_ERR_HANDLE
    L.alv_ffn_release(None)  # no-op


def test_python_layer_validates_before_the_abi():
    import torch

    import alveare_amd as aa

    W = torch.zeros(16 * 2 * 20, dtype=torch.uint8)
    x = torch.zeros(64)
    y = torch.zeros(16)
    with pytest.raises(ValueError, match="GPU"):
        aa.gemv_q(W, x, y, N=16, K=64)
    with pytest.raises(ValueError, match="multiple of 32"):
        aa.gemv_q(W, x, y, N=16, K=48)
    with pytest.raises(ValueError, match="unknown activation"):
        aa.FfnWeights(W, W, W, 64, 64, activation="relu")


def test_weight_row_stride_of_padded_arrays():
    """A 2-D weight array is read with its own row stride: a padded array (the
    reference quantizer pads K and N, tools/quantize_gemma4.py:177-187) yields
    its leading (N, K/32*20) sub-matrix; an array too small, or with rows that
    are not whole 20-byte blocks, or neither 1-D nor 2-D, is rejected; a flat
    1-D buffer may be larger than needed."""
    import torch

    from alveare_amd.ops import _weight

    N, K = 48, 256
    rb = K // 32 * 20
    P = torch.randint(0, 256, (64, 320), dtype=torch.uint8)  # padded to 64 rows, K = 512
    W = _weight(P, N, K)
    assert W.shape == (N, rb) and W.is_contiguous()
    assert torch.equal(W, P[:N, :rb])
    exact = P[:N, :rb].contiguous()
    assert _weight(exact, N, K).data_ptr() == exact.data_ptr()  # no copy when nothing is padded
    flat = P.reshape(-1)
    assert _weight(flat, N, K).data_ptr() == flat.data_ptr()    # oversized flat buffers are allowed
    with pytest.raises(RuntimeError, match="too small"):
        _weight(P[:N - 1], N, K)
    with pytest.raises(RuntimeError, match="too small"):
        _weight(P[:, :rb - 20], N, K)
    with pytest.raises(RuntimeError, match="too small"):
        _weight(flat[: N * rb - 1], N, K)
    with pytest.raises(ValueError, match="20-byte"):
        _weight(P[:, :rb + 7], N, K)
    with pytest.raises(ValueError, match="1-D"):
        _weight(P.reshape(4, 16, 320), N, K)
    with pytest.raises(TypeError, match="uint8"):
        _weight(P.to(torch.int16), N, K)
