"""Torch-facing Q4 ops over the C ABI, mirroring the reference's op interface.

Canonical names and the reference's IRON names (``kernels/*/<name>.py``):

=================  =====================================================
``gemv_q``         ``gemv_q_npu(W, X, Y, *, N, K, m, k_tile)``
                   (kernels/gemv_q/gemv_q.py:33-42)
``gemm_q``         ``gemm_q_npu(W, X, Y, *, B, N, K, m, k_tile)``
                   (kernels/gemm_q/gemm_q.py:28-39)
``ffn_fused``      ``ffn_fused_npu(W_fused, X, Y_partial, *, H, I, m_I,
                   k_tile, activation)`` (kernels/ffn_fused/ffn_fused.py:28-39)
``pack_ffn_fused_weights``  same name, kernels/ffn_fused/ffn_fused.py:330-395
                   and runtime/cpp/src/weights.cpp:94-190
=================  =====================================================

Buffers are torch tensors on the GPU. As in the reference (the
``_patched_validate`` hook, runtime/py/model.py:12-21) a buffer may be larger
than the op needs; only a buffer that is too small raises. Activations may be
float32 or bfloat16; outputs float32 receive the fp32 result before the
reference's final bf16 cast, outputs bfloat16 receive that cast (round to
nearest even). ``m``, ``k_tile`` and ``m_I`` are NPU tiling parameters; they
are accepted for signature compatibility and do not change the result.

Work is enqueued on torch's current stream of the tensors' device.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import ALV_ACT_GELU_TANH, ALV_ACT_SILU, check, lib

_ACTS = {"gelu": ALV_ACT_GELU_TANH, "gelu_tanh": ALV_ACT_GELU_TANH, "silu": ALV_ACT_SILU}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_gpu(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError("alveare_amd ops run on the GPU; got a tensor on " + str(t.device))
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _too_small(name: str, actual: int, expected: int) -> None:
    if actual < expected:
        raise RuntimeError(f"Tensor too small. Actual: {actual}, Expected: {expected} ({name})")


def _weight(W: torch.Tensor, N: int, K: int, name: str = "W") -> torch.Tensor:
    """The (N, K/32*20) combined-layout matrix held by W. A 2-D W is read with
    its own row stride: rows of W.shape[1] bytes, of which the first K/32*20
    are used, and the first N rows (the reference's quantizer pads K and N
    with zero weights, tools/quantize_gemma4.py:158-187); a padded W yields a
    contiguous copy of that sub-matrix. A 1-D W is a flat row-major buffer
    that may be larger than needed (runtime/py/model.py:12-21)."""
    if not isinstance(W, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(W).__name__}")
    if W.dtype != torch.uint8:
        raise TypeError(f"{name} must be uint8 in the combined Q4 layout, got {W.dtype}")
    rb = (K // 32) * 20
    if W.dim() == 2:
        if W.shape[1] < rb or W.shape[0] < N:
            raise RuntimeError(f"Tensor too small. Actual: {tuple(W.shape)}, Expected: ({N}, {rb}) ({name})")
        if W.shape[1] % 20:
            raise ValueError(f"{name} rows of {W.shape[1]} bytes are not whole 20-byte Q4 blocks")
        if W.shape[1] != rb or not W.is_contiguous():
            return W[:N, :rb].contiguous()
        return W
    if W.dim() != 1:
        raise ValueError(f"{name} must be 1-D (flat) or 2-D (rows, K/32*20), got shape {tuple(W.shape)}")
    if not W.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    _too_small(name, W.numel(), N * rb)
    return W


def _act_in(X: torch.Tensor, n: int, name: str) -> torch.Tensor:
    _too_small(name, X.numel(), n)
    X = X.reshape(-1)[:n]
    if X.dtype == torch.bfloat16:
        X = X.float()
    elif X.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 or bfloat16, got {X.dtype}")
    return X.contiguous()


def _check_shape(N: int, K: int) -> None:
    if N < 1 or K < 32 or K % 32:
        raise ValueError(f"bad shape N={N} K={K}: K must be a positive multiple of 32")


def _store(Y: torch.Tensor, y32: torch.Tensor, n: int) -> None:
    flat = Y.view(-1)
    if flat.data_ptr() == y32.data_ptr():
        return
    flat[:n].copy_(y32.reshape(-1))  # bf16 targets: round to nearest even


def _out_buffer(Y: torch.Tensor, n: int, name: str) -> torch.Tensor:
    _too_small(name, Y.numel(), n)
    if Y.dtype == torch.float32 and Y.is_contiguous():
        return Y.view(-1)[:n]
    if Y.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"{name} must be float32 or bfloat16, got {Y.dtype}")
    return torch.empty(n, dtype=torch.float32, device=Y.device)


def gemv_q(W: torch.Tensor, X: torch.Tensor, Y: torch.Tensor, *, N: int, K: int,
           m: int = 32, k_tile: int = 256) -> torch.Tensor:
    """Y[:N] = dequant(W)[N, K] @ X[:K] (tools/ref/gemv_q.py:73-80)."""
    _check_shape(N, K)
    _need_gpu(W, X, Y)
    W = _weight(W, N, K)
    x = _act_in(X, K, "X")
    y = _out_buffer(Y, N, "Y")
    with torch.cuda.device(W.device):
        check(lib().alv_gemv_q(W.data_ptr(), x.data_ptr(), y.data_ptr(), N, K, _stream(W)), "alv_gemv_q")
    _store(Y, y, N)
    return Y


def gemm_q(W: torch.Tensor, X: torch.Tensor, Y: torch.Tensor, *, B: int, N: int, K: int,
           m: int = 32, k_tile: int = 256) -> torch.Tensor:
    """Y[B, N] = X[B, K] @ dequant(W)^T, row-major (runtime/py/model.py:1049-1111)."""
    _check_shape(N, K)
    if B < 1:
        raise ValueError(f"bad batch B={B}")
    _need_gpu(W, X, Y)
    W = _weight(W, N, K)
    x = _act_in(X, B * K, "X")
    y = _out_buffer(Y, B * N, "Y")
    with torch.cuda.device(W.device):
        check(lib().alv_gemm_q(W.data_ptr(), x.data_ptr(), y.data_ptr(), B, N, K, K, N, _stream(W)),
              "alv_gemm_q")
    _store(Y, y, B * N)
    return Y


def dequant_q4(W: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """bf16 (N, K) = dequant(W) (tools/ref/gemv_q.py:39-62); parity entry point."""
    _check_shape(N, K)
    _need_gpu(W)
    W = _weight(W, N, K)
    out = torch.empty((N, K), dtype=torch.bfloat16, device=W.device)
    with torch.cuda.device(W.device):
        check(lib().alv_dequant_q4(W.data_ptr(), out.data_ptr(), N, K, _stream(W)), "alv_dequant_q4")
    return out


def q4_tile(W: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """The kernels' tiled layout of W (uint8, alv_q4_tiled_bytes(N, K) bytes);
    parity entry point for the registration-time repack."""
    _check_shape(N, K)
    _need_gpu(W)
    W = _weight(W, N, K)
    out = torch.empty(int(lib().alv_q4_tiled_bytes(N, K)), dtype=torch.uint8, device=W.device)
    with torch.cuda.device(W.device):
        check(lib().alv_q4_tile(W.data_ptr(), out.data_ptr(), N, K, _stream(W)), "alv_q4_tile")
    return out


def _float_source(W: torch.Tensor, N: int | None, K: int | None):
    if W.dim() != 2 or W.dtype != torch.float32:
        raise ValueError(f"W must be a 2-D float32 tensor (got {tuple(W.shape)} {W.dtype})")
    _need_gpu(W)
    if W.stride(1) != 1:
        W = W.contiguous()
    n_src, k_src = W.shape
    N = n_src if N is None else N
    K = k_src if K is None else K
    if N < n_src or K < k_src:
        raise ValueError(f"target {N} x {K} smaller than the source {n_src} x {k_src}")
    _check_shape(N, K)
    return W, n_src, k_src, N, K


def quantize_q4(W: torch.Tensor, N: int | None = None, K: int | None = None) -> torch.Tensor:
    """quantize_to_q4_0 + pack_to_combined (tools/convert/gemv_q_convert.py:5-85)
    on the GPU: float32 W (n, k) -> uint8 (N, K/32*20), zero-padded to N x K
    as quantize_and_pack_tensor does (tools/quantize_gemma4.py:26-41)."""
    W, n_src, k_src, N, K = _float_source(W, N, K)
    out = torch.empty((N, K // 32 * 20), dtype=torch.uint8, device=W.device)
    with torch.cuda.device(W.device):
        check(lib().alv_quantize_q4(W.data_ptr(), n_src, k_src, W.stride(0), out.data_ptr(), N, K, _stream(W)),
              "alv_quantize_q4")
    return out


class Q4Weight:
    """A registered projection (runtime/cpp/src/npu.cpp:241-253
    create_gemv_weight): a device copy in the kernels' tiled layout, used by
    ``gemv``/``__call__``. Released on ``close()`` or garbage collection.
    ``Q4Weight.quantize(W_fp32, N, K)`` quantizes float32 weights on the GPU
    straight into this layout."""

    @classmethod
    def quantize(cls, W: torch.Tensor, N: int | None = None, K: int | None = None) -> "Q4Weight":
        W, n_src, k_src, N, K = _float_source(W, N, K)
        self = cls.__new__(cls)
        self.N, self.K, self.device = N, K, W.device
        self._h = ctypes.c_void_p()
        with torch.cuda.device(W.device):
            check(lib().alv_weight_quantize(W.data_ptr(), n_src, k_src, W.stride(0), N, K, ctypes.byref(self._h),
                                            _stream(W)), "alv_weight_quantize")
        self.shape = (N, K // 32 * 20)
        return self

    def __init__(self, W: torch.Tensor, N: int, K: int):
        _check_shape(N, K)
        dev = _need_gpu(W)
        W = _weight(W, N, K)
        self.N, self.K, self.device = N, K, dev
        self._h = ctypes.c_void_p()
        with torch.cuda.device(dev):
            check(lib().alv_weight_register(W.data_ptr(), N, K, ctypes.byref(self._h), _stream(W)),
                  "alv_weight_register")
        self.shape = (N, K // 32 * 20)

    @property
    def handle(self) -> int:
        if not self._h:
            raise ValueError("weights were released")
        return self._h.value

    @property
    def exec_shape(self) -> tuple[int, int]:
        """(N, K) the kernels stream: registration drops trailing rows and
        32-column blocks whose weights are all zero (padded shapes)."""
        n, k = ctypes.c_int(), ctypes.c_int()
        check(lib().alv_weight_exec_shape(self.handle, ctypes.byref(n), ctypes.byref(k)), "alv_weight_exec_shape")
        return n.value, k.value

    def close(self) -> None:
        if self._h:
            with torch.cuda.device(self.device):
                lib().alv_weight_release(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __call__(self, X: torch.Tensor, Y: torch.Tensor | None = None, M: int = 1) -> torch.Tensor:
        """Y[M, N] = X[M, K] @ dequant(W)^T (M = 1: the decode GEMV)."""
        x = _act_in(X, M * self.K, "X")
        if x.device != self.device:
            raise ValueError(f"X on {x.device}, weights on {self.device}")
        if Y is None:
            Y = torch.empty((M, self.N) if M > 1 else (self.N,), dtype=torch.float32, device=self.device)
        _need_gpu(Y)
        y = _out_buffer(Y, M * self.N, "Y")
        with torch.cuda.device(self.device):
            check(lib().alv_gemv(self.handle, x.data_ptr(), y.data_ptr(), M, self.K, self.N, _stream(x)),
                  "alv_gemv")
        _store(Y, y, M * self.N)
        return Y


class FfnWeights:
    """A registered FFN layer (the device-resident analogue of the reference's
    fused FFN weight, runtime/cpp/src/npu.cpp:255-267). Owns a device copy of
    gate/up/down and the activation scratch; released on ``close()`` or
    garbage collection."""

    def __init__(self, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                 H: int, I: int, activation: str = "gelu"):
        if activation not in _ACTS:
            raise ValueError(f"unknown activation {activation!r}; expected one of {sorted(_ACTS)}")
        if H < 32 or I < 32 or H % 32 or I % 32:
            raise ValueError(f"bad FFN shape H={H} I={I}: both must be positive multiples of 32")
        dev = _need_gpu(w_gate, w_up, w_down)
        w_gate = _weight(w_gate, I, H, "w_gate")
        w_up = _weight(w_up, I, H, "w_up")
        w_down = _weight(w_down, H, I, "w_down")
        self.H, self.I, self.activation, self.device = H, I, activation, dev
        self._h = ctypes.c_void_p()
        with torch.cuda.device(dev):
            check(lib().alv_ffn_register(w_gate.data_ptr(), w_up.data_ptr(), w_down.data_ptr(), H, I,
                                         _ACTS[activation], ctypes.byref(self._h), _stream(w_gate)),
                  "alv_ffn_register")
        # Lets ffn_fused_npu's caller read .shape like the reference's ResidentWeight.
        self.shape = (H, I)

    @property
    def handle(self) -> int:
        if not self._h:
            raise ValueError("FFN weights were released")
        return self._h.value

    @property
    def exec_shape(self) -> tuple[int, int]:
        """(H, I) the kernels run at after registration dropped trailing
        all-zero hidden / intermediate rows and columns (padded shapes)."""
        h, i = ctypes.c_int(), ctypes.c_int()
        check(lib().alv_ffn_exec_shape(self.handle, ctypes.byref(h), ctypes.byref(i)), "alv_ffn_exec_shape")
        return h.value, i.value

    def close(self) -> None:
        if self._h:
            with torch.cuda.device(self.device):
                lib().alv_ffn_release(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def last_activation(self, M: int = 1) -> torch.Tensor:
        """The bf16-valued activation (M, I) of the last call (parity checks)."""
        out = torch.empty((M, self.I), dtype=torch.float32, device=self.device)
        with torch.cuda.device(self.device):
            check(lib().alv_ffn_activation(self.handle, out.data_ptr(), M, _stream(out)),
                  "alv_ffn_activation")
        return out

    def gate_up(self, X: torch.Tensor, M: int = 1) -> None:
        """Only the gate/up launch of a call (alv_ffn_gate_up): the activation
        lands in the handle's scratch (``last_activation``)."""
        x = _act_in(X, M * self.H, "X")
        if x.device != self.device:
            raise ValueError(f"X on {x.device}, weights on {self.device}")
        with torch.cuda.device(self.device):
            check(lib().alv_ffn_gate_up(self.handle, x.data_ptr(), M, self.H, _stream(x)), "alv_ffn_gate_up")

    def partials(self, X: torch.Tensor, P: torch.Tensor | None = None) -> int:
        """Only the first launch of a one-token call (alv_ffn_partials): the
        activation of every intermediate row and each 64-row slice's partial
        output, G = I / 64 rows of H' floats into P (None: the handle's
        buffer). Returns G."""
        x = _act_in(X, self.H, "X")
        if x.device != self.device:
            raise ValueError(f"X on {x.device}, weights on {self.device}")
        g = ctypes.c_int(0)
        with torch.cuda.device(self.device):
            check(lib().alv_ffn_partials(self.handle, x.data_ptr(), P.data_ptr() if P is not None else None,
                                         ctypes.byref(g), _stream(x)), "alv_ffn_partials")
        return g.value

    def __call__(self, X: torch.Tensor, Y: torch.Tensor | None = None, M: int = 1) -> torch.Tensor:
        x = _act_in(X, M * self.H, "X")
        if x.device != self.device:
            raise ValueError(f"X on {x.device}, weights on {self.device}")
        if Y is None:
            Y = torch.empty((M, self.H) if M > 1 else (self.H,), dtype=torch.float32, device=self.device)
        _need_gpu(Y)
        y = _out_buffer(Y, M * self.H, "Y")
        with torch.cuda.device(self.device):
            check(lib().alv_ffn_fused(self.handle, x.data_ptr(), y.data_ptr(), M, self.H, self.H,
                                      _stream(x)), "alv_ffn_fused")
        _store(Y, y, M * self.H)
        return Y


def pack_ffn_fused_weights(w_gate, w_up, w_down, H: int, I: int, m_I: int = 32,
                           k_tile: int = 256, activation: str = "gelu", device=None) -> FfnWeights:
    """Register gate/up/down (combined Q4 layout, torch uint8 tensors or numpy
    arrays) as one device-resident FFN. The reference packs an NPU tile stream
    here; on the GPU the handle keeps its own copy in the kernels' layout."""
    dev = torch.device(device) if device is not None else None

    def to_dev(w):
        if isinstance(w, torch.Tensor):
            return w.contiguous() if dev is None else w.to(dev).contiguous()
        return torch.from_numpy(w.reshape(w.shape[0], -1).copy()).to(dev or "cuda")

    return FfnWeights(to_dev(w_gate), to_dev(w_up), to_dev(w_down), H, I, activation)


def ffn_fused(W_fused: FfnWeights, X: torch.Tensor, Y_partial: torch.Tensor, *, H: int, I: int,
              m_I: int = 32, k_tile: int = 256, activation: str = "gelu", M: int = 1) -> torch.Tensor:
    """Y_partial[:H] (or [:M*H]) = down(GLU(gate X, up X)). The reference writes
    one partial row per NPU core and its caller sums them
    (runtime/py/model.py:394-395); here the sum is finished on the device, so
    the result is the single row Y_partial[0] (a sum over axis 0 of a (1, H)
    view is the identity)."""
    if not isinstance(W_fused, FfnWeights):
        raise TypeError("W_fused must come from pack_ffn_fused_weights")
    if (H, I) != (W_fused.H, W_fused.I):
        raise ValueError(f"shape mismatch: registered (H={W_fused.H}, I={W_fused.I}), called with (H={H}, I={I})")
    if activation not in _ACTS or _ACTS[activation] != _ACTS[W_fused.activation]:
        raise ValueError(f"activation {activation!r} does not match the registered {W_fused.activation!r}")
    return W_fused(X, Y_partial, M)


def chain_run(ops, M: int = 1) -> None:
    """Enqueue a chain of registered ops with one call and no host waits
    between them (alv_chain_run). ``ops`` is a list of ``(handle, x, y, dep)`` with
    handle a Q4Weight or FfnWeights, x/y float32 GPU tensors (x may be a view
    into an earlier op's y) and dep the index of the op whose output x reads
    (or -1). Equivalent to calling the ops one after another."""
    from ._lib import ChainOp

    arr = (ChainOp * len(ops))()
    dev = None
    for i, (h, x, y, dep) in enumerate(ops):
        if not isinstance(h, (Q4Weight, FfnWeights)):
            raise TypeError("chain ops take Q4Weight or FfnWeights handles")
        d = _need_gpu(x, y)
        dev = dev or d
        if x.dtype != torch.float32 or y.dtype != torch.float32 or not x.is_contiguous() or not y.is_contiguous():
            raise TypeError("chain activations are contiguous float32 tensors")
        K, N = (h.K, h.N) if isinstance(h, Q4Weight) else (h.H, h.H)
        _too_small("x", x.numel(), M * K)
        _too_small("y", y.numel(), M * N)
        arr[i].weight = h.handle if isinstance(h, Q4Weight) else None
        arr[i].ffn = h.handle if isinstance(h, FfnWeights) else None
        arr[i].x = x.data_ptr()
        arr[i].y = y.data_ptr()
        arr[i].dep = int(dep)
    with torch.cuda.device(dev):
        check(lib().alv_chain_run(arr, len(ops), M, torch.cuda.current_stream(dev).cuda_stream), "alv_chain_run")


def lm_head(W: "Q4Weight", x: torch.Tensor, vocab: int | None = None, softcap: float = 30.0,
            logits: torch.Tensor | None = None, token: torch.Tensor | None = None,
            pos: torch.Tensor | None = None, max_pos: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """LM head of a decode step (alv_lm_head): logits[:vocab] =
    softcap * tanh(bf16(W x) / softcap) in float32 (softcap 0: the bf16
    logits) and the greedy token, np.argmax of the logits, as a 1-element
    int32 tensor on the device (runtime/py/model.py:904-916,
    runtime/py/sampler.py:9; runtime/cpp/src/generator.cpp:15-52).
    A bfloat16 x runs alv_lm_head_bf16 (one activation term, the same bits
    as its float32 widening). ``pos`` (bfloat16 x only): a 1-element int32
    device tensor holding the decode position, advanced by one in the head's
    last launch; the token is then -1 when pos >= max_pos."""
    if not isinstance(W, Q4Weight):
        raise TypeError("W must be a registered Q4Weight")
    vocab = W.N if vocab is None else int(vocab)
    bf = x.dtype == torch.bfloat16
    if pos is not None and not bf:
        raise ValueError("pos takes a bfloat16 x (alv_lm_head_bf16)")
    if bf:
        _too_small("x", x.numel(), W.K)
        xv = x.reshape(-1)[:W.K].contiguous()
        if xv.data_ptr() % 16:
            xv = xv.clone()
    else:
        xv = _act_in(x, W.K, "x")
    if xv.device != W.device:
        raise ValueError(f"x on {xv.device}, weights on {W.device}")
    if logits is None:
        logits = torch.empty(vocab, dtype=torch.float32, device=W.device)
    _need_gpu(logits)
    if logits.dtype != torch.float32 or not logits.is_contiguous():
        raise TypeError("logits must be a contiguous float32 tensor")
    _too_small("logits", logits.numel(), vocab)
    if token is None:
        token = torch.empty(1, dtype=torch.int32, device=W.device)
    if token.dtype != torch.int32 or token.device != W.device:
        raise TypeError("token must be an int32 tensor on the weights' device")
    if pos is not None and (pos.dtype != torch.int32 or pos.device != W.device or pos.numel() < 1):
        raise TypeError("pos must be an int32 tensor on the weights' device")
    with torch.cuda.device(W.device):
        if bf:
            check(lib().alv_lm_head_bf16(W.handle, xv.data_ptr(), logits.data_ptr(), vocab, float(softcap),
                                         token.data_ptr(), pos.data_ptr() if pos is not None else None,
                                         int(max_pos), _stream(xv)), "alv_lm_head_bf16")
        else:
            check(lib().alv_lm_head(W.handle, xv.data_ptr(), logits.data_ptr(), vocab, float(softcap),
                                    token.data_ptr(), _stream(xv)), "alv_lm_head")
    return logits, token


# The reference's names for the same ops.
gemv_q_npu = gemv_q
gemm_q_npu = gemm_q
ffn_fused_npu = ffn_fused

__all__ = ["gemv_q", "gemm_q", "ffn_fused", "dequant_q4", "q4_tile", "Q4Weight", "FfnWeights", "chain_run", "lm_head",
           "pack_ffn_fused_weights", "gemv_q_npu", "gemm_q_npu", "ffn_fused_npu"]
