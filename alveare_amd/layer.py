"""Device-resident decode layer: the reference's per-layer host work on the GPU.

The reference runs a decode layer as NPU matmuls with numpy (Python runtime,
``runtime/py/model.py:705-790``) or C++ (``runtime/cpp/src/model.cpp:314-420``)
host code between them: RMSNorms, per-head q/k/v norms, RoPE, the KV-cache
insert, attention, residual adds and the layer output scale, with a host round
trip for every matmul. Here the whole layer is a sequence of launches on one
stream over device tensors (bf16 activations, bf16 KV caches), so the layer
never leaves the GPU and a token step can be captured in one HIP graph.

Op wrappers (bf16 tensors are ``torch.bfloat16``; float32 norm weights):

=====================  ======================================================
``rmsnorm``            run_rmsnorm_cpu (model.py:522-531), bit-exact
``qkv_post``           q/k/v norms + RoPE + cache insert (model.py:742-770)
``attention``          run_attention_host (model.py:577-628), float32
``add_norm``           residual (+ scale) (+ next norm) (model.py:775-788)
``gemv_bf16``          run_gemv_npu: bf16 in, bf16 out (model.py:283-362)
``ffn_fused_bf16``     run_ffn_fused_npu: bf16 in, bf16 out (model.py:363-397)
=====================  ======================================================

``Gemma4DecodeLayer`` composes them into the Gemma-4 layer of model.py:705-790
(sliding layers: 16 q heads of 256, 8 kv heads, window 1024, RoPE base 1e4;
global layers: 16 q heads of 512, one kv head whose v is its un-normalised k,
proportional RoPE base 1e6 on a quarter of the angles; attention scale 1).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import check, lib
import math

from .ops import FfnWeights, Q4Weight, _need_gpu, _stream, lm_head

_GEMMA_EPS = 1e-6


def _bf16(t: torch.Tensor, name: str, n: int) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < n:
        raise ValueError(f"{name} has {t.numel()} elements, needs {n}")
    return t


def _f32(t, name: str, n: int, dev) -> torch.Tensor | None:
    if t is None:
        return None
    t = torch.as_tensor(t, dtype=torch.float32, device=dev).contiguous()
    if t.numel() < n:
        raise ValueError(f"{name} has {t.numel()} elements, needs {n}")
    return t


def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def rmsnorm(x: torch.Tensor, w=None, *, K: int | None = None, rows: int = 1, pad: int | None = None,
            eps: float = _GEMMA_EPS, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(x / sqrt(mean(x^2) + eps) * w) per row of K values, zero-padded to
    `pad` columns (run_rmsnorm_cpu, runtime/py/model.py:522-531)."""
    dev = _need_gpu(x)
    K = x.numel() // rows if K is None else K
    pad = K if pad is None else pad
    _bf16(x, "x", rows * K)
    w = _f32(w, "w", K, dev)
    if out is None:
        out = torch.empty(rows * pad, dtype=torch.bfloat16, device=dev)
    _bf16(out, "out", rows * pad)
    with torch.cuda.device(dev):
        check(lib().alv_rmsnorm(x.data_ptr(), _ptr(w), out.data_ptr(), rows, K, K, pad, pad, ctypes.c_float(eps),
                                _stream(x)), "alv_rmsnorm")
    return out


def qkv_post(qkv: torch.Tensor, pos_dev: torch.Tensor, kcache: torch.Tensor, vcache: torch.Tensor, *,
             heads: int, kv_heads: int, D: int, k_off: int, v_off: int, q_w=None, k_w=None, norm_q: bool = True,
             norm_k: bool = True, norm_v: bool = True, eps: float = _GEMMA_EPS, rope: torch.Tensor | None = None,
             rope_stride: int | None = None, cos_off: int = 0, sin_off: int | None = None, half: int | None = None,
             q_out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-head norms, RoPE of q and k at the device position `pos_dev`, K/V
    cache insert (runtime/py/model.py:742-770). Caches are (kv_heads, max_seq, D)."""
    dev = _need_gpu(qkv)
    n_v = 0 if v_off < 0 else v_off + kv_heads * D
    _bf16(qkv, "qkv", max(k_off + kv_heads * D, n_v))
    if kcache.shape != vcache.shape or kcache.dim() != 3 or kcache.shape[0] != kv_heads or kcache.shape[2] != D:
        raise ValueError(f"caches must be ({kv_heads}, max_seq, {D}), got {tuple(kcache.shape)} / {tuple(vcache.shape)}")
    _bf16(kcache, "kcache", kcache.numel())
    _bf16(vcache, "vcache", vcache.numel())
    if pos_dev.dtype != torch.int32 or pos_dev.device != dev:
        raise ValueError("pos_dev must be an int32 tensor on the activations' device")
    q_w = _f32(q_w, "q_w", D, dev)
    k_w = _f32(k_w, "k_w", D, dev)
    if rope is not None:
        _bf16(rope, "rope", rope.numel())
        rope_stride = D if rope_stride is None else rope_stride
        half = D // 2 if half is None else half
        sin_off = half if sin_off is None else sin_off
        if rope.numel() < kcache.shape[1] * rope_stride:
            raise ValueError(f"rope table of {rope.numel()} values has fewer than the cache's {kcache.shape[1]} rows "
                             f"of {rope_stride}")
    if q_out is None:
        q_out = torch.empty(heads * D, dtype=torch.bfloat16, device=dev)
    _bf16(q_out, "q_out", heads * D)
    with torch.cuda.device(dev):
        check(lib().alv_qkv_post(qkv.data_ptr(), k_off, v_off, heads, kv_heads, D, _ptr(q_w), _ptr(k_w), int(norm_q),
                                 int(norm_k), int(norm_v), ctypes.c_float(eps), _ptr(rope), rope_stride or 0, cos_off,
                                 sin_off or 0, half or 0, pos_dev.data_ptr(), kcache.shape[1], q_out.data_ptr(),
                                 kcache.data_ptr(), vcache.data_ptr(), _stream(qkv)), "alv_qkv_post")
    return q_out


def qkv_attention(qkv: torch.Tensor, pos_dev: torch.Tensor, kcache: torch.Tensor, vcache: torch.Tensor, *,
                  heads: int, kv_heads: int, D: int, k_off: int, v_off: int, q_w=None, k_w=None, norm_q: bool = True,
                  norm_k: bool = True, norm_v: bool = True, eps: float = _GEMMA_EPS, rope: torch.Tensor | None = None,
                  rope_stride: int | None = None, cos_off: int = 0, sin_off: int | None = None,
                  half: int | None = None, q_out: torch.Tensor | None = None, window: int = 0, scale: float = 1.0,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """qkv_post and attention in one: the attention kernel normalises and
    rotates q, k and v itself (the same arithmetic, bit for bit), inserts k
    and v into the caches and writes the rotated q to q_out when given."""
    dev = _need_gpu(qkv)
    n_v = 0 if v_off < 0 else v_off + kv_heads * D
    _bf16(qkv, "qkv", max(k_off + kv_heads * D, n_v))
    if kcache.shape != vcache.shape or kcache.dim() != 3 or kcache.shape[0] != kv_heads or kcache.shape[2] != D:
        raise ValueError(f"caches must be ({kv_heads}, max_seq, {D}), got {tuple(kcache.shape)} / {tuple(vcache.shape)}")
    _bf16(kcache, "kcache", kcache.numel())
    _bf16(vcache, "vcache", vcache.numel())
    if pos_dev.dtype != torch.int32 or pos_dev.device != dev:
        raise ValueError("pos_dev must be an int32 tensor on the activations' device")
    q_w = _f32(q_w, "q_w", D, dev)
    k_w = _f32(k_w, "k_w", D, dev)
    if rope is not None:
        _bf16(rope, "rope", rope.numel())
        rope_stride = D if rope_stride is None else rope_stride
        half = D // 2 if half is None else half
        sin_off = half if sin_off is None else sin_off
        if rope.numel() < kcache.shape[1] * rope_stride:
            raise ValueError(f"rope table of {rope.numel()} values has fewer than the cache's {kcache.shape[1]} rows "
                             f"of {rope_stride}")
    if q_out is not None:
        _bf16(q_out, "q_out", heads * D)
    if out is None:
        out = torch.empty(heads * D, dtype=torch.bfloat16, device=dev)
    _bf16(out, "out", heads * D)
    with torch.cuda.device(dev):
        check(lib().alv_qkv_attention(qkv.data_ptr(), k_off, v_off, heads, kv_heads, D, _ptr(q_w), _ptr(k_w),
                                      int(norm_q), int(norm_k), int(norm_v), ctypes.c_float(eps), _ptr(rope),
                                      rope_stride or 0, cos_off, sin_off or 0, half or 0, pos_dev.data_ptr(),
                                      kcache.shape[1], _ptr(q_out), kcache.data_ptr(), vcache.data_ptr(), window,
                                      ctypes.c_float(scale), out.data_ptr(), _stream(qkv)), "alv_qkv_attention")
    return out


def attention(q: torch.Tensor, kcache: torch.Tensor, vcache: torch.Tensor, pos_dev: torch.Tensor, *, heads: int,
              window: int = 0, scale: float = 1.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """One token's attention over the cache positions up to `pos_dev`
    (run_attention_host, runtime/py/model.py:577-628)."""
    dev = _need_gpu(q)
    kv_heads, max_seq, D = kcache.shape
    _bf16(q, "q", heads * D)
    _bf16(kcache, "kcache", kcache.numel())
    _bf16(vcache, "vcache", vcache.numel())
    if out is None:
        out = torch.empty(heads * D, dtype=torch.bfloat16, device=dev)
    _bf16(out, "out", heads * D)
    with torch.cuda.device(dev):
        check(lib().alv_attention(q.data_ptr(), kcache.data_ptr(), vcache.data_ptr(), out.data_ptr(), heads, kv_heads,
                                  D, max_seq, window, ctypes.c_float(scale), pos_dev.data_ptr(), _stream(q)),
              "alv_attention")
    return out


def add_norm(resid: torch.Tensor, y: torch.Tensor, *, K: int, w_y=None, norm_y: bool = True, scale: float = 1.0,
             scale_mode: int = 0, w_out=None, norm_out: bool = False, pad: int | None = None, rows: int = 1,
             eps: float = _GEMMA_EPS, sum_out: torch.Tensor | None = None, norm_buf: torch.Tensor | None = None):
    """Residual step: s = bf16(resid + (norm_y ? bf16(rmsnorm(y) * w_y) : y)),
    scaled per scale_mode (1: Python runtime, two roundings; 2: C++ runtime, one),
    and optionally the next norm of s zero-padded to `pad`. Returns (s, norm)."""
    dev = _need_gpu(resid)
    pad = K if pad is None else pad
    _bf16(resid, "resid", rows * K)
    _bf16(y, "y", rows * K)
    w_y = _f32(w_y, "w_y", K, dev)
    w_out = _f32(w_out, "w_out", K, dev)
    if sum_out is None:
        sum_out = torch.empty(rows * K, dtype=torch.bfloat16, device=dev)
    _bf16(sum_out, "sum_out", rows * K)
    if norm_out and norm_buf is None:
        norm_buf = torch.empty(rows * pad, dtype=torch.bfloat16, device=dev)
    if norm_out:
        _bf16(norm_buf, "norm_out", rows * pad)
    with torch.cuda.device(dev):
        check(lib().alv_add_norm(resid.data_ptr(), K, y.data_ptr(), K, _ptr(w_y), int(norm_y), ctypes.c_float(scale),
                                 scale_mode, sum_out.data_ptr(), K, _ptr(w_out), _ptr(norm_buf) if norm_out else 0,
                                 pad, rows, K, pad, ctypes.c_float(eps), _stream(resid)), "alv_add_norm")
    return sum_out, (norm_buf if norm_out else None)


def gemv_bf16(W: Q4Weight, X: torch.Tensor, Y: torch.Tensor | None = None, M: int = 1) -> torch.Tensor:
    """Y = bf16(X W^T), bf16 in and out (the reference's run_gemv contract)."""
    _bf16(X, "X", M * W.K)
    if Y is None:
        Y = torch.empty(M * W.N, dtype=torch.bfloat16, device=W.device)
    _bf16(Y, "Y", M * W.N)
    with torch.cuda.device(W.device):
        check(lib().alv_gemv_bf16(W.handle, X.data_ptr(), Y.data_ptr(), M, W.K, W.N, _stream(X)), "alv_gemv_bf16")
    return Y


def ffn_fused_bf16(F: FfnWeights, X: torch.Tensor, Y: torch.Tensor | None = None, M: int = 1) -> torch.Tensor:
    """Y = bf16(down(GLU(gate X, up X))), bf16 in and out (run_ffn_fused)."""
    _bf16(X, "X", M * F.H)
    if Y is None:
        Y = torch.empty(M * F.H, dtype=torch.bfloat16, device=F.device)
    _bf16(Y, "Y", M * F.H)
    with torch.cuda.device(F.device):
        check(lib().alv_ffn_fused_bf16(F.handle, X.data_ptr(), Y.data_ptr(), M, F.H, F.H, _stream(X)),
              "alv_ffn_fused_bf16")
    return Y


def _step_args(resid, y, K, w_y, norm_y, scale, scale_mode, sum_out, w_x, eps, dev):
    _bf16(resid, "resid", K)
    if y is None:  # no residual step: the activation is the norm of resid
        w_x = _f32(w_x, "w_x", K, dev)
        return (resid.data_ptr(), None, None, 0, ctypes.c_float(1.0), 0, None, _ptr(w_x),
                ctypes.c_float(eps)), (w_x,)
    _bf16(y, "y", K)
    if sum_out is None:
        raise ValueError("a residual step needs sum_out")
    _bf16(sum_out, "sum_out", K)
    if sum_out.data_ptr() in (resid.data_ptr(), y.data_ptr()):
        raise ValueError("sum_out must not alias resid or y")
    w_y = _f32(w_y, "w_y", K, dev)
    w_x = _f32(w_x, "w_x", K, dev)
    return (resid.data_ptr(), y.data_ptr(), _ptr(w_y), int(norm_y), ctypes.c_float(scale), scale_mode,
            sum_out.data_ptr(), _ptr(w_x), ctypes.c_float(eps)), (w_y, w_x)


def gemv_bf16_addnorm(W: Q4Weight, resid: torch.Tensor, y: torch.Tensor | None, *,
                      sum_out: torch.Tensor | None = None, w_y=None, norm_y: bool = True, scale: float = 1.0,
                      scale_mode: int = 0, w_x=None, eps: float = _GEMMA_EPS,
                      Y: torch.Tensor | None = None) -> torch.Tensor:
    """add_norm(resid, y, ...) of one row (sum_out = s) and Y = gemv_bf16(W,
    rmsnorm(s) * w_x) in one launch: the matmul's workgroups compute the
    normalised activation themselves, bit for bit as the two calls do.
    y None: no residual step, Y = gemv_bf16(W, rmsnorm(resid) * w_x) (the
    first layer's input norm inside its QKV launch)."""
    args, keep = _step_args(resid, y, W.K, w_y, norm_y, scale, scale_mode, sum_out, w_x, eps, W.device)
    if Y is None:
        Y = torch.empty(W.N, dtype=torch.bfloat16, device=W.device)
    _bf16(Y, "Y", W.N)
    with torch.cuda.device(W.device):
        check(lib().alv_gemv_bf16_addnorm(W.handle, *args, Y.data_ptr(), _stream(resid)), "alv_gemv_bf16_addnorm")
    return Y


def lm_head_addnorm(W: Q4Weight, resid: torch.Tensor, y: torch.Tensor | None, *, hidden: int,
                    sum_out: torch.Tensor | None = None, w_y=None, norm_y: bool = True, scale: float = 1.0,
                    scale_mode: int = 0, w_x=None, eps: float = _GEMMA_EPS, vocab: int | None = None,
                    softcap: float = 30.0, logits: torch.Tensor | None = None, token: torch.Tensor | None = None,
                    pos: torch.Tensor | None = None, max_pos: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """add_norm(resid, y, ..., w_out=w_x, pad=W.K) of one `hidden`-wide row
    and lm_head on its bf16 norm in the head GEMV's launch
    (alv_lm_head_bf16_addnorm): the same sum_out, logits and token bits as
    the two calls. y None: the head on rmsnorm(resid) * w_x."""
    if not isinstance(W, Q4Weight):
        raise TypeError("W must be a registered Q4Weight")
    if not 8 <= hidden <= W.K or hidden % 8:
        raise ValueError(f"hidden={hidden}: a multiple of 8 in [8, {W.K}]")
    args, keep = _step_args(resid, y, hidden, w_y, norm_y, scale, scale_mode, sum_out, w_x, eps, W.device)
    vocab = W.N if vocab is None else int(vocab)
    if logits is None:
        logits = torch.empty(vocab, dtype=torch.float32, device=W.device)
    if logits.dtype != torch.float32 or not logits.is_contiguous() or logits.device != W.device:
        raise TypeError("logits must be a contiguous float32 tensor on the weights' device")
    if logits.numel() < vocab:
        raise ValueError(f"logits holds {logits.numel()} values, vocab is {vocab}")
    if token is None:
        token = torch.empty(1, dtype=torch.int32, device=W.device)
    if token.dtype != torch.int32 or token.device != W.device:
        raise TypeError("token must be an int32 tensor on the weights' device")
    if pos is not None and (pos.dtype != torch.int32 or pos.device != W.device or pos.numel() < 1):
        raise TypeError("pos must be an int32 tensor on the weights' device")
    with torch.cuda.device(W.device):
        check(lib().alv_lm_head_bf16_addnorm(W.handle, *args, int(hidden), logits.data_ptr(), vocab, float(softcap),
                                             token.data_ptr(), pos.data_ptr() if pos is not None else None,
                                             int(max_pos), _stream(resid)), "alv_lm_head_bf16_addnorm")
    return logits, token


def ffn_fused_bf16_addnorm(F: FfnWeights, resid: torch.Tensor, y: torch.Tensor, *, sum_out: torch.Tensor, w_y=None,
                           norm_y: bool = True, scale: float = 1.0, scale_mode: int = 0, w_x=None,
                           eps: float = _GEMMA_EPS, Y: torch.Tensor | None = None) -> torch.Tensor:
    """add_norm(resid, y, ...) of one row (sum_out = s) and Y =
    ffn_fused_bf16(F, rmsnorm(s) * w_x), the residual step inside the FFN's
    gate/up launch."""
    args, keep = _step_args(resid, y, F.H, w_y, norm_y, scale, scale_mode, sum_out, w_x, eps, F.device)
    if Y is None:
        Y = torch.empty(F.H, dtype=torch.bfloat16, device=F.device)
    _bf16(Y, "Y", F.H)
    with torch.cuda.device(F.device):
        check(lib().alv_ffn_fused_bf16_addnorm(F.handle, *args, Y.data_ptr(), _stream(resid)),
              "alv_ffn_fused_bf16_addnorm")
    return Y


def embed(table: torch.Tensor, token_dev: torch.Tensor, scale: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(float(double(table[token]) * scale)) for the token in device memory
    (the Gemma-4 lookup with scale sqrt(hidden), runtime/py/model.py:889-891);
    table is float16 (vocab, H)."""
    dev = _need_gpu(table)
    if table.dtype != torch.float16 or table.dim() != 2 or not table.is_contiguous():
        raise ValueError("table must be a contiguous 2-D float16 tensor")
    if token_dev.dtype != torch.int32 or token_dev.device != dev:
        raise ValueError("token_dev must be an int32 tensor on the table's device")
    vocab, H = table.shape
    if out is None:
        out = torch.empty(H, dtype=torch.bfloat16, device=dev)
    _bf16(out, "out", H)
    with torch.cuda.device(dev):
        check(lib().alv_embed(table.data_ptr(), vocab, H, token_dev.data_ptr(), ctypes.c_double(scale), out.data_ptr(),
                              _stream(table)), "alv_embed")
    return out


def cos_sin_table_gemma(base: float, dim: int, max_seq_len: int, gemma4: bool = True) -> np.ndarray:
    """The reference's RoPE table (precompute_cos_sin_table_gemma,
    runtime/py/model.py:263-280): float32 rows [cos(pos f) | sin(pos f)] in
    numpy, then bf16 (round to nearest even; returned as uint16 bit patterns).
    Gemma-4's 512-wide heads rotate a quarter of the angles."""
    if gemma4 and dim == 512:
        angles = int(0.25 * dim // 2)
        inv_freq = np.zeros(dim // 2, dtype=np.float32)
        inv_freq[:angles] = 1.0 / (base ** (np.arange(0, 2 * angles, 2, dtype=np.float32) / dim))
    else:
        inv_freq = 1.0 / (base ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    table = np.zeros((max_seq_len, dim), dtype=np.float32)
    for pos in range(max_seq_len):
        freqs = pos * inv_freq
        table[pos] = np.concatenate([np.cos(freqs), np.sin(freqs)])
    u = table.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


# Longest attention span (the sliding window, or a global layer's cache) the
# chunked attention takes: its merge holds 1024 chunk partials of 64 positions.
ATTN_MAX_SPAN = 1024 * 64


class Gemma4DecodeLayer:
    """One Gemma-4 decoder layer with every step on the device
    (runtime/py/model.py:705-790 with the NPU matmuls). Weights are combined
    Q4 arrays: ``qkv`` the rows [q | k | v] (sliding) or [q | k] (global) of
    H columns, ``o`` (H, q_size) and the FFN; norms float32. ``forward(x, pos)``
    takes and returns bf16 [H] device tensors and updates the KV caches."""

    def __init__(self, *, qkv, o, gate, up, down, norms: dict, scale: float, sliding: bool, H: int, I: int,
                 max_seq: int, device, rope_table=None, pos_dev: torch.Tensor | None = None, fuse: bool = True):
        dev = torch.device(device)
        self.sliding, self.H, self.I, self.max_seq, self.device = sliding, H, I, max_seq, dev
        self.fuse = fuse
        self.heads = 16
        self.kv_heads = 8 if sliding else 1
        self.D = 256 if sliding else 512
        self.q_size = self.heads * self.D
        self.k_size = self.kv_heads * self.D
        self.n_qkv = self.q_size + (2 if sliding else 1) * self.k_size
        self.window = 1024 if sliding else 0
        span = min(self.window, max_seq) if sliding else max_seq
        if max_seq < 1 or span > ATTN_MAX_SPAN:
            raise ValueError(f"max_seq={max_seq}: attention takes up to {ATTN_MAX_SPAN} positions per "
                             f"{'window' if sliding else 'global'} span (its chunk merge holds 1024 chunks of 64)")
        self.scale = float(np.float32(scale))

        def dev_u8(a):
            return torch.as_tensor(np.ascontiguousarray(a)).to(dev) if isinstance(a, np.ndarray) else a

        self.w_qkv = Q4Weight(dev_u8(qkv), self.n_qkv, H)
        self.w_o = Q4Weight(dev_u8(o), H, self.q_size)
        self.ffn = FfnWeights(dev_u8(gate), dev_u8(up), dev_u8(down), H, I, "gelu")
        self.norms = {k: _f32(v, k, self.D if k in ("q", "k") else H, dev) for k, v in norms.items()}
        if rope_table is None:
            rope_table = cos_sin_table_gemma(10000.0 if sliding else 1000000.0, self.D, max_seq)
        self.rope = torch.as_tensor(np.ascontiguousarray(rope_table)).view(torch.bfloat16).to(dev)
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.kcache = torch.zeros((self.kv_heads, max_seq, self.D), **bf)
        self.vcache = torch.zeros((self.kv_heads, max_seq, self.D), **bf)
        self.pos_dev = torch.zeros(1, dtype=torch.int32, device=dev) if pos_dev is None else pos_dev
        # Intermediates (kept for inspection and for graph capture: fixed addresses).
        self.x_norm = torch.empty(H, **bf)
        self.qkv_out = torch.empty(self.n_qkv, **bf)
        self.q_rope = torch.empty(self.q_size, **bf)
        self.attn_out = torch.empty(self.q_size, **bf)
        self.attn_proj = torch.empty(H, **bf)
        self.x_post = torch.empty(H, **bf)
        self.x_norm2 = torch.empty(H, **bf)
        self.down = torch.empty(H, **bf)
        self.y = torch.empty(H, **bf)

    def enqueue(self, x: torch.Tensor, normed: bool = False, next_norm=None, step_in: dict | None = None,
                defer: bool = False, norm_in_qkv: bool = False):
        """The layer's launches for the position already in ``pos_dev``.
        ``normed``: ``x_norm`` already holds the input norm (written by the
        previous layer's last launch). ``next_norm`` = (weights, out, pad): the
        last launch also writes the next norm of the output into ``out``.
        ``step_in``: the previous layer's deferred residual step (its
        ``defer`` result), run inside this layer's QKV launch, which computes
        the input norm itself (``x`` is that step's sum_out). ``defer``: leave
        this layer's last residual step to the next layer's QKV launch and
        return (y, step) instead of y. ``norm_in_qkv`` (without ``step_in``
        or ``normed``): the QKV launch computes the input norm of ``x``
        itself (``x_norm`` is then not written). With ``fuse`` the q/k/v
        norms, RoPE and cache insert run inside the attention launch, and the
        post-attention step inside the FFN's gate/up launch (``x_norm2`` is
        then not written)."""
        H, n = self.H, self.norms
        if step_in is not None:
            gemv_bf16_addnorm(self.w_qkv, step_in["resid"], step_in["y"], sum_out=step_in["sum_out"],
                              w_y=step_in["w_y"], scale=step_in["scale"], scale_mode=step_in["scale_mode"],
                              w_x=n["attn"], Y=self.qkv_out)
        elif norm_in_qkv and not normed:
            gemv_bf16_addnorm(self.w_qkv, x, None, w_x=n["attn"], Y=self.qkv_out)
        else:
            if not normed:
                rmsnorm(x, n["attn"], K=H, out=self.x_norm)
            gemv_bf16(self.w_qkv, self.x_norm, self.qkv_out)
        post = dict(heads=self.heads, kv_heads=self.kv_heads, D=self.D, k_off=self.q_size,
                    v_off=self.q_size + self.k_size if self.sliding else -1, q_w=n["q"], k_w=n["k"], norm_v=True,
                    rope=self.rope, q_out=self.q_rope)
        if self.fuse:
            qkv_attention(self.qkv_out, self.pos_dev, self.kcache, self.vcache, window=self.window,
                          out=self.attn_out, **post)
        else:
            qkv_post(self.qkv_out, self.pos_dev, self.kcache, self.vcache, **post)
            attention(self.q_rope, self.kcache, self.vcache, self.pos_dev, heads=self.heads, window=self.window,
                      out=self.attn_out)
        gemv_bf16(self.w_o, self.attn_out, self.attn_proj)
        if self.fuse:
            ffn_fused_bf16_addnorm(self.ffn, x, self.attn_proj, sum_out=self.x_post, w_y=n["post_attn"], w_x=n["ffn"],
                                   Y=self.down)
        else:
            add_norm(x, self.attn_proj, K=H, w_y=n["post_attn"], w_out=n["ffn"], norm_out=True, sum_out=self.x_post,
                     norm_buf=self.x_norm2)
            ffn_fused_bf16(self.ffn, self.x_norm2, self.down)
        if defer:
            return self.y, {"resid": self.x_post, "y": self.down, "w_y": n["post_ffw"], "scale": self.scale,
                            "scale_mode": 1, "sum_out": self.y}
        if next_norm is None:
            add_norm(self.x_post, self.down, K=H, w_y=n["post_ffw"], scale=self.scale, scale_mode=1, sum_out=self.y)
        else:
            w_next, out_next, pad_next = next_norm
            add_norm(self.x_post, self.down, K=H, w_y=n["post_ffw"], scale=self.scale, scale_mode=1, sum_out=self.y,
                     w_out=w_next, norm_out=True, norm_buf=out_next, pad=pad_next)
        return self.y

    def forward(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        if not 0 <= pos < self.max_seq:
            raise ValueError(f"position {pos} outside the cache of {self.max_seq}")
        self.pos_dev.fill_(pos)
        return self.enqueue(x)

    def close(self) -> None:
        self.w_qkv.close()
        self.w_o.close()
        self.ffn.close()


def cos_sin_table_llama(max_seq_len: int) -> np.ndarray:
    """The Llama-3.2 RoPE table (precompute_cos_sin_table,
    runtime/py/model.py:230-261): head dim 64, base 500000, the Llama-3
    frequency scaling (factor 32, low/high frequency factors 1 and 4, original
    context 8192), float32 rows [cos | cos | sin | sin] of the 32 angles (128
    values), then bf16 (returned as uint16 bit patterns)."""
    dim, base, factor, lo, hi, old_ctx = 64, 500000.0, 32.0, 1.0, 4.0, 8192
    inv_freq = 1.0 / (base ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    wavelen = 2 * np.pi / inv_freq
    scaled = np.where(wavelen > old_ctx / lo, inv_freq / factor, inv_freq)
    smooth = np.clip((old_ctx / wavelen - lo) / (hi - lo), 0.0, 1.0)
    smoothed = (1 - smooth) * (inv_freq / factor) + smooth * inv_freq
    inv = np.where((wavelen >= old_ctx / hi) & (wavelen <= old_ctx / lo), smoothed, scaled)
    table = np.zeros((max_seq_len, 128), dtype=np.float32)
    for pos in range(max_seq_len):
        freqs = pos * inv
        c, sn = np.cos(freqs), np.sin(freqs)
        table[pos] = np.concatenate([c, c, sn, sn])
    u = table.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


class _DecodeLayer:
    """A Gemma-3 or Llama-3.2 decoder layer with every step on the device,
    composed of the same launches as Gemma4DecodeLayer: the input norm, one
    QKV GEMV over the rows [q | k | v], the q/k norms (Gemma-3), RoPE and the
    cache insert inside the attention launch (``fuse``) or before it, the O
    GEMV, the post-attention residual step (inside the FFN's gate/up launch
    with ``fuse``) and the last residual step. ``forward(x, pos)`` takes and
    returns bf16 [H] device tensors and updates the KV caches. Subclasses set
    the model's constants (norm eps, which norms exist, activation, RoPE
    table, attention window)."""

    eps: float
    post_norms: bool          # residual steps normalise the branch output (Gemma) or add it as is (Llama)
    qk_norms: bool
    act: str

    def __init__(self, *, qkv, o, gate, up, down, norms: dict, H: int, I: int, heads: int, kv_heads: int, D: int,
                 max_seq: int, window: int, rope_table: np.ndarray, rope_stride: int, sin_off: int, half: int,
                 device, pos_dev: torch.Tensor | None = None, fuse: bool = True):
        dev = torch.device(device)
        self.H, self.I, self.heads, self.kv_heads, self.D = H, I, heads, kv_heads, D
        self.max_seq, self.window, self.device, self.fuse = max_seq, window, dev, fuse
        self.q_size, self.k_size = heads * D, kv_heads * D
        self.n_qkv = self.q_size + 2 * self.k_size
        span = min(window, max_seq) if window > 0 else max_seq
        if max_seq < 1 or span > ATTN_MAX_SPAN:
            raise ValueError(f"max_seq={max_seq}: attention takes up to {ATTN_MAX_SPAN} positions per span")
        if heads % kv_heads:
            raise ValueError(f"heads={heads} is not a multiple of kv_heads={kv_heads}")

        def dev_u8(a):
            return torch.as_tensor(np.ascontiguousarray(a)).to(dev) if isinstance(a, np.ndarray) else a

        self.w_qkv = Q4Weight(dev_u8(qkv), self.n_qkv, H)
        self.w_o = Q4Weight(dev_u8(o), H, self.q_size)
        self.ffn = FfnWeights(dev_u8(gate), dev_u8(up), dev_u8(down), H, I, self.act)
        self.norms = {k: _f32(v, k, D if k in ("q", "k") else H, dev) for k, v in norms.items()}
        self.rope = torch.as_tensor(np.ascontiguousarray(rope_table)).view(torch.bfloat16).to(dev)
        self.rope_args = dict(rope=self.rope, rope_stride=rope_stride, cos_off=0, sin_off=sin_off, half=half)
        if self.rope.numel() < max_seq * rope_stride:
            raise ValueError(f"the RoPE table holds fewer than {max_seq} rows of {rope_stride}")
        self.attn_scale = float(np.float32(1.0 / np.sqrt(D)))
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.kcache = torch.zeros((kv_heads, max_seq, D), **bf)
        self.vcache = torch.zeros((kv_heads, max_seq, D), **bf)
        self.pos_dev = torch.zeros(1, dtype=torch.int32, device=dev) if pos_dev is None else pos_dev
        self.x_norm = torch.empty(H, **bf)
        self.qkv_out = torch.empty(self.n_qkv, **bf)
        self.q_rope = torch.empty(self.q_size, **bf)
        self.attn_out = torch.empty(self.q_size, **bf)
        self.attn_proj = torch.empty(H, **bf)
        self.x_post = torch.empty(H, **bf)
        self.x_norm2 = torch.empty(H, **bf)
        self.down = torch.empty(H, **bf)
        self.y = torch.empty(H, **bf)

    def enqueue(self, x: torch.Tensor) -> torch.Tensor:
        H, n, eps = self.H, self.norms, self.eps
        rmsnorm(x, n["attn"], K=H, eps=eps, out=self.x_norm)
        gemv_bf16(self.w_qkv, self.x_norm, self.qkv_out)
        post = dict(heads=self.heads, kv_heads=self.kv_heads, D=self.D, k_off=self.q_size,
                    v_off=self.q_size + self.k_size, q_w=n.get("q"), k_w=n.get("k"), norm_q=self.qk_norms,
                    norm_k=self.qk_norms, norm_v=False, eps=eps, q_out=self.q_rope, **self.rope_args)
        if self.fuse:
            qkv_attention(self.qkv_out, self.pos_dev, self.kcache, self.vcache, window=self.window,
                          scale=self.attn_scale, out=self.attn_out, **post)
        else:
            qkv_post(self.qkv_out, self.pos_dev, self.kcache, self.vcache, **post)
            attention(self.q_rope, self.kcache, self.vcache, self.pos_dev, heads=self.heads, window=self.window,
                      scale=self.attn_scale, out=self.attn_out)
        gemv_bf16(self.w_o, self.attn_out, self.attn_proj)
        w_post = n.get("post_attn") if self.post_norms else None
        if self.fuse:
            ffn_fused_bf16_addnorm(self.ffn, x, self.attn_proj, sum_out=self.x_post, w_y=w_post,
                                   norm_y=self.post_norms, w_x=n["ffn"], eps=eps, Y=self.down)
        else:
            add_norm(x, self.attn_proj, K=H, w_y=w_post, norm_y=self.post_norms, w_out=n["ffn"], norm_out=True,
                     eps=eps, sum_out=self.x_post, norm_buf=self.x_norm2)
            ffn_fused_bf16(self.ffn, self.x_norm2, self.down)
        add_norm(self.x_post, self.down, K=H, w_y=n.get("post_ffw") if self.post_norms else None,
                 norm_y=self.post_norms, eps=eps, sum_out=self.y)
        return self.y

    def forward(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        if not 0 <= pos < self.max_seq:
            raise IndexError(f"position {pos} outside the cache of {self.max_seq}")
        self.pos_dev.fill_(pos)
        return self.enqueue(x)

    def close(self) -> None:
        self.w_qkv.close()
        self.w_o.close()
        self.ffn.close()


class Gemma3DecodeLayer(_DecodeLayer):
    """One Gemma-3 decoder layer (runtime/py/model.py:632-700; Gemma-3 1B:
    H 1152, 4 q heads and 1 kv head of 256, FFN 6912 GeGLU): RMSNorm eps 1e-6,
    per-head q/k norms with weights, no v norm, RoPE over the whole 256-wide
    head (base 10000 on sliding layers, 1e6 on global ones), attention scaled
    by 1/sqrt(256) over a 512-position window on sliding layers, the
    post-attention and post-FFN norms on the residual adds, no output scale.
    ``qkv`` holds the rows [q | k | v]; norms: attn, q, k, post_attn, ffn,
    post_ffw."""

    eps, post_norms, qk_norms, act = _GEMMA_EPS, True, True, "gelu"

    def __init__(self, *, qkv, o, gate, up, down, norms: dict, sliding: bool, H: int = 1152, I: int = 6912,
                 heads: int = 4, kv_heads: int = 1, D: int = 256, max_seq: int, device, rope_table=None,
                 pos_dev: torch.Tensor | None = None, fuse: bool = True):
        self.sliding = sliding
        if rope_table is None:
            rope_table = cos_sin_table_gemma(10000.0 if sliding else 1000000.0, D, max_seq, gemma4=False)
        super().__init__(qkv=qkv, o=o, gate=gate, up=up, down=down, norms=norms, H=H, I=I, heads=heads,
                         kv_heads=kv_heads, D=D, max_seq=max_seq, window=512 if sliding else 0,
                         rope_table=rope_table, rope_stride=D, sin_off=D // 2, half=D // 2, device=device,
                         pos_dev=pos_dev, fuse=fuse)


class LlamaDecodeLayer(_DecodeLayer):
    """One Llama-3.2 decoder layer (runtime/py/model.py:820-860; Llama-3.2 1B:
    H 2048, 32 q heads and 8 kv heads of 64, FFN 8192 SwiGLU): RMSNorm eps
    1e-5, no q/k norms, RoPE on 64-wide heads from the scaled Llama-3 table
    (cos_sin_table_llama; run_rope_cpu, model.py:533-547), full attention
    scaled by 1/8, the branch outputs added to the residual as they are.
    ``qkv`` holds the rows [q | k | v]; norms: attn, ffn."""

    eps, post_norms, qk_norms, act = 1e-5, False, False, "silu"

    def __init__(self, *, qkv, o, gate, up, down, norms: dict, H: int = 2048, I: int = 8192, heads: int = 32,
                 kv_heads: int = 8, max_seq: int, device, rope_table=None, pos_dev: torch.Tensor | None = None,
                 fuse: bool = True):
        if rope_table is None:
            rope_table = cos_sin_table_llama(max_seq)
        super().__init__(qkv=qkv, o=o, gate=gate, up=up, down=down, norms=norms, H=H, I=I, heads=heads,
                         kv_heads=kv_heads, D=64, max_seq=max_seq, window=0, rope_table=rope_table,
                         rope_stride=128, sin_off=64, half=32, device=device, pos_dev=pos_dev, fuse=fuse)


class Gemma4Decoder:
    """A whole Gemma-4 decode step on the device (runtime/py/model.py:889-915):
    embedding of the token in ``token_dev``, every layer, the final RMSNorm
    (zero-padded to the head's K), the LM head with the 30 tanh(x / 30)
    softcap, and the greedy token (np.argmax, runtime/py/sampler.py:9) written
    back into ``token_dev``; then ``pos_dev`` advances. The next step therefore
    needs nothing from the host: a captured step replays token after token."""

    def __init__(self, layers: list, embed_table: torch.Tensor, final_norm, head: Q4Weight, vocab: int,
                 softcap: float = 30.0, fuse: bool = True):
        self.layers = layers
        self.fuse = fuse
        self.device = head.device
        self.H = layers[0].H
        self.pos_dev = layers[0].pos_dev
        for L in layers:
            if L.pos_dev is not self.pos_dev:
                raise ValueError("the layers must share one pos_dev")
        self.table = embed_table
        self.final_norm = _f32(final_norm, "final_norm", self.H, self.device)
        self.head, self.vocab, self.softcap = head, vocab, softcap
        self.scale = math.sqrt(self.H)
        # Positions the KV caches hold: a step at pos >= max_pos would write
        # past them (the reference raises IndexError there). The host tracks
        # the position through step() and replay(); on the device a step at
        # such a position writes token -1 (never a vocabulary token), so raw
        # graph replays past the end cannot yield a plausible token.
        self.max_pos = min(L.max_seq for L in layers) if layers else 1 << 30
        self.pos_host = 0  # the position of the next step, as last seen by the host
        self.token_dev = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.x = torch.empty(self.H, dtype=torch.bfloat16, device=self.device)
        self.x_norm = torch.empty(head.K, dtype=torch.bfloat16, device=self.device)
        self.logits = torch.empty(vocab, dtype=torch.float32, device=self.device)
        # Steps run on the decoder's own stream: the per-stream scratch that
        # eager steps size is then the scratch a captured step uses.
        self.stream = torch.cuda.Stream(device=self.device)

    def enqueue(self) -> None:
        embed(self.table, self.token_dev, self.scale, out=self.x)
        h = self.x
        n = len(self.layers)
        # fuse: the first layer's QKV launch computes its input norm itself,
        # each layer's last residual step runs inside the next layer's QKV
        # launch (which computes its input norm too), and the last layer's
        # inside the head's GEMV launch with the final norm, zero-padded to
        # the head's K (x_norm is then not written). Unfused: each layer's
        # last launch writes the next layer's input norm, the last layer's
        # the final norm.
        step = None
        for i, L in enumerate(self.layers):
            nxt = self.layers[i + 1] if i + 1 < n else None
            if self.fuse:
                h, step = L.enqueue(h, step_in=step, defer=True, norm_in_qkv=i == 0)
                continue
            next_norm = ((nxt.norms["attn"], nxt.x_norm, self.H) if nxt is not None
                         else (self.final_norm, self.x_norm, self.head.K))
            h = L.enqueue(h, normed=i > 0 and step is None, next_norm=next_norm, step_in=step)
            step = None
        # The head on the bf16 final norm; its last launch also writes token -1
        # past the caches and advances pos_dev.
        if step is not None:
            lm_head_addnorm(self.head, step["resid"], step["y"], hidden=self.H, sum_out=step["sum_out"],
                            w_y=step["w_y"], scale=step["scale"], scale_mode=step["scale_mode"], w_x=self.final_norm,
                            vocab=self.vocab, softcap=self.softcap, logits=self.logits, token=self.token_dev,
                            pos=self.pos_dev, max_pos=self.max_pos)
            return
        if n == 0:
            rmsnorm(h, self.final_norm, K=self.H, pad=self.head.K, out=self.x_norm)
        lm_head(self.head, self.x_norm, self.vocab, self.softcap, self.logits, token=self.token_dev,
                pos=self.pos_dev, max_pos=self.max_pos)

    def _check_pos(self, pos: int) -> None:
        if not 0 <= pos < self.max_pos:
            raise IndexError(f"decode position {pos} outside the KV caches' {self.max_pos} positions")

    def _current_pos(self) -> int:
        # The device position is authoritative (callers may set pos_dev
        # themselves); reading it synchronises, as an eager step does anyway.
        self.pos_host = int(self.pos_dev.item())
        return self.pos_host

    def step(self, token: int | None = None, pos: int | None = None) -> int:
        """One eager step (from `token` at `pos` when given, else from the
        device state); returns the greedy next token. Raises IndexError when
        the position is past the KV caches."""
        p = int(pos) if pos is not None else self._current_pos()
        self._check_pos(p)
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            if token is not None:
                self.token_dev.fill_(int(token))
            if pos is not None:
                self.pos_dev.fill_(p)
            self.enqueue()
            tok = int(self.token_dev.item())
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        self.pos_host = p + 1
        return tok

    def replay(self, graph: torch.cuda.CUDAGraph, steps: int = 1) -> None:
        """Replay a captured step `steps` times on the decoder's stream,
        refusing (IndexError, before anything runs) when the last of them
        would be past the KV caches."""
        p = self._current_pos()
        self._check_pos(p + steps - 1)
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            for _ in range(steps):
                graph.replay()
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        self.pos_host = p + steps

    def capture(self) -> torch.cuda.CUDAGraph:
        """A HIP graph of one step on the decoder's stream (run one eager
        step first: it sizes the stream's scratch, which cannot grow during
        capture). Each replay advances the device state by one token; replay
        it with ``graph.replay()`` under ``torch.cuda.stream(decoder.stream)``
        or after synchronising."""
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            self.enqueue()
        return g

    def set_position(self, pos: int) -> None:
        """Point the next step at `pos` (the device position and the host's
        record of it)."""
        self._check_pos(int(pos))
        self.pos_dev.fill_(int(pos))
        self.pos_host = int(pos)
