"""Device dispatch with the semantics of the reference's ``runtime/py`` entry
points (runtime/py/model.py), on PyTorch-ROCm tensors.

``Q4Dispatch`` holds what ``LlamaNPUModel`` keeps for its matmuls -- resident
projection weights and the registered FFN of every layer -- and exposes the
three calls the model graph makes:

* ``run_gemv_npu(W_combined, x_bf16)``  (model.py:283-361)
* ``run_ffn_fused_npu(l, x_bf16)``      (model.py:363-397)
* ``run_gemm_npu(W_combined, x_bf16)``  (model.py:399-485)

Return values follow the reference: bf16 vectors, computed in fp32 and
rounded to nearest even once, with the padding rules of the reference (x
shorter than K is zero-padded; y holds the first N rows). By default they are
torch.bfloat16 tensors on the GPU, so a device-resident caller keeps them
there; ``Q4Dispatch(..., host_io=True)`` returns host NumPy arrays instead,
as the reference's NumPy model graph expects (``ml_dtypes.bfloat16`` when
that package is importable, else the same bits as ``uint16``). The NPU's
per-shape limits (MAX_N/MAX_K chunking, N padded to 256, batch chunks of 16)
do not exist on the GPU, so no chunking happens and the results are the
unchunked fp32 sums.

FFN weights may be the reference quantizer's padded arrays (gate/up
(16384, 4096/32*20), down (4096, 16384/32*20) for a 3840/15360 model,
tools/quantize_gemma4.py:177-187): registration reads the (I, H) and (H, I)
sub-matrices with the arrays' own row stride, as the reference's Python packer
slices them (kernels/ffn_fused/ffn_fused.py:356-392) and its CPU path zeroes
the padded activations (runtime/py/model.py:795-806).
"""
from __future__ import annotations

import os
from pathlib import Path

import numpy as np
import torch

from .ops import FfnWeights, Q4Weight, gemm_q, gemv_q, lm_head, pack_ffn_fused_weights

PROJECTIONS = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]


class ResidentWeight:
    """A device-resident combined-Q4 matrix (model.py:31-35). The first call
    through Q4Dispatch also registers it (the kernels' tiled copy, kept next to
    ``tensor``), so resident weights take the registered-weight kernels."""

    def __init__(self, tensor: torch.Tensor, shape):
        self.tensor = tensor
        self.shape = tuple(int(s) for s in shape)
        self.size = int(np.prod(self.shape))
        self.registered: Q4Weight | None = None

    def q4(self) -> Q4Weight:
        if self.registered is None:
            N, K = _shape_of(self)
            self.registered = Q4Weight(self.tensor.view(self.shape), N, K)
        return self.registered


def _to_device_u8(data, device) -> torch.Tensor:
    if isinstance(data, torch.Tensor):
        return data.to(device=device, dtype=torch.uint8).contiguous()
    arr = np.ascontiguousarray(np.asarray(data, dtype=np.uint8))
    return torch.from_numpy(arr).to(device)


class LazyLayerWeights:
    """Upload a layer's packed projections once and keep them resident
    (model.py:37-56): reads ``blk.{l}.{proj}.weight_packed.npy``."""

    def __init__(self, weights_dir, layer_idx: int, device="cuda"):
        self.weights_dir = Path(weights_dir)
        self.layer_idx = layer_idx
        self._cache: dict[str, ResidentWeight] = {}
        for proj in PROJECTIONS:
            path = self.weights_dir / f"blk.{layer_idx}.{proj}.weight_packed.npy"
            if path.exists():
                data = np.load(path, allow_pickle=False)
                self._cache[proj] = ResidentWeight(_to_device_u8(data.reshape(-1), device), data.shape)

    def __getitem__(self, key: str) -> ResidentWeight:
        return self._cache[key]

    def __contains__(self, key: str) -> bool:
        return key in self._cache

    def clear(self) -> None:
        # Weights stay resident, as in the reference.
        pass


def _shape_of(W) -> tuple[int, int]:
    N = int(W.shape[0])
    K = int(W.shape[1]) // 20 * 32
    return N, K


class Q4Dispatch:
    """The matmul dispatch of the reference model, on one GPU."""

    def __init__(self, hidden_size: int, intermediate_size: int, model_type: str = "gemma4",
                 device: str | torch.device = "cuda", host_io: bool = False):
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.model_type = model_type
        self.device = torch.device(device)
        self.host_io = host_io
        self.layer_ffn_fused_tensors: list[FfnWeights] = []

    # -- registration (model.py:176-194) ------------------------------------
    def activation(self) -> str:
        return "silu" if self.model_type not in ("gemma3", "gemma4") else "gelu"

    def register_ffn(self, w_gate, w_up, w_down) -> int:
        """Register one layer's FFN; returns its layer index. The arrays are
        2-D combined-layout matrices at least (I, H/32*20) and (H, I/32*20);
        larger (padded) arrays contribute their leading sub-matrices."""
        for name, w, rows, K in (("w_gate", w_gate, self.intermediate_size, self.hidden_size),
                                 ("w_up", w_up, self.intermediate_size, self.hidden_size),
                                 ("w_down", w_down, self.hidden_size, self.intermediate_size)):
            shp = tuple(w.shape)
            if len(shp) != 2:
                raise ValueError(f"{name} must be 2-D (rows, K/32*20) so its row stride is known, got {shp}")
            if shp[0] < rows or shp[1] < K // 32 * 20:
                raise ValueError(f"{name} of shape {shp} is smaller than ({rows}, {K // 32 * 20})")
        ffn = pack_ffn_fused_weights(w_gate, w_up, w_down, H=self.hidden_size,
                                     I=self.intermediate_size, activation=self.activation(),
                                     device=self.device)
        self.layer_ffn_fused_tensors.append(ffn)
        return len(self.layer_ffn_fused_tensors) - 1

    def resident(self, W) -> ResidentWeight:
        if isinstance(W, ResidentWeight):
            return W
        arr = W if isinstance(W, torch.Tensor) else np.asarray(W, dtype=np.uint8)
        return ResidentWeight(_to_device_u8(arr, self.device).reshape(-1), tuple(arr.shape))

    def _x(self, x, K: int) -> torch.Tensor:
        x = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x, dtype=np.float32))
        x = x.to(self.device)
        if x.dtype not in (torch.float32, torch.bfloat16):
            x = x.float()
        n = x.shape[-1]
        if n > K:
            raise ValueError(f"activation length {n} exceeds K={K}")
        if n < K:  # model.py:343-346: zero-pad x to K
            pad = torch.zeros(x.shape[:-1] + (K - n,), dtype=x.dtype, device=self.device)
            x = torch.cat([x, pad], dim=-1)
        return x.contiguous()

    def _out(self, y32: torch.Tensor):
        """fp32 result -> the reference's bf16 (round to nearest even), on the
        GPU or, with host_io, as a host NumPy array."""
        yb = y32.to(torch.bfloat16)
        if not self.host_io:
            return yb
        return bf16_to_numpy(yb)

    # -- the three entry points ---------------------------------------------
    def run_gemv_npu(self, W_combined, x_bf16):
        rw = self.resident(W_combined)
        N, K = _shape_of(rw)
        x = self._x(x_bf16, K)
        y = torch.empty(N, dtype=torch.float32, device=self.device)
        if isinstance(W_combined, ResidentWeight):
            rw.q4()(x.float(), y)
        else:  # a per-call array, as the reference's non-resident path uploads per call
            gemv_q(rw.tensor.view(rw.shape), x, y, N=N, K=K)
        return self._out(y)

    def run_ffn_fused_npu(self, l: int, x_bf16):
        ffn = self.layer_ffn_fused_tensors[l]
        x = self._x(x_bf16, self.hidden_size)
        y = ffn(x)
        return self._out(y)

    def run_lm_head(self, W_head, x_norm, vocab_size: int | None = None, softcap: float = 30.0):
        """The head of the reference's decode step (runtime/py/model.py:904-916
        for Gemma; softcap 0 for models without one): x_norm zero-padded to the
        head's K, logits = bf16(W x) sliced to the vocabulary and softcapped in
        float32, plus the greedy token (runtime/py/sampler.py:9). Returns
        (logits, token): float32 logits on the GPU (host NumPy with host_io)
        and the token as an int."""
        rw = self.resident(W_head)
        N, K = _shape_of(rw)
        x = self._x(x_norm, K).float()
        logits, token = lm_head(rw.q4(), x, vocab_size or N, softcap)
        tok = int(token.item())
        if self.host_io:
            return logits.cpu().numpy(), tok
        return logits, tok

    def run_gemm_npu(self, W_combined, x_bf16):
        rw = self.resident(W_combined)
        N, K = _shape_of(rw)
        X = self._x(x_bf16, K)
        if X.ndim != 2:
            raise ValueError("run_gemm_npu takes a (B, K) batch")
        B = X.shape[0]
        Y = torch.empty((B, N), dtype=torch.float32, device=self.device)
        if isinstance(W_combined, ResidentWeight):
            rw.q4()(X.float(), Y, M=B)
        else:
            gemm_q(rw.tensor.view(rw.shape), X, Y, B=B, N=N, K=K)
        return self._out(Y)


def bf16_to_numpy(t: torch.Tensor) -> np.ndarray:
    """A bf16 torch tensor as a host NumPy array with the same bits: dtype
    ml_dtypes.bfloat16 (the reference's array type) when ml_dtypes is
    importable, else uint16 bit patterns."""
    bits = t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    try:
        import ml_dtypes
    except ImportError:
        return bits
    return bits.view(ml_dtypes.bfloat16)


def load_layer_weights(weights_dir, num_layers: int, device="cuda") -> list[LazyLayerWeights]:
    """Resident weights of every layer (model.py:118-120)."""
    return [LazyLayerWeights(weights_dir, l, device) for l in range(num_layers)]


__all__ = ["ResidentWeight", "LazyLayerWeights", "Q4Dispatch", "load_layer_weights", "bf16_to_numpy", "PROJECTIONS"]
