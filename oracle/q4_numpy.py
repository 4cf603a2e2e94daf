"""Second, independent restatement of the reference's CPU path in numpy.

TEST INFRASTRUCTURE ONLY. ``ml_dtypes`` (the reference's bf16 dtype) is not
installed, so bf16 values are carried as float32 arrays holding bf16-exact
numbers, with round-to-nearest-even done on the uint32 view
(``runtime/cpp/src/bf16.cpp:7-20``). Everything else is the reference's own
numpy expressions, so numpy decides dtype promotion and the matmul order:

* ``dequantize_combined``   -- ``tools/ref/gemv_q.py:4-62``
* ``gemv_q_combined``       -- ``tools/ref/gemv_q.py:73-80`` (value before the cast)
* ``ffn_cpu``               -- ``runtime/py/model.py:797-806`` (gelu) and
                              ``:853-860`` (silu)
* ``quantize_to_q4_0``      -- ``tools/convert/gemv_q_convert.py:5-51`` and
                              ``pack_to_combined`` ``:53-85``
* ``lm_head_cpu``           -- ``runtime/py/model.py:904-916`` (bf16 logits,
                              vocabulary slice, float32 softcap) and
                              ``runtime/py/sampler.py:9`` (greedy np.argmax)
"""
from __future__ import annotations

import numpy as np


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bf16, returned as float32 (NaN -> 0x7FC0)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    h = (u >> 16).astype(np.uint32)
    h = np.where(np.isnan(x), np.uint32(0x7FC0), h)
    return (h << 16).astype(np.uint32).view(np.float32)


def dequantize_combined(w_combined: np.ndarray) -> np.ndarray:
    N, kb20 = w_combined.shape
    nb = kb20 // 20
    w = w_combined.reshape(N, nb, 20)
    w_q4 = w[:, :, :16].copy().reshape(N, nb * 16)
    sbits = w[:, :, 16].astype(np.uint32) | (w[:, :, 17].astype(np.uint32) << 8)
    scales = (sbits << 16).view(np.float32)
    q0 = (w_q4 & 0x0F).astype(np.int8)
    q1 = ((w_q4 >> 4) & 0x0F).astype(np.int8)
    q0[q0 >= 8] -= 16
    q1[q1 >= 8] -= 16
    q = np.empty((N, nb * 32), dtype=np.int8)
    q[:, 0::2] = q0
    q[:, 1::2] = q1
    scales_expanded = np.repeat(scales.astype(np.float32), 32, axis=1)
    return bf16_rne(q.astype(np.float32) * scales_expanded)


def gemv_q_combined(w_combined: np.ndarray, x: np.ndarray) -> np.ndarray:
    W = dequantize_combined(w_combined)
    return W.astype(np.float32) @ np.asarray(x).astype(np.float32)


def ffn_cpu(Wg: np.ndarray, Wu: np.ndarray, Wd: np.ndarray, x: np.ndarray, act: str = "gelu",
            return_act: bool = False):
    x = np.asarray(x, np.float32)
    gate = bf16_rne(dequantize_combined(Wg).astype(np.float32) @ x)
    up = bf16_rne(dequantize_combined(Wu).astype(np.float32) @ x)
    gate_fp32 = gate.astype(np.float32)
    up_fp32 = up.astype(np.float32)
    if act == "gelu":
        gelu_out = 0.5 * gate_fp32 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (gate_fp32 + 0.044715 * (gate_fp32 ** 3))))
        geglu_out = gelu_out * up_fp32
    else:
        geglu_out = (gate_fp32 * (1.0 / (1.0 + np.exp(-gate_fp32)))) * up_fp32
    # ml_dtypes casts float64 to bf16 through float32.
    a = bf16_rne(np.asarray(geglu_out).astype(np.float32))
    y = dequantize_combined(Wd).astype(np.float32) @ a.astype(np.float32)
    return (y, a) if return_act else y


def lm_head_cpu(y_fp32: np.ndarray, vocab: int, softcap: float = 30.0):
    """The reference's head after its GEMV: y_fp32 is the GEMV's fp32 value
    (the oracle's gemv_q); the GEMV returns bf16, the model slices to the
    vocabulary and softcaps in float32 (numpy's own division and tanh), the
    sampler takes np.argmax. softcap 0: the C++ generator's raw logits
    (runtime/cpp/src/generator.cpp:48)."""
    logits = bf16_rne(np.asarray(y_fp32, np.float32))
    logits_unmasked = logits[:vocab].astype(np.float32)
    if softcap:
        out = softcap * np.tanh(logits_unmasked / softcap)
    else:
        out = logits_unmasked
    out = np.asarray(out, np.float32)
    return out, int(np.argmax(out))


def quantize_to_q4_0(W: np.ndarray) -> np.ndarray:
    """The reference quantizer followed by pack_to_combined, in the
    reference's numpy expressions: (N, K/32*20) uint8. bf16 scales by
    bf16_rne (ml_dtypes' float32 -> bfloat16 is round-to-nearest-even)."""
    W = np.asarray(W, dtype=np.float32)
    N, K = W.shape
    W_blocks = W.reshape(N, K // 32, 32)
    max_vals = np.max(np.abs(W_blocks), axis=2)
    scales = max_vals / 7.0
    scales[scales == 0.0] = 1.0
    with np.errstate(invalid="ignore"):
        q_blocks = np.round(W_blocks / np.expand_dims(scales, axis=2)).astype(np.int32)
    q = np.clip(q_blocks, -8, 7).reshape(N, K)
    w_q4 = ((q[:, 0::2] & 0x0F) | ((q[:, 1::2] & 0x0F) << 4)).astype(np.uint8)
    sb = (bf16_rne(scales).view(np.uint32) >> 16).astype(np.uint16)
    out = np.zeros((N, K // 32, 20), np.uint8)
    out[:, :, :16] = w_q4.reshape(N, K // 32, 16)
    out[:, :, 16] = sb & 0xFF
    out[:, :, 17] = sb >> 8
    return out.reshape(N, K // 32 * 20)
