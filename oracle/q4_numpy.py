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
* ``rmsnorm_cpu``           -- ``runtime/py/model.py:522-531``
* ``rope_cpu_gemma``        -- ``runtime/py/model.py:549-575``
* ``cos_sin_table_gemma``   -- ``runtime/py/model.py:263-280``
* ``attention_host``        -- ``runtime/py/model.py:577-628``
* ``gemma4_decode_layer``   -- ``runtime/py/model.py:705-790`` (the NPU path:
                              the projections and the FFN are callables)
* ``gemma3_decode_layer``   -- ``runtime/py/model.py:632-700``
* ``llama_decode_layer``    -- ``runtime/py/model.py:820-860``
* ``cos_sin_table_llama``   -- ``runtime/py/model.py:230-261``
* ``rope_cpu_llama``        -- ``runtime/py/model.py:533-547``

bf16 arrays of the reference are float32 arrays of bf16-exact values here, so
``x.astype(np.float32)`` of a bf16 array is the identity and
``.astype(bfloat16)`` is ``bf16_rne``.
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


# ---- host ops of a decode layer (runtime/py/model.py) ------------------------------

def rmsnorm_cpu(x: np.ndarray, w, eps: float = 1e-6) -> np.ndarray:
    """run_rmsnorm_cpu (model.py:522-531): Gemma eps 1e-6 (weights optional),
    Llama eps 1e-5. numpy >= 2 evaluates the scalar arithmetic in float32."""
    x32 = np.asarray(x, np.float32)
    variance = np.mean(x32 ** 2)
    normed = x32 * (1.0 / np.sqrt(variance + eps))
    if w is not None:
        normed = normed * np.asarray(w, np.float32)
    return bf16_rne(normed)


def cos_sin_table_gemma(base: float, dim: int, max_seq_len: int, gemma4: bool = True) -> np.ndarray:
    """precompute_cos_sin_table_gemma (model.py:263-280): (max_seq_len, dim)
    bf16 rows [cos | sin]; Gemma-4's 512-wide global heads rotate only the
    first quarter of the angles (the rest have inv_freq 0: cos 1, sin 0)."""
    if gemma4 and dim == 512:
        rope_angles = int(0.25 * dim // 2)
        inv_freq_rotated = 1.0 / (base ** (np.arange(0, 2 * rope_angles, 2, dtype=np.float32) / dim))
        inv_freq = np.zeros(dim // 2, dtype=np.float32)
        inv_freq[:rope_angles] = inv_freq_rotated
    else:
        inv_freq = 1.0 / (base ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    table = np.zeros((max_seq_len, dim), dtype=np.float32)
    for pos in range(max_seq_len):
        freqs = pos * inv_freq
        table[pos] = np.concatenate([np.cos(freqs), np.sin(freqs)])
    return bf16_rne(table)


def rope_cpu_gemma(x: np.ndarray, cos_sin_row: np.ndarray, dim: int) -> np.ndarray:
    """run_rope_cpu_gemma (model.py:549-575) on one table row: rotate-half
    pairs (i, i + dim/2) of every dim-wide head, float32, then bf16."""
    x_flat = np.asarray(x, np.float32).reshape(-1)
    num_heads = x_flat.shape[0] // dim
    cos = np.asarray(cos_sin_row[:dim // 2], np.float32)
    sin = np.asarray(cos_sin_row[dim // 2:dim], np.float32)
    x_fp32 = x_flat.reshape(num_heads, dim)
    y_fp32 = np.zeros_like(x_fp32)
    for h in range(num_heads):
        x1 = x_fp32[h, :dim // 2]
        x2 = x_fp32[h, dim // 2:]
        y_fp32[h, :dim // 2] = x1 * cos - x2 * sin
        y_fp32[h, dim // 2:] = x2 * cos + x1 * sin
    return bf16_rne(y_fp32.reshape(-1))


def attention_host(q_rope: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, pos: int, num_heads: int,
                   num_kv_heads: int, dim: int, scale: float, window: int = 0) -> np.ndarray:
    """run_attention_host (model.py:577-628) for one token at `pos`: caches are
    (kv_heads, max_seq, dim); window > 0 is a sliding layer's window. float32
    scores, softmax and weighted sum; bf16 out."""
    q = np.asarray(q_rope, np.float32).reshape(num_heads, dim)
    seq_len = pos + 1
    if window > 0:
        W = min(seq_len, window)
        k = np.asarray(k_cache[:, pos + 1 - W:pos + 1, :], np.float32)
        v = np.asarray(v_cache[:, pos + 1 - W:pos + 1, :], np.float32)
    else:
        k = np.asarray(k_cache[:, :seq_len, :], np.float32)
        v = np.asarray(v_cache[:, :seq_len, :], np.float32)
        W = seq_len
    group_ratio = num_heads // num_kv_heads
    if group_ratio > 1:
        k = np.repeat(k, group_ratio, axis=0)
        v = np.repeat(v, group_ratio, axis=0)
    scores = np.zeros((num_heads, W), dtype=np.float32)
    for h in range(num_heads):
        scores[h] = np.dot(k[h], q[h]) * scale
    max_scores = np.max(scores, axis=-1, keepdims=True)
    exp_scores = np.exp(scores - max_scores)
    probs = exp_scores / np.sum(exp_scores, axis=-1, keepdims=True)
    output = np.zeros((num_heads, dim), dtype=np.float32)
    for h in range(num_heads):
        output[h] = np.dot(probs[h], v[h])
    return bf16_rne(output.reshape(-1))


def gemma4_decode_layer(x: np.ndarray, pos: int, sliding: bool, w: dict, qkv_proj, o_proj, ffn,
                        k_cache: np.ndarray, v_cache: np.ndarray, cos_sin_row: np.ndarray, stages: dict | None = None):
    """run_layer for gemma4 (model.py:705-790), NPU path. qkv_proj(x_norm)
    returns the bf16 [q | k | v] rows (v absent on global layers, where v is
    the raw k), o_proj(attn_out) and ffn(x_norm2) the bf16 outputs (first 3840
    used). w holds the float32 norm weights (attn, q, k, post_attn, ffn,
    post_ffw) and the layer output scale. The caches are updated at `pos`.
    `stages` (optional) receives every intermediate."""
    H = x.shape[0]
    q_size = 4096 if sliding else 8192
    k_size = 2048 if sliding else 512
    h_dim = 256 if sliding else 512
    n_heads, n_kv = 16, (8 if sliding else 1)
    st = {} if stages is None else stages
    st["x_norm"] = x_norm = rmsnorm_cpu(x, w["attn"])
    qkv = qkv_proj(x_norm)
    q = qkv[:q_size]
    k = qkv[q_size:q_size + k_size]
    v = qkv[q_size + k_size:q_size + 2 * k_size] if sliding else k
    q_n = np.concatenate([rmsnorm_cpu(q[h * h_dim:(h + 1) * h_dim], w["q"]) for h in range(n_heads)])
    k_n = np.concatenate([rmsnorm_cpu(k[h * h_dim:(h + 1) * h_dim], w["k"]) for h in range(n_kv)])
    v_n = np.concatenate([rmsnorm_cpu(v[h * h_dim:(h + 1) * h_dim], None) for h in range(n_kv)])
    st["q_rope"] = q_rope = rope_cpu_gemma(q_n, cos_sin_row, h_dim)
    k_rope = rope_cpu_gemma(k_n, cos_sin_row, h_dim)
    k_cache[:, pos, :] = k_rope.reshape(n_kv, h_dim)
    v_cache[:, pos, :] = v_n.reshape(n_kv, h_dim)
    st["attn_out"] = attn_out = attention_host(q_rope, k_cache, v_cache, pos, n_heads, n_kv, h_dim, 1.0,
                                               1024 if sliding else 0)
    st["attn_proj"] = attn_proj = o_proj(attn_out)[:H]
    normed = rmsnorm_cpu(attn_proj, w["post_attn"])
    st["x_post"] = x_post = bf16_rne(x + normed)
    st["x_norm2"] = x_norm2 = rmsnorm_cpu(x_post, w["ffn"])
    st["down"] = down = ffn(x_norm2)[:H]
    down_normed = rmsnorm_cpu(down, w["post_ffw"])
    y = bf16_rne(x_post + down_normed)
    st["y"] = y = bf16_rne(y * np.float32(w["scale"]))
    return y


def cos_sin_table_llama(max_seq_len: int) -> np.ndarray:
    """precompute_cos_sin_table (model.py:230-261): Llama-3.2's RoPE for
    64-wide heads, base 500000, the Llama-3 frequency scaling (factor 32,
    low / high frequency factors 1 / 4, original context 8192); rows
    [cos | cos | sin | sin] of the 32 angles, float32, then bf16."""
    dim = 64
    base = 500000.0
    factor = 32.0
    low_freq_factor = 1.0
    high_freq_factor = 4.0
    old_context_len = 8192
    inv_freq = 1.0 / (base ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    low_freq_wavelen = old_context_len / low_freq_factor
    high_freq_wavelen = old_context_len / high_freq_factor
    wavelen = 2 * np.pi / inv_freq
    inv_freq_llama = np.where(wavelen > low_freq_wavelen, inv_freq / factor, inv_freq)
    smooth_factor = np.clip((old_context_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor),
                            0.0, 1.0)
    smoothed_inv_freq = (1 - smooth_factor) * (inv_freq / factor) + smooth_factor * inv_freq
    is_medium_freq = (wavelen >= high_freq_wavelen) & (wavelen <= low_freq_wavelen)
    inv_freq_llama = np.where(is_medium_freq, smoothed_inv_freq, inv_freq_llama)
    table = np.zeros((max_seq_len, 128), dtype=np.float32)
    for pos in range(max_seq_len):
        freqs = pos * inv_freq_llama
        cos_val, sin_val = np.cos(freqs), np.sin(freqs)
        table[pos] = np.concatenate([cos_val, cos_val, sin_val, sin_val])
    return bf16_rne(table)


def rope_cpu_llama(x: np.ndarray, cos_sin_row: np.ndarray) -> np.ndarray:
    """run_rope_cpu (model.py:533-547) on one table row: 64-wide heads, cos
    from the row's first 32 values and sin from values 64..95, rotate-half
    pairs (i, i + 32), float32, then bf16."""
    x_flat = np.asarray(x, np.float32).reshape(-1)
    cos = np.asarray(cos_sin_row[:32], np.float32)
    sin = np.asarray(cos_sin_row[64:96], np.float32)
    num_heads = x_flat.shape[0] // 64
    x_fp32 = x_flat.reshape(num_heads, 64)
    y_fp32 = np.zeros_like(x_fp32)
    for h in range(num_heads):
        x1 = x_fp32[h, :32]
        x2 = x_fp32[h, 32:]
        y_fp32[h, :32] = x1 * cos - x2 * sin
        y_fp32[h, 32:] = x2 * cos + x1 * sin
    return bf16_rne(y_fp32.reshape(-1))


def gemma3_decode_layer(x: np.ndarray, pos: int, sliding: bool, w: dict, qkv_proj, o_proj, ffn,
                        k_cache: np.ndarray, v_cache: np.ndarray, cos_sin_row: np.ndarray, n_heads: int = 4,
                        n_kv: int = 1, h_dim: int = 256, stages: dict | None = None):
    """run_layer for gemma3 (model.py:632-700), NPU path. qkv_proj(x_norm)
    returns the bf16 rows [q | k | v] (the reference's three GEMVs over the
    same input), o_proj and ffn the bf16 outputs (first H used); w holds the
    float32 norm weights (attn, q, k, post_attn, ffn, post_ffw). q and k are
    normalised per head, v is not; attention is scaled by 1/sqrt(h_dim) over
    a 512-position window on sliding layers; no output scale."""
    H = x.shape[0]
    q_size, k_size = n_heads * h_dim, n_kv * h_dim
    st = {} if stages is None else stages
    st["x_norm"] = x_norm = rmsnorm_cpu(x, w["attn"])
    qkv = qkv_proj(x_norm)
    q, k, v = qkv[:q_size], qkv[q_size:q_size + k_size], qkv[q_size + k_size:q_size + 2 * k_size]
    q_n = np.concatenate([rmsnorm_cpu(q[h * h_dim:(h + 1) * h_dim], w["q"]) for h in range(n_heads)])
    k_n = np.concatenate([rmsnorm_cpu(k[h * h_dim:(h + 1) * h_dim], w["k"]) for h in range(n_kv)])
    st["q_rope"] = q_rope = rope_cpu_gemma(q_n, cos_sin_row, h_dim)
    k_rope = rope_cpu_gemma(k_n, cos_sin_row, h_dim)
    k_cache[:, pos, :] = k_rope.reshape(n_kv, h_dim)
    v_cache[:, pos, :] = np.asarray(v, np.float32).reshape(n_kv, h_dim)
    st["attn_out"] = attn_out = attention_host(q_rope, k_cache, v_cache, pos, n_heads, n_kv, h_dim,
                                               1.0 / np.sqrt(h_dim), 512 if sliding else 0)
    st["attn_proj"] = attn_proj = o_proj(attn_out)[:H]
    st["x_post"] = x_post = bf16_rne(x + rmsnorm_cpu(attn_proj, w["post_attn"]))
    st["x_norm2"] = x_norm2 = rmsnorm_cpu(x_post, w["ffn"])
    st["down"] = down = ffn(x_norm2)[:H]
    st["y"] = y = bf16_rne(x_post + rmsnorm_cpu(down, w["post_ffw"]))
    return y


def llama_decode_layer(x: np.ndarray, pos: int, w: dict, qkv_proj, o_proj, ffn, k_cache: np.ndarray,
                       v_cache: np.ndarray, cos_sin_row: np.ndarray, n_heads: int = 32, n_kv: int = 8,
                       stages: dict | None = None):
    """The Llama-3.2 branch of run_layer (model.py:820-860), NPU path:
    RMSNorm eps 1e-5 with weights (attn, ffn), no q/k norms, RoPE on 64-wide
    heads (rope_cpu_llama), full attention scaled by 1/8, the attention and
    FFN outputs added to the residual without a norm."""
    H = x.shape[0]
    q_size, k_size = n_heads * 64, n_kv * 64
    st = {} if stages is None else stages
    st["x_norm"] = x_norm = rmsnorm_cpu(x, w["attn"], eps=1e-5)
    qkv = qkv_proj(x_norm)
    q, k, v = qkv[:q_size], qkv[q_size:q_size + k_size], qkv[q_size + k_size:q_size + 2 * k_size]
    st["q_rope"] = q_rope = rope_cpu_llama(q, cos_sin_row)
    k_rope = rope_cpu_llama(k, cos_sin_row)
    k_cache[:, pos, :] = k_rope.reshape(n_kv, 64)
    v_cache[:, pos, :] = np.asarray(v, np.float32).reshape(n_kv, 64)
    st["attn_out"] = attn_out = attention_host(q_rope, k_cache, v_cache, pos, n_heads, n_kv, 64,
                                               1.0 / np.sqrt(64), 0)
    st["attn_proj"] = attn_proj = o_proj(attn_out)[:H]
    st["x_post"] = x_post = bf16_rne(x + attn_proj)
    st["x_norm2"] = x_norm2 = rmsnorm_cpu(x_post, w["ffn"], eps=1e-5)
    st["down"] = down = ffn(x_norm2)[:H]
    st["y"] = y = bf16_rne(x_post + down)
    return y


def pack_ffn_fused_weights_ref(w_gate: np.ndarray, w_up: np.ndarray, w_down: np.ndarray, H: int, I: int,
                               m_I: int = 32, k_tile: int = 256) -> np.ndarray:
    """The reference's registration-time FFN packing
    (runtime/cpp/src/weights.cpp:94-190), restated: per NPU core, gate and up
    tiles of m_I rows x k_tile columns for every I-block, then four passes of
    down tiles of k_tile rows x m_I columns; cores concatenated (<= 8) or
    interleaved tile by tile per column of 8 (16 or 32 cores). Produces the
    blob NpuRegistry::create_ffn_fused_weight receives."""
    m_H = k_tile
    n_cores = 1
    for c in (32, 16, 8, 4, 2):
        if I % (c * m_I) == 0:
            n_cores = c
            break
    I_div = I // n_cores
    nb_I = I_div // m_I
    cpg = k_tile // 32
    gs, ds = H // 32 * 20, I // 32 * 20
    g = np.asarray(w_gate, np.uint8).reshape(-1)
    u = np.asarray(w_up, np.uint8).reshape(-1)
    d = np.asarray(w_down, np.uint8).reshape(-1)
    tile = m_I * cpg * 20
    n_passes = 4
    dtpp = (H // m_H) // n_passes
    per_core = []
    for c in range(n_cores):
        parts = []
        start_I = c * I_div

        def tile_rows(w, r0, r1, b0, b1, stride):
            for r in range(r0, r1):
                parts.append(w[r * stride + b0:r * stride + b1])

        for b in range(nb_I):
            r0 = start_I + b * m_I
            for hb in range(H // k_tile):
                tile_rows(g, r0, r0 + m_I, hb * cpg * 20, (hb + 1) * cpg * 20, gs)
                tile_rows(u, r0, r0 + m_I, hb * cpg * 20, (hb + 1) * cpg * 20, gs)
        for p in range(n_passes):
            for b in range(nb_I):
                c0 = (start_I // 32) * 20 + b * (m_I // 32) * 20
                for hd in range(p * dtpp, (p + 1) * dtpp):
                    tile_rows(d, hd * m_H, (hd + 1) * m_H, c0, c0 + (m_I // 32) * 20, ds)
        per_core.append(np.concatenate(parts))
    if n_cores in (16, 32):
        rows_per_col = n_cores // 8
        n_tiles = len(per_core[0]) // tile
        out = []
        for col in range(8):
            for t in range(n_tiles):
                for r in range(rows_per_col):
                    out.append(per_core[rows_per_col * col + r][t * tile:(t + 1) * tile])
        return np.concatenate(out)
    return np.concatenate(per_core)
