"""GPU parity of the device-resident decode layer (host ops on the GPU).

Bars: RMSNorm, the q/k/v post-processing (norms, RoPE, cache insert) and the
residual steps bit-exact against the reference's numpy expressions
(oracle/q4_numpy.py); attention within the float32 bound of an fp64
evaluation (the reference's own np.dot order is its BLAS's); bf16 GEMV / FFN
outputs between the bf16 roundings of the fp64 value +- its float32 bound; the
whole layer checked stage by stage, each stage's oracle fed the GPU's own
inputs to that stage, so every stage meets its own bar.
"""
import sys

import numpy as np
import pytest
import torch

import parity
from oracle import q4_numpy as qn

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bf_dev(a, dev):
    """float32 array of bf16-exact values -> torch bfloat16 on dev."""
    bits = parity.f32_bits_bf16(np.asarray(a, np.float32)).view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(bits)).view(torch.bfloat16).to(dev)


def bf_np(t):
    return parity.bits_bf16_f32(parity.bf16_bits(t))


def rnd_bf16(rng, shape, sd=1.0):
    return qn.bf16_rne(rng.normal(0, sd, shape).astype(np.float32))


# ---- RMSNorm (runtime/py/model.py:522-531) ----------------------------------------

@pytest.mark.parametrize("rows,K,weighted", [(1, 3840, True), (16, 256, True), (1, 512, True), (3, 1152, True),
                                              (2, 1000, True), (1, 20480, True), (4, 100, False), (8, 256, False)])
def test_rmsnorm_bit_exact(dev, rows, K, weighted):
    from alveare_amd import layer

    _say(f"rmsnorm rows={rows} K={K} weighted={weighted}")
    rng = np.random.default_rng(K + rows)
    x = rnd_bf16(rng, (rows, K), rng.uniform(0.05, 20))
    w = rng.uniform(0.3, 2.0, K).astype(np.float32) if weighted else None
    pad = K + 64
    out = layer.rmsnorm(bf_dev(x, dev), w, K=K, rows=rows, pad=pad)
    got = bf_np(out).reshape(rows, pad)
    for r in range(rows):
        assert np.array_equal(got[r, :K], qn.rmsnorm_cpu(x[r], w)), f"row {r}"
    assert not got[:, K:].any()


def test_rmsnorm_rounding_edges(dev):
    """bf16 rounding at its edges, through RMSNorm's final products x * inv * w:
    weights that drive them into float32 subnormals (including values that
    round up into the normal range), past the largest bf16 to inf, to NaN
    (canonical 0x7FC0), signed zeros, and exact rounding ties (w chosen so
    that x * inv * w lands halfway between two bf16 values)."""
    from alveare_amd import layer

    rng = np.random.default_rng(1234)
    rows, K = 8, 4096
    x = rnd_bf16(rng, (rows, K), 1.0)
    w = rng.uniform(0.3, 2.0, K).astype(np.float32)
    w[0:512] = rng.uniform(1e-45, 1e-37, 512).astype(np.float32)       # subnormal and just-normal products
    w[512:576] = np.float32(3.0e38)                                     # overflow to +-inf
    w[576:580] = np.float32("nan")
    w[580:584] = [0.0, -0.0, np.float32(1e-45), np.float32(-1e-45)]
    w[584:600] = -w[600:616]                                            # sign flips
    # ties: pick w so that the float32 product is exactly halfway (odd and even
    # bf16 neighbours) for row 0.
    x0 = x[0].astype(np.float32)
    n0 = x0 * (1.0 / np.sqrt(np.mean(x0 ** 2) + 1e-6))
    ties = 0
    for k in range(600, 1100):
        if n0[k] == 0:
            continue
        # (2n + 1) 2^(s - 1), n in [128, 256): halfway between two bf16 values
        target = np.float32((2 * int(rng.integers(128, 256)) + 1) * 2.0 ** int(rng.integers(-30, 10)))
        wk = np.float32(target / n0[k])
        if n0[k] * wk == target:
            w[k] = wk
            ties += 1
    assert ties > 100
    out = layer.rmsnorm(bf_dev(x, dev), w, K=K, rows=rows, pad=K)
    got = parity.bf16_bits(out).reshape(rows, K)
    for r in range(rows):
        want = parity.f32_bits_bf16(qn.rmsnorm_cpu(x[r], w))
        assert np.array_equal(got[r], want), f"row {r}: {np.flatnonzero(got[r] != want)[:8]}"
    assert (got[:, 576:580] == 0x7FC0).all()


# ---- q/k/v post-processing (model.py:742-770) ---------------------------------------

@pytest.mark.parametrize("sliding,pos", [(True, 0), (True, 7), (True, 1500), (False, 0), (False, 2047)])
def test_qkv_post_bit_exact(dev, sliding, pos):
    from alveare_amd import layer

    _say(f"qkv_post sliding={sliding} pos={pos}")
    rng = np.random.default_rng(pos + (1 if sliding else 2))
    D, kv = (256, 8) if sliding else (512, 1)
    q_size, k_size, S = 16 * D, kv * D, 2048
    qkv = rnd_bf16(rng, q_size + (2 if sliding else 1) * k_size, 2.0)
    qw, kw = rng.uniform(0.5, 1.5, D).astype(np.float32), rng.uniform(0.5, 1.5, D).astype(np.float32)
    table = qn.cos_sin_table_gemma(10000.0 if sliding else 1e6, D, S)
    assert np.array_equal(layer.cos_sin_table_gemma(10000.0 if sliding else 1e6, D, S), parity.f32_bits_bf16(table))
    kc = torch.zeros((kv, S, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    pos_dev = torch.tensor([pos], dtype=torch.int32, device=dev)
    q_out = layer.qkv_post(bf_dev(qkv, dev), pos_dev, kc, vc, heads=16, kv_heads=kv, D=D, k_off=q_size,
                           v_off=q_size + k_size if sliding else -1, q_w=qw, k_w=kw, norm_v=True,
                           rope=bf_dev(table, dev))
    q = qkv[:q_size]
    k = qkv[q_size:q_size + k_size]
    v = qkv[q_size + k_size:] if sliding else k
    q_n = np.concatenate([qn.rmsnorm_cpu(q[h * D:(h + 1) * D], qw) for h in range(16)])
    k_n = np.concatenate([qn.rmsnorm_cpu(k[h * D:(h + 1) * D], kw) for h in range(kv)])
    v_n = np.concatenate([qn.rmsnorm_cpu(v[h * D:(h + 1) * D], None) for h in range(kv)])
    assert np.array_equal(bf_np(q_out), qn.rope_cpu_gemma(q_n, table[pos], D))
    kcn, vcn = bf_np(kc).reshape(kv, S, D), bf_np(vc).reshape(kv, S, D)
    assert np.array_equal(kcn[:, pos].reshape(-1), qn.rope_cpu_gemma(k_n, table[pos], D))
    assert np.array_equal(vcn[:, pos].reshape(-1), v_n)
    kcn[:, pos] = 0
    vcn[:, pos] = 0
    assert not kcn.any() and not vcn.any()


# ---- attention (model.py:577-628) ---------------------------------------------------

def _attn_check(q, kc, vc, pos, heads, kv, D, window, got_bits, scale=1.0):
    """fp64 softmax(scale K q) V with the float32 bound (scale a power of two);
    returns the bf16 mismatch count against numpy's own float32 evaluation."""
    g = heads // kv
    seq = pos + 1
    st = max(0, seq - window) if window else 0
    ref = np.empty(heads * D)
    bound = np.empty(heads * D)
    for h in range(heads):
        k64 = kc[h // g, st:seq].astype(np.float64)
        v64 = vc[h // g, st:seq].astype(np.float64)
        qh = q[h * D:(h + 1) * D].astype(np.float64)
        s = (k64 @ qh) * scale
        ds = (D + 2) * 2.0 ** -24 * (np.abs(k64) @ np.abs(qh)) * scale  # float32 score error
        p = np.exp(s - s.max())
        p /= p.sum()
        ref[h * D:(h + 1) * D] = p @ v64
        # score errors move the weights by exp(+-2 ds); plus float32 sums over W and D
        bound[h * D:(h + 1) * D] = (np.expm1(2 * ds.max()) + (seq - st + 16) * 2.0 ** -23) * (p @ np.abs(v64)) + 1e-30
    parity.bf16_interval_check(got_bits, ref, bound, "attention")
    npy = qn.attention_host(q, kc, vc, pos, heads, kv, D, scale, window)
    return int((parity.bits_bf16_f32(got_bits) != npy).sum())


@pytest.mark.parametrize("sliding,pos", [(True, 0), (True, 100), (True, 1023), (True, 1500), (True, 2047),
                                          (False, 0), (False, 700), (False, 2047)])
def test_attention_bound(dev, sliding, pos):
    from alveare_amd import layer

    _say(f"attention sliding={sliding} pos={pos}")
    rng = np.random.default_rng(10 * pos + sliding)
    D, kv, S = (256, 8, 2048) if sliding else (512, 1, 2048)
    kc = rnd_bf16(rng, (kv, S, D), 1.0)
    vc = rnd_bf16(rng, (kv, S, D), 1.0)
    q = rnd_bf16(rng, 16 * D, 0.15)  # scores of a few units: a peaked, not one-hot, softmax
    pos_dev = torch.tensor([pos], dtype=torch.int32, device=dev)
    out = layer.attention(bf_dev(q, dev), bf_dev(kc, dev), bf_dev(vc, dev), pos_dev, heads=16,
                          window=1024 if sliding else 0)
    mism = _attn_check(q, kc, vc, pos, 16, kv, D, 1024 if sliding else 0, parity.bf16_bits(out))
    _say(f"  bf16 outputs differing from numpy's float32 evaluation: {mism} of {16 * D}")
    assert mism <= 16 * D // 50


@pytest.mark.parametrize("D,kv,S,window,pos", [(512, 1, 65536, 0, 60000), (128, 4, 4096, 0, 3000),
                                                (64, 16, 2048, 512, 1800), (128, 2, 1024, 0, 0)])
def test_attention_head_groups(dev, D, kv, S, window, pos):
    """Other head widths and the other head groupings per workgroup (2 q
    heads of 512 over a 65536-position cache, 1024 chunks to merge; 4 at
    D 128; 1 with one q head per kv head) within the same bound."""
    from alveare_amd import layer

    _say(f"attention D={D} kv={kv} S={S} window={window} pos={pos}")
    rng = np.random.default_rng(D + kv + pos)
    kc = rnd_bf16(rng, (kv, S, D), 1.0)
    vc = rnd_bf16(rng, (kv, S, D), 1.0)
    q = rnd_bf16(rng, 16 * D, 0.15)
    pos_dev = torch.tensor([pos], dtype=torch.int32, device=dev)
    out = layer.attention(bf_dev(q, dev), bf_dev(kc, dev), bf_dev(vc, dev), pos_dev, heads=16, window=window)
    mism = _attn_check(q, kc, vc, pos, 16, kv, D, window, parity.bf16_bits(out))
    assert mism <= 16 * D // 50


@pytest.mark.parametrize("sliding,pos", [(True, 0), (True, 63), (True, 64), (True, 1500), (False, 0), (False, 1023),
                                          (False, 2047)])
def test_qkv_attention_fused_bit_identical(dev, sliding, pos):
    """alv_qkv_attention gives what alv_qkv_post then alv_attention give,
    bit for bit -- attention output, rotated q and both caches -- also when
    the cache row at pos holds NaN beforehand (the fused kernel must use the
    new k and v, not the row it loaded)."""
    from alveare_amd import layer

    _say(f"qkv_attention sliding={sliding} pos={pos}")
    rng = np.random.default_rng(50 + pos + sliding)
    D, kv, S = (256, 8, 2048) if sliding else (512, 1, 2048)
    heads, q_size, k_size = 16, 16 * D, kv * D
    n_qkv = q_size + (2 if sliding else 1) * k_size
    qkv = bf_dev(rnd_bf16(rng, n_qkv, 1.0), dev)
    kc0 = rnd_bf16(rng, (kv, S, D), 1.0)
    vc0 = rnd_bf16(rng, (kv, S, D), 1.0)
    qw = rng.uniform(0.5, 1.5, D).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, D).astype(np.float32)
    table = torch.as_tensor(layer.cos_sin_table_gemma(1e4 if sliding else 1e6, D, S)).view(torch.bfloat16).to(dev)
    pos_dev = torch.tensor([pos], dtype=torch.int32, device=dev)
    post = dict(heads=heads, kv_heads=kv, D=D, k_off=q_size, v_off=q_size + k_size if sliding else -1, q_w=qw,
                k_w=kw, norm_v=True, rope=table)
    window = 1024 if sliding else 0
    kc_a, vc_a = bf_dev(kc0, dev), bf_dev(vc0, dev)
    q_a = torch.empty(heads * D, dtype=torch.bfloat16, device=dev)
    layer.qkv_post(qkv, pos_dev, kc_a.view(kv, S, D), vc_a.view(kv, S, D), q_out=q_a, **post)
    out_a = layer.attention(q_a, kc_a.view(kv, S, D), vc_a.view(kv, S, D), pos_dev, heads=heads, window=window)
    kc_b, vc_b = bf_dev(kc0, dev), bf_dev(vc0, dev)
    kc_b.view(kv, S, D)[:, pos].fill_(float("nan"))
    vc_b.view(kv, S, D)[:, pos].fill_(float("nan"))
    q_b = torch.empty(heads * D, dtype=torch.bfloat16, device=dev)
    out_b = layer.qkv_attention(qkv, pos_dev, kc_b.view(kv, S, D), vc_b.view(kv, S, D), q_out=q_b, window=window,
                                **post)
    torch.cuda.synchronize()
    assert np.array_equal(bf_np(out_a), bf_np(out_b))
    assert np.array_equal(bf_np(q_a), bf_np(q_b))
    assert np.array_equal(bf_np(kc_a), bf_np(kc_b))
    assert np.array_equal(bf_np(vc_a), bf_np(vc_b))


# ---- residual steps (model.py:775-788; model.cpp:409-420) ---------------------------

@pytest.mark.parametrize("mode,norm_y,norm_out,K,pad", [(0, True, True, 3840, 4096), (1, True, False, 3840, 4096),
                                                         (2, True, False, 3840, 4096), (0, False, True, 3840, 4096),
                                                         (0, True, True, 1152, 1152), (1, True, True, 5000, 5120),
                                                         (0, True, True, 1001, 1008), (2, False, True, 4096, 4096)])
def test_add_norm_bit_exact(dev, mode, norm_y, norm_out, K, pad):
    """Rows held in registers (K a multiple of 8, pad <= 4096) and the LDS
    paths (wider rows, K not a multiple of 8) give the reference's bits."""
    from alveare_amd import layer

    _say(f"add_norm mode={mode} norm_y={norm_y} norm_out={norm_out} K={K} pad={pad}")
    rng = np.random.default_rng(mode * 4 + norm_y * 2 + norm_out + K)
    rows = 2
    r = rnd_bf16(rng, (rows, K), 4.0)
    y = rnd_bf16(rng, (rows, K), 0.7)
    wy = rng.uniform(0.3, 2.0, K).astype(np.float32)
    wo = rng.uniform(0.3, 2.0, K).astype(np.float32)
    scale = np.float32(0.8125 if mode else 1.0) * np.float32(1.0001)
    s_out, n_out = layer.add_norm(bf_dev(r, dev), bf_dev(y, dev), K=K, rows=rows, w_y=wy, norm_y=norm_y,
                                  scale=float(scale), scale_mode=mode, w_out=wo, norm_out=norm_out, pad=pad)
    got_s = bf_np(s_out).reshape(rows, K)
    for i in range(rows):
        t = qn.rmsnorm_cpu(y[i], wy) if norm_y else y[i]
        s = qn.bf16_rne(r[i] + t)
        if mode == 1:
            s = qn.bf16_rne(s * scale)
        elif mode == 2:
            s = qn.bf16_rne((r[i] + t) * scale)
        assert np.array_equal(got_s[i], s), f"row {i}"
        if norm_out:
            got_n = bf_np(n_out).reshape(rows, pad)
            assert np.array_equal(got_n[i, :K], qn.rmsnorm_cpu(s, wo))
            assert not got_n[i, K:].any()


# ---- bf16 GEMV and FFN (the reference's run_gemv / run_ffn_fused contract) ----------

@pytest.mark.parametrize("M,N,K", [(1, 8192, 3840), (1, 3840, 4096), (4, 2048, 2048), (16, 1024, 3840),
                                   (17, 1024, 3840), (24, 2048, 2048), (64, 1024, 3840)])
def test_gemv_bf16(orc, dev, M, N, K):
    import alveare_amd as aa
    from alveare_amd import layer

    _say(f"gemv_bf16 M={M} N={N} K={K}")
    W = orc.synth_q4(N, K, 100 + M)
    X = qn.bf16_rne(orc.synth_normal(M * K, 101 + M)).reshape(M, K)
    w = aa.Q4Weight(torch.from_numpy(W).to(dev), N, K)
    Y = layer.gemv_bf16(w, bf_dev(X, dev), M=M)
    torch.cuda.synchronize()
    yb = parity.bf16_bits(Y).reshape(M, N)
    flips = sum(parity.gemv_bf16_check(orc, W, X[m], yb[m], N, K) for m in range(M))
    _say(f"  rows rounding away from the fp64 value's bf16: {flips} of {M * N}")
    w.close()


@pytest.mark.parametrize("H,I,M", [(1152, 6912, 1), (3840, 15360, 1), (1152, 6912, 4), (1152, 6912, 20),
                                   (1024, 2048, 64)])
def test_ffn_fused_bf16(orc, dev, H, I, M, monkeypatch):
    """bf16 ends on the same device FFN: gate/up reads the bf16 activation as
    its one term and gives the activation alv_ffn_fused gives for the same
    (bf16-valued) input, bit for bit; the bf16 output is the rounding of
    alv_ffn_fused's float32 output (which meets the FFN bar against the oracle).
    From 17 to 32 tokens the bf16 call takes the tiled kernel and the fp32 one
    the streaming kernel: both are held to the tiled kernel there, so that the
    two runs share one summation order."""
    import alveare_amd as aa
    from alveare_amd import layer

    if 17 <= M < 33:
        monkeypatch.setenv("ALV_TILED_MIN_M", "17")

    _say(f"ffn_fused_bf16 H={H} I={I} M={M}")
    Wg, Wu, Wd = orc.synth_q4(I, H, 200), orc.synth_q4(I, H, 201), orc.synth_q4(H, I, 202)
    X = qn.bf16_rne(orc.synth_normal(M * H, 203)).reshape(M, H)
    F = aa.FfnWeights(*(torch.from_numpy(w).to(dev) for w in (Wg, Wu, Wd)), H, I, "gelu")
    Yb = layer.ffn_fused_bf16(F, bf_dev(X, dev), M=M)
    a_bf = F.last_activation(M).cpu().numpy()
    Y32 = F(torch.from_numpy(X.reshape(-1)).to(dev), M=M)
    a_32 = F.last_activation(M).cpu().numpy()
    torch.cuda.synchronize()
    assert np.array_equal(a_bf, a_32)
    y32 = Y32.cpu().numpy().reshape(M, H)
    got = parity.bits_bf16_f32(parity.bf16_bits(Yb)).reshape(M, H)
    same = got == qn.bf16_rne(y32)
    # where they differ, y32 sits within float32 noise of a bf16 rounding point
    if not same.all():
        off = np.abs(y32[~same].astype(np.float64) - got[~same].astype(np.float64))
        half_ulp = np.abs(got[~same].astype(np.float64)) * 2.0 ** -9
        assert np.all(np.abs(off - half_ulp) <= np.abs(y32[~same]) * 2.0 ** -20 + 1e-30)
    F.close()


# ---- the whole layer, stage by stage (model.py:705-790) -----------------------------

@pytest.mark.parametrize("sliding,fuse", [(True, True), (False, True), (True, False)])
def test_gemma4_layer_stagewise(orc, dev, sliding, fuse):
    """Every stage of a layer against the reference's arithmetic; fused, the
    post-attention residual step runs inside the FFN's launch (x_norm2 is
    then the reference's norm of the GPU's x_post, never written)."""
    from alveare_amd import layer

    H, I, S = 512, 1024, 64
    D, kv = (256, 8) if sliding else (512, 1)
    q_size, k_size = 16 * D, kv * D
    n_qkv = q_size + (2 if sliding else 1) * k_size
    _say(f"gemma4 layer sliding={sliding} H={H} I={I}")
    rng = np.random.default_rng(300 + sliding)
    Wqkv = orc.synth_q4(n_qkv, H, 301)
    Wo = orc.synth_q4(H, q_size, 302)
    Wg, Wu, Wd = orc.synth_q4(I, H, 303), orc.synth_q4(I, H, 304), orc.synth_q4(H, I, 305)
    norms = {k: rng.uniform(0.5, 1.5, D if k in ("q", "k") else H).astype(np.float32)
             for k in ("attn", "q", "k", "post_attn", "ffn", "post_ffw")}
    scale = np.float32(0.6)
    L = layer.Gemma4DecodeLayer(qkv=Wqkv, o=Wo, gate=Wg, up=Wu, down=Wd, norms=norms, scale=float(scale),
                                sliding=sliding, H=H, I=I, max_seq=S, device=dev, fuse=fuse)
    table = qn.cos_sin_table_gemma(10000.0 if sliding else 1e6, D, S)
    kc = np.zeros((kv, S, D), np.float32)
    vc = np.zeros((kv, S, D), np.float32)
    for pos in range(6):
        x = rnd_bf16(rng, H, 1.0)
        y = L.forward(bf_dev(x, dev), pos)
        torch.cuda.synchronize()
        g = {k: bf_np(getattr(L, k)) for k in ("x_norm", "qkv_out", "q_rope", "attn_out", "attn_proj", "x_post",
                                                "x_norm2", "down")}
        assert np.array_equal(g["x_norm"], qn.rmsnorm_cpu(x, norms["attn"]))
        parity.gemv_bf16_check(orc, Wqkv, g["x_norm"], parity.bf16_bits(L.qkv_out), n_qkv, H)
        # norms + rope + cache insert from the GPU's qkv
        qkv = g["qkv_out"]
        q, k = qkv[:q_size], qkv[q_size:q_size + k_size]
        v = qkv[q_size + k_size:] if sliding else k
        q_n = np.concatenate([qn.rmsnorm_cpu(q[h * D:(h + 1) * D], norms["q"]) for h in range(16)])
        k_n = np.concatenate([qn.rmsnorm_cpu(k[h * D:(h + 1) * D], norms["k"]) for h in range(kv)])
        v_n = np.concatenate([qn.rmsnorm_cpu(v[h * D:(h + 1) * D], None) for h in range(kv)])
        assert np.array_equal(g["q_rope"], qn.rope_cpu_gemma(q_n, table[pos], D))
        kc[:, pos] = qn.rope_cpu_gemma(k_n, table[pos], D).reshape(kv, D)
        vc[:, pos] = v_n.reshape(kv, D)
        assert np.array_equal(bf_np(L.kcache).reshape(kv, S, D), kc)
        assert np.array_equal(bf_np(L.vcache).reshape(kv, S, D), vc)
        _attn_check(g["q_rope"], kc, vc, pos, 16, kv, D, 1024 if sliding else 0, parity.bf16_bits(L.attn_out))
        parity.gemv_bf16_check(orc, Wo, g["attn_out"], parity.bf16_bits(L.attn_proj), H, q_size)
        x_post = qn.bf16_rne(x + qn.rmsnorm_cpu(g["attn_proj"], norms["post_attn"]))
        assert np.array_equal(g["x_post"], x_post)
        if fuse:
            g["x_norm2"] = qn.rmsnorm_cpu(x_post, norms["ffn"])
        assert np.array_equal(g["x_norm2"], qn.rmsnorm_cpu(x_post, norms["ffn"]))
        # FFN from the GPU's x_norm2: the layer's bf16 FFN is the rounding of the
        # float32 FFN on the same input, which meets the flip-aware FFN bar.
        a_layer = L.ffn.last_activation().cpu().numpy().reshape(-1)
        y32 = L.ffn(torch.from_numpy(g["x_norm2"]).to(dev)).cpu().numpy().reshape(-1)
        a32 = L.ffn.last_activation().cpu().numpy().reshape(-1)
        assert np.array_equal(a_layer, a32)
        parity.ffn_check(orc, Wg, Wu, Wd, g["x_norm2"], H, I, 0, y32, a_test=a32)
        assert np.array_equal(g["down"], qn.bf16_rne(y32))
        y_ref = qn.bf16_rne(qn.bf16_rne(x_post + qn.rmsnorm_cpu(g["down"], norms["post_ffw"])) * scale)
        assert np.array_equal(bf_np(y), y_ref)
    L.close()


@pytest.mark.parametrize("kind,sliding,fuse", [("gemma3", True, True), ("gemma3", False, False),
                                               ("llama", False, True), ("llama", False, False)])
def test_gemma3_llama_layer_stagewise(orc, dev, kind, sliding, fuse):
    """The Gemma-3 (1B: H 1152, 4 q heads and 1 kv head of 256, FFN 6912
    GeGLU) and Llama-3.2 (1B: H 2048, 32 q heads and 8 kv heads of 64, FFN
    8192 SwiGLU) layers at their real shapes, every stage against the
    reference's arithmetic as the oracle restates it
    (gemma3_decode_layer, llama_decode_layer): norms, RoPE, cache insert and
    the residual steps bit-exact; the projections within the GEMV bound;
    attention within its fp64 bound; the FFN on the GPU's own input."""
    from alveare_amd import layer

    S = 96
    if kind == "gemma3":
        H, I, heads, kv, D = 1152, 6912, 4, 1, 256
        eps, act = 1e-6, 0
    else:
        H, I, heads, kv, D = 2048, 8192, 32, 8, 64
        eps, act = 1e-5, 1
    q_size, k_size = heads * D, kv * D
    n_qkv = q_size + 2 * k_size
    _say(f"{kind} layer sliding={sliding} fuse={fuse} H={H} I={I}")
    rng = np.random.default_rng(400 + sliding + 2 * fuse + (10 if kind == "llama" else 0))
    base = 410 if kind == "gemma3" else 420
    Wqkv = orc.synth_q4(n_qkv, H, base + 1)
    Wo = orc.synth_q4(H, q_size, base + 2)
    Wg, Wu, Wd = orc.synth_q4(I, H, base + 3), orc.synth_q4(I, H, base + 4), orc.synth_q4(H, I, base + 5)
    names = ("attn", "q", "k", "post_attn", "ffn", "post_ffw") if kind == "gemma3" else ("attn", "ffn")
    norms = {k: rng.uniform(0.5, 1.5, D if k in ("q", "k") else H).astype(np.float32) for k in names}
    if kind == "gemma3":
        L = layer.Gemma3DecodeLayer(qkv=Wqkv, o=Wo, gate=Wg, up=Wu, down=Wd, norms=norms, sliding=sliding,
                                    max_seq=S, device=dev, fuse=fuse)
        table = qn.cos_sin_table_gemma(10000.0 if sliding else 1e6, D, S, gemma4=False)
        window = 512 if sliding else 0
    else:
        L = layer.LlamaDecodeLayer(qkv=Wqkv, o=Wo, gate=Wg, up=Wu, down=Wd, norms=norms, max_seq=S, device=dev,
                                   fuse=fuse)
        table = qn.cos_sin_table_llama(S)
        window = 0
    assert np.array_equal(bf_np(L.rope).reshape(S, -1), table)
    kc = np.zeros((kv, S, D), np.float32)
    vc = np.zeros((kv, S, D), np.float32)
    for pos in (0, 1, 2, 40, 95):
        x = rnd_bf16(rng, H, 1.0)
        y = L.forward(bf_dev(x, dev), pos)
        torch.cuda.synchronize()
        g = {k: bf_np(getattr(L, k)) for k in ("x_norm", "qkv_out", "q_rope", "attn_out", "attn_proj", "x_post",
                                                "down")}
        assert np.array_equal(g["x_norm"], qn.rmsnorm_cpu(x, norms["attn"], eps=eps))
        parity.gemv_bf16_check(orc, Wqkv, g["x_norm"], parity.bf16_bits(L.qkv_out), n_qkv, H)
        qkv = g["qkv_out"]
        q, k, v = qkv[:q_size], qkv[q_size:q_size + k_size], qkv[q_size + k_size:]
        if kind == "gemma3":
            q_n = np.concatenate([qn.rmsnorm_cpu(q[h * D:(h + 1) * D], norms["q"]) for h in range(heads)])
            k_n = np.concatenate([qn.rmsnorm_cpu(k[h * D:(h + 1) * D], norms["k"]) for h in range(kv)])
            q_r, k_r = qn.rope_cpu_gemma(q_n, table[pos], D), qn.rope_cpu_gemma(k_n, table[pos], D)
        else:
            q_r, k_r = qn.rope_cpu_llama(q, table[pos]), qn.rope_cpu_llama(k, table[pos])
        assert np.array_equal(g["q_rope"], q_r)
        kc[:, pos] = k_r.reshape(kv, D)
        vc[:, pos] = v.reshape(kv, D)
        assert np.array_equal(bf_np(L.kcache).reshape(kv, S, D), kc)
        assert np.array_equal(bf_np(L.vcache).reshape(kv, S, D), vc)
        _attn_check(g["q_rope"], kc, vc, pos, heads, kv, D, window, parity.bf16_bits(L.attn_out),
                    scale=1.0 / np.sqrt(D))
        parity.gemv_bf16_check(orc, Wo, g["attn_out"], parity.bf16_bits(L.attn_proj), H, q_size)
        branch = qn.rmsnorm_cpu(g["attn_proj"], norms["post_attn"]) if kind == "gemma3" else g["attn_proj"]
        x_post = qn.bf16_rne(x + branch)
        assert np.array_equal(g["x_post"], x_post)
        x_norm2 = qn.rmsnorm_cpu(x_post, norms["ffn"], eps=eps)
        if not fuse:
            assert np.array_equal(bf_np(L.x_norm2), x_norm2)
        y32 = L.ffn(torch.from_numpy(x_norm2).to(dev)).cpu().numpy().reshape(-1)
        parity.ffn_check(orc, Wg, Wu, Wd, x_norm2, H, I, act, y32, a_test=L.ffn.last_activation().cpu().numpy().reshape(-1))
        assert np.array_equal(g["down"], qn.bf16_rne(y32))
        down_b = qn.rmsnorm_cpu(g["down"], norms["post_ffw"]) if kind == "gemma3" else g["down"]
        assert np.array_equal(bf_np(y), qn.bf16_rne(x_post + down_b))
    L.close()


# ---- a whole decode step on the device (model.py:889-915) ---------------------------

def test_gemma4_decoder_step_and_graph(orc, dev):
    """Embedding, two layers (sliding, global), final norm, head and greedy
    token entirely on the device: the embedding and final norm bit-exact, the
    head's bf16 logits within the GEMV bound, the token their np.argmax; a
    captured step replayed from the same state gives the eager steps' logits
    and tokens bit for bit. The head is 64 columns wider than the hidden size
    (the reference pads Gemma-4's K to 4096): the fused decoder computes the
    final norm inside the head's launch, zero-padded, and the first layer's
    input norm inside its QKV launch, with every bit of the unfused
    decoder's launches."""
    import math

    import alveare_amd as aa
    from alveare_amd import layer

    H, I, S, V = 512, 1024, 32, 1000
    rng = np.random.default_rng(400)
    pos_dev = torch.zeros(1, dtype=torch.int32, device=dev)
    layers = []
    for sliding in (True, False):
        D, kv = (256, 8) if sliding else (512, 1)
        n_qkv = 16 * D + (2 if sliding else 1) * kv * D
        norms = {k: rng.uniform(0.5, 1.5, D if k in ("q", "k") else H).astype(np.float32)
                 for k in ("attn", "q", "k", "post_attn", "ffn", "post_ffw")}
        layers.append(layer.Gemma4DecodeLayer(
            qkv=orc.synth_q4(n_qkv, H, 401 + sliding), o=orc.synth_q4(H, 16 * D, 403 + sliding),
            gate=orc.synth_q4(I, H, 405), up=orc.synth_q4(I, H, 406), down=orc.synth_q4(H, I, 407), norms=norms,
            scale=0.7, sliding=sliding, H=H, I=I, max_seq=S, device=dev, pos_dev=pos_dev))
    table_np = rng.normal(0, 0.05, (V, H)).astype(np.float16)
    fnorm = rng.uniform(0.5, 1.5, H).astype(np.float32)
    KH = H + 64
    Wh = orc.synth_q4(V, KH, 408)
    head = aa.Q4Weight(torch.from_numpy(Wh).to(dev), V, KH)
    dec = layer.Gemma4Decoder(layers, torch.from_numpy(table_np).to(dev), fnorm, head, V, softcap=0.0)
    # The same layers unfused (separate residual-step launches): the fused
    # step must give every bit the unfused one gives.
    ref = layer.Gemma4Decoder(layers, torch.from_numpy(table_np).to(dev), fnorm, head, V, softcap=0.0, fuse=False)

    def reset():
        torch.cuda.synchronize()
        for L in layers:
            L.kcache.zero_()
            L.vcache.zero_()
        dec.token_dev.fill_(7)
        pos_dev.fill_(0)
        torch.cuda.synchronize()

    def reset_ref():
        reset()
        ref.token_dev.fill_(7)
        torch.cuda.synchronize()

    reset_ref()
    unfused = []
    for L in layers:
        L.fuse = False
    for step in range(4):
        tok = ref.step()
        torch.cuda.synchronize()
        xn = bf_np(ref.x_norm)
        assert np.array_equal(xn[:H], qn.rmsnorm_cpu(bf_np(layers[-1].y), fnorm))
        assert not xn[H:].any()
        unfused.append((ref.logits.cpu().numpy().copy(), tok, [bf_np(L.y).copy() for L in layers]))
    for L in layers:
        L.fuse = True

    reset()
    eager = []
    for step in range(4):
        _say(f"decoder eager step {step}")
        tok_in = int(dec.token_dev.item())
        tok = dec.step()
        torch.cuda.synchronize()
        assert np.array_equal(dec.logits.cpu().numpy(), unfused[step][0]), f"step {step}: fused logits differ"
        assert tok == unfused[step][1]
        for L, y_ref in zip(layers, unfused[step][2]):
            assert np.array_equal(bf_np(L.y), y_ref)
        x = (table_np[tok_in].astype(np.float32) * np.sqrt(H)).astype(np.float32)
        assert np.array_equal(bf_np(dec.x), qn.bf16_rne(x))
        # The final norm the head's launch computed (zero past H).
        xn = np.zeros(KH, np.float32)
        xn[:H] = qn.rmsnorm_cpu(bf_np(layers[-1].y), fnorm)
        logits = dec.logits.cpu().numpy()
        parity.gemv_bf16_check(orc, Wh, xn, parity.f32_bits_bf16(logits), V, KH)
        assert tok == int(np.argmax(logits))
        eager.append((logits.copy(), tok))
    reset()
    g = dec.capture()
    reset()
    for step in range(4):
        _say(f"decoder graph replay {step}")
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dec.logits.cpu().numpy(), eager[step][0])
        assert int(dec.token_dev.item()) == eager[step][1]
        assert int(pos_dev.item()) == step + 1
    del g
    for L in layers:
        L.close()
    head.close()


@pytest.mark.parametrize("H,KH,softcap", [(3840, 4096, 30.0), (512, 512, 0.0), (992, 1024, 30.0)])
def test_fused_input_and_final_norms(orc, dev, H, KH, softcap):
    """The norms a decode step folds into its matmul launches give the bits
    of the separate launches: the first layer's input norm inside its QKV
    launch (alv_gemv_bf16_addnorm without y) against alv_rmsnorm then
    alv_gemv_bf16; the last residual step and the final norm inside the LM
    head's launch (alv_lm_head_bf16_addnorm, rows H wide on a head K wide,
    the norm zero-padded) against alv_add_norm(pad = K) then
    alv_lm_head_bf16 -- sum_out, logits and token -- and the head on the
    norm of a row alone (no y) against alv_rmsnorm(pad = K) then the head."""
    import alveare_amd as aa
    from alveare_amd import layer

    _say(f"fused input/final norms H={H} KH={KH} softcap={softcap}")
    rng = np.random.default_rng(600 + H)
    V, NQ = 3000, 384
    Wq = aa.Q4Weight(torch.from_numpy(orc.synth_q4(NQ, H, 601)).to(dev), NQ, H)
    head = aa.Q4Weight(torch.from_numpy(orc.synth_q4(V, KH, 602)).to(dev), V, KH)
    resid = bf_dev(rnd_bf16(rng, H, 2.0), dev)
    y = bf_dev(rnd_bf16(rng, H, 0.5), dev)
    w_x = rng.uniform(0.5, 1.5, H).astype(np.float32)
    w_y = rng.uniform(0.5, 1.5, H).astype(np.float32)

    # Input norm inside the QKV launch.
    xn = layer.rmsnorm(resid, w_x, K=H)
    ref_q = layer.gemv_bf16(Wq, xn)
    got_q = layer.gemv_bf16_addnorm(Wq, resid, None, w_x=w_x)
    torch.cuda.synchronize()
    assert torch.equal(got_q.view(torch.int16), ref_q.view(torch.int16))
    parity.gemv_bf16_check(orc, orc.synth_q4(NQ, H, 601), bf_np(xn), parity.bf16_bits(got_q), NQ, H)

    # Last residual step + final norm inside the head's launch.
    s_ref, n_ref = layer.add_norm(resid, y, K=H, w_y=w_y, scale=0.7, scale_mode=1, w_out=w_x, norm_out=True,
                                  pad=KH)
    lg_ref, tok_ref = aa.lm_head(head, n_ref, V, softcap)
    lg_ref, tok_ref = lg_ref.clone(), tok_ref.clone()
    s_got = torch.empty(H, dtype=torch.bfloat16, device=dev)
    lg, tok = layer.lm_head_addnorm(head, resid, y, hidden=H, sum_out=s_got, w_y=w_y, scale=0.7, scale_mode=1,
                                    w_x=w_x, vocab=V, softcap=softcap)
    torch.cuda.synchronize()
    assert torch.equal(s_got.view(torch.int16), s_ref.view(torch.int16))
    assert torch.equal(lg.view(torch.int32), lg_ref.view(torch.int32))
    assert int(tok.item()) == int(tok_ref.item())
    assert not bf_np(n_ref)[H:].any()

    # The head on the norm of a row alone.
    n2 = layer.rmsnorm(resid, w_x, K=H, pad=KH)
    lg2_ref, tok2_ref = aa.lm_head(head, n2, V, softcap)
    lg2_ref, tok2_ref = lg2_ref.clone(), tok2_ref.clone()
    lg2, tok2 = layer.lm_head_addnorm(head, resid, None, hidden=H, w_x=w_x, vocab=V, softcap=softcap)
    torch.cuda.synchronize()
    assert torch.equal(lg2.view(torch.int32), lg2_ref.view(torch.int32))
    assert int(tok2.item()) == int(tok2_ref.item())

    with pytest.raises(ValueError):
        layer.lm_head_addnorm(head, resid, None, hidden=KH + 8, w_x=w_x)
    with pytest.raises(ValueError):
        layer.lm_head_addnorm(head, resid, y, hidden=H, w_x=w_x)  # a step needs sum_out
    Wq.close()
    head.close()


def test_gemma4_decoder_position_bounds(orc, dev):
    """Steps past the KV caches: an eager step or a checked replay at
    position >= max_seq raises IndexError before anything runs (the
    reference raises IndexError writing the cache past max_seq_len); a raw
    graph replay there writes token -1 rather than a token from stale
    attention."""
    import alveare_amd as aa
    from alveare_amd import layer

    H, I, S, V = 256, 512, 3, 300
    rng = np.random.default_rng(500)
    pos_dev = torch.zeros(1, dtype=torch.int32, device=dev)
    D, kv = 256, 8
    n_qkv = 16 * D + 2 * kv * D
    norms = {k: rng.uniform(0.5, 1.5, D if k in ("q", "k") else H).astype(np.float32)
             for k in ("attn", "q", "k", "post_attn", "ffn", "post_ffw")}
    L = layer.Gemma4DecodeLayer(qkv=orc.synth_q4(n_qkv, H, 501), o=orc.synth_q4(H, 16 * D, 502),
                                gate=orc.synth_q4(I, H, 503), up=orc.synth_q4(I, H, 504),
                                down=orc.synth_q4(H, I, 505), norms=norms, scale=0.7, sliding=True, H=H, I=I,
                                max_seq=S, device=dev, pos_dev=pos_dev)
    table = torch.from_numpy(rng.normal(0, 0.05, (V, H)).astype(np.float16)).to(dev)
    head = aa.Q4Weight(torch.from_numpy(orc.synth_q4(V, H, 506)).to(dev), V, H)
    dec = layer.Gemma4Decoder([L], table, rng.uniform(0.5, 1.5, H).astype(np.float32), head, V, softcap=30.0)
    assert dec.max_pos == S
    toks = [dec.step(token=5, pos=0)] + [dec.step() for _ in range(S - 1)]
    assert all(0 <= t < V for t in toks)
    assert int(pos_dev.item()) == S
    with pytest.raises(IndexError):
        dec.step()
    with pytest.raises(IndexError):
        dec.step(token=1, pos=S)
    assert int(pos_dev.item()) == S  # nothing ran
    dec.set_position(S - 1)
    g = dec.capture()  # the captured step itself advances nothing until replayed
    dec.set_position(S - 1)
    dec.replay(g)  # the last position the caches hold
    torch.cuda.synchronize()
    assert 0 <= int(dec.token_dev.item()) < V
    with pytest.raises(IndexError):
        dec.replay(g)
    g.replay()  # unchecked: the device guard marks the token
    torch.cuda.synchronize()
    assert int(dec.token_dev.item()) == -1
    with pytest.raises(ValueError, match="positions"):
        layer.Gemma4DecodeLayer(qkv=orc.synth_q4(8704, H, 1), o=orc.synth_q4(H, 16 * 512, 2), gate=orc.synth_q4(I, H, 3),
                                up=orc.synth_q4(I, H, 4), down=orc.synth_q4(H, I, 5), norms=norms, scale=0.7,
                                sliding=False, H=H, I=I, max_seq=layer.ATTN_MAX_SPAN + 64, device=dev)
    del g
    L.close()
    head.close()
