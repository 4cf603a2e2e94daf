"""GPU parity of the HIP path against the oracle (C ABI through alveare_amd).

Bars (tests/parity.py): dequant bit-exact; GEMV/GEMM max-relative error
<= 1e-4 against the oracle plus the per-element fp32 bound against fp64; FFN
flip-aware (down projection <= 1e-4 at the GPU's own activation, every
activation flip on a bf16 rounding midpoint within the fp32 bound, end to end
<= 1e-4 plus the flips' exact contribution).
"""
import sys

import numpy as np
import pytest
import torch

import parity

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def run_gemv(W, x, N, K, dev):
    import alveare_amd as aa

    y = torch.empty(N, dtype=torch.float32, device=dev)
    aa.gemv_q(to_dev(W, dev), to_dev(x, dev), y, N=N, K=K)
    torch.cuda.synchronize()
    return y.cpu().numpy()


# ---- dequant -------------------------------------------------------------------

def test_dequant_exhaustive_scales(orc, dev):
    import alveare_amd as aa

    _say("dequant: all bf16 scales with |s| < 2^119, 16 codes x 2 nibble positions")
    W = np.zeros((65536, 20), np.uint8)
    lo = np.arange(16, dtype=np.uint8)
    W[:, :16] = lo | ((15 - lo) << 4)
    s = np.arange(65536, dtype=np.uint32)
    W[:, 16], W[:, 17] = s & 0xFF, s >> 8
    got = aa.dequant_q4(to_dev(W, dev), 65536, 32).view(torch.int16).cpu().numpy().view(np.uint16)
    want = orc.dequant_q4(W, 65536, 32)
    exp_field = (s >> 7) & 0xFF
    dom = exp_field <= 127 + 118  # documented domain: |s| < 2^119
    assert dom.sum() == 2 * 246 * 128
    assert np.array_equal(got[dom], want[dom])


def test_single_token_dequant_exact_scales(orc, dev):
    """The streaming kernel dequantizes with its own instruction
    sequence (q4_device.h::dequant8_mix): a one-hot x selects a dequantized
    column exactly, so every (code, scale) pair of its domain |s| < 2^112 --
    all 16 codes in both nibble positions, every such bf16 scale, subnormal
    ones included -- must match the oracle's dequant bit for bit."""
    import alveare_amd as aa

    _say("streaming-kernel dequant: one-hot GEMV over all bf16 scales with |s| < 2^112")
    s = np.arange(65536, dtype=np.uint32)
    exp_field = (s >> 7) & 0xFF
    s = s[exp_field <= 127 + 111]
    N, K = len(s), 32
    W = np.zeros((N, 20), np.uint8)
    lo = np.arange(16, dtype=np.uint8)
    W[:, :16] = lo | ((15 - lo) << 4)
    W[:, 16], W[:, 17] = s & 0xFF, s >> 8
    want = parity.bf16_f32(orc.dequant_q4(W, N, K).reshape(N, K))
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    for k in range(K):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        y = w(to_dev(x, dev))
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        # -0.0 vs +0.0 of an exactly zero product is not distinguished.
        assert np.array_equal(got, want[:, k]), f"column {k}"
    w.close()


def test_dequant_random_matches_oracle(orc, dev):
    import alveare_amd as aa

    N, K = 300, 1152
    W = orc.synth_q4(N, K, 77)
    got = aa.dequant_q4(to_dev(W, dev), N, K).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, orc.dequant_q4(W, N, K))


# ---- GEMV ------------------------------------------------------------------------

GEMV_SHAPES = [
    (2048, 2048, "c1"),       # single gemv_q at the reference CPU path's size
    (256, 256, "ref42"),      # tests/test_gemv_q.py:76-91 style (seed 42, U(-1,1) quantized)
    (2560, 2560, "ref42"),    # tests/test_gemv_q.py:93-114
    (1, 32, "syn"), (17, 96, "syn"), (333, 1152, "syn"), (31, 6912, "syn"),
    (3840, 4096, "syn"),      # O projection
    (8192, 3840, "syn"),      # fused QKV at the 12B-class shape
    (3840, 15360, "syn"),     # FFN down shape
    (100, 480, "syn"),        # K not a multiple of 128 (partial super-steps)
    (64, 16896, "syn"),       # 33 super-steps: K split over workgroups
]


@pytest.mark.parametrize("N,K,kind", GEMV_SHAPES)
def test_gemv_parity(orc, dev, N, K, kind):
    _say(f"gemv N={N} K={K} {kind}")
    if kind == "ref42":
        rng = np.random.default_rng(42)
        Wf = rng.uniform(-1.0, 1.0, size=(N, K)).astype(np.float32)
        x = rng.uniform(-1.0, 1.0, size=(K,)).astype(np.float32)
        W = orc.quantize_q4_0(Wf)
    else:
        W = orc.synth_q4(N, K, orc.seed_for(1, 0) + N + K)
        x = orc.synth_normal(K, orc.seed_for(1, 1) + K)
    y = run_gemv(W, x, N, K, dev)
    err = parity.gemv_check(orc, W, x, y, N, K)
    _say(f"  max-rel {err:.2e}")


def test_gemv_one_hot_and_zero(orc, dev):
    N, K = 4096, 3840
    W = orc.synth_q4(N, K, 5)
    Wd = to_dev(W, dev)
    import alveare_amd as aa

    deq = aa.dequant_q4(Wd, N, K).float().cpu().numpy()
    for k in (0, 7, 31, 32, 1000, K - 1):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        assert np.array_equal(run_gemv(W, x, N, K, dev), deq[:, k])
    assert np.all(run_gemv(W, np.zeros(K, np.float32), N, K, dev) == 0.0)


def test_gemv_deterministic_and_linear(orc, dev):
    N, K = 3840, 15360  # split-K across workgroups
    W = orc.synth_q4(N, K, 8)
    x = orc.synth_normal(K, 9)
    y1 = run_gemv(W, x, N, K, dev)
    y2 = run_gemv(W, x, N, K, dev)
    assert np.array_equal(y1, y2)
    # Scaling x by a power of two scales every product and sum exactly.
    y4 = run_gemv(W, 4.0 * x, N, K, dev)
    assert np.array_equal(y4, 4.0 * y1)


def test_gemv_bf16_activation_and_padded_buffers(orc, dev):
    import alveare_amd as aa

    N, K = 1000, 2048
    W = orc.synth_q4(N, K, 12)
    x = orc.bf16_round(orc.synth_normal(K, 13))
    big_w = torch.zeros(W.size + 4096, dtype=torch.uint8, device=dev)  # oversized buffers are allowed
    big_w[: W.size] = to_dev(W.reshape(-1), dev)
    xb = to_dev(x, dev).to(torch.bfloat16)
    y = torch.full((N + 10,), 7.0, device=dev)
    aa.gemv_q(big_w, xb, y, N=N, K=K)
    yc = y.cpu().numpy()
    parity.gemv_check(orc, W, x, yc[:N], N, K)
    assert np.all(yc[N:] == 7.0)
    yb = torch.empty(N, dtype=torch.bfloat16, device=dev)
    aa.gemv_q(big_w, xb, yb, N=N, K=K)
    assert torch.equal(yb, y[:N].to(torch.bfloat16))
    with pytest.raises(RuntimeError, match="too small"):
        aa.gemv_q(big_w[:100], xb, y, N=N, K=K)


# ---- tiled layout and registered weights ---------------------------------------------

@pytest.mark.parametrize("N,K", [(37, 1152), (16, 96), (300, 3840), (5, 32), (64, 15360)])
def test_tile_layout_matches_definition(orc, dev, N, K):
    import alveare_amd as aa

    _say(f"tile N={N} K={K}")
    W = orc.synth_q4(N, K, 4000 + N + K)
    got = aa.q4_tile(to_dev(W, dev), N, K).cpu().numpy()
    assert np.array_equal(got, parity.tile_layout_np(W, N, K))


REG_SHAPES = [(2048, 2048), (8192, 3840), (3840, 4096), (3840, 15360), (333, 1152), (17, 96), (1, 32),
              (100, 480),
              (8704, 3840), (3840, 8192)]  # Gemma-4 global layers: fused q (16 x 512) + k (512), and O


@pytest.mark.parametrize("N,K", REG_SHAPES)
def test_registered_gemv_parity(orc, dev, N, K):
    import alveare_amd as aa

    _say(f"registered gemv N={N} K={K}")
    W = orc.synth_q4(N, K, orc.seed_for(1, 2) + N + K)
    x = orc.synth_normal(K, orc.seed_for(1, 3) + K)
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    y = w(to_dev(x, dev))
    torch.cuda.synchronize()
    err = parity.gemv_check(orc, W, x, y.cpu().numpy(), N, K)
    _say(f"  max-rel {err:.2e}")
    w.close()


@pytest.mark.parametrize("M,N,K", [(3, 3840, 3840), (5, 2000, 2048), (16, 1000, 1152), (8, 3840, 15360),
                                   (40, 700, 3840)])
def test_registered_gemm_parity(orc, dev, M, N, K):
    import alveare_amd as aa

    _say(f"registered gemm M={M} N={N} K={K}")
    W = orc.synth_q4(N, K, 5000 + M)
    X = orc.synth_normal(M * K, 6000 + M).reshape(M, K)
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    Y = w(to_dev(X, dev), M=M).cpu().numpy()
    err = parity.max_rel(Y, orc.gemm_q(W, X, M, N, K))
    _say(f"  max-rel {err:.2e}")
    assert err <= parity.TOL
    for m in sorted({0, M - 1}):
        parity.gemv_check(orc, W, X[m], Y[m], N, K)
    w.close()


def test_registered_split_k_deterministic(orc, dev):
    """Eight tokens against a long K: the launch splits K over workgroups and
    the last of each tile group adds the shares in split order, so repeated
    launches agree bit for bit (and the arrival counters reset themselves)."""
    import alveare_amd as aa

    M, N, K = 8, 3840, 15360
    _say(f"split-K determinism M={M} N={N} K={K}")
    W = orc.synth_q4(N, K, 8100)
    X = orc.synth_normal(M * K, 8101).reshape(M, K)
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    Xd = to_dev(X, dev)
    ys = [w(Xd, M=M).cpu().numpy() for _ in range(3)]
    for y in ys[1:]:
        assert np.array_equal(y, ys[0])
    for m in (0, M - 1):
        parity.gemv_check(orc, W, X[m], ys[0][m], N, K)
    w.close()


def test_prefill_split_k_deterministic(orc, dev):
    """A prefill-sized product whose grid is small enough that K is split over
    workgroups (the last of each tile adds the partial tiles in split order):
    repeated launches agree bit for bit and rows pass the GEMV check."""
    import alveare_amd as aa

    M, N, K = 64, 384, 8192
    _say(f"prefill split-K determinism M={M} N={N} K={K}")
    W = orc.synth_q4(N, K, 8200)
    X = orc.synth_normal(M * K, 8201).reshape(M, K)
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    Xd = to_dev(X, dev)
    ys = [w(Xd, M=M).cpu().numpy() for _ in range(3)]
    for y in ys[1:]:
        assert np.array_equal(y, ys[0])
    for m in (0, 31, M - 1):
        parity.gemv_check(orc, W, X[m], ys[0][m], N, K)
    w.close()


def test_registered_matches_raw_path(orc, dev):
    """Same products through the combined-layout entry point and the registered
    one: equal up to summation order (both within the fp32 bound)."""
    import alveare_amd as aa

    N, K = 3840, 4096
    W = orc.synth_q4(N, K, 77)
    x = orc.synth_normal(K, 78)
    Wd = to_dev(W, dev)
    y_raw = run_gemv(W, x, N, K, dev)
    w = aa.Q4Weight(Wd, N, K)
    y_reg = w(to_dev(x, dev)).cpu().numpy()
    assert parity.max_rel(y_reg, y_raw) <= 1e-6
    w.close()


def test_ffn_gate_up_alone(orc, dev):
    """alv_ffn_gate_up leaves the same activation as the full FFN call."""
    import alveare_amd as aa

    H, I = 1152, 3456
    Wg, Wu, Wd = orc.synth_q4(I, H, 81), orc.synth_q4(I, H, 82), orc.synth_q4(H, I, 83)
    f = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    for M in (1, 3):
        _say(f"ffn gate_up M={M}")
        x = to_dev(orc.synth_normal(M * H, 84 + M), dev)
        f(x, M=M)
        full = f.last_activation(M).cpu().numpy()
        f.gate_up(x, M=M)
        alone = f.last_activation(M).cpu().numpy()
        assert np.array_equal(full, alone)
    f.close()


# ---- op chains ------------------------------------------------------------------------

def test_chain_matches_separate_calls(orc, dev):
    """A layer-shaped chain -- projection, projection reading a slice of the
    first output, FFN reading the second, projection reading the FFN output --
    run as one chain equals the same ops called one by one, and each op passes
    the oracle on the inputs it actually saw."""
    import alveare_amd as aa

    _say("chain layer")
    H, I, NQ, KO = 1152, 3456, 2048, 1024
    Wq, Wo = orc.synth_q4(NQ, H, 61), orc.synth_q4(H, KO, 62)
    Wg, Wu, Wd = orc.synth_q4(I, H, 63), orc.synth_q4(I, H, 64), orc.synth_q4(H, I, 65)
    Wn = orc.synth_q4(NQ, H, 66)
    q = aa.Q4Weight(to_dev(Wq, dev), NQ, H)
    o = aa.Q4Weight(to_dev(Wo, dev), H, KO)
    f = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    n = aa.Q4Weight(to_dev(Wn, dev), NQ, H)
    x = to_dev(orc.synth_normal(H, 67), dev)
    yq, yo, yf, yn = (torch.empty(NQ, device=dev), torch.empty(H, device=dev), torch.empty(H, device=dev),
                      torch.empty(NQ, device=dev))
    for rep in range(3):  # repeated launches reuse (and must reset) the chain counters
        yq.fill_(float("nan")); yo.fill_(float("nan")); yf.fill_(float("nan")); yn.fill_(float("nan"))
        aa.chain_run([(q, x, yq, -1), (o, yq[:KO], yo, 0), (f, yo, yf, 1), (n, yf, yn, 2)])
        got = [t.cpu().numpy().copy() for t in (yq, yo, yf, yn)]
        if rep == 0:
            first = got
        else:
            for a_, b_ in zip(first, got):
                assert np.array_equal(a_, b_), "chain results differ between launches"
    sq = q(x).cpu().numpy()
    so = o(torch.from_numpy(got[0][:KO]).to(dev)).cpu().numpy()
    sf = f(torch.from_numpy(got[1]).to(dev)).cpu().numpy()
    sn = n(torch.from_numpy(got[2]).to(dev)).cpu().numpy()
    # Projections differ from separate calls by summation order only; the FFN
    # may also flip a bf16 rounding of its activation (checked below).
    for a_, b_, tol in zip(got, (sq, so, sf, sn), (1e-6, 1e-6, 2e-3, 1e-6)):
        assert parity.max_rel(a_, b_) <= tol
    parity.gemv_check(orc, Wq, x.cpu().numpy(), got[0], NQ, H)
    parity.gemv_check(orc, Wo, got[0][:KO], got[1], H, KO)
    parity.ffn_check(orc, Wg, Wu, Wd, got[1], H, I, 0, got[2], f.last_activation(1).cpu().numpy()[0])
    parity.gemv_check(orc, Wn, got[2], got[3], NQ, H)
    for h in (q, o, n, f):
        h.close()


def test_chain_long_and_repeated_ffn(orc, dev):
    """A chain longer than one launch holds (the split is transparent) and an
    FFN handle used twice in a row."""
    import alveare_amd as aa

    _say("chain long")
    H, I = 512, 1024
    Wg, Wu, Wd = orc.synth_q4(I, H, 71), orc.synth_q4(I, H, 72), orc.synth_q4(H, I, 73)
    f = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    p = aa.Q4Weight(to_dev(orc.synth_q4(H, H, 74), dev), H, H)
    x = to_dev(orc.bf16_round(orc.synth_normal(H, 75)) * 0.25, dev)
    steps = 12
    ys = [torch.empty(H, device=dev) for _ in range(steps)]
    ops = []
    for i in range(steps):
        h = f if i % 3 else p
        ops.append((h, x if i == 0 else ys[i - 1], ys[i], i - 1))
    aa.chain_run(ops)
    torch.cuda.synchronize()
    cur = x
    for i in range(steps):
        h = f if i % 3 else p
        ref = h(cur).clone()
        tol = 2e-3 if h is f else 1e-6  # the FFN may flip a bf16 rounding of its activation
        assert parity.max_rel(ys[i].cpu().numpy(), ref.cpu().numpy()) <= tol, f"step {i}"
        cur = ys[i]
    f.close()
    p.close()


# ---- GEMM (small M: streaming kernel; from 17 bf16 / 33 fp32 tokens: MFMA tiled kernel) ---

@pytest.mark.parametrize("M,N,K,bf16x", [(2, 3840, 3840, False), (4, 15360, 3840, False),
                                          (8, 3840, 15360, False), (16, 3840, 3840, False),
                                          (19, 1000, 1152, False), (32, 512, 1024, False),
                                          (64, 2048, 3840, True), (100, 777, 2048, False),
                                          (512, 1024, 3840, True), (300, 640, 1024, "mixed"),
                                          (257, 384, 15360, False)])
def test_gemm_parity(orc, dev, M, N, K, bf16x):
    import alveare_amd as aa

    _say(f"gemm M={M} N={N} K={K} bf16x={bf16x}")
    W = orc.synth_q4(N, K, 1000 + M)
    X = orc.synth_normal(M * K, 2000 + M).reshape(M, K)
    if bf16x == "mixed":
        # First 256-token tile fp32-valued except its first row, the second
        # bf16-valued: each tile takes its own number of activation terms.
        X = X.copy()
        X[256:] = orc.bf16_round(X[256:]).reshape(M - 256, K)
        X[0] = orc.bf16_round(X[0])
    elif bf16x:
        X = orc.bf16_round(X).reshape(M, K)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    aa.gemm_q(to_dev(W, dev), to_dev(X, dev), Y, B=M, N=N, K=K)
    torch.cuda.synchronize()
    Yc = Y.cpu().numpy()
    Yr = orc.gemm_q(W, X, M, N, K)
    err = parity.max_rel(Yc, Yr)
    _say(f"  max-rel {err:.2e}")
    assert err <= parity.TOL
    for m in sorted({0, M // 2, M - 1}):
        parity.gemv_check(orc, W, X[m], Yc[m], N, K)


# ---- FFN ---------------------------------------------------------------------------

def _ffn_inputs(orc, H, I, kind, seed):
    if kind == "ref":
        # tests/test_ffn_fused.py:38-58: seed 1726250518, U(-1,1) weights quantized.
        rng = np.random.default_rng(1726250518)
        Wg = orc.quantize_q4_0(rng.uniform(-1, 1, size=(I, H)).astype(np.float32))
        Wu = orc.quantize_q4_0(rng.uniform(-1, 1, size=(I, H)).astype(np.float32))
        Wd = orc.quantize_q4_0(rng.uniform(-1, 1, size=(H, I)).astype(np.float32))
        x = rng.uniform(-1, 1, size=(H,)).astype(np.float32)
        return Wg, Wu, Wd, x[None, :]
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    return Wg, Wu, Wd, None


@pytest.mark.parametrize("H,I,M,act,kind", [(256, 512, 1, "gelu", "ref"), (1024, 2048, 1, "gelu", "syn"),
                                            (1152, 6912, 1, "gelu", "syn"), (1152, 6912, 1, "silu", "syn"),
                                            (3840, 15360, 1, "gelu", "syn"), (3840, 15360, 2, "gelu", "syn"),
                                            (3840, 15360, 4, "gelu", "syn"), (3840, 15360, 8, "gelu", "syn"),
                                            (3840, 15360, 16, "gelu", "syn"),
                                            (1152, 6912, 16, "gelu", "syn"), (1152, 6912, 64, "gelu", "syn")])
def test_ffn_parity(orc, dev, H, I, M, act, kind):
    import alveare_amd as aa

    _say(f"ffn H={H} I={I} M={M} {act} {kind}")
    seed = orc.seed_for(2, 0) + H + M
    Wg, Wu, Wd, X = _ffn_inputs(orc, H, I, kind, seed)
    if X is None:
        X = orc.synth_normal(M * H, seed + 7).reshape(M, H)
    ffn = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I,
                                    activation=act)
    Y = torch.empty((M, H), dtype=torch.float32, device=dev)
    ffn(to_dev(X, dev), Y, M)
    A = ffn.last_activation(M).cpu().numpy()
    Yc = Y.cpu().numpy()
    a_id = 0 if act == "gelu" else 1
    worst, flips, cache = 0.0, 0, {}
    for m in range(M):
        st = parity.ffn_check(orc, Wg, Wu, Wd, X[m], H, I, a_id, Yc[m], A[m], cache=cache)
        worst = max(worst, st["max_rel"])
        flips += st["flips"]
        if m == 0:
            _say(f"  token0 {st}")
    _say(f"  FFN-PARITY H={H} I={I} M={M} {act}: worst end-to-end max-rel {worst:.2e}, "
         f"activation flips {flips} over {M} tokens")
    ffn.close()


@pytest.mark.parametrize("xkind", ["bf16", "fp32"])
def test_ffn_prefill_12b(orc, dev, xkind):
    """Prefill FFN at M = 512 on the 12B-class shape (MFMA tiled kernel, GLU
    epilogue with its second pass, down projection with K = 15360 split over
    workgroups). bf16-valued activations are the reference's prefill input
    (x_bf16); fp32 ones take the three-term passes. Every one of the 512
    tokens is checked (the batched flip-aware check against float64), and
    two tokens also against the float32 oracle."""
    import alveare_amd as aa

    H, I, M = 3840, 15360, 512
    _say(f"ffn prefill H={H} I={I} M={M} x={xkind}")
    seed = orc.seed_for(5, 0)
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    X = orc.synth_normal(M * H, seed + 3).reshape(M, H)
    if xkind == "bf16":
        X = orc.bf16_round(X).reshape(M, H)
    ffn = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    Y = torch.empty((M, H), dtype=torch.float32, device=dev)
    ffn(to_dev(X, dev), Y, M)
    A = ffn.last_activation(M).cpu().numpy()
    Yc = Y.cpu().numpy()
    st = parity.ffn_check_batch(orc, Wg, Wu, Wd, X, H, I, 0, Yc, A)
    _say(f"  FFN-PARITY H={H} I={I} M={M} x={xkind} all {M} tokens: worst end-to-end max-rel {st['max_rel']:.2e} "
         f"(down projection {st['down_max_rel']:.2e}), activation flips {st['flips']} in {st['tokens_with_flips']} "
         f"tokens, {st['tokens_over_tol']} tokens above 1e-4 before the flip budget")
    cache = {}
    for m in (0, M - 1):
        parity.ffn_check(orc, Wg, Wu, Wd, X[m], H, I, 0, Yc[m], A[m], cache=cache)
    ffn.close()


def test_ffn_padded_arrays_dispatch(orc, dev):
    """The reference quantizer's padded FFN arrays (K and N padded past the
    model's H and I, tools/quantize_gemma4.py:177-187) registered through the
    dispatch with the model's H and I: the kernels read the (I, H) and (H, I)
    sub-matrices with the arrays' row stride, which is the reference's CPU
    path (runtime/py/model.py:795-806: x zero-padded, padded activations
    zeroed). The padding holds garbage here, so reading it would show."""
    from alveare_amd.runtime import Q4Dispatch

    H, I, Hp, Ip = 1152, 3456, 1280, 4096
    seed = orc.seed_for(2, 9)
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)

    def padded(W, N, K, Np, Kp, s):
        P = orc.synth_q4(Np, Kp, s)  # garbage everywhere, then the real matrix in the corner
        P = P.reshape(Np, Kp // 32 * 20)
        P[:N, :K // 32 * 20] = W.reshape(N, K // 32 * 20)
        return P

    Pg, Pu, Pd = padded(Wg, I, H, Ip, Hp, seed + 3), padded(Wu, I, H, Ip, Hp, seed + 4), padded(Wd, H, I, Hp, Ip, seed + 5)
    d = Q4Dispatch(H, I, "gemma3", dev)
    l = d.register_ffn(Pg, Pu, Pd)
    x = orc.bf16_round(orc.synth_normal(H, seed + 6))
    y = d.run_ffn_fused_npu(l, torch.from_numpy(x).to(torch.bfloat16))
    assert y.shape == (H,)
    parity.ffn_check(orc, Wg, Wu, Wd, x, H, I, 0, y.float().cpu().numpy(),
                     d.layer_ffn_fused_tensors[l].last_activation(1).cpu().numpy()[0], tol=2 ** -8)
    # host NumPy in and out, as the reference's model graph uses it
    dh = Q4Dispatch(H, I, "gemma3", dev, host_io=True)
    dh.layer_ffn_fused_tensors = d.layer_ffn_fused_tensors
    yh = dh.run_ffn_fused_npu(l, x)
    assert isinstance(yh, np.ndarray) and yh.shape == (H,)
    assert np.array_equal(yh.view(np.uint16), y.view(torch.int16).cpu().numpy().view(np.uint16))
    with pytest.raises(ValueError, match="smaller than"):
        d.register_ffn(Pg[:I - 16], Pu, Pd)
    with pytest.raises(ValueError, match="2-D"):
        d.register_ffn(Pg.reshape(-1), Pu, Pd)


def test_ffn_graph_survives_prefill(orc, dev):
    """A decode FFN captured in a HIP graph keeps working after prefill-sized
    calls (which allocate larger per-stream buffers) and a multi-token decode
    call: replays after them still equal the eager result."""
    import alveare_amd as aa

    H, I = 1152, 3456
    Wg, Wu, Wd = orc.synth_q4(I, H, 91), orc.synth_q4(I, H, 92), orc.synth_q4(H, I, 93)
    f = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    s = torch.cuda.Stream()
    x = to_dev(orc.synth_normal(H, 94), dev)
    y = torch.empty(H, device=dev)
    with torch.cuda.stream(s):
        f(x, y)  # eager call on the capture stream first: its buffers exist before capture
        torch.cuda.synchronize()
        want = y.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            f(x, y)
    for M in (64, 300, 16):
        xm = to_dev(orc.synth_normal(M * H, 95 + M), dev)
        with torch.cuda.stream(s):
            ym = f(xm, M=M)
        torch.cuda.synchronize()
        for m in (0, M - 1):
            parity.ffn_check(orc, Wg, Wu, Wd, xm[m * H:(m + 1) * H].cpu().numpy(), H, I, 0, ym[m].cpu().numpy(),
                             f.last_activation(M).cpu().numpy()[m])
        for _ in range(2):
            y.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, want), f"graph replay after an M={M} call"
    del g
    f.close()


def test_ffn_one_token_sequence(orc, dev):
    """One-token calls back to back: each token's output follows its own
    activation, never the one a previous call left in the handle's scratch, and
    a repeated token repeats bit for bit."""
    import alveare_amd as aa

    H, I = 3840, 15360
    seed = orc.seed_for(2, 0) + 11
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    ffn = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    xs = [orc.synth_normal(H, seed + 10 + t) for t in range(3)]
    outs = []
    for t, x in enumerate(xs):
        y = torch.empty((1, H), dtype=torch.float32, device=dev)
        ffn(to_dev(x[None, :], dev), y, 1)
        A = ffn.last_activation(1).cpu().numpy()
        st = parity.ffn_check(orc, Wg, Wu, Wd, x, H, I, 0, y.cpu().numpy()[0], A[0])
        _say(f"  token {t}: {st}")
        outs.append(y.clone())
    y = torch.empty((1, H), dtype=torch.float32, device=dev)
    ffn(to_dev(xs[0][None, :], dev), y, 1)
    assert torch.equal(y, outs[0])
    ffn.close()


def test_ffn_deterministic(orc, dev):
    import alveare_amd as aa

    H, I = 3840, 15360
    Wg, Wu, Wd = orc.synth_q4(I, H, 1), orc.synth_q4(I, H, 2), orc.synth_q4(H, I, 3)
    ffn = aa.pack_ffn_fused_weights(Wg, Wu, Wd, H, I, device=dev)
    x = to_dev(orc.synth_normal(H, 4), dev)
    y1 = ffn(x).clone()
    y2 = ffn(x).clone()
    assert torch.equal(y1, y2)
    with pytest.raises(ValueError, match="shape mismatch"):
        aa.ffn_fused(ffn, x, y1, H=H, I=I + 32)
    ffn.close()


@pytest.mark.parametrize("H,I", [(3840, 15360), (1152, 6912), (1024, 2048)])
def test_ffn_one_token_both_forms(orc, dev, monkeypatch, H, I):
    """The one-token FFN in one launch (q4_ffn1_kernel: 64 intermediate rows per
    workgroup, the down slice's partial outputs summed in a fixed order by a
    second launch) and in two (gate/up, then down) both meet the oracle, with
    the same activation bit for bit; the one-launch form is deterministic."""
    import alveare_amd as aa

    _say(f"ffn one-token forms H={H} I={I}")
    seed = orc.seed_for(2, 7) + H
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    ffn = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    x = orc.synth_normal(H, seed + 3)
    acts = {}
    for form in ("1", "0"):
        monkeypatch.setenv("ALV_FFN_ONE", form)
        Y = torch.empty((1, H), dtype=torch.float32, device=dev)
        ffn(to_dev(x[None, :], dev), Y, 1)
        acts[form] = ffn.last_activation(1).cpu().numpy()[0]
        st = parity.ffn_check(orc, Wg, Wu, Wd, x, H, I, 0, Y.cpu().numpy()[0], acts[form])
        _say(f"  ALV_FFN_ONE={form}: {st}")
        if form == "1":
            Y2 = torch.empty_like(Y)
            ffn(to_dev(x[None, :], dev), Y2, 1)
            assert torch.equal(Y, Y2)
            # The first launch alone (alv_ffn_partials): one partial output per
            # 64-row slice; the output is their sum in the summing launch's
            # order (group q of 32 adds slices q, q + 32, ..., then the groups
            # in order), bit for bit.
            P = torch.empty((I // 64) * H, dtype=torch.float32, device=dev)
            G = ffn.partials(to_dev(x, dev), P)
            assert G == I // 64
            Pn = P.cpu().numpy().reshape(G, H)
            grp = [np.zeros(H, np.float32) for _ in range(32)]
            for q in range(32):
                for b in range(q, G, 32):
                    grp[q] = (grp[q] + Pn[b]).astype(np.float32)
            want = np.zeros(H, np.float32)
            for q in range(32):
                want = (want + grp[q]).astype(np.float32)
            assert np.array_equal(want, Y.cpu().numpy()[0])
    assert np.array_equal(acts["1"], acts["0"])
    ffn.close()


# ---- runtime/py dispatch -------------------------------------------------------------

def test_dispatch_entry_points(orc, dev):
    from alveare_amd.runtime import Q4Dispatch, ResidentWeight

    H, I = 1152, 6912
    d = Q4Dispatch(H, I, "gemma3", dev)
    Wg, Wu, Wd = orc.synth_q4(I, H, 51), orc.synth_q4(I, H, 52), orc.synth_q4(H, I, 53)
    l = d.register_ffn(Wg, Wu, Wd)
    x = orc.bf16_round(orc.synth_normal(H, 54))
    xb = torch.from_numpy(x).to(torch.bfloat16)
    y = d.run_ffn_fused_npu(l, xb)
    assert y.dtype == torch.bfloat16 and y.shape == (H,)
    st = parity.ffn_check(orc, Wg, Wu, Wd, x, H, I, 0, y.float().cpu().numpy(),
                          d.layer_ffn_fused_tensors[l].last_activation(1).cpu().numpy()[0], tol=2 ** -8)
    # gemv with x shorter than K (zero-padded, model.py:343-346), numpy weights
    N, K = 1024, 2048
    W = orc.synth_q4(N, K, 55)
    xs = orc.bf16_round(orc.synth_normal(1152, 56))
    yg = d.run_gemv_npu(W, torch.from_numpy(xs).to(torch.bfloat16)).float().cpu().numpy()
    xp = np.zeros(K, np.float32)
    xp[:1152] = xs
    ref = orc.bf16_round(orc.gemv_q(W, xp, N, K))
    assert parity.max_rel(yg, ref) <= 2 ** -8
    # resident weights (registered on first use) and a batch
    rw = ResidentWeight(to_dev(W.reshape(-1), dev), W.shape)
    yr = d.run_gemv_npu(rw, torch.from_numpy(xs).to(torch.bfloat16)).float().cpu().numpy()
    assert parity.max_rel(yr, ref) <= 2 ** -8
    Xb = orc.bf16_round(orc.synth_normal(5 * K, 57)).reshape(5, K)
    Yb = d.run_gemm_npu(rw, torch.from_numpy(Xb).to(torch.bfloat16)).float().cpu().numpy()
    assert parity.max_rel(Yb, orc.bf16_round(orc.gemm_q(W, Xb, 5, N, K))) <= 2 ** -8
    del st


@pytest.mark.parametrize("act", [0, 1])
def test_glu_bit_exact(orc, dev, act):
    """The FFN epilogue's GLU (float32 fast path where it provably rounds like
    the reference, float64 otherwise) equals the oracle's bit for bit: every
    bf16 gate value with 2^-24 <= |g| < 2^8, both signs, against 256 up values
    each, plus normally distributed pairs as the FFN produces them."""
    import alveare_amd as aa

    rng = np.random.default_rng(0xA1E0 + act)
    mags = ((np.arange(127 - 24, 127 + 8, dtype=np.uint32)[:, None] << 7)
            | np.arange(128, dtype=np.uint32)[None, :]).ravel() << 16
    gs = np.concatenate([mags, mags | 0x80000000]).view(np.float32)
    ug = orc.bf16_round((rng.standard_normal(256) * np.exp2(rng.integers(-8, 6, 256))).astype(np.float32))
    g1 = np.repeat(gs, ug.size)
    u1 = np.tile(ug, gs.size)
    g2 = orc.bf16_round((rng.standard_normal(1 << 20) * 3.0).astype(np.float32))
    u2 = orc.bf16_round((rng.standard_normal(1 << 20) * 3.0).astype(np.float32))
    g = np.concatenate([g1, g2, np.zeros(4, np.float32)])
    u = np.concatenate([u1, u2, np.array([1.0, -0.0, 0.0, 3.0], np.float32)])
    out = torch.empty(g.size, dtype=torch.float32, device=dev)
    gd, ud = to_dev(g, dev), to_dev(u, dev)
    rc = aa.lib().alv_glu(gd.data_ptr(), ud.data_ptr(), out.data_ptr(), g.size, act,
                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    got = out.cpu().numpy()
    want = orc.glu(g, u, act)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    _say(f"  glu act={act}: {g.size} pairs, {bad.size} mismatches")
    assert bad.size == 0, f"first mismatches at g={g[bad[:4]]}, u={u[bad[:4]]}: {got[bad[:4]]} vs {want[bad[:4]]}"


# ---- LM head ---------------------------------------------------------------------

def _absdot(orc, W, x, N, K, chunk=4096):
    """sum_k |w_ik x_k| per row in fp64 (the scale of row i's fp32 rounding
    error), in row chunks so a 262144-row head fits in memory."""
    W = np.asarray(W).reshape(N, K // 32 * 20)
    xa = np.abs(np.asarray(x, np.float64))
    out = np.empty(N)
    for r0 in range(0, N, chunk):
        n = min(chunk, N - r0)
        out[r0:r0 + n] = np.abs(parity.deq_f64(orc, np.ascontiguousarray(W[r0:r0 + n]), n, K)) @ xa
    return out


def _head_check(orc, W, x, N, K, vocab, softcap, logits, token, y_ref=None):
    """Logits of the GPU head against the reference's head evaluated by NumPy
    (oracle/q4_numpy.py::lm_head_cpu on the oracle's fp32 GEMV). The two fp32
    GEMVs add in different orders: each logit may differ by the fp32 bound
    2 gamma_K sum|w x| of its row, plus one bf16 ulp where that difference
    straddles a rounding midpoint (the softcap's slope is at most 1), plus
    float32 ulps of NumPy's tanh (1 ulp from the correctly rounded one) and
    the product. The token is NumPy's argmax unless the two candidates are
    within those tolerances of each other."""
    from oracle import q4_numpy

    if y_ref is None:
        y_ref = orc.gemv_q(W, x, N, K)
    want, tok_ref = q4_numpy.lm_head_cpu(y_ref, vocab, softcap)
    got = np.asarray(logits, np.float32)
    assert got.shape == (vocab,)
    nan_w, nan_g = np.isnan(want), np.isnan(got)
    assert np.array_equal(nan_w, nan_g), "NaN logits differ"
    ok = ~nan_w
    gamma = K * parity.U32 / (1 - K * parity.U32)
    tol_y = 2 * gamma * _absdot(orc, W, x, N, K)[:vocab]
    yv = np.abs(np.asarray(y_ref[:vocab], np.float64))
    tol = tol_y + (yv + tol_y) * 2.0 ** -7 + np.abs(want.astype(np.float64)) * 2.0 ** -21 + 1e-30
    diff = np.abs(got[ok].astype(np.float64) - want[ok])
    bad = diff > tol[ok]
    if bad.any():
        i = np.nonzero(ok)[0][np.argmax(bad)]
        raise AssertionError(f"{bad.sum()} logits outside tolerance, first {i}: got {got[i]!r} want {want[i]!r} "
                             f"y_ref {y_ref[i]!r} tol {tol[i]:.3e}")
    exact = np.mean(got[ok] == want[ok])
    if token != tok_ref:
        assert not np.isnan(want[tok_ref]) and want[token] >= want[tok_ref] - tol[tok_ref] - tol[token], \
            f"token {token} vs reference {tok_ref}: {want[token]} vs {want[tok_ref]}"
    return exact, tok_ref


@pytest.mark.parametrize("softcap", [30.0, 0.0])
def test_lm_head_reduced_vocab(orc, dev, softcap):
    """A head of 20000 x 4096 (K padded as the reference pads it, x zero past
    3840) sliced to a 19990-token vocabulary; then a row duplicated before the
    maximum (the first index of equal logits wins) and a NaN row (NaN wins,
    the first one)."""
    import alveare_amd as aa

    N, K, vocab = 20000, 4096, 19990
    seed = orc.seed_for(6, 0)
    W = orc.synth_q4(N, K, seed)
    x = np.zeros(K, np.float32)
    x[:3840] = orc.synth_normal(3840, seed + 1)
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    logits, tok = aa.lm_head(w, to_dev(x, dev), vocab, softcap)
    exact, tref = _head_check(orc, W, x, N, K, vocab, softcap, logits.cpu().numpy(), int(tok.item()))
    _say(f"  head softcap={softcap}: token {int(tok.item())} (reference {tref}), {exact:.4%} logits bit-equal")
    w.close()

    best = int(tok.item())
    W2 = W.copy().reshape(N, K // 32 * 20)
    W2[best // 2] = W2[best]          # an earlier row with the same logit wins
    W2[vocab - 3, 16:18] = [0xC0, 0x7F]  # a NaN scale: NaN logit near the end ...
    W2[vocab - 7, 16:18] = [0xC0, 0x7F]  # ... and an earlier one, which wins
    w2 = aa.Q4Weight(to_dev(W2, dev), N, K)
    logits2, tok2 = aa.lm_head(w2, to_dev(x, dev), vocab, softcap)
    _head_check(orc, W2, x, N, K, vocab, softcap, logits2.cpu().numpy(), int(tok2.item()))
    assert int(tok2.item()) == vocab - 7
    W2[vocab - 3, 16:18] = W2[vocab - 7, 16:18] = 0x00
    w2.close()
    w3 = aa.Q4Weight(to_dev(W2, dev), N, K)
    _, tok3 = aa.lm_head(w3, to_dev(x, dev), vocab, softcap)
    assert int(tok3.item()) == best // 2
    w3.close()


def test_lm_head_bf16_and_position(orc, dev):
    """alv_lm_head_bf16: the head on bf16 activations (one MFMA term) gives
    the logits and token of alv_lm_head on the same values widened to fp32,
    bit for bit, also with a NaN row; with a decode position it advances the
    position by one per call and writes token -1 once the position reaches
    max_pos (the decoder's bookkeeping, folded into the head's last launch)."""
    import torch

    import alveare_amd as aa

    N, K, vocab = 20000, 4096, 19990
    seed = orc.seed_for(6, 2)
    W = orc.synth_q4(N, K, seed)
    W = W.reshape(N, K // 32 * 20)
    W[vocab - 11, 16:18] = [0xC0, 0x7F]  # a NaN logit
    x = np.zeros(K, np.float32)
    x[:3840] = orc.bf16_round(orc.synth_normal(3840, seed + 1))
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    xd = to_dev(x, dev)
    for softcap in (30.0, 0.0):
        l32, t32 = aa.lm_head(w, xd, vocab, softcap)
        l16, t16 = aa.lm_head(w, xd.bfloat16(), vocab, softcap)
        assert int(t16.item()) == int(t32.item()) == vocab - 11
        assert np.array_equal(l16.cpu().numpy().view(np.uint32), l32.cpu().numpy().view(np.uint32))
    W[vocab - 11, 16:18] = 0x00
    w.close()
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    lref, tref = aa.lm_head(w, xd, vocab, 30.0)
    exact, tok_ref = _head_check(orc, W.reshape(-1), x, N, K, vocab, 30.0, lref.cpu().numpy(), int(tref.item()))
    pos = torch.tensor([5], dtype=torch.int32, device=dev)
    for p_before, want in ((5, int(tref.item())), (6, int(tref.item())), (7, -1), (8, -1)):
        _, tok = aa.lm_head(w, xd.bfloat16(), vocab, 30.0, pos=pos, max_pos=7)
        assert int(tok.item()) == want, (p_before, int(tok.item()), want)
        assert int(pos.item()) == p_before + 1
    _say(f"  bf16 head: token {int(tref.item())} (reference {tok_ref}), {exact:.4%} logits bit-equal; position advanced")
    w.close()


def test_lm_head_fold_group_counts(orc, dev):
    """The token fold at every grid size the head takes (1 to 256
    workgroups of logits), calls back to back on one stream: the token is
    the np.argmax of the logits the call wrote, a tie of the largest logit
    across workgroups (the lower index wins) and a NaN included."""
    import alveare_amd as aa

    N, K = 20000, 256
    seed = orc.seed_for(6, 3)
    W = orc.synth_q4(N, K, seed).reshape(N, K // 32 * 20)
    w0 = aa.Q4Weight(to_dev(W, dev), N, K)
    x = to_dev(orc.bf16_round(orc.synth_normal(K, seed + 1)), dev)
    r = int(aa.lm_head(w0, x, N, 30.0)[1].item())
    w0.close()
    j = (r + 9000) % N
    W[j] = W[r]  # the largest logit twice, in workgroups far apart: the lower index wins
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    for vocab in (1, 2, 63, 64, 65, 1000, 12346, 16383, 16385, 20000, 7, 20000):
        for softcap in (30.0, 0.0):
            logits, tok = aa.lm_head(w, x, vocab, softcap)
            lg = logits.cpu().numpy()
            assert int(tok.item()) == int(np.argmax(lg)), (vocab, softcap)
            if vocab == N:
                assert int(tok.item()) == min(r, j)
    Wn = W.copy()
    Wn[15000, 16:18] = [0xC0, 0x7F]  # NaN scale: a NaN logit outranks every value
    wn = aa.Q4Weight(to_dev(Wn, dev), N, K)
    _, tok = aa.lm_head(wn, x, 20000, 30.0)
    assert int(tok.item()) == 15000
    _, tok = aa.lm_head(wn, x, 15000, 30.0)  # the NaN row past the vocabulary
    assert int(tok.item()) == int(np.argmax(aa.lm_head(w, x, 15000, 30.0)[0].cpu().numpy()))
    w.close()
    wn.close()


def test_lm_head_full_vocab(orc, dev):
    """The reference's head shape: 262144 x 4096 (671 MB of Q4 weights, the
    largest GEMV of a decode step), softcap 30, whole vocabulary; then through
    the dispatch with host NumPy output, as the reference's model graph takes
    it."""
    import alveare_amd as aa
    from alveare_amd.runtime import Q4Dispatch, ResidentWeight

    N, K = 262144, 4096
    seed = orc.seed_for(6, 1)
    W = orc.synth_q4(N, K, seed)
    x = np.zeros(K, np.float32)
    x[:3840] = orc.bf16_round(orc.synth_normal(3840, seed + 1))
    Wd = to_dev(W, dev)
    w = aa.Q4Weight(Wd, N, K)
    logits, tok = aa.lm_head(w, to_dev(x, dev), N, 30.0)
    y_ref = orc.gemv_q(W, x, N, K)
    exact, tref = _head_check(orc, W, x, N, K, N, 30.0, logits.cpu().numpy(), int(tok.item()), y_ref)
    _say(f"  head 262144x4096: token {int(tok.item())} (reference {tref}), {exact:.4%} logits bit-equal")
    w.close()
    d = Q4Dispatch(3840, 15360, "gemma4", dev, host_io=True)
    rw = ResidentWeight(Wd.reshape(-1), (N, K // 32 * 20))
    lh, th = d.run_lm_head(rw, x[:3840], N)
    assert isinstance(lh, np.ndarray) and th == int(tok.item())
    assert np.array_equal(lh, logits.cpu().numpy())


def test_tiled_split_counters_survive_other_shapes(orc, dev, monkeypatch):
    """The tiled kernel's split-K arrival counters are zero at every launch
    whatever ran on the stream before: fp32 GEMMs whose token flags and
    activation terms fill the stream's scratch alternate with a wider GEMM
    that splits K over more tiles (a counter left non-zero makes a workgroup
    add the partial tiles before the others have written theirs). Every result
    matches the oracle on the first pass and is bit-identical after."""
    import alveare_amd as aa

    monkeypatch.setenv("ALV_TILED_MIN_M", "1")
    cases = []
    for i, (N, K) in enumerate([(3840, 15360), (15360, 3840), (3840, 4096)]):
        W = orc.synth_q4(N, K, 7300 + i)
        x = orc.synth_normal(K, 7310 + i)
        cases.append((N, K, W, x, aa.Q4Weight(to_dev(W, dev), N, K), to_dev(x, dev)))
    first = {}
    for rep in range(4):
        for N, K, W, x, w, xd in cases:
            y = w(xd, M=1).cpu().numpy().reshape(-1)
            if rep == 0:
                parity.gemv_check(orc, W, x, y, N, K)
                first[(N, K)] = y
            else:
                assert np.array_equal(y, first[(N, K)]), f"{N}x{K} pass {rep} differs from pass 0"
    for *_, w, _ in cases:
        w.close()


@pytest.mark.parametrize("M", [1, 8, 16])
def test_tiled_kernel_at_small_m(orc, dev, monkeypatch, M):
    """The MFMA tiled kernel at decode-sized M (ALV_TILED_MIN_M=1 routes every
    product to it, as the benchmark's crossover measurement does): GEMM rows
    and FFN tokens pass the oracle."""
    import alveare_amd as aa

    monkeypatch.setenv("ALV_TILED_MIN_M", "1")
    N, K = 3840, 15360
    W = orc.synth_q4(N, K, 7000 + M)
    X = orc.synth_normal(M * K, 7100 + M).reshape(M, K)
    w = aa.Q4Weight(to_dev(W, dev), N, K)
    Y = w(to_dev(X, dev), M=M).reshape(M, N).cpu().numpy()
    for m in sorted({0, M - 1}):
        parity.gemv_check(orc, W, X[m], Y[m], N, K)
    w.close()
    H, I = 3840, 15360
    seed = orc.seed_for(4, 7)
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    Xf = orc.synth_normal(M * H, seed + 3).reshape(M, H)
    f = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    Yf = torch.empty((M, H), device=dev)
    f(to_dev(Xf, dev), Yf, M)
    A = f.last_activation(M).cpu().numpy()
    cache = {}
    for m in sorted({0, M - 1}):
        parity.ffn_check(orc, Wg, Wu, Wd, Xf[m], H, I, 0, Yf.cpu().numpy()[m], A[m], cache=cache)
    f.close()


# ---- quantizer (tools/convert/gemv_q_convert.py:5-85) ----------------------------

def test_quantize_matches_oracle(orc, dev):
    import alveare_amd as aa

    _say("quantize: edge-case blocks (ties, zeros, subnormals, NaN, inf) and 512 x 4096 N(0, 0.02)")
    w = parity.quant_cases()
    got = aa.quantize_q4(to_dev(w, dev)).cpu().numpy()
    assert np.array_equal(got, orc.quantize_q4_0(w))
    rng = np.random.default_rng(11)
    w2 = rng.normal(0.0, 0.02, size=(512, 4096)).astype(np.float32)
    got2 = aa.quantize_q4(to_dev(w2, dev)).cpu().numpy()
    assert np.array_equal(got2, orc.quantize_q4_0(w2))


def test_quantize_padded_source(orc, dev):
    """quantize_and_pack_tensor (tools/quantize_gemma4.py:26-41): a 300 x 3800
    view with row stride 3840 zero-padded to 320 x 4096, as the reference pads
    the Gemma-4 projections before quantizing."""
    import alveare_amd as aa

    rng = np.random.default_rng(12)
    big = rng.normal(0.0, 0.02, size=(300, 3840)).astype(np.float32)
    src = to_dev(big, dev)[:, :3800]
    assert src.stride(0) == 3840
    got = aa.quantize_q4(src, 320, 4096).cpu().numpy()
    pad = np.zeros((320, 4096), np.float32)
    pad[:300, :3800] = big[:, :3800]
    assert np.array_equal(got, orc.quantize_q4_0(pad))


def test_quantize_into_registered_weight(orc, dev):
    """Q4Weight.quantize gives the weight registering the quantized bytes
    gives: the same GEMV output, bit for bit, and that output passes the GEMV
    bar against the oracle on the oracle's quantization."""
    import alveare_amd as aa

    rng = np.random.default_rng(13)
    N, K = 1000, 2048
    w = rng.normal(0.0, 0.02, size=(N, K)).astype(np.float32)
    x = orc.synth_normal(K, 14)
    wd, xd = to_dev(w, dev), to_dev(x, dev)
    a = aa.Q4Weight.quantize(wd)
    b = aa.Q4Weight(aa.quantize_q4(wd), N, K)
    ya, yb = a(xd).cpu().numpy(), b(xd).cpu().numpy()
    a.close()
    b.close()
    assert np.array_equal(ya, yb)
    parity.gemv_check(orc, orc.quantize_q4_0(w), x, ya, N, K)
