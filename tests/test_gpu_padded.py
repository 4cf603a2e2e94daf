"""Padded shapes: the reference's quantizer and C++ runtime register Gemma-4's
matrices zero-padded (K 3840 stored as 4096, tools/quantize_gemma4.py:145-187;
the sliding O projection padded to 8192 rows so it shares the QKV context,
runtime/cpp/src/weights.cpp:318-327; the FFN 15360 x 3840 stored as 16384 x
4096). Registration trims trailing all-zero rows and 32-column blocks, so a
call streams the real matrix only. These tests check that a padded
registration executes the real shape and returns what the reference computes
on the padded arrays: the real rows bit for bit equal to the unpadded
registration's (the same kernels on the same bytes), the trimmed rows exact
zeros (the reference's 0 * x sums, up to the sign of zero), and the oracle on
the padded arrays within the contract."""
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


def pad_q4(W, N, K, Np, Kp):
    """The combined-layout matrix W (N x K) zero-padded to Np x Kp, as the
    reference's quantizer writes it (zero weights, zero scales)."""
    P = np.zeros((Np, Kp // 32 * 20), np.uint8)
    P[:N, :K // 32 * 20] = W.reshape(N, K // 32 * 20)
    return P


# (padded N, padded K, real N, real K): the reference runtime's registered
# shapes for a 3840-hidden Gemma-4 layer, and a small one the oracle checks.
GEMV_PADDED = [
    (8192, 4096, 8192, 3840),    # sliding fused QKV, K padded
    (8192, 4096, 3840, 4096),    # sliding O padded to the QKV context's 8192 rows
    (10240, 4096, 8704, 3840),   # global fused QK: q 8192 + k 512 padded to 2048 rows, K padded
    (4096, 8192, 3840, 8192),    # global O, rows padded
    (16384, 4096, 16384, 3840),  # LM-head chunk, K padded
    (333, 1184, 250, 1056),
]


@pytest.mark.parametrize("Np,Kp,N,K", GEMV_PADDED)
def test_padded_gemv_equals_unpadded(orc, dev, Np, Kp, N, K):
    import alveare_amd as aa

    _say(f"padded gemv {Np}x{Kp} (real {N}x{K})")
    W = orc.synth_q4(N, K, orc.seed_for(3, 1) + N + K)
    P = pad_q4(W, N, K, Np, Kp)
    x = orc.synth_normal(Kp, orc.seed_for(3, 2) + Kp)  # finite values in the padding too: 0 * x is 0
    wp = aa.Q4Weight(to_dev(P, dev), Np, Kp)
    wr = aa.Q4Weight(to_dev(W, dev), N, K)
    assert wp.exec_shape == (N, K)
    assert wr.exec_shape == (N, K)
    yp = wp(to_dev(x, dev)).cpu().numpy()
    yr = wr(to_dev(x[:K].copy(), dev)).cpu().numpy()
    assert np.array_equal(yp[:N].view(np.uint32), yr.view(np.uint32)), "real rows differ from the unpadded call"
    assert np.all(yp[N:] == 0.0), "trimmed rows must be zero"
    if Np * Kp <= 1 << 20:
        err = parity.gemv_check(orc, P, x, yp, Np, Kp)  # the oracle on the padded arrays
        _say(f"  max-rel vs oracle on the padded matrix {err:.2e}")
    wp.close()
    wr.close()


@pytest.mark.parametrize("M", [4, 16, 40])
def test_padded_multi_token(orc, dev, M):
    """Several tokens (the streaming kernel's token groups at 4 and 16, the
    prefill GEMM at 40): trimmed rows are zero for every token."""
    import alveare_amd as aa

    Np, Kp, N, K = 1200, 1088, 1000, 960
    _say(f"padded gemm M={M} {Np}x{Kp} (real {N}x{K})")
    W = orc.synth_q4(N, K, 777 + M)
    P = pad_q4(W, N, K, Np, Kp)
    X = orc.synth_normal(M * Kp, 778 + M).reshape(M, Kp)
    wp = aa.Q4Weight(to_dev(P, dev), Np, Kp)
    wr = aa.Q4Weight(to_dev(W, dev), N, K)
    Yp = torch.full((M, Np), float("nan"), device=dev)  # every element must be written
    wp(to_dev(X, dev), Yp, M=M)
    Yr = wr(to_dev(np.ascontiguousarray(X[:, :K]), dev), M=M).cpu().numpy()
    Yp = Yp.cpu().numpy()
    assert np.array_equal(Yp[:, :N].view(np.uint32), Yr.view(np.uint32))
    assert np.all(Yp[:, N:] == 0.0)
    err = parity.max_rel(Yp, orc.gemm_q(P, X, M, Np, Kp))
    _say(f"  max-rel vs oracle {err:.2e}")
    assert err <= parity.TOL
    wp.close()
    wr.close()


def test_padded_bf16_entry_point(orc, dev):
    import alveare_amd as aa
    from alveare_amd._lib import check, lib

    Np, Kp, N, K = 512, 1024, 400, 992
    W = orc.synth_q4(N, K, 4242)
    P = pad_q4(W, N, K, Np, Kp)
    x = orc.bf16_round(orc.synth_normal(Kp, 4243))
    xb = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    wp = aa.Q4Weight(to_dev(P, dev), Np, Kp)
    wr = aa.Q4Weight(to_dev(W, dev), N, K)
    yp = torch.full((Np,), float("nan"), dtype=torch.bfloat16, device=dev)
    yr = torch.empty(N, dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    check(lib().alv_gemv_bf16(wp.handle, xb.data_ptr(), yp.data_ptr(), 1, Kp, Np, st), "alv_gemv_bf16")
    check(lib().alv_gemv_bf16(wr.handle, xb.data_ptr(), yr.data_ptr(), 1, K, N, st), "alv_gemv_bf16")
    a, b = yp.view(torch.int16).cpu().numpy(), yr.view(torch.int16).cpu().numpy()
    assert np.array_equal(a[:N], b)
    assert np.all(a[N:] & 0x7FFF == 0)
    wp.close()
    wr.close()


def test_padded_lm_head(orc, dev):
    """A head whose last rows and columns are zero padding: the padded rows'
    logits are softcap(0) = 0 and take part in the greedy pick."""
    import alveare_amd as aa

    Np, Kp, N, K = 3000, 1024, 2800, 960
    W = orc.synth_q4(N, K, 5151)
    P = pad_q4(W, N, K, Np, Kp)
    x = orc.synth_normal(Kp, 5152)
    wp = aa.Q4Weight(to_dev(P, dev), Np, Kp)
    wr = aa.Q4Weight(to_dev(W, dev), N, K)
    lp, tp = aa.lm_head(wp, to_dev(x, dev), Np, 30.0)
    lr, tr = aa.lm_head(wr, to_dev(x[:K].copy(), dev), N, 30.0)
    lp, lr = lp.cpu().numpy(), lr.cpu().numpy()
    assert np.array_equal(lp[:N].view(np.uint32), lr.view(np.uint32))
    assert np.all(lp[N:] == 0.0)
    assert int(tp.item()) == int(np.argmax(lp))
    assert int(tr.item()) == int(np.argmax(lr))
    wp.close()
    wr.close()


@pytest.mark.parametrize("H,I,Hp,Ip,Ms", [(1152, 6912, 1280, 7168, (1, 5, 16, 40)),
                                           (3840, 15360, 4096, 16384, (1, 16))])
def test_padded_ffn_equals_unpadded(orc, dev, H, I, Hp, Ip, Ms):
    """The reference's padded FFN (15360 x 3840 stored as 16384 x 4096)
    registered at its padded shape executes the real one: outputs and
    activation equal the unpadded registration's, padded entries zero."""
    import alveare_amd as aa

    _say(f"padded ffn {Hp}x{Ip} (real {H}x{I})")
    seed = orc.seed_for(3, 7) + H
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    Pg, Pu, Pd = pad_q4(Wg, I, H, Ip, Hp), pad_q4(Wu, I, H, Ip, Hp), pad_q4(Wd, H, I, Hp, Ip)
    fp = aa.FfnWeights(to_dev(Pg, dev), to_dev(Pu, dev), to_dev(Pd, dev), Hp, Ip, "gelu")
    fr = aa.FfnWeights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I, "gelu")
    assert fp.exec_shape == (H, I)
    for M in Ms:
        X = orc.synth_normal(M * Hp, seed + 10 + M).reshape(M, Hp)
        Yp = torch.full((M, Hp), float("nan"), device=dev)
        fp(to_dev(X, dev), Yp, M=M)
        ap = fp.last_activation(M).cpu().numpy()
        Yr = fr(to_dev(np.ascontiguousarray(X[:, :H]), dev), M=M).cpu().numpy().reshape(M, H)
        ar = fr.last_activation(M).cpu().numpy()
        Yp = Yp.cpu().numpy()
        assert np.array_equal(Yp[:, :H].view(np.uint32), Yr.view(np.uint32)), f"M={M}: outputs differ"
        assert np.all(Yp[:, H:] == 0.0), f"M={M}: padded outputs not zero"
        assert np.array_equal(ap[:, :I], ar), f"M={M}: activations differ"
        assert np.all(ap[:, I:] == 0.0), f"M={M}: padded activations not zero"
        _say(f"  M={M} ok")
    if H * I <= 1 << 23:
        x = orc.synth_normal(Hp, seed + 99)
        y = fp(to_dev(x, dev)).cpu().numpy()
        a = fp.last_activation(1).cpu().numpy()[0]
        st = parity.ffn_check(orc, Pg, Pu, Pd, x, Hp, Ip, 0, y, a)
        _say(f"  oracle on the padded arrays: max-rel {st['max_rel']:.2e}, flips {st['flips']}")
    fp.close()
    fr.close()


def test_fused_residual_rejects_trimmed_columns(orc, dev):
    """A fused residual step normalises the whole row, so it refuses a
    registration whose trailing columns were trimmed."""
    import alveare_amd as aa
    from alveare_amd._lib import lib

    W = pad_q4(orc.synth_q4(64, 96, 31), 64, 96, 64, 128)
    w = aa.Q4Weight(to_dev(W, dev), 64, 128)
    z = torch.zeros(128, dtype=torch.bfloat16, device=dev)
    y = torch.empty(64, dtype=torch.bfloat16, device=dev)
    rc = lib().alv_gemv_bf16_addnorm(w.handle, z.data_ptr(), z.data_ptr(), None, 1, 1.0, 0, z.data_ptr(), None,
                                     1e-6, y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc != 0
    assert b"trimmed" in lib().alv_last_error()
    w.close()
