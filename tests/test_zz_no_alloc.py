"""alv_ffn_fused_noalloc against alv_ffn_fused, through the C ABI: two calls in
a row on the 12B-class FFN (the second with fewer tokens), both bit-identical
to the allocating entry point and within the oracle's bar; a shape whose
split-K partial sums exceed the fixed scratch, and M > 16, are rejected
before anything runs."""
import ctypes
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


def test_ffn_noalloc_matches_allocating_entry_point(orc, dev):
    import alveare_amd as aa
    from alveare_amd._lib import ALV_ERR_ARG, ALV_ERR_RANGE

    L = aa.lib()
    H, I = 3840, 15360
    seed = orc.seed_for(4, 0)
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    ffn = aa.pack_ffn_fused_weights(to_dev(Wg, dev), to_dev(Wu, dev), to_dev(Wd, dev), H, I)
    st = torch.cuda.current_stream().cuda_stream
    for M in (16, 3, 1):  # 16 tokens split K in gate/up and down; then smaller calls (1: the one-launch form)
        _say(f"ffn noalloc M={M}")
        X = orc.synth_normal(M * H, seed + 10 + M).reshape(M, H)
        Xd = to_dev(X, dev)
        want = torch.empty((M, H), device=dev)
        got = torch.full((M, H), float("nan"), device=dev)
        assert L.alv_ffn_fused(ffn.handle, Xd.data_ptr(), want.data_ptr(), M, H, H, st) == 0
        torch.cuda.synchronize()
        a_want = ffn.last_activation(M).cpu().numpy()
        rc = L.alv_ffn_fused_noalloc(ffn.handle, Xd.data_ptr(), got.data_ptr(), M, H, H, st)
        assert rc == 0, L.alv_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"M={M}: noalloc result differs from alv_ffn_fused"
        assert np.array_equal(ffn.last_activation(M).cpu().numpy(), a_want)
        Yc = got.cpu().numpy()
        for m in (0, M - 1):
            parity.ffn_check(orc, Wg, Wu, Wd, X[m], H, I, 0, Yc[m], a_want[m])
    big = torch.empty((17, H), device=dev)
    assert L.alv_ffn_fused_noalloc(ffn.handle, big.data_ptr(), big.data_ptr(), 17, H, H, st) == ALV_ERR_ARG

    # Captured in a HIP graph on a stream that has never run a call (no
    # per-stream buffers exist for it): replays equal the eager result.
    M = 16
    X = to_dev(orc.synth_normal(M * H, seed + 40).reshape(M, H), dev)
    want = torch.empty((M, H), device=dev)
    assert L.alv_ffn_fused(ffn.handle, X.data_ptr(), want.data_ptr(), M, H, H, st) == 0
    torch.cuda.synchronize()
    got = torch.empty((M, H), device=dev)
    cs = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        rc = L.alv_ffn_fused_noalloc(ffn.handle, X.data_ptr(), got.data_ptr(), M, H, H, cs.cuda_stream)
    assert rc == 0, L.alv_last_error()
    for _ in range(3):
        got.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), "graph replay of the no-allocation FFN differs"
    del g
    ffn.close()

    # H = 4096, I = 65536 at 16 tokens: the gate/up launch needs 32 MiB of
    # split-K partial sums, beyond the fixed 16 MiB, so the call is refused and
    # writes nothing. The weights' values do not matter as long as they are
    # nonzero (registration trims all-zero trailing rows and columns).
    H2, I2 = 4096, 65536
    Wz = torch.full((I2, H2 // 32 * 20), 0x11, dtype=torch.uint8, device=dev)
    Wdz = torch.full((H2, I2 // 32 * 20), 0x11, dtype=torch.uint8, device=dev)
    f2 = aa.FfnWeights(Wz, Wz, Wdz, H2, I2, "gelu")
    del Wz, Wdz
    X2 = torch.zeros((16, H2), device=dev)
    Y2 = torch.full((16, H2), 7.0, device=dev)
    assert L.alv_ffn_fused_noalloc(f2.handle, X2.data_ptr(), Y2.data_ptr(), 16, H2, H2, st) == ALV_ERR_RANGE
    assert b"fixed scratch" in L.alv_last_error()
    torch.cuda.synchronize()
    assert torch.all(Y2 == 7.0)
    f2.close()
