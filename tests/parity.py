"""Parity criteria shared by the CPU and GPU tests.

GEMV / GEMM outputs are fp32 values before the reference's final bf16 cast, so
they are compared directly: max|y - y*| / max|y*| <= 1e-4 (the contract), plus
the per-element fp32 bound |y - y64| <= 2 gamma_K sum|w x| against fp64.

The FFN has three bf16 rounding points inside the reference's "fp32" path
(runtime/py/model.py:798-803): g = bf16(Wg x), u = bf16(Wu x),
a = bf16(act(g) u). Two correct fp32 implementations that add in different
orders (numpy's BLAS order is not specified) round a few g/u/a elements to
different neighbouring bf16 values, and one flipped element of `a` moves every
output by Wd[:, i] * ulp(a_i) -- up to ~4e-4 of max|y| at the 12B-class shape
(two CPU orders of the reference's own computation already differ by 1.8e-4
there). So the FFN check is split into parts that each have an exact bar:
  (1) down projection: y vs Wd @ a_test (the tested activation), <= 1e-4;
  (2) activation flips are rare (<= 5e-3 of I) and every one is legitimate:
      the exact (fp64) g or u of that element lies within the fp32 error bound
      of a bf16 rounding midpoint, or a's own pre-rounding value does;
  (3) end to end: |y - y*| <= 1e-4 max|y*| + sum over flips |Wd[h, i]| |da_i|.
"""
from __future__ import annotations

import numpy as np

TOL = 1e-4          # max-relative error, the reference contract
FLIP_RATE = 5e-3    # sanity bound on the fraction of activation elements that flip
U32 = 2.0 ** -24


def bf16_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits).astype(np.uint32) << 16).view(np.float32)


def deq_f64(orc, W, N, K) -> np.ndarray:
    return bf16_f32(orc.dequant_q4(W, N, K)).astype(np.float64)


def max_rel(y: np.ndarray, ref: np.ndarray) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def gemv_check(orc, W, x, y, N, K, tol=TOL):
    """Assert GEMV parity of y (fp32, N) against the oracle; returns max-rel."""
    y_ref = orc.gemv_q(W, x, N, K)
    y64 = orc.gemv_q_f64(W, x, N, K)
    absdot = np.abs(deq_f64(orc, W, N, K)) @ np.abs(np.asarray(x, np.float64))
    gamma = K * U32 / (1 - K * U32)
    err = max_rel(y, y_ref)
    assert err <= tol, f"GEMV max-rel {err:.3e} > {tol}"
    bad = np.abs(np.asarray(y, np.float64) - y64) > 2 * gamma * absdot + 1e-30
    assert not bad.any(), f"{bad.sum()} elements outside the fp32 bound, first row {np.argmax(bad)}"
    return err


def _midpoint_dist(v: np.ndarray) -> np.ndarray:
    """Distance of fp64 values to the nearest bf16 rounding midpoint."""
    v = np.asarray(v, np.float64)
    f = v.astype(np.float32)
    hi = (f.view(np.uint32) >> 16).astype(np.uint32)
    lo_v = (hi << 16).view(np.float32).astype(np.float64)
    nxt = ((hi + 1) << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    prv = ((hi - 1) << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    m1 = (lo_v + nxt) / 2
    m0 = (lo_v + prv) / 2
    return np.minimum(np.abs(v - m1), np.abs(v - m0))


def ffn_check(orc, Wg, Wu, Wd, x, H, I, act, y_test, a_test=None, tol=TOL, cache=None):
    """Flip-aware FFN parity of one token (see module docstring). Returns a
    dict with the end-to-end max-rel and the flip count. `cache` (a dict kept
    across the tokens of one weight set) holds the fp64 dequantized matrices."""
    if cache is None:
        cache = {}

    def deq(name, W, N, K):
        if name not in cache:
            cache[name] = deq_f64(orc, W, N, K)
        return cache[name]

    x = np.asarray(x, np.float32)
    g = orc.gemv_q(Wg, x, I, H)
    u = orc.gemv_q(Wu, x, I, H)
    a_ref = orc.glu(orc.bf16_round(g), orc.bf16_round(u), act)
    y_ref = orc.gemv_q(Wd, a_ref, H, I)
    scale = float(np.max(np.abs(y_ref)))
    y_test = np.asarray(y_test, np.float64)
    if a_test is None:
        a_test = a_ref
    a_test = np.asarray(a_test, np.float32)

    # (1) the down projection at the tested activation
    e1 = max_rel(y_test, orc.gemv_q(Wd, a_test, H, I))
    assert e1 <= tol, f"down projection max-rel {e1:.3e} > {tol}"

    # (2) flips are rare and sit on rounding midpoints within the fp32 bound
    flips = np.nonzero(a_test != a_ref)[0]
    assert len(flips) <= max(2, FLIP_RATE * I), f"{len(flips)} activation flips of {I}"
    if len(flips):
        g64 = orc.gemv_q_f64(Wg, x, I, H)[flips]
        u64 = orc.gemv_q_f64(Wu, x, I, H)[flips]
        xa = np.abs(x.astype(np.float64))
        bg = (np.abs(deq("g", Wg, I, H)[flips]) @ xa) * 2 * H * U32
        bu = (np.abs(deq("u", Wu, I, H)[flips]) @ xa) * 2 * H * U32
        near_g = _midpoint_dist(g64) <= bg
        near_u = _midpoint_dist(u64) <= bu
        # a's own rounding: the unrounded product in fp64
        gb = orc.bf16_round(g)[flips].astype(np.float64)
        ub = orc.bf16_round(u)[flips].astype(np.float64)
        if act == 0:
            inner = (gb + 0.044715 * gb ** 3)
            raw = 0.5 * gb * (1 + np.tanh(np.sqrt(2 / np.pi) * inner)) * ub
        else:
            raw = gb / (1 + np.exp(-gb)) * ub
        near_a = _midpoint_dist(raw) <= 1e-6 * np.abs(raw) + 1e-30
        tiny = np.abs(a_test[flips].astype(np.float64) - a_ref[flips]) <= 1e-9 * (np.abs(ub) + 1)
        legit = near_g | near_u | near_a | tiny
        assert legit.all(), f"unexplained activation flips at {flips[~legit][:8]}"

    # (3) end to end with the flip budget
    da = np.abs(a_test.astype(np.float64) - a_ref)
    budget = np.zeros(H)
    if len(flips):
        budget = np.abs(deq("d", Wd, H, I)[:, flips]) @ da[flips]
    bad = np.abs(y_test - y_ref) > tol * scale + budget
    assert not bad.any(), f"{bad.sum()} outputs outside tolerance + flip budget"
    return {"max_rel": max_rel(y_test, y_ref), "flips": int(len(flips)), "down_max_rel": e1}


def ffn_check_batch(orc, Wg, Wu, Wd, X, H, I, act, Y_test, A_test, tol=TOL):
    """ffn_check for every token of a batch at once, against the exact
    (float64) arithmetic on the oracle's dequantized matrices instead of the
    float32 oracle (whose per-token cost is a full dequantization): for each
    token, (1) the down projection of the tested activation within tol of
    max|y|, (2) activation flips against a64 = GLU(bf16(g64), bf16(u64)) rare
    and each on a bf16 rounding midpoint within the fp32 error bound of g, u
    or the GLU product, (3) y within tol * max|y| plus the flips' exact
    contribution. Returns per-batch figures: the worst end-to-end max-rel, the
    worst down-projection max-rel, flip counts, and how many tokens exceed tol
    end to end before the flip budget."""
    X = np.asarray(X, np.float32).reshape(-1, H)
    M = X.shape[0]
    X64 = X.astype(np.float64)
    G = deq_f64(orc, Wg, I, H).reshape(I, H)
    U = deq_f64(orc, Wu, I, H).reshape(I, H)
    D = deq_f64(orc, Wd, H, I).reshape(H, I)
    g64 = X64 @ G.T
    u64 = X64 @ U.T
    gb = orc.bf16_round(g64.astype(np.float32)).reshape(M, I)
    ub = orc.bf16_round(u64.astype(np.float32)).reshape(M, I)
    a64 = orc.glu(gb, ub, act).reshape(M, I)
    A_test = np.asarray(A_test, np.float32).reshape(M, I)
    Y_test = np.asarray(Y_test, np.float64).reshape(M, H)
    y_ref = a64.astype(np.float64) @ D.T
    y_at = A_test.astype(np.float64) @ D.T
    scale = np.max(np.abs(y_ref), axis=1)
    e_down = np.max(np.abs(Y_test - y_at), axis=1) / np.maximum(np.max(np.abs(y_at), axis=1), 1e-30)
    assert np.all(e_down <= tol), f"down projection max-rel {e_down.max():.3e} > {tol} (token {int(np.argmax(e_down))})"
    flip_m, flip_i = np.nonzero(A_test != a64)
    per_tok = np.bincount(flip_m, minlength=M)
    assert np.all(per_tok <= max(2, FLIP_RATE * I)), f"{per_tok.max()} activation flips in one token of {I}"
    if len(flip_m):
        xa = np.abs(X64[flip_m])
        bg = np.sum(np.abs(G[flip_i]) * xa, axis=1) * 2 * H * U32
        bu = np.sum(np.abs(U[flip_i]) * xa, axis=1) * 2 * H * U32
        near_g = _midpoint_dist(g64[flip_m, flip_i]) <= bg
        near_u = _midpoint_dist(u64[flip_m, flip_i]) <= bu
        gf = gb[flip_m, flip_i].astype(np.float64)
        uf = ub[flip_m, flip_i].astype(np.float64)
        if act == 0:
            raw = 0.5 * gf * (1 + np.tanh(np.sqrt(2 / np.pi) * (gf + 0.044715 * gf ** 3))) * uf
        else:
            raw = gf / (1 + np.exp(-gf)) * uf
        near_a = _midpoint_dist(raw) <= 1e-6 * np.abs(raw) + 1e-30
        tiny = np.abs(A_test[flip_m, flip_i].astype(np.float64) - a64[flip_m, flip_i]) <= 1e-9 * (np.abs(uf) + 1)
        legit = near_g | near_u | near_a | tiny
        assert legit.all(), f"unexplained activation flips at (token, row) {list(zip(flip_m[~legit][:8], flip_i[~legit][:8]))}"
    da = np.abs(A_test.astype(np.float64) - a64)
    budget = da @ np.abs(D).T
    err = np.abs(Y_test - y_ref)
    bad = err > tol * scale[:, None] + budget
    assert not bad.any(), f"{bad.sum()} outputs outside tolerance + flip budget (token {int(np.argmax(bad.any(1)))})"
    rel = np.max(err, axis=1) / np.maximum(scale, 1e-30)
    return {"tokens": M, "max_rel": float(rel.max()), "down_max_rel": float(e_down.max()), "flips": int(len(flip_m)),
            "tokens_with_flips": int(np.count_nonzero(per_tok)), "tokens_over_tol": int(np.count_nonzero(rel > tol))}


def tile_layout_np(W: np.ndarray, N: int, K: int) -> np.ndarray:
    """The kernels' tiled layout, restated from its definition: per 16-row tile
    and 512-column super-step, lane (g, j) owns the 80-byte run of row j over
    blocks 4g..4g+3; its five 16-byte pieces go to planes i at
    tile + i*256*ng + 16*(16g + j). ng = 4 except the last super-step
    (ceil(blocks left / 4)); bytes past the row or past N are zero."""
    nb = K // 32
    nss = (nb + 15) // 16
    ngl = (nb - 16 * (nss - 1) + 3) // 4
    rtb = (nss - 1) * 5120 + 1280 * ngl
    RT = (N + 15) // 16
    rs = nb * 20
    Wp = np.zeros((RT * 16, nss * 320), np.uint8)
    Wp[:N, :rs] = np.asarray(W).reshape(N, rs)
    out = np.zeros(RT * rtb, np.uint8)
    for rt in range(RT):
        for ss in range(nss):
            ng = 4 if ss < nss - 1 else ngl
            for g in range(ng):
                runs = Wp[rt * 16:(rt + 1) * 16, (ss * 16 + g * 4) * 20:(ss * 16 + g * 4) * 20 + 80]
                for i in range(5):
                    dst = rt * rtb + ss * 5120 + i * 256 * ng + g * 256
                    out[dst:dst + 256] = runs[:, 16 * i:16 * i + 16].reshape(-1)
    return out


def quant_cases():
    """Random blocks plus the edge cases of quantize_to_q4_0: exact ties of
    w / s at +-0.5, 1.5, ... (np.round to even), all-zero blocks, subnormal
    blocks whose max / 7 underflows to 0 (scale 1.0), a NaN and an inf block."""
    rng = np.random.default_rng(7)
    w = rng.normal(0.0, 0.05, size=(24, 256)).astype(np.float32)
    w[0, :32] = np.array([7.0, 0.5, 1.5, 2.5, 3.5, -0.5, -2.5, -3.5] + [0.25] * 24, np.float32)  # s = 1: ties
    w[1, :32] = np.arange(-16, 16, dtype=np.float32) * np.float32(0.5)  # max 8 -> s = 8/7
    w[2, :64] = 0.0
    w[3, :32] = np.float32(1e-45) * np.arange(32, dtype=np.float32)  # subnormals
    w[4, :32] = np.float32(3e-38)
    w[5, 32:64] = np.nan
    w[6, 64] = np.nan
    w[7, 96] = np.inf
    w[8, 128:160] = -np.inf
    w[9, :32] = -0.0
    w[10, :32] = np.float32(1e-45) * np.array([0, 1, 2, 3] * 8, np.float32)  # max / 7 underflows to 0
    return w


# ---- host ops of a decode layer ---------------------------------------------------

def pw_sum_gpu_order(a: np.ndarray) -> np.float32:
    """The GPU's float32 sum of a (layer_ops.hip pw_sum_wave): per buffer of
    8192 values (buffer sums added in order), leaves of a halving tree summed
    by the 8-accumulator rule and combined pairwise up the tree, or the full
    recursion on one lane for other widths. Meant to equal np.add.reduce(a)
    bit for bit."""
    a = np.asarray(a, np.float32)
    if len(a) > 8192:
        r = _pw_chunk(a[:8192])
        for off in range(8192, len(a), 8192):
            r = np.float32(r + _pw_chunk(a[off:off + 8192]))
        return r
    return _pw_chunk(a)


def _pw_chunk(a: np.ndarray) -> np.float32:
    n = len(a)

    def leaf(x):
        if len(x) < 8:
            r = np.float32(0)
            for v in x:
                r = np.float32(r + v)
            return r
        r = [np.float32(v) for v in x[:8]]
        i = 8
        while i < len(x) - len(x) % 8:
            for j in range(8):
                r[j] = np.float32(r[j] + x[i + j])
            i += 8
        res = np.float32(np.float32(np.float32(r[0] + r[1]) + np.float32(r[2] + r[3])) +
                         np.float32(np.float32(r[4] + r[5]) + np.float32(r[6] + r[7])))
        for v in x[i:]:
            res = np.float32(res + v)
        return res

    def rec(x):
        if len(x) <= 128:
            return leaf(x)
        n2 = len(x) // 2
        n2 -= n2 % 8
        return np.float32(rec(x[:n2]) + rec(x[n2:]))

    lf, leaves = n, 1
    halving = True
    while lf > 128:
        if lf % 2 or (lf // 2) % 8:
            halving = False
            break
        lf //= 2
        leaves *= 2
    if not (halving and leaves <= 64):
        return rec(a)
    v = [leaf(a[i * lf:(i + 1) * lf]) for i in range(leaves)]
    s = 1
    while s < leaves:
        v = [np.float32(v[i] + v[i + 1]) for i in range(0, len(v), 2)]
        s *= 2
    return v[0]


def bf16_bits(t) -> np.ndarray:
    """uint16 bit patterns of a torch bfloat16 tensor (on any device)."""
    return t.detach().cpu().view(__import__("torch").int16).numpy().view(np.uint16)


def bits_bf16_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_bits_bf16(x: np.ndarray) -> np.ndarray:
    from oracle import q4_numpy
    return (q4_numpy.bf16_rne(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_interval_check(out_bits: np.ndarray, ref64: np.ndarray, bound: np.ndarray, what: str) -> int:
    """Every bf16 output lies between the bf16 roundings of ref64 - bound and
    ref64 + bound (a float32 value within `bound` of the exact one, rounded to
    bf16); returns how many differ from the rounding of ref64 itself."""
    from oracle import q4_numpy
    out = bits_bf16_f32(out_bits).astype(np.float64)
    lo = q4_numpy.bf16_rne(np.nextafter((ref64 - bound).astype(np.float32), np.float32(-np.inf))).astype(np.float64)
    hi = q4_numpy.bf16_rne(np.nextafter((ref64 + bound).astype(np.float32), np.float32(np.inf))).astype(np.float64)
    bad = (out < lo) | (out > hi)
    assert not bad.any(), f"{what}: {bad.sum()} bf16 outputs outside the bound, first at {np.argmax(bad)}"
    mid = q4_numpy.bf16_rne(ref64.astype(np.float32)).astype(np.float64)
    return int((out != mid).sum())


def gemv_bf16_check(orc, W, x, y_bits, N, K) -> int:
    """bf16 GEMV output against the fp64 value with the fp32 bound (rows can
    round either way only when the bound straddles a bf16 rounding point)."""
    y64 = orc.gemv_q_f64(W, x, N, K)
    absdot = np.abs(deq_f64(orc, W, N, K)) @ np.abs(np.asarray(x, np.float64))
    gamma = K * U32 / (1 - K * U32)
    return bf16_interval_check(y_bits, y64, 2 * gamma * absdot + 1e-30, "bf16 GEMV")
