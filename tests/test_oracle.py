"""Pins of the CPU oracle (oracle/) -- CPU only.

Each check is independent of the oracle's own code path: the reference's
compiled bf16.cpp (oracle/_ref), torch's bf16 cast, the AIE kernel's
shift-based sign extension, numpy evaluating the reference's own expressions
(oracle/q4_numpy.py), fp64 brute force, exhaustive tables and closed forms.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import q4_numpy

import parity


def _bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return bits.astype(np.uint32).view(np.float32)


def _torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# ---- bf16 (runtime/cpp/src/bf16.cpp:7-27) -----------------------------------

def test_bf16_exhaustive_vs_reference_bf16_cpp(orc):
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference tree: make -C oracle ref)")
    first = ctypes.c_uint32(0)
    fn = ctypes.cast(ref.ref_bf16_from_f32, ctypes.c_void_p)
    bad = orc.lib().orc_bf16_sweep(fn, ctypes.byref(first))
    assert bad == 0, f"{bad} of 2^32 patterns differ from bf16.cpp, first 0x{first.value:08x}"


def test_bf16_vs_torch_and_specials(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFFFFFFFF,
                         0x00000001, 0x007FFFFF, 0x00800000, 0x3F808000, 0x3F818000, 0x3F807FFF,
                         0x3F808001, 0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF], dtype=np.uint32)
    # Every tie pattern (low 16 bits exactly 0x8000) for a spread of high halves.
    ties = (np.arange(0, 1 << 16, 7, dtype=np.uint32) << 16) | 0x8000
    f = _bits_to_f32(np.concatenate([bits, specials, ties]))
    # NaN payloads are outside the comparison: torch's vectorised cast keeps
    # them, the reference's bf16.cpp (pinned exhaustively above) makes 0x7FC0.
    f = f[~np.isnan(f)]
    assert np.array_equal(orc.bf16_bits(f), _torch_bf16_bits(f))
    # NaN -> 0x7FC0 (bf16.cpp:9-11), ties to even, overflow to inf.
    tb = orc.bf16_bits(_bits_to_f32(np.array([0x7FC00000, 0x3F808000, 0x3F818000, 0x7F7FFFFF], np.uint32)))
    assert tb.tolist() == [0x7FC0, 0x3F80, 0x3F82, 0x7F80]


def test_bf16_numpy_restatement_matches(orc):
    rng = np.random.default_rng(8)
    f = _bits_to_f32(rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32))
    a = q4_numpy.bf16_rne(f).view(np.uint32) >> 16
    assert np.array_equal(a.astype(np.uint16), orc.bf16_bits(f))


# ---- unpack (tools/ref/gemv_q.py:19-31) ---------------------------------------

def _all_bytes_matrix() -> np.ndarray:
    """16 rows x one block: row r holds bytes 16r .. 16r+15, so all 256 byte
    values appear once; scale 1.0."""
    W = np.zeros((16, 20), np.uint8)
    W[:, :16] = np.arange(256, dtype=np.uint8).reshape(16, 16)
    W[:, 16], W[:, 17] = 0x80, 0x3F
    return W


def test_unpack_exhaustive_vs_aie_shift_form(orc):
    W = _all_bytes_matrix()
    q = orc.unpack_q4(W, 16, 32).reshape(256, 2)
    b = np.arange(256, dtype=np.int32)
    # kernels/gemv_q/gemv_q.cc:46-47 sign-extends by int16 shifts: (x<<12)>>12, (x<<8)>>12.
    lo = ((b << 12).astype(np.int16) >> 12).astype(np.int8)
    hi = ((b << 8).astype(np.int16) >> 12).astype(np.int8)
    assert np.array_equal(q[:, 0], lo) and np.array_equal(q[:, 1], hi)


def test_pack_unpack_round_trip_all_pairs(orc):
    q0, q1 = np.meshgrid(np.arange(-8, 8), np.arange(-8, 8), indexing="ij")
    q0, q1 = q0.ravel(), q1.ravel()
    # tools/convert/gemv_q_convert.py:46-48 packing.
    byte = ((q0 & 0x0F) | ((q1 & 0x0F) << 4)).astype(np.uint8)
    W = np.zeros((16, 20), np.uint8)
    W[:, :16] = byte.reshape(16, 16)
    q = orc.unpack_q4(W, 16, 32).reshape(256, 2)
    assert np.array_equal(q[:, 0], q0) and np.array_equal(q[:, 1], q1)


# ---- dequant (tools/ref/gemv_q.py:33-37) ----------------------------------------

def exhaustive_scale_matrix() -> np.ndarray:
    """65536 rows x one block: row s has bf16 scale bits s and codes covering
    all 16 values in both nibble positions."""
    W = np.zeros((65536, 20), np.uint8)
    lo = np.arange(16, dtype=np.uint8)
    W[:, :16] = lo | ((15 - lo) << 4)
    s = np.arange(65536, dtype=np.uint32)
    W[:, 16] = s & 0xFF
    W[:, 17] = s >> 8
    return W


def test_dequant_exhaustive_vs_torch(orc):
    W = exhaustive_scale_matrix()
    got = orc.dequant_q4(W, 65536, 32)
    q = orc.unpack_q4(W, 65536, 32).astype(np.float32)
    s = _bits_to_f32(np.arange(65536, dtype=np.uint32) << 16)[:, None]
    prod32 = torch.from_numpy(q).mul(torch.from_numpy(np.ascontiguousarray(np.broadcast_to(s, q.shape))))
    want = prod32.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    # NaN products (NaN scales, 0 * inf) become 0x7FC0 as in bf16.cpp:9-11;
    # torch keeps NaN payloads, so they are compared separately.
    nan = torch.isnan(prod32).numpy()
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(got[nan] == 0x7FC0) and nan.sum() == 254 * 32 + 2 * 2
    # Powers of two (|q| in {0,1,2,4,8}) are exact products for finite scales.
    fin = np.isfinite(s[:, 0])
    exact = np.isin(np.abs(q), [0, 1, 2, 4, 8])
    with np.errstate(over="ignore", invalid="ignore"):
        prod = (q * s)[fin][exact[fin]]
    deq = _bits_to_f32(got.astype(np.uint32) << 16)[fin][exact[fin]]
    nz = np.abs(prod) >= np.float32(2.0 ** -126)  # keep normal results
    assert np.array_equal(deq[nz], prod[nz])


def test_dequant_numpy_restatement(orc):
    W = orc.synth_q4(64, 256, 11)
    a = orc.dequant_q4(W, 64, 256)
    b = (q4_numpy.dequantize_combined(W).view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(a, b)


# ---- gemv (tools/ref/gemv_q.py:73-80) --------------------------------------------

@pytest.mark.parametrize("N,K,seed", [(64, 256, 1), (256, 256, 42), (333, 1152, 5), (128, 4096, 9)])
def test_gemv_fp64_bound_and_numpy(orc, N, K, seed):
    W = orc.synth_q4(N, K, seed)
    x = orc.synth_normal(K, seed + 1)
    y = orc.gemv_q(W, x, N, K)
    y64 = orc.gemv_q_f64(W, x, N, K)
    w = _bits_to_f32(orc.dequant_q4(W, N, K).astype(np.uint32) << 16).astype(np.float64)
    absdot = np.abs(w) @ np.abs(x.astype(np.float64))
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    assert np.all(np.abs(y - y64) <= gamma * absdot + 1e-30)
    # numpy with the reference's own expression (BLAS order) agrees to fp32 rounding.
    yn = q4_numpy.gemv_q_combined(W, x)
    assert np.all(np.abs(y - yn) <= 2 * gamma * absdot + 1e-30)


def test_gemv_one_hot_selects_column(orc):
    N, K = 48, 320
    W = orc.synth_q4(N, K, 3)
    deq = _bits_to_f32(orc.dequant_q4(W, N, K).astype(np.uint32) << 16)
    for k in (0, 1, 31, 32, 100, K - 1):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        assert np.array_equal(orc.gemv_q(W, x, N, K), deq[:, k])


def test_gemv_zero_scale_rows(orc):
    N, K = 8, 128
    W = orc.synth_q4(N, K, 4)
    W.reshape(N, K // 32, 20)[3, :, 16:18] = 0  # row 3: all scales +0
    y = orc.gemv_q(W, orc.synth_normal(K, 5), N, K)
    assert y[3] == 0.0 and np.all(y[[0, 1, 2, 4]] != 0.0)


def test_dropped_dequant_rounding_fails_tolerance(orc):
    """A plausible mistake -- factoring the scale out (s * sum q x, no bf16
    rounding of the dequantized weight, as runtime/cpp/src/generator.cpp:80-101
    does) -- is caught by the 1e-4 max-relative tolerance."""
    N, K = 3840, 3840
    W = orc.synth_q4(N, K, 21)
    x = orc.synth_normal(K, 22)
    y = orc.gemv_q(W, x, N, K)
    q = orc.unpack_q4(W, N, K).astype(np.float64)
    s = _bits_to_f32(orc.scales_q4(W, N, K).astype(np.uint32) << 16).astype(np.float64)
    y_bad = ((q.reshape(N, K // 32, 32) * x.reshape(1, K // 32, 32)).sum(-1) * s).sum(-1)
    err = np.max(np.abs(y_bad - y)) / np.max(np.abs(y))
    assert err > 1e-4, err


# ---- gemm (runtime/py/model.py:1049-1111; runtime/cpp/src/main.cpp:98-108) ----------

def test_gemm_rows_equal_gemv(orc):
    M, N, K = 5, 96, 512
    W = orc.synth_q4(N, K, 12)
    X = orc.synth_normal(M * K, 13).reshape(M, K)
    Y = orc.gemm_q(W, X, M, N, K)
    for m in range(M):
        assert np.array_equal(Y[m], orc.gemv_q(W, X[m], N, K))


# ---- GLU and FFN (runtime/py/model.py:797-806, :853-860) ---------------------------

def _numpy_gelu_mul(g, u):
    # runtime/py/model.py:802-803, evaluated by numpy.
    gelu_out = 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * (g ** 3))))
    return q4_numpy.bf16_rne(np.asarray(gelu_out * u).astype(np.float32))


def _numpy_silu_mul(g, u):
    return q4_numpy.bf16_rne((g * (1.0 / (1.0 + np.exp(-g)))) * u)


def test_glu_matches_numpy_expression(orc):
    rng = np.random.default_rng(3)
    g = q4_numpy.bf16_rne(rng.standard_normal(1 << 18).astype(np.float32) * 4)
    u = q4_numpy.bf16_rne(rng.standard_normal(1 << 18).astype(np.float32) * 4)
    a = orc.glu(g, u, 0)
    want = _numpy_gelu_mul(g, u)
    diff = a != want
    # numpy's float32 g**3 is a SIMD routine, not correctly rounded: at most a
    # rare one-ulp flip of the bf16 result.
    assert diff.mean() < 1e-3, diff.mean()
    # Where 1 + tanh cancels (g < -4.5) the libm tanh ulps are amplified, but
    # the values are below 1e-9 * |u|; elsewhere the flips are single bf16 ulps.
    deep = g[diff] < -4.5
    ulp = np.abs(a[diff].view(np.int32) - want[diff].view(np.int32))
    assert np.all(ulp[~deep] == 1 << 16)
    assert np.all(np.abs(a[diff][deep] - want[diff][deep]) <= 1e-9 * np.abs(u[diff][deep]))
    a_s = orc.glu(g, u, 1)
    ws = _numpy_silu_mul(g, u)
    ds = a_s != ws
    assert ds.mean() < 1e-3
    deep = g[ds] < -20
    assert np.all(np.abs(a_s[ds].view(np.int32) - ws[ds].view(np.int32))[~deep] == 1 << 16)


def test_glu_vs_longdouble_tanh(orc):
    rng = np.random.default_rng(4)
    g = q4_numpy.bf16_rne(rng.standard_normal(1 << 16).astype(np.float32) * 3)
    u = np.ones_like(g)
    a = orc.glu(g, u, 0)
    gl = g.astype(np.longdouble)
    inner = (g + np.float32(0.044715) * ((g * g) * g)).astype(np.longdouble)
    c = np.sqrt(np.longdouble(2) / np.pi)
    ref = np.longdouble(0.5) * gl * (1 + np.tanh(c * inner))
    want = q4_numpy.bf16_rne(ref.astype(np.float64).astype(np.float32))
    ok = g > -4.5  # outside the 1 + tanh cancellation, where float64 itself loses digits
    assert (a[ok] != want[ok]).mean() < 1e-3
    assert np.all(np.abs(a[~ok] - want[~ok]) <= 1e-9)


def test_glu_special_cases(orc):
    g = np.array([0.0, 0.0, 3.0, -3.0, 40.0, -40.0, 1.0], np.float32)
    u = np.array([5.0, 0.0, 0.0, 0.0, 2.0, 2.0, 1.0], np.float32)
    a = orc.glu(g, u, 0)
    assert a[0] == 0 and a[1] == 0 and a[2] == 0 and a[3] == 0
    assert a[4] == 80.0 and a[5] == 0.0  # gelu(g) -> g, -> 0
    # gelu_tanh(1) = 0.841192 -> bf16 0.83984375
    assert a[6] == np.float32(0.83984375)


@pytest.mark.parametrize("H,I,act,seed", [(256, 512, "gelu", 31), (384, 1152, "silu", 31),
                                         (1152, 6912, "gelu", 31), (1152, 6912, "gelu", 100)])
def test_ffn_vs_numpy(orc, H, I, act, seed):
    """The oracle against numpy evaluating the reference's expressions, with
    the flip-aware criterion of tests/parity.py (numpy's BLAS adds in another
    order, so a few bf16 rounding points may legitimately differ)."""
    Wg, Wu, Wd = orc.synth_q4(I, H, seed), orc.synth_q4(I, H, seed + 1), orc.synth_q4(H, I, seed + 2)
    x = orc.synth_normal(H, seed + 3)
    yn, an = q4_numpy.ffn_cpu(Wg, Wu, Wd, x, act, return_act=True)
    st = parity.ffn_check(orc, Wg, Wu, Wd, x, H, I, 0 if act == "gelu" else 1, yn, an)
    assert st["down_max_rel"] < 1e-5


def test_ffn_fp64_accumulation_within_flip_bound(orc):
    """fp64 accumulation of gate/up is another legitimate order."""
    H, I = 1152, 6912
    Wg, Wu, Wd = orc.synth_q4(I, H, 31), orc.synth_q4(I, H, 32), orc.synth_q4(H, I, 33)
    x = orc.synth_normal(H, 34)
    g = orc.bf16_round(orc.gemv_q_f64(Wg, x, I, H).astype(np.float32))
    u = orc.bf16_round(orc.gemv_q_f64(Wu, x, I, H).astype(np.float32))
    a = orc.glu(g, u, 0)
    y = orc.gemv_q(Wd, a, H, I)
    st = parity.ffn_check(orc, Wg, Wu, Wd, x, H, I, 0, y, a)
    assert st["flips"] >= 1  # this seed does flip, so the flip path is exercised


def test_ffn_batch_rows_equal(orc):
    H, I, M = 128, 256, 3
    Wg, Wu, Wd = orc.synth_q4(I, H, 41), orc.synth_q4(I, H, 42), orc.synth_q4(H, I, 43)
    X = orc.synth_normal(M * H, 44).reshape(M, H)
    Y = orc.ffn(Wg, Wu, Wd, X, H, I, 0)
    for m in range(M):
        assert np.array_equal(Y[m], orc.ffn(Wg, Wu, Wd, X[m], H, I, 0))


# ---- quantizer (tools/convert/gemv_q_convert.py:5-85) ----------------------------

def test_quantize_hand_block(orc):
    w = np.zeros((1, 64), np.float32)
    # block 0: max 7 -> scale 1.0; halves tie to even (np.round).
    w[0, :10] = [7, -7, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.49, -6.51]
    # block 1 all zero -> scale 1.0, codes 0.
    W = orc.quantize_q4_0(w)
    q = orc.unpack_q4(W, 1, 64)[0]
    assert q[:10].tolist() == [7, -7, 0, 2, 2, 0, -2, -2, 3, -7]
    assert np.all(q[10:] == 0)
    s = orc.scales_q4(W, 1, 64)[0]
    assert s.tolist() == [0x3F80, 0x3F80]
    assert W[0, 18:20].tolist() == [0, 0] and W[0, 38:40].tolist() == [0, 0]


def test_quantize_round_trip_bound(orc):
    rng = np.random.default_rng(42)
    w = rng.uniform(-1.0, 1.0, size=(256, 256)).astype(np.float32)
    W = orc.quantize_q4_0(w)
    deq = _bits_to_f32(orc.dequant_q4(W, 256, 256).astype(np.uint32) << 16)
    s = np.repeat(np.abs(w).reshape(256, 8, 32).max(-1) / np.float32(7), 32, axis=1)
    # half a step, plus half a bf16 ulp (2^-8 relative) on the scale and on the product
    assert np.all(np.abs(deq - w) <= s * (0.5 + 2 * 7 * 2.0 ** -8))


# ---- synthetic inputs -------------------------------------------------------------

def test_synth_deterministic_and_distributed(orc):
    a = orc.synth_q4(64, 512, 123)
    assert np.array_equal(a, orc.synth_q4(64, 512, 123))
    assert not np.array_equal(a, orc.synth_q4(64, 512, 124))
    blk = a.reshape(64, 16, 20)
    assert np.all(blk[:, :, 18:] == 0)
    s = _bits_to_f32(orc.scales_q4(a, 64, 512).astype(np.uint32) << 16)
    assert s.min() >= 0.00099 and s.max() <= 0.0201
    q = orc.unpack_q4(a, 64, 512)
    hist = np.bincount(q.ravel() + 8, minlength=16)
    assert hist.min() > 0.8 * q.size / 16
    x = orc.synth_normal(1 << 16, 5)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    # Counter-based SplitMix64 (Steele et al.): first outputs for seed 0.
    assert orc.lib().orc_splitmix64_at(0, 0) == 0xE220A8397B1DCDAF


def test_lm_head_restatement_pins():
    """oracle/q4_numpy.py::lm_head_cpu against what the mathematics fixes:
    bf16 logits first (a value rounds before the softcap), 30 tanh(l / 30)
    within 4 float32 ulps of the float64 value (three float32 roundings), |logit| < 30, odd, ~l for
    small l; softcap 0 leaves the bf16 logits; the token is the first index of
    the maximum, NaN first."""
    from oracle import q4_numpy

    rng = np.random.default_rng(11)
    y = (rng.standard_normal(5000) * 40).astype(np.float32)
    out, tok = q4_numpy.lm_head_cpu(y, 4000, 30.0)
    lb = q4_numpy.bf16_rne(y[:4000]).astype(np.float64)
    exact = 30.0 * np.tanh(lb / 30.0)
    assert out.dtype == np.float32 and out.shape == (4000,)
    assert np.all(np.abs(out - exact) <= 4 * np.spacing(np.abs(exact).astype(np.float32)))
    assert np.all(np.abs(out) <= 30.0)
    assert tok == int(np.argmax(exact))
    o2, _ = q4_numpy.lm_head_cpu(-y, 4000, 30.0)
    assert np.array_equal(o2, -out)
    small, _ = q4_numpy.lm_head_cpu(np.array([2.0 ** -10], np.float32), 1, 30.0)
    assert small[0] == np.float32(2.0 ** -10)
    raw, t0 = q4_numpy.lm_head_cpu(y, 4000, 0.0)
    assert np.array_equal(raw, q4_numpy.bf16_rne(y[:4000])) and t0 == int(np.argmax(lb))
    ties = np.array([1.0, 5.0, 5.0, np.float32(5.0009765625)], np.float32)  # the last rounds to 5.0 in bf16
    assert q4_numpy.lm_head_cpu(ties, 4, 30.0)[1] == 1
    assert q4_numpy.lm_head_cpu(np.array([1.0, np.nan, 9.0, np.nan], np.float32), 4, 30.0)[1] == 1


def test_quantize_matches_numpy_restatement(orc):
    w = parity.quant_cases()
    a = orc.quantize_q4_0(w)
    b = q4_numpy.quantize_to_q4_0(w)
    assert np.array_equal(a, b)
    # NaN blocks: every code -8, scale the quiet NaN 0x7FC0; an inf block: its
    # finite weights quantize to 0, the inf (inf / inf) to -8, scale 0x7F80.
    q = orc.unpack_q4(a, 24, 256)
    s = orc.scales_q4(a, 24, 256)
    assert np.all(q[5, 32:64] == -8) and s[5, 1] == 0x7FC0
    assert q[6, 64] == -8 and np.all(q[6, 65:96] == -8) and s[6, 2] == 0x7FC0
    assert q[7, 96] == -8 and np.all(q[7, 97:128] == 0) and s[7, 3] == 0x7F80
    assert np.all(q[10, :32] == 0) and s[10, 0] == 0x3F80
    assert q[3, 31] == 7 and s[3, 0] == 0  # subnormal scale 3 * 2^-149 rounds to bf16 +0


# ---- host ops of a decode layer (runtime/py/model.py:522-628, :705-790) ------------

@pytest.mark.parametrize("n", [1, 7, 8, 100, 128, 129, 256, 512, 1000, 1152, 2048, 2560, 3840, 4096, 5376,
                               8192, 12288, 15360, 16384, 20480])
def test_gpu_summation_order_is_numpys(n):
    """The GPU RMSNorm sums squares in numpy's pairwise order: its algorithm,
    restated in parity.pw_sum_gpu_order, equals np.add.reduce (and np.mean is
    that sum / n in float32) bit for bit, for halving widths and others."""
    rng = np.random.default_rng(n)
    for _ in range(3):
        x = q4_numpy.bf16_rne(rng.normal(0, rng.uniform(0.01, 30), n).astype(np.float32))
        sq = x ** 2
        s = np.add.reduce(sq)
        assert parity.pw_sum_gpu_order(sq) == s
        assert np.mean(sq) == np.float32(s / np.float32(n))


def test_rmsnorm_restatement_pins():
    rng = np.random.default_rng(3)
    w = rng.uniform(0.5, 1.5, 3840).astype(np.float32)
    # Constant +-2^k rows: mean(x^2) = 4^k exactly, sqrt(4^k + eps) rounds to
    # 2^k (k >= 3), so the output is bf16(+-w).
    for k in (3, 5, -1 + 10):
        c = np.float32(2.0 ** k)
        x = np.full(3840, c, np.float32)
        x[::3] = -c
        assert np.array_equal(q4_numpy.rmsnorm_cpu(x, w), q4_numpy.bf16_rne(np.sign(x) * w))
    # fp64 brute force: within one bf16 ulp.
    x = q4_numpy.bf16_rne(rng.normal(0, 3, 3840).astype(np.float32))
    y = q4_numpy.rmsnorm_cpu(x, w).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6) * w
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-30)
    # No weights (Gemma-4's v norm): unit RMS.
    z = q4_numpy.rmsnorm_cpu(x, None).astype(np.float64)
    assert abs(np.sqrt(np.mean(z ** 2)) - 1.0) < 5e-3


def test_rope_restatement_pins():
    t = q4_numpy.cos_sin_table_gemma(10000.0, 256, 64)
    assert np.all(t[0, :128] == 1.0) and np.all(t[0, 128:] == 0.0)
    g = q4_numpy.cos_sin_table_gemma(1e6, 512, 8)
    assert np.all(g[5, 64:256] == 1.0) and np.all(g[5, 256 + 64:] == 0.0)  # unrotated three quarters
    rng = np.random.default_rng(4)
    x = q4_numpy.bf16_rne(rng.normal(0, 1, 16 * 256).astype(np.float32))
    assert np.array_equal(q4_numpy.rope_cpu_gemma(x, t[0], 256), x)  # position 0: identity
    # A rotation: per pair, within one bf16 ulp of the fp64 rotation by the table's angles.
    pos = 37
    y = q4_numpy.rope_cpu_gemma(x, t[pos], 256).astype(np.float64).reshape(16, 256)
    c, s = t[pos, :128].astype(np.float64), t[pos, 128:].astype(np.float64)
    xr = x.astype(np.float64).reshape(16, 256)
    ref = np.concatenate([xr[:, :128] * c - xr[:, 128:] * s, xr[:, 128:] * c + xr[:, :128] * s], axis=1)
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + 2.0 ** -24 * (np.abs(xr) @ np.ones((256, 256))))
    # the table holds cos/sin of pos * base^(-2i/dim) to bf16 precision
    f = pos * 10000.0 ** (-np.arange(0, 256, 2) / 256)
    assert np.all(np.abs(t[pos, :128] - np.cos(f)) <= 2.0 ** -8 + 1e-6)


def test_attention_restatement_pins():
    rng = np.random.default_rng(5)
    kv, D, S, heads = 2, 64, 40, 4
    kc = q4_numpy.bf16_rne(rng.normal(0, 1, (kv, S, D)).astype(np.float32))
    vc = q4_numpy.bf16_rne(rng.normal(0, 1, (kv, S, D)).astype(np.float32))
    q = q4_numpy.bf16_rne(rng.normal(0, 1, heads * D).astype(np.float32))
    # One position: softmax 1, the output is v itself (bf16 exact).
    out = q4_numpy.attention_host(q, kc, vc, 0, heads, kv, D, 1.0)
    assert np.array_equal(out.reshape(heads, D), np.repeat(vc[:, 0], 2, axis=0))
    # q = 0: uniform weights, the mean of v over the window (GQA: heads 2k, 2k+1 share kv head k).
    out = q4_numpy.attention_host(np.zeros(heads * D, np.float32), kc, vc, 29, heads, kv, D, 1.0, window=10)
    mean = vc[:, 20:30].astype(np.float64).mean(1)
    assert np.all(np.abs(out.reshape(heads, D) - np.repeat(mean, 2, axis=0)) <= np.abs(np.repeat(mean, 2, 0)) * 2.0 ** -8 + 1e-6)
    # fp64 brute force, global attention.
    out = q4_numpy.attention_host(q, kc, vc, 33, heads, kv, D, 0.125).astype(np.float64).reshape(heads, D)
    for h in range(heads):
        k64, v64 = kc[h // 2, :34].astype(np.float64), vc[h // 2, :34].astype(np.float64)
        sc = k64 @ q[h * D:(h + 1) * D].astype(np.float64) * 0.125
        p = np.exp(sc - sc.max())
        ref = (p / p.sum()) @ v64
        assert np.all(np.abs(out[h] - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-5 * (p / p.sum()) @ np.abs(v64) + 1e-6)


def test_gemma4_layer_restatement_closed_form():
    """With zero O and down projections both branches vanish (rmsnorm(0) = 0),
    so the layer is y = bf16(bf16(x) * scale) and the caches still receive k
    and v at pos."""
    rng = np.random.default_rng(6)
    H = 256
    x = q4_numpy.bf16_rne(rng.normal(0, 1, H).astype(np.float32))
    w = {k: rng.uniform(0.5, 1.5, 256).astype(np.float32) for k in ("attn", "q", "k", "post_attn", "ffn", "post_ffw")}
    w["scale"] = np.float32(0.75)
    qkv_val = q4_numpy.bf16_rne(rng.normal(0, 1, 8192).astype(np.float32))
    kc = np.zeros((8, 16, 256), np.float32)
    vc = np.zeros((8, 16, 256), np.float32)
    t = q4_numpy.cos_sin_table_gemma(10000.0, 256, 16)
    y = q4_numpy.gemma4_decode_layer(x, 3, True, w, lambda xn: qkv_val, lambda a: np.zeros(H, np.float32),
                                     lambda xn: np.zeros(H, np.float32), kc, vc, t[3])
    assert np.array_equal(y, q4_numpy.bf16_rne(x * np.float32(0.75)))
    v_n = np.concatenate([q4_numpy.rmsnorm_cpu(qkv_val[6144 + 256 * h:6144 + 256 * (h + 1)], None) for h in range(8)])
    assert np.array_equal(vc[:, 3].reshape(-1), v_n)
    assert np.any(kc[:, 3] != 0) and not np.any(kc[:, 4])


def test_llama_rope_restatement_pins():
    """cos_sin_table_llama against closed forms: position 0 is (cos 1, sin 0);
    each row repeats its 32 cosines and 32 sines; the fastest angle (inverse
    frequency 1, wavelength 2 pi below the high-frequency bound 2048) is the
    position itself, the slowest (wavelength above 8192) is divided by the
    factor 32, and a medium one follows the smoothing between the two. Then
    rope_cpu_llama: identity at position 0, and on a made-up row whose
    cosines are 0 and whose sines (values 64..95) are 1 the exact swap
    y1 = -x2, y2 = x1 -- with values 32..63 set to a decoy that a reader of
    the wrong offset would pick up."""
    t = q4_numpy.cos_sin_table_llama(300)
    assert np.all(t[0, :64] == 1.0) and np.all(t[0, 64:] == 0.0)
    assert np.array_equal(t[:, 32:64], t[:, :32]) and np.array_equal(t[:, 96:], t[:, 64:96])
    pos = np.arange(300, dtype=np.float64)
    inv = 500000.0 ** (-np.arange(0, 64, 2) / 64.0)
    wl = 2 * np.pi / inv
    assert wl[0] < 2048 and wl[31] > 8192
    assert np.all(np.abs(t[:, 0] - np.cos(pos)) <= 2.0 ** -8 + 1e-6)
    assert np.all(np.abs(t[:, 64] - np.sin(pos)) <= 2.0 ** -8 + 1e-6)
    assert np.all(np.abs(t[:, 31] - np.cos(pos * inv[31] / 32)) <= 2.0 ** -8 + 1e-6)
    med = [i for i in range(32) if 2048 <= wl[i] <= 8192]
    assert med
    i = med[0]
    sm = (8192 / wl[i] - 1.0) / 3.0
    f = (1 - sm) * inv[i] / 32 + sm * inv[i]
    assert np.all(np.abs(t[:, i] - np.cos(pos * f)) <= 2.0 ** -8 + 1e-5)
    assert not np.allclose(t[:, i], np.cos(pos * inv[i]), atol=1e-2)  # not the unscaled angle
    rng = np.random.default_rng(8)
    x = q4_numpy.bf16_rne(rng.normal(0, 1, 8 * 64).astype(np.float32))
    assert np.array_equal(q4_numpy.rope_cpu_llama(x, t[0]), x)
    row = np.zeros(128, np.float32)
    row[32:64] = 0.5  # decoy
    row[64:96] = 1.0
    y = q4_numpy.rope_cpu_llama(x, row).reshape(8, 64)
    xr = x.reshape(8, 64)
    assert np.array_equal(y[:, :32], -xr[:, 32:]) and np.array_equal(y[:, 32:], xr[:, :32])


def test_gemma3_llama_layer_restatement_closed_forms():
    """With the FFN's output zero and the O projection returning a fixed c,
    a Llama layer is y = bf16(x + c) (no norm on the residual adds) and a
    Gemma-3 layer y = bf16(x + rmsnorm(c) * w_post_attn) (the post-attention
    norm, no output scale); with both zero, y = x. The caches receive the
    rotated k (Gemma-3: after its norm) and the raw v at pos."""
    rng = np.random.default_rng(9)
    # Llama: H 256, 4 q heads and 2 kv heads of 64.
    H = 256
    x = q4_numpy.bf16_rne(rng.normal(0, 1, H).astype(np.float32))
    c = q4_numpy.bf16_rne(rng.normal(0, 1, H).astype(np.float32))
    w = {k: rng.uniform(0.5, 1.5, H).astype(np.float32) for k in ("attn", "ffn")}
    qkv_val = q4_numpy.bf16_rne(rng.normal(0, 1, 8 * 64).astype(np.float32))
    kc, vc = np.zeros((2, 16, 64), np.float32), np.zeros((2, 16, 64), np.float32)
    t = q4_numpy.cos_sin_table_llama(16)
    zero = lambda a: np.zeros(H, np.float32)  # noqa: E731
    y = q4_numpy.llama_decode_layer(x, 5, w, lambda xn: qkv_val, lambda a: c, zero, kc, vc, t[5], 4, 2)
    assert np.array_equal(y, q4_numpy.bf16_rne(x + c))
    y0 = q4_numpy.llama_decode_layer(x, 6, w, lambda xn: qkv_val, zero, zero, kc, vc, t[6], 4, 2)
    assert np.array_equal(y0, x)
    assert np.array_equal(kc[:, 5].reshape(-1), q4_numpy.rope_cpu_llama(qkv_val[256:384], t[5]))
    assert np.array_equal(vc[:, 5].reshape(-1), qkv_val[384:512])
    # Gemma-3: H 256, 2 q heads and 1 kv head of 256.
    wg = {k: rng.uniform(0.5, 1.5, 256).astype(np.float32) for k in ("attn", "q", "k", "post_attn", "ffn", "post_ffw")}
    qkv3 = q4_numpy.bf16_rne(rng.normal(0, 1, 4 * 256).astype(np.float32))
    kc3, vc3 = np.zeros((1, 16, 256), np.float32), np.zeros((1, 16, 256), np.float32)
    tg = q4_numpy.cos_sin_table_gemma(10000.0, 256, 16)
    y3 = q4_numpy.gemma3_decode_layer(x, 4, True, wg, lambda xn: qkv3, lambda a: c, zero, kc3, vc3, tg[4], 2, 1)
    assert np.array_equal(y3, q4_numpy.bf16_rne(x + q4_numpy.rmsnorm_cpu(c, wg["post_attn"])))
    assert not np.array_equal(y3, q4_numpy.bf16_rne(x + c))
    y30 = q4_numpy.gemma3_decode_layer(x, 5, False, wg, lambda xn: qkv3, zero, zero, kc3, vc3, tg[5], 2, 1)
    assert np.array_equal(y30, x)
    k_n = q4_numpy.rmsnorm_cpu(qkv3[512:768], wg["k"])
    assert np.array_equal(kc3[0, 4], q4_numpy.rope_cpu_gemma(k_n, tg[4], 256))
    assert np.array_equal(vc3[0, 4], qkv3[768:1024])


def test_ffn_check_batch_pins(orc):
    """The batched flip-aware FFN check (tests/parity.py::ffn_check_batch)
    accepts the float32 oracle's own outputs and rejects a planted mistake:
    the GLU applied to g before its bf16 rounding."""
    import parity

    H, I, M = 256, 512, 7
    Wg, Wu, Wd = orc.synth_q4(I, H, 1), orc.synth_q4(I, H, 2), orc.synth_q4(H, I, 3)
    X = orc.synth_normal(M * H, 4).reshape(M, H)
    G, U = orc.gemm_q(Wg, X, M, I, H), orc.gemm_q(Wu, X, M, I, H)
    A = orc.glu(orc.bf16_round(G), orc.bf16_round(U), 0).reshape(M, I)
    st = parity.ffn_check_batch(orc, Wg, Wu, Wd, X, H, I, 0, orc.gemm_q(Wd, A, M, H, I), A)
    assert st["tokens"] == M and st["max_rel"] <= parity.TOL
    A2 = orc.glu(G.reshape(-1), orc.bf16_round(U), 0).reshape(M, I)
    with pytest.raises(AssertionError):
        parity.ffn_check_batch(orc, Wg, Wu, Wd, X, H, I, 0, orc.gemm_q(Wd, A2, M, H, I), A2)
