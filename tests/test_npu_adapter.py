"""The C++ NpuRegistry adapter's host side (no GPU): unpacking the reference's
packed FFN blob (runtime/cpp/src/weights.cpp:94-190) back into gate / up /
down, through libalveare_npu.so's alvnpu_unpack_ffn."""
import ctypes
import os

import numpy as np
import pytest

from oracle import q4_numpy

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NPU_LIB = os.path.join(ROOT, "alveare_amd", "libalveare_npu.so")


@pytest.fixture(scope="module")
def npu():
    if not os.path.exists(NPU_LIB):
        from alveare_amd import build
        build.build(verbose=False)
    lib = ctypes.CDLL(NPU_LIB)
    lib.alvnpu_unpack_ffn.restype = ctypes.c_int
    lib.alvnpu_unpack_ffn.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.alvnpu_last_error.restype = ctypes.c_char_p
    return lib


def _rand(rng, rows, cols):
    return rng.integers(0, 256, size=(rows, cols // 32 * 20), dtype=np.uint8)


def _unpack(npu, blob, H, I, m_I, k_tile):
    g = np.zeros((I, H // 32 * 20), np.uint8)
    u = np.zeros_like(g)
    d = np.zeros((H, I // 32 * 20), np.uint8)
    rc = npu.alvnpu_unpack_ffn(blob.ctypes.data, blob.nbytes, H, I, m_I, k_tile, g.ctypes.data, u.ctypes.data,
                               d.ctypes.data)
    return rc, g, u, d


def test_packing_restatement_hand_tiles():
    """One core (I = 96 is not a multiple of 2 * m_I): the blob starts with
    gate rows 0..31 over the first k_tile columns, then up's, then gate's next
    column block; down tiles follow after every gate/up tile."""
    rng = np.random.default_rng(1)
    H, I, m_I, kt = 512, 96, 32, 128
    g, u, d = _rand(rng, I, H), _rand(rng, I, H), _rand(rng, H, I)
    blob = q4_numpy.pack_ffn_fused_weights_ref(g, u, d, H, I, m_I, kt)
    w = kt // 32 * 20
    tile = m_I * w
    assert blob.nbytes == 3 * I * H // 32 * 20
    assert np.array_equal(blob[:tile].reshape(m_I, w), g[:32, :w])
    assert np.array_equal(blob[tile:2 * tile].reshape(m_I, w), u[:32, :w])
    assert np.array_equal(blob[2 * tile:3 * tile].reshape(m_I, w), g[:32, w:2 * w])
    gu = 2 * (I // m_I) * (H // kt) * tile
    # first down tile: rows 0..k_tile-1 of down, the core's first m_I columns
    assert np.array_equal(blob[gu:gu + tile].reshape(kt, m_I // 32 * 20), d[:kt, :m_I // 32 * 20])


@pytest.mark.parametrize("H,I,m_I,k_tile", [(512, 96, 32, 128), (256, 128, 32, 64), (512, 512, 32, 128),
                                             (1024, 2048, 32, 256), (1024, 1024, 64, 256), (2048, 4096, 32, 256)])
def test_unpack_inverts_packing(npu, H, I, m_I, k_tile):
    rng = np.random.default_rng(H + I)
    g, u, d = _rand(rng, I, H), _rand(rng, I, H), _rand(rng, H, I)
    blob = q4_numpy.pack_ffn_fused_weights_ref(g, u, d, H, I, m_I, k_tile)
    rc, g2, u2, d2 = _unpack(npu, blob, H, I, m_I, k_tile)
    assert rc == 0, npu.alvnpu_last_error()
    assert np.array_equal(g2, g) and np.array_equal(u2, u) and np.array_equal(d2, d)


def test_unpack_rejects_lossy_packing_and_bad_sizes(npu):
    """Gemma-3-1B's shape (H = 1152, k_tile = 128) packs only 8 of its 9 down
    row tiles (the four passes take (H / k_tile) / 4 each); the adapter
    refuses it rather than register a down projection with missing rows."""
    rng = np.random.default_rng(3)
    H, I = 1152, 6912
    blob = np.zeros(3 * I * H // 32 * 20, np.uint8)
    rc, *_ = _unpack(npu, blob, H, I, 32, 128)
    assert rc == -1 and b"leaves out rows" in npu.alvnpu_last_error()
    H, I = 512, 512
    blob = q4_numpy.pack_ffn_fused_weights_ref(_rand(rng, I, H), _rand(rng, I, H), _rand(rng, H, I), H, I, 32, 128)
    rc, *_ = _unpack(npu, blob[:-20], H, I, 32, 128)
    assert rc == -1 and b"expected" in npu.alvnpu_last_error()


REF = "/root/reference"
REF_SRC = os.path.join(REF, "runtime", "cpp", "src")


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="the reference tree is not mounted here")
@pytest.mark.parametrize("unit", ["weights", "model", "generator", "main"])
def test_reference_runtime_compiles_against_adapter(tmp_path, unit):
    """The reference's C++ runtime sources compile unchanged against this
    build's alveare/npu.h (syntax only: the XRT-free translation units the
    registry is used from). The adapter's include directory comes first, and
    the header list shows that its npu.h, not the reference's, was used."""
    import subprocess

    inc = [os.path.join(ROOT, "alveare_amd", "cpp"), os.path.join(REF, "runtime", "cpp", "include")]
    tp = os.path.join(REF, "third_party")
    if os.path.isdir(tp):
        inc.append(tp)
    cmd = ["g++", "-std=c++17", "-fsyntax-only", "-H", *[f"-I{d}" for d in inc], os.path.join(REF_SRC, unit + ".cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    headers = [l.lstrip(". ").strip() for l in r.stderr.splitlines() if l.startswith(".")]
    ours = os.path.join(ROOT, "alveare_amd", "cpp", "alveare", "npu.h")
    theirs = os.path.join(REF, "runtime", "cpp", "include", "alveare", "npu.h")
    if any(os.path.basename(h) == "npu.h" for h in headers):
        assert any(os.path.realpath(h) == os.path.realpath(ours) for h in headers), "adapter npu.h not used"
        assert not any(os.path.realpath(h) == os.path.realpath(theirs) for h in headers), "reference npu.h used"
