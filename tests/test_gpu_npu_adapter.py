"""The C++ NpuRegistry adapter on the GPU: tests/cpp/npu_registry_check drives
alveare::NpuRegistry as the reference runtime drives its registry
(runtime/cpp/src/main.cpp:54-132, weights.cpp:192-380): register, then run on
host bf16 buffers. Outputs against the oracle (GEMV / GEMM: every bf16 value
between the bf16 roundings of the fp64 value +- its float32 bound) and, for the
FFN, against the same registered FFN run directly (the FFN kernels' own
oracle parity is covered elsewhere)."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import parity
from oracle import q4_numpy as qn

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "alveare_amd", "npu_registry_check")


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run(args, tmp_path):
    if not os.path.exists(CHECK):
        pytest.fail("alveare_amd/npu_registry_check is not built")
    _say("npu_registry_check", *args[:4])
    r = subprocess.run([CHECK, *[str(a) for a in args]], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


def _bf16_file(path, x):
    parity.f32_bits_bf16(np.asarray(x, np.float32)).tofile(path)


@pytest.mark.parametrize("mode,B,N,K", [("gemv", 1, 2048, 2048), ("gemv", 1, 8192, 3840), ("gemm", 16, 1024, 3840),
                                        ("gemm", 64, 1024, 3840), ("gemm_streamed", 8, 1152, 2048),
                                        ("gemm_streamed", 64, 512, 1024)])
def test_registry_matmuls(orc, dev, tmp_path, mode, B, N, K):
    W = orc.synth_q4(N, K, 500 + B)
    X = qn.bf16_rne(orc.synth_normal(B * K, 501 + B)).reshape(B, K)
    W.tofile(tmp_path / "W")
    _bf16_file(tmp_path / "x", X)
    if mode == "gemv":
        _run([mode, N, K, tmp_path / "W", tmp_path / "x", tmp_path / "y"], tmp_path)
    else:
        _run([mode, B, N, K, tmp_path / "W", tmp_path / "x", tmp_path / "y"], tmp_path)
    y = np.fromfile(tmp_path / "y", np.uint16).reshape(B, N)
    for b in range(B):
        parity.gemv_bf16_check(orc, W, X[b], y[b], N, K)


# Gemma-4's FFN goes through the registry at its padded shape 4096 x 16384
# (runtime/cpp/src/weights.cpp:336-337): at 3840 the packing's four down
# passes would drop rows, which the adapter refuses (tests/test_npu_adapter.py).
@pytest.mark.parametrize("H,I,act,packing", [(1024, 2048, "gelu", None), (4096, 16384, "gelu", None),
                                              (512, 1536, "silu", (32, 128))])
def test_registry_ffn_from_reference_blob(orc, dev, tmp_path, H, I, act, packing):
    import alveare_amd as aa
    from alveare_amd import layer

    m_I, kt = packing or (32, 128 if H == 1152 else 256)
    Wg, Wu, Wd = orc.synth_q4(I, H, 510), orc.synth_q4(I, H, 511), orc.synth_q4(H, I, 512)
    x = qn.bf16_rne(orc.synth_normal(H, 513))
    qn.pack_ffn_fused_weights_ref(Wg, Wu, Wd, H, I, m_I, kt).tofile(tmp_path / "P")
    _bf16_file(tmp_path / "x", x)
    args = ["ffn", H, I, act, tmp_path / "P", tmp_path / "x", tmp_path / "y"]
    if packing:
        args += list(packing)
    _run(args, tmp_path)
    y = np.fromfile(tmp_path / "y", np.uint16)
    F = aa.FfnWeights(*(torch.from_numpy(w).to(dev) for w in (Wg, Wu, Wd)), H, I, act)
    xd = torch.from_numpy(parity.f32_bits_bf16(x).view(np.int16)).view(torch.bfloat16).to(dev)
    direct = parity.bf16_bits(layer.ffn_fused_bf16(F, xd))
    F.close()
    assert np.array_equal(y, direct)


def test_registry_errors(orc, dev, tmp_path):
    """Invalid handle, shape mismatch, wrong weight kind and a short blob all
    raise std::runtime_error (runtime/cpp/src/npu.cpp:272-276, :295-299)."""
    orc.synth_q4(256, 512, 520).tofile(tmp_path / "W")
    _run(["errors", 256, 512, tmp_path / "W"], tmp_path)


MANIFEST = """{
  "model_type": "gemma4",
  "kernel_name": "MLIR_AIE",
  "kernels": [
    {"kind": "gemv", "N": 8192, "K": 4096, "m": 32, "k_tile": 256, "n_cores": 32,
     "xclbin": "gemv_8192x4096.xclbin", "insts": "gemv_8192x4096.bin"},
    {"kind": "gemm", "B": 16, "N": 16384, "K": 4096, "m": 32, "k_tile": 256, "n_cores": 32,
     "xclbin": "gemm.xclbin", "insts": "gemm.bin", "extra": {"nested": [1, 2, "x\\"y"]}},
    {"kind": "ffn_fused", "H": 1024, "I": 2048, "activation": "gelu", "m": 32, "k_tile": 128,
     "n_cores": 32, "xclbin": "ffn.xclbin", "insts": "ffn.bin"}
  ]
}
"""


def test_registry_reads_manifest(dev, tmp_path):
    """kernels() lists the manifest's kernels (the reference's parity driver,
    runtime/cpp/test/parity_test.cpp:30, walks it), model_type comes from it,
    and unknown fields are skipped."""
    (tmp_path / "manifest.json").write_text(MANIFEST)
    env = dict(os.environ, NPU_MANIFEST=str(tmp_path / "manifest.json"))
    r = subprocess.run([CHECK, "manifest", str(tmp_path / "k.txt")], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
    lines = (tmp_path / "k.txt").read_text().splitlines()
    assert lines[0] == "model_type gemma4"
    assert lines[1:] == ["gemv 8192 4096 0 0 0  32 256 32 gemv_8192x4096.xclbin",
                         "gemm 16384 4096 16 0 0  32 256 32 gemm.xclbin",
                         "ffn_fused 0 0 0 1024 2048 gelu 32 128 32 ffn.xclbin"]


def test_registry_ffn_packing_from_manifest(orc, dev, tmp_path):
    """A blob packed with k_tile = 128 at H = 1024 (the loader's rule would
    say 256): the manifest's ffn_fused entry for the shape gives the packing,
    so the blob unpacks to the right weights."""
    import alveare_amd as aa
    from alveare_amd import layer

    H, I = 1024, 2048
    Wg, Wu, Wd = orc.synth_q4(I, H, 530), orc.synth_q4(I, H, 531), orc.synth_q4(H, I, 532)
    x = qn.bf16_rne(orc.synth_normal(H, 533))
    qn.pack_ffn_fused_weights_ref(Wg, Wu, Wd, H, I, 32, 128).tofile(tmp_path / "P")
    _bf16_file(tmp_path / "x", x)
    (tmp_path / "manifest.json").write_text(MANIFEST)
    env = dict(os.environ, NPU_MANIFEST=str(tmp_path / "manifest.json"))
    args = [CHECK, "ffn", H, I, "gelu", tmp_path / "P", tmp_path / "x", tmp_path / "y"]
    r = subprocess.run([str(a) for a in args], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
    y = np.fromfile(tmp_path / "y", np.uint16)
    F = aa.FfnWeights(*(torch.from_numpy(w).to(dev) for w in (Wg, Wu, Wd)), H, I, "gelu")
    xd = torch.from_numpy(parity.f32_bits_bf16(x).view(np.int16)).view(torch.bfloat16).to(dev)
    direct = parity.bf16_bits(layer.ffn_fused_bf16(F, xd))
    F.close()
    assert np.array_equal(y, direct)
