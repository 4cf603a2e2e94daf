"""The reference's own C++ runtime driving this build through the NpuRegistry
adapter on the GPU.

oracle/Makefile's `ref-runtime` target compiles runtime/cpp/src (main.cpp,
model.cpp, weights.cpp, ...) from the reference's sources, unchanged, against
alveare_amd/cpp/alveare/npu.h and libalveare_npu.so, into
oracle/_ref/alveare_runtime_ref. These tests give it a synthetic one-layer
Gemma-4 model directory in the reference's on-disk format (weights.cpp:192-380:
packed Q4 .npy per projection, float32 norms, config.json) and run the
self-check main.cpp carries for the registry, ALVEARE_TEST_GEMM
(main.cpp:76-152): it registers the 16384x4096 FFN gate, runs run_gemv and
run_gemm(16) on equal rows and prints their largest difference, then
run_gemm_streamed, run_ffn_fused and the up GEMV. (Its ALVEARE_TEST_LAUNCH
probe reads separate q and k handles, which the reference's own loader does
not create for Gemma-4.) The weights are loaded by the reference's loader (weights.cpp), which also
packs the FFN blob (pack_ffn_fused_weights) that the adapter unpacks.
"""
import json
import os
import re
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "oracle", "_ref", "alveare_runtime_ref")


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


VOCAB = 16384  # one 16384-row LM-head tile, registered on the GPU by the reference's loader


def _model_dir(orc, d, layers=1, head=False):
    """Gemma-4 layers (every sixth global) at the shapes the reference's
    quantizer writes (K padded to 4096, FFN 16384 x 4096, global q 8192 rows
    and O 4096 x 8192), float32 norms, output scale 1; with `head`, a
    16384-token fp16 embedding, the final norm and the packed LM head."""
    H = 3840
    cfg = {"model_type": "gemma4", "num_hidden_layers": layers, "hidden_size": H, "intermediate_size": 15360,
           "num_attention_heads": 16, "num_key_value_heads": 8, "head_dim": 256, "vocab_size": VOCAB}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)
    rng = np.random.default_rng(5)
    for l in range(layers):
        sliding = (l + 1) % 6 != 0
        hd = 256 if sliding else 512
        for name, n in (("attn_norm", H), ("ffn_norm", H), ("post_attention_norm", H), ("post_ffw_norm", H),
                        ("attn_q_norm", hd), ("attn_k_norm", hd)):
            np.save(os.path.join(d, f"blk.{l}.{name}.weight.npy"), rng.uniform(0.5, 1.5, n).astype(np.float32))
        np.save(os.path.join(d, f"blk.{l}.layer_output_scale.weight.npy"), np.ones(1, np.float32))
        shapes = {"attn_q": (4096 if sliding else 8192, 4096), "attn_k": (2048, 4096),
                  "attn_output": (4096, 4096 if sliding else 8192),
                  "ffn_gate": (16384, 4096), "ffn_up": (16384, 4096), "ffn_down": (4096, 16384)}
        if sliding:
            shapes["attn_v"] = (2048, 4096)
        for i, (name, (N, K)) in enumerate(shapes.items()):
            W = orc.synth_q4(N, K, orc.seed_for(9, 16 * l + i)).reshape(N, K // 32 * 20)
            np.save(os.path.join(d, f"blk.{l}.{name}.weight_packed.npy"), W)
    if head:
        np.save(os.path.join(d, "token_embd.npy"), (rng.normal(0, 0.05, (VOCAB, H))).astype(np.float16))
        np.save(os.path.join(d, "output_norm.weight.npy"), rng.uniform(0.5, 1.5, H).astype(np.float32))
        np.save(os.path.join(d, "lm_head_packed.npy"),
                orc.synth_q4(VOCAB, 4096, orc.seed_for(9, 999)).reshape(VOCAB, 4096 // 32 * 20))
    manifest = os.path.join(d, "manifest.json")
    with open(manifest, "w") as f:
        json.dump({"model_type": "gemma4", "kernels": []}, f)
    return manifest


def _run(args, env_flag, timeout=240):
    env = dict(os.environ)
    env[env_flag] = "1"
    r = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=timeout, env=env)
    return r.returncode, r.stdout + r.stderr


@pytest.fixture(scope="module")
def model(orc, tmp_path_factory):
    if not os.path.exists(EXE):
        pytest.skip("oracle/_ref/alveare_runtime_ref not built (needs the reference's runtime sources)")
    d = str(tmp_path_factory.mktemp("gemma4_1layer"))
    return d, _model_dir(orc, d)


def test_reference_runtime_gemm_self_check(model):
    """main.cpp's ALVEARE_TEST_GEMM through the adapter: the 16 rows of
    run_gemm on equal inputs match run_gemv (the reference prints the largest
    difference; here every row is within one bf16 ulp of the largest output),
    and the streamed GEMM, fused FFN and up GEMV calls complete."""
    d, manifest = model
    _say("reference runtime: ALVEARE_TEST_GEMM")
    rc, out = _run([d, manifest], "ALVEARE_TEST_GEMM")
    _say(out[-2500:])
    assert rc == 0, out[-4000:]
    m = re.search(r"GEMM-vs-GEMV correctness: signal_max=(\S+) row0_maxdiff=(\S+) row15_maxdiff=(\S+)", out)
    assert m, "no correctness line"
    sig, d0, d15 = (float(v) for v in m.groups())
    assert sig > 0
    assert d0 <= sig * 2.0 ** -7 and d15 <= sig * 2.0 ** -7
    assert "fused (gate+up+gelu+down)" in out and "gemm(16) streamed" in out


@pytest.fixture(scope="module")
def model6(orc, tmp_path_factory):
    if not os.path.exists(EXE):
        pytest.skip("oracle/_ref/alveare_runtime_ref not built (needs the reference's runtime sources)")
    d = str(tmp_path_factory.mktemp("gemma4_6layer"))
    return d, _model_dir(orc, d, layers=6, head=True)


def test_reference_runtime_bench(model6):
    """main.cpp's ALVEARE_BENCH (main.cpp:226-293) through the adapter on six
    Gemma-4 layers (five sliding, one global) with a 16384-token head: its
    per-shape kernel timings (the reference's own harness and shapes, the
    rows its published NPU report lists), then a real generation of 8 tokens
    after the prompt's batched prefill -- the reference's model.cpp and
    generator.cpp driving every matmul on the GPU."""
    d, manifest = model6
    _say("reference runtime: ALVEARE_BENCH (6 layers)")
    rc, out = _run([d, manifest], "ALVEARE_BENCH", timeout=600)
    _say(out[-4000:])
    assert rc == 0, out[-4000:]
    kern = re.findall(r"^KERNEL (\S+) (\S+) (\d+) (\d+) (\S+) (\S+)$", out, re.M)
    names = {(k[0], k[1]) for k in kern}
    for want in (("gemv", "qkv_sliding"), ("gemv", "o_sliding"), ("gemv", "qkv_global"), ("gemv", "o_global"),
                 ("gemv", "lm_head"), ("ffn_fused", "ffn"), ("gemm16", "gate")):
        assert want in names, (want, names)
    assert all(float(k[4]) > 0 for k in kern)
    assert "=== ALVEARE BENCH END ===" in out
    assert re.search(r"Token \d+/\d+", out) or "Prefill" in out
