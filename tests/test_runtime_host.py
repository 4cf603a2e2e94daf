"""Host-side pieces of the Python dispatch (no GPU): LazyLayerWeights loads a
layer's packed projections from ``blk.{l}.{proj}.weight_packed.npy`` files
(runtime/py/model.py:37-56) into ResidentWeight (model.py:31-35) with their
2-D shapes, skips projections that have no file, and refuses pickled
arrays (the files are loaded with allow_pickle=False)."""
import numpy as np
import pytest
import torch

from alveare_amd.runtime import PROJECTIONS, LazyLayerWeights, ResidentWeight, _shape_of, load_layer_weights


def _write(tmp_path, layer, proj, arr):
    np.save(tmp_path / f"blk.{layer}.{proj}.weight_packed.npy", arr, allow_pickle=False)


def test_lazy_layer_weights_loads_packed_files(tmp_path):
    rng = np.random.default_rng(7)
    shapes = {"attn_q": (64, 96 // 32 * 20), "attn_k": (32, 96 // 32 * 20), "ffn_down": (96, 128 // 32 * 20)}
    arrs = {p: rng.integers(0, 256, size=s, dtype=np.uint8) for p, s in shapes.items()}
    for p, a in arrs.items():
        _write(tmp_path, 3, p, a)
    _write(tmp_path, 4, "attn_q", arrs["attn_q"][:16])
    lw = LazyLayerWeights(tmp_path, 3, device="cpu")
    for p in PROJECTIONS:
        assert (p in lw) == (p in arrs)
    for p, a in arrs.items():
        rw = lw[p]
        assert isinstance(rw, ResidentWeight)
        assert rw.shape == a.shape and rw.size == a.size
        assert rw.tensor.dtype == torch.uint8 and rw.tensor.dim() == 1
        assert np.array_equal(rw.tensor.numpy(), a.reshape(-1))
        N, K = _shape_of(rw)
        assert N == a.shape[0] and K == a.shape[1] // 20 * 32
    with pytest.raises(KeyError):
        lw["attn_v"]
    lw.clear()  # weights stay resident, as in the reference
    assert "attn_q" in lw
    layers = load_layer_weights(tmp_path, 5, device="cpu")
    assert len(layers) == 5
    assert "attn_q" in layers[3] and "attn_q" in layers[4] and "attn_q" not in layers[0]
    assert layers[4]["attn_q"].shape == (16, shapes["attn_q"][1])


def test_lazy_layer_weights_refuses_pickles(tmp_path):
    np.save(tmp_path / "blk.0.attn_q.weight_packed.npy", np.array([{"x": 1}], dtype=object), allow_pickle=True)
    with pytest.raises(ValueError):
        LazyLayerWeights(tmp_path, 0, device="cpu")


def test_rope_tables_match_the_oracle():
    """The layers' RoPE tables (built on the host when a layer is created)
    equal the oracle's restatements bit for bit: Llama-3.2's scaled table and
    Gemma-3's 256-wide one."""
    import parity
    from alveare_amd import layer
    from oracle import q4_numpy as qn

    assert np.array_equal(layer.cos_sin_table_llama(300), parity.f32_bits_bf16(qn.cos_sin_table_llama(300)))
    for base in (10000.0, 1e6):
        assert np.array_equal(layer.cos_sin_table_gemma(base, 256, 64, gemma4=False),
                              parity.f32_bits_bf16(qn.cos_sin_table_gemma(base, 256, 64, gemma4=False)))
