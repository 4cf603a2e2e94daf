"""alveare_amd -- MI355X-native (gfx950) Q4 decode hot path of Alveare.

HIP kernels behind a C ABI (``include/alveare_q4.h``, ``libalveare_q4.so``)
for the three quantized matmuls of Alveare's runtime -- ``gemv_q``,
``ffn_fused`` and ``gemm_q`` -- with torch-facing ops (``alveare_amd.ops``)
and the ``runtime/py`` dispatch (``alveare_amd.runtime``) on top.
"""
from ._lib import LibraryNotBuilt, Q4Error, Q4ValueError, lib
from .ops import (FfnWeights, Q4Weight, chain_run, dequant_q4, ffn_fused, ffn_fused_npu,
                  gemm_q, gemm_q_npu, gemv_q, gemv_q_npu, lm_head, pack_ffn_fused_weights, q4_tile,
                  quantize_q4)
from .runtime import LazyLayerWeights, Q4Dispatch, ResidentWeight

__all__ = [
    "FfnWeights", "LazyLayerWeights", "LibraryNotBuilt", "Q4Dispatch", "Q4Error", "Q4ValueError",
    "Q4Weight", "ResidentWeight", "chain_run", "dequant_q4", "ffn_fused", "ffn_fused_npu", "gemm_q", "gemm_q_npu",
    "gemv_q", "gemv_q_npu", "lib", "lm_head", "pack_ffn_fused_weights", "q4_tile", "quantize_q4",
]
