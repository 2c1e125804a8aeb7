"""MI355X-native gated-delta linear attention.

A drop-in for the gated-delta path of ``mlx-lean-moe``
(``src/mlx_lean_moe/model/qwen3_5/{gated_delta,linear_attention}.py``,
``src/mlx_lean_moe/cache/recurrent_cache.py``): the same Python surface over
hand-written HIP kernels for gfx950 in ``libgdn.so`` (C ABI in
``include/gdn.h``). Importable as ``mlx_lean_moe_amd``.
"""

from .config import QWEN3_5_LINEAR, LinearAttentionDims
from .gated_delta import (beta_gate, forget_gate, gated_delta_scan, gated_delta_step,
                          gated_delta_update)
from .linear_attention import (DecodeGraph, PrefillGraph, Qwen3_5LinearAttention, conv_frontend,
                               fused_decode_step, fused_prefill_ok, gated_rms_norm, prefill_fused)
from .quant import LinearWeights, QuantScheme, dequantize, quantized_linear
from .recurrent_cache import RecurrentCache, RecurrentStatePool

__all__ = [
    "DecodeGraph",
    "PrefillGraph",
    "LinearAttentionDims",
    "LinearWeights",
    "QuantScheme",
    "QWEN3_5_LINEAR",
    "Qwen3_5LinearAttention",
    "RecurrentCache",
    "RecurrentStatePool",
    "beta_gate",
    "conv_frontend",
    "dequantize",
    "forget_gate",
    "fused_decode_step",
    "fused_prefill_ok",
    "gated_delta_scan",
    "gated_delta_step",
    "gated_delta_update",
    "gated_rms_norm",
    "prefill_fused",
    "quantized_linear",
]
