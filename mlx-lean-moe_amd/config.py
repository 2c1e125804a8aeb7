"""Shape of a gated-delta layer (the reference's ``Qwen3_5LinearAttention``
dataclass, ``src/mlx_lean_moe/model/qwen3_5/config.py:10-32``)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class LinearAttentionDims:
    """Key and value head counts differ; q/k are shared by ``num_value_heads //
    num_key_heads`` consecutive value heads."""

    num_key_heads: int
    num_value_heads: int
    key_head_dim: int
    value_head_dim: int
    conv_kernel_dim: int

    @property
    def key_dim(self) -> int:
        return self.num_key_heads * self.key_head_dim

    @property
    def value_dim(self) -> int:
        return self.num_value_heads * self.value_head_dim

    @property
    def conv_dim(self) -> int:
        """Channels of the depthwise conv: the q, k and v projections side by
        side (two key_dim blocks, then value_dim)."""
        return self.key_dim * 2 + self.value_dim


# The production shape of the path (Hk=16, Hv=32, d=128, K=4).
QWEN3_5_LINEAR = LinearAttentionDims(16, 32, 128, 128, 4)
