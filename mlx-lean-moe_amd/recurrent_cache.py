"""Fixed-size state of a gated-delta layer.

:class:`RecurrentCache` mirrors the reference's per-layer, single-sequence
cache (``src/mlx_lean_moe/cache/recurrent_cache.py:11-41``): the last
``K - 1`` conv inputs and a float32 ``(Hv, Dv, Dk)`` state, replaced
functionally by ``update``. :class:`RecurrentStatePool` is the batched device
form a serving loop decodes from: ``B`` slots of both pieces, updated in place
by the fused decode kernel.
"""

from __future__ import annotations

import torch


class RecurrentCache:
    """One gated-delta layer's rolling state for one sequence."""

    def __init__(self, conv_kernel_dim: int, conv_dim: int, num_value_heads: int,
                 value_head_dim: int, key_head_dim: int, dtype: torch.dtype = torch.float32,
                 device: torch.device | str = "cuda") -> None:
        if conv_kernel_dim < 1:
            raise ValueError(f"conv_kernel_dim must be positive, got {conv_kernel_dim}")
        self.conv_state = torch.zeros((conv_kernel_dim - 1, conv_dim), dtype=dtype, device=device)
        # float32 whatever the activation dtype: it accumulates over the whole sequence.
        self.ssm_state = torch.zeros((num_value_heads, value_head_dim, key_head_dim),
                                     dtype=torch.float32, device=device)
        self.size = 0

    def state(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self.conv_state, self.ssm_state

    def update(self, conv_state: torch.Tensor, ssm_state: torch.Tensor, advance: int) -> None:
        self.conv_state = conv_state
        self.ssm_state = ssm_state
        self.size += advance


class RecurrentStatePool:
    """``B`` sequences' states for batched decode: conv ``(B, K-1, C)`` in the
    activation dtype and ssm ``(B, Hv, Dv, Dk)`` float32.

    The decode kernel reads the ssm slots and writes them back in place; the
    conv state is double-buffered (``conv_state`` / ``conv_spare``) because a
    key head's conv channels are read by several workgroups."""

    def __init__(self, batch: int, conv_kernel_dim: int, conv_dim: int, num_value_heads: int,
                 value_head_dim: int, key_head_dim: int, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cuda") -> None:
        shape = (batch, conv_kernel_dim - 1, conv_dim)
        self.conv_state = torch.zeros(shape, dtype=dtype, device=device)
        self.conv_spare = torch.zeros(shape, dtype=dtype, device=device)
        self.ssm_state = torch.zeros((batch, num_value_heads, value_head_dim, key_head_dim),
                                     dtype=torch.float32, device=device)
        self.size = torch.zeros(batch, dtype=torch.int64)

    @property
    def batch(self) -> int:
        return self.ssm_state.shape[0]

    def state(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self.conv_state, self.ssm_state

    def swap_conv(self) -> None:
        """Make the freshly written spare conv buffer current."""
        self.conv_state, self.conv_spare = self.conv_spare, self.conv_state

    def load(self, slot: int, cache: RecurrentCache) -> None:
        """Copy one sequence's state (e.g. after its prefill) into ``slot``."""
        conv, ssm = cache.state()
        self.conv_state[slot].copy_(conv)
        self.ssm_state[slot].copy_(ssm)
        self.size[slot] = cache.size
