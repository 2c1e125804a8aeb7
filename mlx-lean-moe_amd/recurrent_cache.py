"""Fixed-size state of a gated-delta layer.

:class:`RecurrentCache` mirrors the reference's per-layer, single-sequence
cache (``src/mlx_lean_moe/cache/recurrent_cache.py:11-41``): the last
``K - 1`` conv inputs and a float32 ``(Hv, Dv, Dk)`` state, replaced
functionally by ``update``. :class:`RecurrentStatePool` is the batched device
form a serving loop decodes from: ``B`` slots of both pieces, updated in place
by the fused decode kernel.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib


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

    def device_halves(self) -> torch.Tensor:
        """The slots' current halves as the decode kernel reads them: the
        device bit, XOR bit 16 of the slot's counter."""
        return (self.conv_half_dev ^ (self.conv_arrivals >> 16)) & 1

    def update(self, conv_state: torch.Tensor, ssm_state: torch.Tensor, advance: int) -> None:
        self.conv_state = conv_state
        self.ssm_state = ssm_state
        self.size += advance


class RecurrentStatePool:
    """``B`` sequences' states for batched decode: ssm ``(B, Hv, Dv, Dk)``
    float32 and conv ``(K-1, C)`` per slot in the activation dtype.

    The decode kernel updates a slot's ssm tiles in place. A key head's conv
    channels are read by several workgroups, so a slot's conv state cannot
    be rolled in place: ``conv_buf`` holds two ``(B, K-1, C)`` halves and
    slot ``s`` currently lives in row ``s + B * conv_half[s]``; a decode reads
    that row and writes the rolled state into the slot's other half, then
    the slot's half flips (no copy, and slots decode independently). The
    bits live on the device (``conv_half_dev``, read by the decode kernel, or
    flipped by ``advance``) with a host copy (``conv_half``) for host-side
    reads. A decode step given the ``conv_arrivals`` counters flips a slot's
    half itself: it adds 2^16 to the slot's counter, and the device half is
    the bit XOR bit 16 of the counter (:meth:`device_halves`); a pool's steps
    then pass the counters every time."""

    def __init__(self, batch: int, conv_kernel_dim: int, conv_dim: int, num_value_heads: int,
                 value_head_dim: int, key_head_dim: int, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cuda") -> None:
        self.conv_buf = torch.zeros((2 * batch, conv_kernel_dim - 1, conv_dim), dtype=dtype,
                                    device=device)
        self.conv_half = torch.zeros(batch, dtype=torch.int64)
        self.conv_half_dev = torch.zeros(batch, dtype=torch.int32, device=device)
        self.conv_arrivals = torch.zeros(batch, dtype=torch.int32, device=device)
        self._slot_sets: dict[tuple[int, ...], torch.Tensor] = {}
        self.ssm_state = torch.zeros((batch, num_value_heads, value_head_dim, key_head_dim),
                                     dtype=torch.float32, device=device)
        self.size = torch.zeros(batch, dtype=torch.int64)
        # NumPy views of the two host arrays: a decode step's bookkeeping
        # costs ~1 us through them (a torch CPU index op costs several)
        self._half_np, self._size_np = self.conv_half.numpy(), self.size.numpy()
        self._counted = False  # a step has flipped halves through conv_arrivals

    @property
    def batch(self) -> int:
        return self.ssm_state.shape[0]

    def _current_rows(self) -> torch.Tensor:
        return torch.arange(self.batch) + self.batch * self.conv_half

    @property
    def conv_state(self) -> torch.Tensor:
        """Every slot's current conv state ``(B, K-1, C)`` (a gathered copy)."""
        return self.conv_buf[self._current_rows().to(self.conv_buf.device)]

    def state(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self.conv_state, self.ssm_state

    def device_halves(self) -> torch.Tensor:
        """The slots' current halves as the decode kernel reads them: the
        device bit, XOR bit 16 of the slot's counter."""
        return (self.conv_half_dev ^ (self.conv_arrivals >> 16)) & 1

    def device_slots(self, slots: list[int]) -> torch.Tensor:
        """``slots`` as an int32 device array, kept per active set (a serving
        loop decodes the same set for many steps), copied without blocking."""
        key = tuple(slots)
        t = self._slot_sets.get(key)
        if t is None:
            if len(self._slot_sets) >= 64:
                self._slot_sets.clear()
            host = torch.tensor(key, dtype=torch.int32).pin_memory()
            t = self._slot_sets[key] = host.to(self.ssm_state.device, non_blocking=True)
        return t

    def advance(self, slots: list[int], slot_t: torch.Tensor | None = None, *,
                device_flipped: bool = False) -> None:
        """After a decode of ``slots`` (distinct; ``slot_t`` the same as an
        int32 device array, if the caller has it): their conv state now lives
        in the other half, and each holds one more token. ``device_flipped``:
        the decode kernel has flipped the halves already (it was given
        ``conv_arrivals``); only the host copy and sizes change. Once a step
        has, the bits alone no longer give a slot's half, so flipping them
        here instead is refused."""
        if device_flipped:
            self._counted = True
        elif self._counted:
            raise ValueError("this pool's decode steps flip the halves through conv_arrivals; "
                             "pass them on every step (advance(..., device_flipped=True))")
        self.flip_host(np.asarray(slots, dtype=np.int64))
        if device_flipped:
            return
        if slot_t is None:
            slot_t = self.device_slots(slots)
        device = self.conv_half_dev.device
        _lib.call("gdn_pool_advance", _lib.ptr(slot_t), len(slots), _lib.ptr(self.conv_half_dev),
                  self.batch, _lib.stream_ptr(device))

    def flip_host(self, idx: np.ndarray, tokens: int = 1) -> None:
        """Host bookkeeping of a decode of the distinct slots ``idx``: flip
        their half bits and add ``tokens`` (-1 undoes a step) to their sizes."""
        self._half_np[idx] ^= 1
        self._size_np[idx] += tokens

    def load(self, slot: int, cache: RecurrentCache) -> None:
        """Copy one sequence's state (e.g. after its prefill) into ``slot``."""
        conv, ssm = cache.state()
        self.conv_buf[slot + self.batch * int(self.conv_half[slot])].copy_(conv)
        self.ssm_state[slot].copy_(ssm)
        self.size[slot] = cache.size
