"""qwen3_5's gated-delta linear-attention layer on MI355X.

Mirrors ``Qwen3_5LinearAttention`` and ``_gated_rms_norm``
(``src/mlx_lean_moe/model/qwen3_5/linear_attention.py:22-127``): four input
projections, the causal depthwise conv with SiLU and conv-state roll, q/k
scaling, the gates, the gated-delta recurrence, the gated RMSNorm and
out_proj. Projections go through :func:`quant.quantized_linear`
(moe_block.py:27-55): affine-quantized weights (the reference's
``other_quant``, e.g. 4-bit groups of 64) on this library's quantized matmul
kernel — the four input projections stacked into one launch when they share a
scheme — and dense weights as ``x @ W.T`` on the vendor BLAS; everything
between them runs in this library's kernels:

* one decode token (1-D ``x``) with Dk = Dv = 128 and K = 4: the fused decode
  kernel (front-end, recurrence and gated norm in one launch);
* otherwise: the front-end kernel, then :func:`gated_delta_update` (chunked
  prefill or sequential scan), then the gated-norm kernel.

:meth:`Qwen3_5LinearAttention.decode_batch` decodes ``B`` sequences at once
from a :class:`RecurrentStatePool`.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .config import LinearAttentionDims
from .gated_delta import (PREFILL_MIN_TOKENS, _c, _check_cu_seqlens, _check_out, _require_device,
                          _stream, gated_delta_update)
from .quant import (LinearWeights, QuantScheme, concat_quantized, quantized_linear,
                    quantized_linear_split)
from .recurrent_cache import RecurrentCache, RecurrentStatePool


def gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float,
                   out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``silu(gate) * rms_norm(x, weight)``, the product in float32, the result
    in ``out_dtype`` (x's dtype by default) (linear_attention.py:22-32).
    Passing ``out_dtype=z.dtype`` folds in the call site's ``y.astype(z.dtype)``."""

    if gate.shape != x.shape or weight.shape != x.shape[-1:]:
        raise ValueError("gate must match x and weight its last axis")
    device = _require_device(x, gate, weight)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    x = _c(x)
    w = _c(weight.float())
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    # the gate may be a (T, H, D) column view of a stacked projection output,
    # read in place: row r at (r / H) * stride(0) + (r % H) * D
    if (gate.dim() == 3 and gate.stride(2) == 1 and gate.stride(1) == D
            and gate.stride(0) >= gate.shape[1] * D and not gate.is_contiguous()):
        heads, z_stride = gate.shape[1], gate.stride(0)
    else:
        gate = _c(gate)
        heads, z_stride = 1, D
    out = torch.empty(x.shape, dtype=out_dtype, device=device)
    _lib.call("gdn_gated_rmsnorm", _lib.ptr(x), _lib.dtype_code(x.dtype), _lib.ptr(gate),
              _lib.dtype_code(gate.dtype), z_stride, heads, _lib.ptr(w), float(eps), _lib.ptr(out),
              _lib.dtype_code(out_dtype), rows, D, _stream(device))
    return out


def conv_frontend(qkv: torch.Tensor, conv_state: torch.Tensor, conv_weight: torch.Tensor,
                  dims: LinearAttentionDims, cu_seqlens: torch.Tensor | None = None,
                  conv_out: torch.Tensor | None = None):
    """Conv + SiLU + roll and q/k scaling for N packed runs
    (linear_attention.py:61-79,103-113).

    ``qkv (T, C)`` in the activation dtype; ``conv_state (N, K-1, C)`` (any
    float dtype); ``conv_weight (C, K)``; ``cu_seqlens`` the N+1 int32
    offsets of the runs (a host sequence, or a device tensor, which is read
    back to the host once for the check below), or None for N equal runs.
    The offsets are checked before anything is launched: N+1 of them,
    from 0 to T, non-decreasing (``ValueError`` otherwise). Returns
    ``q, k (T, Hk, Dk)``, ``v (T, Hv, Dv)`` and the new conv state
    ``(N, K-1, C)`` in the activation dtype (written into ``conv_out`` if
    given: contiguous, not overlapping ``conv_state``)."""

    device = _require_device(qkv, conv_state, conv_weight)
    T, C = qkv.shape
    N = conv_state.shape[0]
    K = dims.conv_kernel_dim
    if C != dims.conv_dim or tuple(conv_state.shape[1:]) != (K - 1, C):
        raise ValueError("qkv/conv_state do not match the layer's conv_dim and kernel")
    cu_seqlens = _runs_on_device(cu_seqlens, N, T, device)
    act = qkv.dtype
    if act not in (torch.float32, torch.bfloat16):
        raise ValueError(f"activations must be float32 or bfloat16, got {act}")
    # qkv may be the first columns of a stacked projection output: read in
    # place with its row stride
    if not (qkv.stride(1) == 1 and qkv.stride(0) >= C):
        qkv = qkv.contiguous()
    conv_state = _c(conv_state)
    w = _c(conv_weight.float().reshape(C, K))
    q = torch.empty((T, dims.num_key_heads, dims.key_head_dim), dtype=act, device=device)
    k = torch.empty_like(q)
    v = torch.empty((T, dims.num_value_heads, dims.value_head_dim), dtype=act, device=device)
    if conv_out is None:
        new_conv = torch.empty((N, K - 1, C), dtype=act, device=device)
    else:
        _check_out(conv_out, (N, K - 1, C), act, device, conv_state, "conv_out")
        new_conv = conv_out
    _lib.call("gdn_frontend", _lib.ptr(qkv), qkv.stride(0), _lib.ptr(conv_state), _lib.ptr(new_conv),
              _lib.dtype_code(conv_state.dtype), _lib.ptr(w), _lib.ptr(cu_seqlens), N, T,
              _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), dims.num_key_heads, dims.num_value_heads,
              dims.key_head_dim, dims.value_head_dim, K, _lib.dtype_code(act), _stream(device))
    return q, k, v, new_conv


def fused_prefill_ok(qkv, a, b, conv_state, ssm_state, dims: LinearAttentionDims, N: int) -> bool:
    """Whether :func:`prefill_fused` takes these operands: bf16 activations,
    Dk = Dv = 128, K = 4, a bf16 or float32 conv state, a float32 ssm state,
    a and b of one dtype (bf16 or float32), and runs long enough (on
    average) for the chunked prefill, i.e. the inputs for which
    ``conv_frontend`` and ``gated_delta_update`` take the tiled front-end and
    the chunked prefill."""

    T = qkv.shape[0]
    return (qkv.dtype == torch.bfloat16 and dims.key_head_dim == 128
            and dims.value_head_dim == 128 and dims.conv_kernel_dim == 4
            and conv_state.dtype in (torch.bfloat16, torch.float32)
            and ssm_state.dtype == torch.float32 and a.dtype == b.dtype
            and a.dtype in (torch.bfloat16, torch.float32)
            and T > 0 and T / N >= PREFILL_MIN_TOKENS)


def _aligned(t: torch.Tensor) -> torch.Tensor:
    return t if t.data_ptr() % 16 == 0 else t.clone()


def prefill_fused(qkv, a, b, conv_state, ssm_state, conv_weight, A_log, dt_bias,
                  dims: LinearAttentionDims, cu_seqlens=None, *, y_dtype=None, conv_out=None,
                  state_out=None):
    """The layer's prompt path between the projections, short of the gated
    norm, in one call: the front-end of :func:`conv_frontend` computed
    inside the chunked prefill's chunk pass, then the state pass
    (linear_attention.py:103-121). The same results, to the bit, as
    ``conv_frontend`` followed by ``gated_delta_update`` on these inputs
    (:func:`fused_prefill_ok` says which).

    ``qkv (T, C)`` bf16 (a column view of a stacked projection output is
    read in place), ``a, b (T, Hv)``, ``conv_state (N, K-1, C)``,
    ``ssm_state (N, Hv, Dv, Dk)`` float32, ``cu_seqlens`` as in
    :func:`conv_frontend`. Returns ``(y (T, Hv, Dv), new_conv (N, K-1, C)
    bf16, new_ssm)``, y in ``y_dtype`` (float32 by default); the new states
    go to ``conv_out`` / ``state_out`` when given."""

    device = _require_device(qkv, a, b, conv_state, ssm_state, conv_weight, A_log, dt_bias)
    T, C = qkv.shape
    N = conv_state.shape[0]
    Hk, Hv, D, K = (dims.num_key_heads, dims.num_value_heads, dims.value_head_dim,
                    dims.conv_kernel_dim)
    if C != dims.conv_dim or tuple(conv_state.shape[1:]) != (K - 1, C):
        raise ValueError("qkv/conv_state do not match the layer's conv_dim and kernel")
    if a.shape != (T, Hv) or b.shape != a.shape or tuple(ssm_state.shape) != (N, Hv, D, D):
        raise ValueError("prefill_fused: inconsistent shapes")
    if not fused_prefill_ok(qkv, a, b, conv_state, ssm_state, dims, N):
        raise ValueError("prefill_fused needs bf16 activations, Dk = Dv = 128, K = 4, a bf16 or "
                         "float32 conv state, a float32 ssm state and runs of at least "
                         f"{PREFILL_MIN_TOKENS} tokens on average")
    cu = _runs_on_device(cu_seqlens, N, T, device)
    if not (qkv.stride(1) == 1 and qkv.stride(0) >= C and qkv.stride(0) % 8 == 0
            and qkv.data_ptr() % 16 == 0):
        qkv = qkv.contiguous()
    conv_state, ssm_in = _aligned(_c(conv_state)), _aligned(_c(ssm_state))
    w = _aligned(_c(conv_weight.float().reshape(C, K)))
    if not (a.stride() == b.stride() and a.stride(1) == 1 and a.stride(0) >= Hv):
        a, b = _c(a), _c(b)
    y = torch.empty((T, Hv, D), dtype=y_dtype or torch.float32, device=device)
    if conv_out is None:
        conv_out = torch.empty((N, K - 1, C), dtype=torch.bfloat16, device=device)
    else:
        _check_out(conv_out, (N, K - 1, C), torch.bfloat16, device, conv_state, "conv_out")
    if state_out is None:
        state_out = torch.empty_like(ssm_in)
    else:
        _check_out(state_out, (N, Hv, D, D), torch.float32, device, ssm_in, "state_out")
    nbytes = int(_lib.load().gdn_prefill_fused_workspace_size(N, T, Hk, Hv, D, D))
    if nbytes < 0:
        raise RuntimeError("gdn_prefill_fused_workspace_size: " + _lib.load().gdn_last_error().decode())
    workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    _lib.call("gdn_prefill_fused", _lib.ptr(qkv), qkv.stride(0), _lib.ptr(conv_state),
              _lib.ptr(conv_out), _lib.dtype_code(conv_state.dtype), _lib.ptr(w), K, _lib.ptr(a),
              _lib.ptr(b), _lib.dtype_code(a.dtype), a.stride(0), _lib.ptr(_c(A_log.float())),
              _lib.ptr(_c(dt_bias.float())), _lib.ptr(ssm_in), _lib.ptr(state_out), _lib.ptr(y),
              _lib.dtype_code(y.dtype), _lib.ptr(cu), N, T, Hk, Hv, D, D, _lib.ptr(workspace),
              workspace.numel(), _stream(device))
    return y, conv_out, state_out


def _runs_on_device(cu_seqlens, N: int, T: int, device) -> torch.Tensor | None:
    """Checked run offsets as an int32 device tensor (None: N equal runs,
    T a multiple of N)."""

    if cu_seqlens is None:
        if N <= 0 or T % N:
            raise ValueError(f"{T} tokens do not split into {N} equal runs; pass cu_seqlens")
        return None
    offsets = _check_cu_seqlens(cu_seqlens, T)
    if len(offsets) != N + 1:
        raise ValueError(f"cu_seqlens must hold {N + 1} offsets (one more than the "
                         f"{N} conv states), got {len(offsets)}")
    if (isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.device == device
            and cu_seqlens.dtype == torch.int32 and cu_seqlens.is_contiguous()):
        return cu_seqlens
    return torch.tensor(offsets, dtype=torch.int32).to(device)


def _fused_decode_ok(dims: LinearAttentionDims, act: torch.dtype) -> bool:
    return (dims.key_head_dim == dims.value_head_dim == 128 and dims.conv_kernel_dim == 4
            and act in (torch.float32, torch.bfloat16))


def check_slots(slots, batch: int, pool: int) -> list[int]:
    """Host-side check of decode slot indices: ``batch`` distinct integers in
    ``[0, pool)`` (two rows on one slot would race on its state)."""

    if isinstance(slots, torch.Tensor):
        if slots.ndim != 1:
            raise ValueError("slots must be one-dimensional")
        if slots.dtype not in (torch.int32, torch.int64):
            raise ValueError("slots must be integers")
        slots = slots.tolist()
    slots = [int(v) for v in slots]
    if len(slots) != batch:
        raise ValueError(f"expected {batch} slots, got {len(slots)}")
    if any(v < 0 or v >= pool for v in slots):
        raise ValueError(f"slots must lie in [0, {pool})")
    if len(set(slots)) != len(slots):
        raise ValueError("slots must be distinct")
    return slots


def check_half_bits(bits, pool: int) -> list[int]:
    """Host-side check of a pool's conv half bits: ``pool`` entries, each 0
    or 1."""

    bits = [int(v) for v in bits]
    if len(bits) != pool or any(v not in (0, 1) for v in bits):
        raise ValueError(f"conv_half must be {pool} bits (0 or 1)")
    return bits


def _rows(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """``t`` as the decode kernel reads it in place: every row packed (the
    trailing dims contiguous) and rows at any stride of at least a row's
    width, e.g. a column slice of a stacked projection output; anything else
    is copied. Returns the tensor and its row stride in elements."""

    width, packed = 1, True
    for n, st in zip(reversed(t.shape[1:]), reversed(t.stride()[1:])):
        packed &= n == 1 or st == width
        width *= n
    if t.shape[0] <= 1:
        return (t if packed else t.contiguous()), width
    if not packed or t.stride(0) < width:
        t = t.contiguous()
    return t, t.stride(0)


def _index_array(values, n: int, device, check, name: str) -> torch.Tensor:
    """A kernel index array: an int32 device tensor of ``n`` entries is used
    as given; anything else is checked on the host and copied."""

    if isinstance(values, torch.Tensor) and values.device.type == "cuda":
        if values.dtype != torch.int32 or values.shape != (n,) or not values.is_contiguous():
            raise ValueError(f"{name} on the device must be a contiguous int32 tensor of {n} entries")
        return values
    return torch.tensor(check(values), dtype=torch.int32, device=device)


def fused_decode_step(qkv, z, a, b, conv_state, ssm_state, conv_weight, A_log, dt_bias,
                      norm_weight, eps, dims: LinearAttentionDims, *, conv_out=None,
                      state_out=None, y_dtype=None, slots=None, conv_half=None,
                      conv_arrivals=None):
    """One decode token for ``B`` sequences in a single kernel launch: conv +
    SiLU + roll, q/k scaling, gates, recurrence and gated RMSNorm
    (linear_attention.py:103-124 at L = 1).

    ``qkv (B, C)``, ``z (B, Hv, Dv)`` or None, ``a, b (B, Hv)`` in the
    activation dtype; ``conv_state (B, K-1, C)`` in the activation dtype;
    ``ssm_state (B, Hv, Dv, Dk)`` float32. ``state_out`` may be ``ssm_state``
    (in-place update); ``conv_out`` must be a different buffer. With ``z`` the
    result is the gated-norm output in the activation dtype; without, the
    recurrence output ``y`` in ``y_dtype`` (float32 by default).

    With ``slots`` (``B`` distinct indices into a pool of ``P`` sequences),
    ``conv_state`` is the pool's ``(P, K-1, C)`` and ``ssm_state`` its
    ``(P, Hv, Dv, Dk)``: row ``b`` reads its conv state at ``slots[b]`` and
    updates the state tiles of ``slots[b]`` in place (``state_out`` must be
    ``ssm_state`` or None); ``conv_out`` is ``(B, K-1, C)`` with the rolled
    rows in batch order, for the caller to put back at the slots. With
    ``conv_half`` as well (the pool's ``P`` bits, 0 or 1), ``conv_state`` is
    the pool's two-half ``(2 P, K-1, C)`` array: slot ``s`` reads its conv
    state at row ``s + P * conv_half[s]`` and rolls it into the other half,
    so nothing is left to copy back (``conv_out`` must be ``conv_state`` or
    None). The bits are read, not flipped (:meth:`RecurrentStatePool.advance`
    flips them after the step), unless ``conv_arrivals`` is given as well
    (power-of-two ``Hv``): the pool's ``P`` int32 counters, to which the
    kernel adds 2^16 per decoded slot, flipping its half (the bit XOR bit 16
    of the counter). ``slots`` and ``conv_half`` given as host
    sequences are checked on the host; given as int32 device tensors they
    are used as they are (no host round trip), and the caller guarantees the
    slots are distinct — the kernel itself still refuses slots outside the
    pool. ``qkv``, ``z``, ``a`` and ``b`` may be row-strided views (column
    slices of one stacked projection output); they are read in place.
    Returns ``(out (B, Hv, Dv), conv_out, state_out)``."""

    device = _require_device(qkv, z, a, b, conv_state, ssm_state)
    B = qkv.shape[0]
    act = qkv.dtype
    if not _fused_decode_ok(dims, act):
        raise ValueError("the fused decode kernel needs Dk = Dv = 128, K = 4 and float32 or "
                         "bfloat16 activations")
    P = B
    slot_t = half_t = None
    if slots is not None:
        P = ssm_state.shape[0]
        slot_t = _index_array(slots, B, device, lambda v: check_slots(v, B, P), "slots")
        if state_out is not None and state_out is not ssm_state:
            raise ValueError("with slots the state is updated in place (state_out=ssm_state)")
        state_out = ssm_state
    conv_rows = P
    if conv_half is not None:
        if slots is None:
            raise ValueError("conv_half needs slots")
        if conv_out is not None and conv_out is not conv_state:
            raise ValueError("with conv_half the conv state rolls within conv_state "
                             "(conv_out=conv_state or None)")
        if not conv_state.is_contiguous():
            raise ValueError("with conv_half, conv_state must be contiguous")
        half_t = _index_array(conv_half, P, device, lambda v: check_half_bits(v, P), "conv_half")
        conv_rows = 2 * P
        conv_out = conv_state
    if conv_arrivals is not None:
        Hv = dims.num_value_heads
        if Hv & (Hv - 1):
            raise ValueError(f"conv_arrivals needs a power-of-two number of value heads (got {Hv})")
        if half_t is None or half_t is not conv_half:
            raise ValueError("conv_arrivals needs conv_half as an int32 device tensor")
        if (not isinstance(conv_arrivals, torch.Tensor) or conv_arrivals.device != device
                or conv_arrivals.dtype != torch.int32 or conv_arrivals.shape != (P,)
                or not conv_arrivals.is_contiguous()):
            raise ValueError(f"conv_arrivals must be a contiguous int32 device tensor of {P} counters")
    if (tuple(qkv.shape) != (B, dims.conv_dim) or tuple(a.shape) != (B, dims.num_value_heads)
            or b.shape != a.shape
            or tuple(conv_state.shape) != (conv_rows, dims.conv_kernel_dim - 1, dims.conv_dim)
            or tuple(ssm_state.shape) != (P, dims.num_value_heads, dims.value_head_dim,
                                           dims.key_head_dim)
            or (z is not None and tuple(z.shape) != (B, dims.num_value_heads, dims.value_head_dim))):
        raise ValueError("fused_decode_step: inconsistent shapes")
    if conv_state.dtype != act or a.dtype != act or b.dtype != act or (z is not None and z.dtype != act):
        raise ValueError("qkv, z, a, b and conv_state must share the activation dtype")
    if ssm_state.dtype != torch.float32 or not ssm_state.is_contiguous():
        raise ValueError("ssm state must be contiguous float32")
    (qkv, s_qkv), (a, s_a), (b, s_b) = _rows(qkv), _rows(a), _rows(b)
    z, s_z = _rows(z) if z is not None else (None, dims.value_dim)
    conv_state = _c(conv_state)
    strides = (s_qkv, s_z, s_a, s_b)
    dense = (dims.conv_dim, dims.value_dim, dims.num_value_heads, dims.num_value_heads)
    row_strides = None if strides == dense else (ctypes.c_int64 * 4)(*strides)
    conv_weight = _c(conv_weight.float().reshape(dims.conv_dim, dims.conv_kernel_dim))
    A_log, dt_bias = _c(A_log.float()), _c(dt_bias.float())
    norm_weight = _c(norm_weight.float()) if z is not None else None
    if conv_out is None:
        conv_out = torch.empty((B,) + tuple(conv_state.shape[1:]), dtype=act, device=device)
    elif half_t is None and (tuple(conv_out.shape) != (B, dims.conv_kernel_dim - 1, dims.conv_dim)
                             or conv_out.dtype != act or not conv_out.is_contiguous()):
        raise ValueError("conv_out must be contiguous (B, K-1, C) in the activation dtype")
    if state_out is None:
        state_out = torch.empty_like(ssm_state)
    out_dtype = act if z is not None else (y_dtype or torch.float32)
    out = torch.empty((B, dims.num_value_heads, dims.value_head_dim), dtype=out_dtype,
                      device=device)
    _lib.call("gdn_decode_step", _lib.ptr(qkv), _lib.ptr(conv_state), _lib.ptr(conv_out),
              _lib.ptr(conv_weight), _lib.ptr(a), _lib.ptr(b), _lib.ptr(A_log),
              _lib.ptr(dt_bias), _lib.ptr(ssm_state), _lib.ptr(state_out), _lib.ptr(z),
              _lib.ptr(norm_weight), float(eps), _lib.ptr(out), _lib.dtype_code(out_dtype), B,
              dims.num_key_heads, dims.num_value_heads, dims.key_head_dim, dims.value_head_dim,
              dims.conv_kernel_dim, _lib.dtype_code(act), _lib.ptr(slot_t), P, _lib.ptr(half_t),
              row_strides, _lib.ptr(conv_arrivals), _stream(device))
    return out, conv_out, state_out


class Qwen3_5LinearAttention:
    """The gated-delta layer. Weights are dense ``(out, in)`` matrices for the
    projections, ``conv1d_weight (C, K, 1)``, ``A_log``, ``dt_bias``
    ``(Hv,)`` and ``norm_weight (Dv,)`` (linear_attention.py:35-59)."""

    def __init__(self, dims: LinearAttentionDims, in_proj_qkv, in_proj_z, in_proj_a, in_proj_b,
                 conv1d_weight, A_log, dt_bias, norm_weight, out_proj,
                 rms_norm_eps: float = 1e-6, quant: QuantScheme | None = None) -> None:
        """Projections are dense ``(N, K)`` tensors, quantized dicts
        ``{"weight", "scales", "biases"}`` (scheme ``quant``, the reference's
        ``config.other_quant``) or :class:`LinearWeights` carrying their own
        scheme (linear_attention.py:95-101)."""

        self.linear = dims
        self.rms_norm_eps = rms_norm_eps
        self.quant = quant
        self.in_proj_qkv = in_proj_qkv
        self.in_proj_z = in_proj_z
        self.in_proj_a = in_proj_a
        self.in_proj_b = in_proj_b
        self.out_proj = out_proj
        self._in_stacked = self._stack_inputs()
        C, K = dims.conv_dim, dims.conv_kernel_dim
        self.conv1d_weight = conv1d_weight.float().reshape(C, K).contiguous()
        self.A_log = A_log.float().contiguous()
        self.dt_bias = dt_bias.float().contiguous()
        self.norm_weight = norm_weight.float().contiguous()

    def new_cache(self, dtype: torch.dtype = torch.float32) -> RecurrentCache:
        d = self.linear
        return RecurrentCache(d.conv_kernel_dim, d.conv_dim, d.num_value_heads, d.value_head_dim,
                              d.key_head_dim, dtype=dtype, device=self.A_log.device)

    def _scheme_of(self, weights):
        if isinstance(weights, LinearWeights):
            return weights.tensors, weights.quant
        if isinstance(weights, torch.Tensor):
            return weights, None
        return weights, self.quant

    def _stack_inputs(self):
        """One quantized projection for qkv|z|a|b when all four are quantized
        with one scheme and one scales dtype (one launch instead of four)."""

        parts = [self._scheme_of(w) for w in (self.in_proj_qkv, self.in_proj_z,
                                             self.in_proj_a, self.in_proj_b)]
        schemes = {q for _, q in parts}
        if len(schemes) != 1 or None in schemes:
            return None
        tensors = [t for t, _ in parts]
        if len({t["scales"].dtype for t in tensors}) != 1:
            return None
        return LinearWeights(concat_quantized(tensors), schemes.pop())

    def keep_dense_weights(self) -> None:
        """Keep the bf16 dequantization of the quantized projections (the
        stacked input one and out_proj) next to them: prompt-sized calls then
        skip converting the weights each time (23 us of a 512-token chunk at
        hidden 2048), for 2 bytes per weight of memory. Results are
        unchanged; decode-sized calls do not use the copies."""

        if self._in_stacked is not None and self._in_stacked.dense is None:
            self._in_stacked = self._in_stacked.with_dense()
        tensors, quant = self._scheme_of(self.out_proj)
        if quant is not None and not (isinstance(self.out_proj, LinearWeights) and self.out_proj.dense is not None):
            self.out_proj = LinearWeights(tensors, quant).with_dense()

    def _proj(self, rows: torch.Tensor, weights, residual: torch.Tensor | None = None) -> torch.Tensor:
        if isinstance(weights, LinearWeights) and weights.dense is not None:
            return quantized_linear(rows, weights, residual=residual)
        tensors, quant = self._scheme_of(weights)
        if quant is None and tensors.dtype != rows.dtype:
            tensors = tensors.to(rows.dtype)
        return quantized_linear(rows, tensors, quant, residual=residual)

    def _project(self, rows: torch.Tensor):
        d = self.linear
        L = rows.shape[0]
        if self._in_stacked is not None:
            qkv, z, ab = quantized_linear_split(rows, self._in_stacked,
                                                [d.conv_dim, d.value_dim, 2 * d.num_value_heads])
            a, b = torch.split(ab, [d.num_value_heads, d.num_value_heads], dim=-1)
            # at decode sizes column slices of one output (the fused decode
            # reads them in place, every other consumer copies what it needs
            # packed); at prefill sizes qkv and z are packed
            return qkv, z.reshape(L, d.num_value_heads, d.value_head_dim), a, b
        qkv = self._proj(rows, self.in_proj_qkv)
        z = self._proj(rows, self.in_proj_z).reshape(L, d.num_value_heads, d.value_head_dim)
        a = self._proj(rows, self.in_proj_a)
        b = self._proj(rows, self.in_proj_b)
        return qkv, z, a, b

    def core(self, qkv, z, a, b, conv_state, ssm_state, cu_seqlens=None, conv_out=None,
             ssm_out=None):
        """Everything between the projections for N packed runs (one run if
        ``cu_seqlens`` is None): ``qkv (T, C)``, ``z (T, Hv, Dv)``,
        ``a, b (T, Hv)``, ``conv_state (N, K-1, C)``, ``ssm_state (N, Hv, Dv, Dk)``.
        Returns ``(out (T, Hv*Dv), new_conv, new_ssm)``, the new states in
        ``conv_out`` and ``ssm_out`` when given."""

        d = self.linear
        T = qkv.shape[0]
        # the offsets are read to the host once and checked there before
        # the first launch (each launch below checks the host list again)
        if cu_seqlens is not None:
            cu_seqlens = _check_cu_seqlens(cu_seqlens, T)
        N = conv_state.shape[0]
        if fused_prefill_ok(qkv, a, b, conv_state, ssm_state, d, N):
            # front-end inside the chunk pass: the same bits, no q/k/v round trip
            y, new_conv, new_ssm = prefill_fused(qkv, a, b, conv_state, ssm_state,
                                                 self.conv1d_weight, self.A_log, self.dt_bias, d,
                                                 cu_seqlens, y_dtype=z.dtype, conv_out=conv_out,
                                                 state_out=ssm_out)
            out = gated_rms_norm(y, z, self.norm_weight, self.rms_norm_eps, out_dtype=z.dtype)
            return out.reshape(T, d.value_dim), new_conv, new_ssm
        q, k, v, new_conv = conv_frontend(qkv, conv_state, self.conv1d_weight, d, cu_seqlens,
                                          conv_out=conv_out)
        # y straight in z's dtype: the norm's first step rounds it there
        if cu_seqlens is None:
            y, new_ssm = gated_delta_update(q[None], k[None], v[None], a[None], b[None],
                                            self.A_log, self.dt_bias, ssm_state, y_dtype=z.dtype,
                                            state_out=ssm_out)
            y = y[0]
        else:
            y, new_ssm = gated_delta_update(q, k, v, a, b, self.A_log, self.dt_bias, ssm_state,
                                            cu_seqlens=cu_seqlens, y_dtype=z.dtype,
                                            state_out=ssm_out)
        out = gated_rms_norm(y, z, self.norm_weight, self.rms_norm_eps, out_dtype=z.dtype)
        return out.reshape(T, d.value_dim), new_conv, new_ssm

    def __call__(self, x: torch.Tensor, cache: RecurrentCache,
                 residual: torch.Tensor | None = None) -> torch.Tensor:
        """``x``: ``(hidden,)`` for one decode step or ``(L, hidden)`` for a
        prompt; returns the same rank (linear_attention.py:81-127). With
        ``residual`` (x's shape and dtype) the result is ``residual +
        layer(x)``, the decoder layer's ``h = rows + attention(rms_norm(rows))``
        (transformer.py:110-112), added in out_proj's store."""

        if x.ndim not in (1, 2):
            raise ValueError(f"Qwen3_5LinearAttention expects 1-D or 2-D x, got shape {tuple(x.shape)}")
        squeeze = x.ndim == 1
        rows = x[None, :] if squeeze else x
        if residual is not None and squeeze:
            residual = residual[None, :]
        conv_state, ssm_state = cache.state()
        out, new_conv, new_ssm = self._rows_step(rows, conv_state, ssm_state, residual)
        cache.update(new_conv, new_ssm, advance=rows.shape[0])
        return out[0] if squeeze else out

    def _rows_step(self, rows, conv_state, ssm_state, residual=None, conv_out=None, ssm_out=None):
        """The layer over ``rows (L, hidden)`` of one sequence from
        ``conv_state (K-1, C)`` and ``ssm_state (Hv, Dv, Dk)``: returns
        ``(out (L, hidden), new_conv, new_ssm)``, the new states in fresh
        tensors, or in ``conv_out`` and ``ssm_out`` when given."""

        d = self.linear
        qkv, z, a, b = self._project(rows)
        act = qkv.dtype
        outs = conv_out is not None or ssm_out is not None
        if rows.shape[0] == 1 and _fused_decode_ok(d, act) and not outs:
            out, new_conv, new_ssm = self._decode_fused(qkv, z, a, b, conv_state[None].to(act),
                                                        ssm_state[None], in_place=False)
            out = out.reshape(1, d.value_dim)
        else:
            out, new_conv, new_ssm = self.core(
                qkv, z, a, b, conv_state[None], ssm_state[None],
                conv_out=None if conv_out is None else conv_out[None],
                ssm_out=None if ssm_out is None else ssm_out[None])
        return self._proj(out, self.out_proj, residual), new_conv[0], new_ssm[0]

    def _decode_fused(self, qkv, z, a, b, conv_state, ssm_state, in_place: bool,
                      conv_out: torch.Tensor | None = None):
        return fused_decode_step(qkv, z, a, b, conv_state, ssm_state, self.conv1d_weight,
                                 self.A_log, self.dt_bias, self.norm_weight, self.rms_norm_eps,
                                 self.linear, conv_out=conv_out,
                                 state_out=ssm_state if in_place else None)

    def decode_batch(self, x: torch.Tensor, pool: RecurrentStatePool, slots=None,
                     residual: torch.Tensor | None = None) -> torch.Tensor:
        """One decode token for each of the pool's sequences: ``x (pool.batch,
        hidden)`` -> ``(pool.batch, hidden)``; or, with ``slots`` (distinct
        pool indices, e.g. the sequences a scheduler has active this step),
        ``x (len(slots), hidden)`` for those slots only. One kernel launch
        updates the slots' ssm tiles in place and rolls their conv state into
        the other half of the pool's conv buffer. ``residual`` as in
        ``__call__``."""

        d = self.linear
        rows = pool.batch if slots is None else len(slots)
        if x.ndim != 2 or x.shape[0] != rows:
            raise ValueError("decode_batch expects x of shape (pool.batch, hidden), or "
                             "(len(slots), hidden) with slots")
        qkv, z, a, b = self._project(x)
        if not _fused_decode_ok(d, qkv.dtype) or pool.conv_buf.dtype != qkv.dtype:
            raise ValueError("decode_batch needs Dk = Dv = 128, K = 4 and a pool in the "
                             "activation dtype (float32 or bfloat16)")
        slot_list = list(range(rows)) if slots is None else check_slots(slots, rows, pool.batch)
        slot_t = pool.device_slots(slot_list)
        # the kernel flips the slots' halves itself where Hv is a power of two
        counted = d.num_value_heads & (d.num_value_heads - 1) == 0
        out, _, _ = fused_decode_step(
            qkv, z, a, b, pool.conv_buf, pool.ssm_state, self.conv1d_weight, self.A_log,
            self.dt_bias, self.norm_weight, self.rms_norm_eps, d, slots=slot_t,
            conv_half=pool.conv_half_dev, conv_arrivals=pool.conv_arrivals if counted else None)
        pool.advance(slot_list, slot_t, device_flipped=counted)
        return self._proj(out.reshape(rows, d.value_dim), self.out_proj, residual)


class DecodeGraph:
    """One ``decode_batch`` step of ``layer`` for a fixed set of pool slots,
    captured in a HIP graph: a replay launches the step's kernels (the
    stacked projection, the fused decode, which also flips the pool's conv
    half bits, and out_proj) without the host work of issuing them one by
    one.

    The graph reads ``self.x`` and writes ``self.out``; ``step(x)`` copies
    ``x`` into ``self.x`` (skip it by writing ``self.x`` directly), replays
    and keeps the pool's host-side bits and sizes in step with the device.
    With ``residual_example`` the step adds a residual as ``decode_batch``
    does, read from ``self.residual`` (``step(x, residual)`` copies it in).
    Shapes, slots and every buffer are fixed at capture; the pool's contents
    may change between steps (e.g. ``pool.load``)."""

    def __init__(self, layer: "Qwen3_5LinearAttention", pool: RecurrentStatePool, slots,
                 x_example: torch.Tensor, residual_example: torch.Tensor | None = None) -> None:
        self.layer, self.pool = layer, pool
        self.slots = check_slots(slots, len(slots), pool.batch)
        if x_example.ndim != 2 or x_example.shape[0] != len(self.slots):
            raise ValueError("x_example must be (len(slots), hidden)")
        self.x = x_example.detach().clone()
        self.residual = None if residual_example is None else residual_example.detach().clone()
        self._idx = np.asarray(self.slots, dtype=np.int64)
        # One eager step first, on a throwaway pool of the same shapes, so
        # that everything the step creates lazily (the vendor BLAS handle and
        # its kernels, torch's workspaces, the first launch of each kernel)
        # exists before capture: library set-up under stream capture is not
        # allowed, and the process can end inside it without a Python error.
        # The real pool is not touched.
        n = len(self.slots)
        warm = RecurrentStatePool(n, pool.conv_buf.shape[1] + 1, pool.conv_buf.shape[2],
                                  pool.ssm_state.shape[1], pool.ssm_state.shape[2],
                                  pool.ssm_state.shape[3], dtype=pool.conv_buf.dtype,
                                  device=self.x.device)
        layer.decode_batch(self.x, warm, slots=list(range(n)), residual=self.residual)
        torch.cuda.synchronize(self.x.device)
        del warm
        # the slot array must exist before capture (no host copy in the
        # graph), and the graph holds it: the pool's cache of slot arrays may
        # drop it later, and a replay must not read freed (reused) memory
        side = torch.cuda.Stream(self.x.device)
        side.wait_stream(torch.cuda.current_stream(self.x.device))
        with torch.cuda.stream(side):
            self._slot_t = pool.device_slots(self.slots)
        torch.cuda.current_stream(self.x.device).wait_stream(side)
        torch.cuda.synchronize(self.x.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = layer.decode_batch(self.x, pool, slots=self.slots, residual=self.residual)
        # capture ran decode_batch's host bookkeeping once and none of its
        # device work: undo the former
        pool.flip_host(self._idx, tokens=-1)

    def step(self, x: torch.Tensor | None = None, residual: torch.Tensor | None = None) -> torch.Tensor:
        if x is not None and x is not self.x:
            self.x.copy_(x)
        if residual is not None:
            if self.residual is None:
                raise ValueError("this step was captured without a residual")
            if residual is not self.residual:
                self.residual.copy_(residual)
        self.graph.replay()
        self.pool.flip_host(self._idx)
        return self.out



class PrefillGraph:
    """One ``layer(x, cache)`` call over a fixed-length chunk of a prompt,
    captured in a HIP graph: a serving loop that prefills prompts in chunks
    of ``len(x_example)`` tokens replays the chunk's kernels (projections,
    front-end, chunked prefill, gated norm, out_proj) without issuing them
    one by one from Python, which at a few hundred tokens per chunk takes
    longer than the kernels themselves.

    The graph reads ``self.x`` (and ``self.residual`` when captured with
    ``residual_example``) and writes ``self.out``. The sequence's state lives
    in two buffer sets the chunks alternate between (the kernels read one
    and write the other; two graphs over one memory pool). ``step(cache,
    x)`` copies ``x`` in, copies the cache's state into the first set unless
    the cache already holds one of the sets, replays, and points the cache
    at the set just written (``cache.update``): consecutive chunks of one
    sequence run without copies, and the cache's state tensors are then
    overwritten two steps later on this graph: clone them to keep a
    snapshot, and before another sequence's step on the same graph. The
    returned output holds until the next step. Writing the chunk straight
    into ``self.x`` (and calling ``step(cache)``) skips its copy. Shapes and
    buffers are fixed at capture; a prompt's last, shorter chunk runs through
    ``layer`` as usual."""

    def __init__(self, layer: "Qwen3_5LinearAttention", x_example: torch.Tensor,
                 residual_example: torch.Tensor | None = None) -> None:
        if x_example.ndim != 2 or x_example.shape[0] < 2:
            raise ValueError("x_example must be (chunk, hidden) with at least two tokens")
        d = layer.linear
        dev = x_example.device
        self.layer = layer
        self.chunk = x_example.shape[0]
        self.x = x_example.detach().clone()
        self.residual = None if residual_example is None else residual_example.detach().clone()
        self._conv = [torch.zeros((d.conv_kernel_dim - 1, d.conv_dim), dtype=self.x.dtype, device=dev)
                      for _ in range(2)]
        self._ssm = [torch.zeros((d.num_value_heads, d.value_head_dim, d.key_head_dim),
                                 dtype=torch.float32, device=dev) for _ in range(2)]
        # one eager call first: lazily built operands (workspace sizes, BLAS
        # handles) exist before capture
        layer._rows_step(self.x, self._conv[0], self._ssm[0], self.residual)
        torch.cuda.synchronize(dev)
        self._graphs, self._outs = [], []
        for i in (0, 1):
            graph = torch.cuda.CUDAGraph()
            pool = self._graphs[0].pool() if self._graphs else None
            with torch.cuda.graph(graph, pool=pool):
                out, _, _ = layer._rows_step(self.x, self._conv[i], self._ssm[i], self.residual,
                                             conv_out=self._conv[1 - i], ssm_out=self._ssm[1 - i])
            self._graphs.append(graph)
            self._outs.append(out)
        self.out = self._outs[0]

    def step(self, cache: RecurrentCache, x: torch.Tensor | None = None,
             residual: torch.Tensor | None = None) -> torch.Tensor:
        if x is not None and x is not self.x:
            if tuple(x.shape) != tuple(self.x.shape):
                raise ValueError(f"x must be {tuple(self.x.shape)}, got {tuple(x.shape)}")
            self.x.copy_(x)
        if residual is not None:
            if self.residual is None:
                raise ValueError("this chunk was captured without a residual")
            if residual is not self.residual:
                self.residual.copy_(residual)
        conv, ssm = cache.state()
        held = [i for i in (0, 1) if conv is self._conv[i] and ssm is self._ssm[i]]
        i = held[0] if held else 0
        if not held:
            self._conv[0].copy_(conv)
            self._ssm[0].copy_(ssm)
        self._graphs[i].replay()
        cache.update(self._conv[1 - i], self._ssm[1 - i], advance=self.chunk)
        self.out = self._outs[i]
        return self.out
