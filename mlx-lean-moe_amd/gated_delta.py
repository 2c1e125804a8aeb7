"""The gated-delta recurrence on MI355X: the reference's Python surface
(``src/mlx_lean_moe/model/qwen3_5/gated_delta.py``) over hand-written HIP
kernels.

Same names, arguments, shape checks (``ValueError`` before any launch) and
result dtypes as the reference:

* :func:`forget_gate`       -- ``gated_delta.py:14-21``
* :func:`gated_delta_step`  -- ``gated_delta.py:24-41``
* :func:`gated_delta_scan`  -- ``gated_delta.py:44-90``; ``use_kernel=False``
  selects the plain one-thread-per-row GPU kernel, as the reference's flag
  selects its op-by-op path.

plus the batch-first / packed-varlen update with the gates fused,
:func:`gated_delta_update` (the upstream signature the reference's tests call,
``tests/test_qwen3_5_gated_delta.py:59-69``).

Every call runs on the GPU that holds its tensors; CPU tensors are rejected
(the reference would run its ops path on the CPU device; this library has no
CPU path).
"""

from __future__ import annotations

import torch

from . import _lib

# Token runs at least this long (bf16, Dk = Dv = 128) take the chunked MFMA
# prefill instead of the sequential scan.
PREFILL_MIN_TOKENS = 64


def _promote(*tensors: torch.Tensor) -> torch.dtype:
    dtype = tensors[0].dtype
    for t in tensors[1:]:
        dtype = torch.promote_types(dtype, t.dtype)
    return dtype


def _require_device(*tensors: torch.Tensor | None) -> torch.device:
    devices = {t.device for t in tensors if t is not None}
    if len(devices) != 1:
        raise ValueError(f"all tensors must be on one device, got {sorted(map(str, devices))}")
    (device,) = devices
    if device.type != "cuda":
        raise RuntimeError(
            f"gated-delta kernels run on ROCm devices only; got tensors on {device}")
    for t in tensors:
        if t is not None and t.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise ValueError(f"unsupported dtype {t.dtype}")
    return device


def _c(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _check_out(out: torch.Tensor, shape, dtype: torch.dtype, device, src: torch.Tensor, name: str):
    """A caller-provided output buffer: the shape and dtype the call would
    allocate, contiguous, on the call's device, and not overlapping ``src``
    (the kernels read their inputs while they write their outputs)."""

    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or not out.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {tuple(shape)} {dtype} tensor")
    if out.device != device:
        raise ValueError(f"{name} must be on {device}")
    a0, a1 = out.data_ptr(), out.data_ptr() + out.numel() * out.element_size()
    b0, b1 = src.data_ptr(), src.data_ptr() + src.numel() * src.element_size()
    if a0 < b1 and b0 < a1:
        raise ValueError(f"{name} must not overlap its input")


def _stream(device: torch.device):
    return _lib.stream_ptr(device)


# ---------------------------------------------------------------------------
# gates
# ---------------------------------------------------------------------------


def _gates(a, b, A_log, dt_bias, want_g=True, want_beta=True):
    src = a if a is not None else b
    device = _require_device(a, b, A_log if want_g else None, dt_bias if want_g else None)
    Hv = src.shape[-1]
    rows = src.numel() // Hv if Hv else 0
    a = _c(a) if a is not None else None
    b = _c(b) if b is not None else None
    A_log = _c(A_log.float()) if want_g else None
    dt_bias = _c(dt_bias.float()) if want_g else None
    g = torch.empty(src.shape, dtype=torch.float32, device=device) if want_g else None
    beta = torch.empty(b.shape, dtype=b.dtype, device=device) if want_beta else None
    _lib.call("gdn_gates", _lib.ptr(a), _lib.ptr(b), _lib.dtype_code(src.dtype),
              _lib.ptr(A_log), _lib.ptr(dt_bias), _lib.ptr(g), _lib.ptr(beta),
              _lib.dtype_code(b.dtype) if want_beta else 0, rows, Hv, _stream(device))
    return g, beta


def forget_gate(a: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor) -> torch.Tensor:
    """Per-value-head decay in (0, 1]: ``exp(-exp(A_log) * softplus(a + dt_bias))``
    in float32 (gated_delta.py:14-21). ``a``: ``(..., Hv)``."""

    if a.shape[-1:] != A_log.shape or A_log.shape != dt_bias.shape:
        raise ValueError("a must end in A_log's (value_heads,) shape, as must dt_bias")
    g, _ = _gates(a, None, A_log, dt_bias, want_g=True, want_beta=False)
    return g


def beta_gate(b: torch.Tensor) -> torch.Tensor:
    """``sigmoid(b)`` in b's dtype (linear_attention.py:116)."""

    _, beta = _gates(None, b, None, None, want_g=False, want_beta=True)
    return beta


# ---------------------------------------------------------------------------
# shape checks (gated_delta.py:57-79)
# ---------------------------------------------------------------------------


def _check_scan_shapes(q, k, v, g, beta, state):
    if q.ndim != 3 or k.shape != q.shape or v.ndim != 3:
        raise ValueError("q/k must have matching (L, key_heads, key_dim) shapes; v must be 3-D")
    length, key_heads, key_dim = q.shape
    _, value_heads, value_dim = v.shape
    if min(length, key_heads, key_dim, value_heads, value_dim) <= 0:
        raise ValueError("gated_delta_scan requires nonempty sequence and head dimensions")
    if v.shape[0] != length or value_heads % key_heads:
        raise ValueError("v must match q's sequence length and have a multiple of its head count")
    if tuple(g.shape) != (length, value_heads) or beta.shape != g.shape:
        raise ValueError("g and beta must have shape (L, value_heads)")
    if tuple(state.shape) != (value_heads, value_dim, key_dim):
        raise ValueError("state must have shape (value_heads, value_dim, key_dim)")


# ---------------------------------------------------------------------------
# launches (shapes already checked, tensors contiguous on one device)
# ---------------------------------------------------------------------------


def _launch_scan(name, q, k, v, g, beta, state_in, state_out, y, cu, N, T, Hk, Hv, Dk, Dv,
                 device):
    _lib.call(name, _lib.ptr(q), _lib.ptr(k), _lib.dtype_code(q.dtype), _lib.ptr(v), _lib.dtype_code(v.dtype),
              _lib.ptr(g), _lib.dtype_code(g.dtype), _lib.ptr(beta), _lib.dtype_code(beta.dtype),
              _lib.ptr(state_in), _lib.ptr(state_out), _lib.dtype_code(state_in.dtype),
              _lib.ptr(y), _lib.dtype_code(y.dtype), _lib.ptr(cu), N, T, Hk, Hv, Dk, Dv,
              _stream(device))


def prefill_workspace_bytes(N: int, T: int, Hk: int, Hv: int, Dk: int, Dv: int) -> int:
    return int(_lib.load().gdn_prefill_workspace_size(N, T, Hk, Hv, Dk, Dv))


def _launch_prefill(q, k, v, ga, gb, A_log, dt_bias, gate_mode, state_in, state_out, y, cu, N, T,
                    Hk, Hv, Dk, Dv, device, workspace=None, gate_stride=None):
    nbytes = prefill_workspace_bytes(N, T, Hk, Hv, Dk, Dv)
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    _lib.call("gdn_prefill_chunked", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.dtype_code(q.dtype), _lib.ptr(ga),
              _lib.ptr(gb), _lib.dtype_code(gb.dtype), Hv if gate_stride is None else gate_stride,
              _lib.ptr(A_log), _lib.ptr(dt_bias),
              gate_mode, _lib.ptr(state_in), _lib.ptr(state_out), _lib.ptr(y),
              _lib.dtype_code(y.dtype), _lib.ptr(cu), N, T, Hk, Hv, Dk, Dv,
              _lib.ptr(workspace), workspace.numel(), _stream(device))


def _prefill_eligible(q, k, v, tokens_per_run: float) -> bool:
    """The chunked prefill's shapes, dtypes and operand alignment: q, k, v
    all bfloat16 (q, k 16-byte aligned, v 8) or all float32 (each 16-byte
    aligned); a contiguous view may start anywhere in its storage."""

    if q.dtype == k.dtype == v.dtype == torch.bfloat16:
        v_align = 8
    elif q.dtype == k.dtype == v.dtype == torch.float32:
        v_align = 16
    else:
        return False
    return (q.shape[-1] == 128 and v.shape[-1] == 128
            and tokens_per_run >= PREFILL_MIN_TOKENS
            and q.data_ptr() % 16 == 0 and k.data_ptr() % 16 == 0 and v.data_ptr() % v_align == 0)


# ---------------------------------------------------------------------------
# public surface
# ---------------------------------------------------------------------------


def gated_delta_scan(q, k, v, g, beta, state, *, use_kernel: bool = True):
    """Runs the gated-delta step over ``L`` positions in order
    (gated_delta.py:44-90). ``q, k``: ``(L, Hk, Dk)``; ``v``: ``(L, Hv, Dv)``;
    ``g, beta``: ``(L, Hv)``; ``state``: ``(Hv, Dv, Dk)``. Returns
    ``(y (L, Hv, Dv), new_state)`` in the dtypes the reference's ops promote
    to. The input state is never modified.

    ``use_kernel=True`` picks the register-resident scan (``Dk`` in
    {32, 64, 128, 256}) or, for bf16 q/k/v with ``Dk = Dv = 128`` and at
    least ``PREFILL_MIN_TOKENS`` tokens, the chunked MFMA prefill;
    ``use_kernel=False`` (or any other ``Dk``) runs the plain per-row kernel."""

    _check_scan_shapes(q, k, v, g, beta, state)
    device = _require_device(q, k, v, g, beta, state)
    L, Hk, Dk = q.shape
    Hv, Dv = v.shape[1:]
    y_dtype = _promote(q, k, v, g, beta, state)
    s_dtype = _promote(k, v, g, beta, state)
    qk_dtype = _promote(q, k)  # one dtype for both; the widening is exact
    q, k = q.to(qk_dtype), k.to(qk_dtype)
    q, k, v, g, beta = map(_c, (q, k, v, g, beta))
    state_in = _c(state.to(s_dtype))
    y = torch.empty((L, Hv, Dv), dtype=y_dtype, device=device)
    state_out = torch.empty((Hv, Dv, Dk), dtype=s_dtype, device=device)
    if (use_kernel and s_dtype == torch.float32 and g.dtype == torch.float32
            and _prefill_eligible(q, k, v, L)):
        _launch_prefill(q, k, v, g, beta, None, None, 1, state_in, state_out, y, None, 1, L, Hk,
                        Hv, Dk, Dv, device)
    else:
        name = "gdn_scan" if use_kernel and Dk in (32, 64, 128, 256) else "gdn_scan_reference"
        _launch_scan(name, q, k, v, g, beta, state_in, state_out, y, None, 1, L, Hk, Hv, Dk, Dv,
                     device)
    return y, state_out


def gated_delta_step(q, k, v, g, beta, state):
    """One recurrent step (gated_delta.py:24-41). ``q``/``k`` are
    ``(Hv, Dk)``, already repeated out to the value heads; ``v`` ``(Hv, Dv)``;
    ``g, beta`` ``(Hv,)``; ``state`` ``(Hv, Dv, Dk)``."""

    if q.ndim != 2 or k.shape != q.shape or v.ndim != 2 or v.shape[0] != q.shape[0]:
        raise ValueError("q/k must be (value_heads, key_dim) and v (value_heads, value_dim)")
    y, new_state = gated_delta_scan(q[None], k[None], v[None], g[None], beta[None], state)
    return y[0], new_state


def _check_cu_seqlens(cu_seqlens, T: int) -> list[int]:
    offsets = torch.as_tensor(cu_seqlens).to("cpu", torch.int64)
    if offsets.ndim != 1 or offsets.numel() < 2:
        raise ValueError("cu_seqlens must be 1-D with at least two offsets")
    offsets = offsets.tolist()
    if offsets[0] != 0 or offsets[-1] != T:
        raise ValueError(f"cu_seqlens must run from 0 to the token count {T}")
    if any(b < a for a, b in zip(offsets, offsets[1:])):
        raise ValueError("cu_seqlens must be non-decreasing")
    if T >= 2 ** 31:
        raise ValueError("packed token count must fit int32")
    return offsets


def gated_delta_update(q, k, v, a, b, A_log, dt_bias, state=None, *, cu_seqlens=None,
                       use_kernel: bool = True, y_dtype: torch.dtype | None = None,
                       state_out: torch.Tensor | None = None):
    """Gated-delta update with the gates computed from ``a, b`` inside
    (beta = sigmoid(b), g = forget_gate(a, A_log, dt_bias)).

    Batch-first: ``q, k (B, L, Hk, Dk)``, ``v (B, L, Hv, Dv)``,
    ``a, b (B, L, Hv)``, ``state (B, Hv, Dv, Dk)`` or None (zeros, float32).
    Packed: with ``cu_seqlens`` (N+1 offsets) ``q, k (T, Hk, Dk)``,
    ``v (T, Hv, Dv)``, ``a, b (T, Hv)``, ``state (N, Hv, Dv, Dk)``; each run
    starts from its own state. Returns ``(y, new_state)``.

    ``y`` comes in the promotion of the inputs' dtypes (float32 with a
    float32 state); ``y_dtype`` asks for it rounded to nearest even into that
    dtype instead, the values of ``y.to(y_dtype)`` without the float32 copy
    (the layer's output cast, linear_attention.py:122-124). ``state_out``
    receives the new state instead of a fresh tensor (its shape and dtype,
    contiguous, not overlapping ``state``) and is returned."""

    packed = cu_seqlens is not None
    lead = 1 if packed else 2
    if q.ndim != lead + 2 or k.shape != q.shape or v.ndim != lead + 2:
        raise ValueError("q/k must share a shape and v must match their rank")
    if v.shape[:lead] != q.shape[:lead] or a.shape != v.shape[:-1] or b.shape != a.shape:
        raise ValueError("v, a and b must match q's leading (token) axes")
    Hk, Dk = q.shape[-2:]
    Hv, Dv = v.shape[-2:]
    if min(Hk, Dk, Hv, Dv) <= 0 or Hv % Hk:
        raise ValueError("value heads must be a nonzero multiple of the key heads")
    if A_log.shape != (Hv,) or dt_bias.shape != (Hv,):
        raise ValueError("A_log and dt_bias must have shape (value_heads,)")
    if packed:
        T = q.shape[0]
        offsets = _check_cu_seqlens(cu_seqlens, T)
        N = len(offsets) - 1
        mean_run = T / N
    else:
        N, L = q.shape[:2]
        T = N * L
        mean_run = L
    if N == 0:
        raise ValueError("gated_delta_update needs at least one sequence")
    if state is not None and tuple(state.shape) != (N, Hv, Dv, Dk):
        raise ValueError(f"state must have shape {(N, Hv, Dv, Dk)}")
    device = _require_device(q, k, v, a, b, A_log, dt_bias, state)
    cu = (torch.tensor(offsets, dtype=torch.int32, device=device) if packed else None)
    if state is None:
        state = torch.zeros((N, Hv, Dv, Dk), dtype=torch.float32, device=device)
    if y_dtype is None:
        y_dtype = _promote(q, k, v, b, state, torch.empty(0, dtype=torch.float32))
    elif y_dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"y_dtype must be a float dtype, got {y_dtype}")
    s_dtype = _promote(k, v, b, state, torch.empty(0, dtype=torch.float32))
    qk_dtype = _promote(q, k)
    q, k = q.to(qk_dtype), k.to(qk_dtype)
    q, k, v = (_c(t.reshape((T,) + tuple(t.shape[lead:]))) for t in (q, k, v))
    a, b = a.reshape(T, Hv), b.reshape(T, Hv)
    # a and b may be column slices of one projection output: the chunked
    # prefill reads them with their row stride, every other path packs them
    rows_ok = a.stride() == b.stride() and a.stride(1) == 1 and a.stride(0) >= Hv
    state_in = _c(state.to(s_dtype))
    y = torch.empty((T, Hv, Dv), dtype=y_dtype, device=device)
    if state_out is None:
        state_out = torch.empty((N, Hv, Dv, Dk), dtype=s_dtype, device=device)
    else:
        _check_out(state_out, (N, Hv, Dv, Dk), s_dtype, device, state_in, "state_out")
    if T > 0:
        if (use_kernel and s_dtype == torch.float32 and a.dtype == b.dtype
                and a.dtype in (torch.bfloat16, torch.float32)
                and _prefill_eligible(q, k, v, mean_run)):
            if not rows_ok:
                a, b = _c(a), _c(b)
            _launch_prefill(q, k, v, a, b, _c(A_log.float()), _c(dt_bias.float()), 0, state_in,
                            state_out, y, cu, N, T, Hk, Hv, Dk, Dv, device, gate_stride=a.stride(0))
        else:
            g, beta = _gates(_c(a), _c(b), A_log, dt_bias)
            name = "gdn_scan" if use_kernel and Dk in (32, 64, 128, 256) else "gdn_scan_reference"
            _launch_scan(name, q, k, v, g, beta, state_in, state_out, y, cu, N, T, Hk, Hv, Dk, Dv,
                         device)
    else:
        state_out.copy_(state_in)
    if not packed:
        y = y.reshape(N, T // N, Hv, Dv)
    return y, state_out
