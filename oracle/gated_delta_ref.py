"""CPU restatement of the reference's gated-delta path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU comparator), never as a product code path.

Every function restates one piece of the reference (paths relative to the
reference root, ``src/mlx_lean_moe/`` unless they start with ``tests/``):

=============================  ==============================================
function                       reference
=============================  ==============================================
``forget_gate``                ``model/qwen3_5/gated_delta.py:14-21``
``gated_delta_step``           ``model/qwen3_5/gated_delta.py:24-41``
``gated_delta_scan``           ``model/qwen3_5/gated_delta.py:44-90`` (checks)
``gated_delta_scan_ops``       ``model/qwen3_5/gated_delta.py:93-109``
``convolve``                   ``model/qwen3_5/linear_attention.py:61-79``
``qk_scale``                   ``model/qwen3_5/linear_attention.py:109-113``
``gated_rms_norm``             ``model/qwen3_5/linear_attention.py:22-32``
``linear_attention_core``      ``model/qwen3_5/linear_attention.py:96-124``
``linear_attention``           ``model/qwen3_5/linear_attention.py:81-127``
``metal_test_inputs``          ``tests/test_gated_delta_metal.py:10-23``
``metal_test_reference``       ``tests/test_gated_delta_metal.py:26-39``
=============================  ==============================================

Arithmetic runs in ``dtype`` (float64 by default, float32 for the timed
op-for-op CPU comparator).  ``act="bf16"`` additionally rounds to bfloat16 at
the points where the reference holds bfloat16 activations (conv output, SiLU,
q/k scaling, ``sigmoid(b)``, the y cast before the gated norm, the gated-norm
output); in float64 each of these is the exact value's one rounding.  Those rounding points follow the reference's dtype flow; where they
depend on MLX's internal bf16 kernels (``mx.fast.rms_norm``, ``mx.conv1d``,
Python-scalar promotion) they are a best restatement and parity is unpinned
at the bit level, which the bf16 tolerance (2e-2 max-abs) absorbs.

Pinning (tests/test_oracle.py): closed forms (g=1/beta=0 identity, exact
overwrite at beta=1, g=0 reset), an index-loop brute force on the reference
test's small shapes, split/carry invariants, the chunked WY form agreeing with
the sequential recurrence, and torch's CPU conv1d / rms_norm / softplus /
silu / sigmoid as library cross-checks of the front-end and gated norm.
"""

from __future__ import annotations

import numpy as np

EPS_QK = 1e-6  # hard-coded q/k eps, model/qwen3_5/linear_attention.py:109-113


# --------------------------------------------------------------------------
# rounding helpers
# --------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even), once, from the value as
    given; returns float32 values. float64 input is rounded on its own bits
    (8 significant bits kept), not through float32, whose own rounding would
    otherwise decide values within a float32 ulp of a bf16 tie; below 2^-126,
    bfloat16's subnormal range, to a multiple of 2^-133."""

    x = np.asarray(x)
    if x.dtype == np.float64:
        u = np.ascontiguousarray(x).view(np.uint64)
        drop = np.uint64(45)  # 52 - 7 stored mantissa bits
        half = np.uint64((1 << 44) - 1)
        keep = np.uint64(0xFFFF_FFFF_FFFF_FFFF ^ ((1 << 45) - 1))
        u = (u + half + ((u >> drop) & np.uint64(1))) & keep
        out = u.view(np.float64)
        with np.errstate(invalid="ignore"):
            tiny = np.abs(x) < 2.0 ** -126
        if tiny.any():  # np.rint: nearest, ties to even; the scalings are exact
            out = np.where(tiny, np.rint(x * 2.0 ** 133) * 2.0 ** -133, out)
        return np.asarray(out).astype(np.float32)
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def f16_round(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float16).astype(np.float32)


def act_round(x, act: str | None, dtype=np.float64) -> np.ndarray:
    """Round ``x`` to the activation dtype ``act`` (None/"f32"/"bf16"/"f16"),
    keeping the values in the arithmetic ``dtype``."""

    if act is None or act == "f64":
        return np.asarray(x, dtype=dtype)
    if act == "f32":
        return np.asarray(x, dtype=np.float32).astype(dtype)
    if act == "bf16":
        return bf16_round(x).astype(dtype)
    if act == "f16":
        return f16_round(x).astype(dtype)
    raise ValueError(f"unknown activation dtype {act!r}")


# --------------------------------------------------------------------------
# elementwise pieces (MLX semantics)
# --------------------------------------------------------------------------


def softplus(x):
    """``mlx.nn.softplus``: log(1 + e^x) in its logaddexp form."""

    return np.logaddexp(x, 0.0)


def sigmoid(x):
    x = np.asarray(x)
    return np.exp(-np.logaddexp(0.0, -x))


def silu(x):
    return x * sigmoid(x)


def rms_norm(x, weight, eps):
    """``mx.fast.rms_norm``: x * rsqrt(mean(x^2, -1) + eps) * weight."""

    ms = np.mean(np.square(x), axis=-1, keepdims=True)
    out = x / np.sqrt(ms + eps)
    return out if weight is None else out * weight


def forget_gate(a, A_log, dt_bias, dtype=np.float64):
    """g = exp(-exp(A_log) * softplus(a + dt_bias)) in float (gated_delta.py:14-21)."""

    a = np.asarray(a, dtype=dtype)
    A_log = np.asarray(A_log, dtype=dtype)
    dt_bias = np.asarray(dt_bias, dtype=dtype)
    return np.exp(-np.exp(A_log) * softplus(a + dt_bias)).astype(dtype)


def beta_gate(b, act=None, dtype=np.float64):
    """beta = sigmoid(b) held in b's dtype (linear_attention.py:116)."""

    return act_round(sigmoid(np.asarray(b, dtype=dtype)), act, dtype)


# --------------------------------------------------------------------------
# the recurrence
# --------------------------------------------------------------------------


def gated_delta_step(q, k, v, g, beta, state):
    """One step for all value heads (gated_delta.py:24-41). q/k are
    ``(Hv, Dk)`` already repeated out; v ``(Hv, Dv)``; g/beta ``(Hv,)``;
    state ``(Hv, Dv, Dk)``. Returns ``(y (Hv, Dv), new_state)``."""

    state = state * g[:, None, None]
    read = (state * k[:, None, :]).sum(axis=-1)
    delta = (v - read) * beta[:, None]
    state = state + k[:, None, :] * delta[:, :, None]
    y = (state * q[:, None, :]).sum(axis=-1)
    return y, state


def repeat_heads(x, repeat: int):
    """``mx.repeat(x, repeat, axis=-2)``: each key head is repeated in place,
    so value head ``h`` reads key head ``h // repeat`` (gated_delta.py:99-101)."""

    return np.repeat(x, repeat, axis=-2) if repeat > 1 else x


def gated_delta_scan_ops(q, k, v, g, beta, state, dtype=np.float64):
    """The pure-ops recurrence over L positions (gated_delta.py:93-109)."""

    q, k, v, g, beta, state = (np.asarray(t, dtype=dtype) for t in (q, k, v, g, beta, state))
    repeat = v.shape[-2] // q.shape[-2]
    q = repeat_heads(q, repeat)
    k = repeat_heads(k, repeat)
    outputs = []
    for t in range(q.shape[0]):
        y, state = gated_delta_step(q[t], k[t], v[t], g[t], beta[t], state)
        outputs.append(y)
    return np.stack(outputs), state


def check_scan_shapes(q, k, v, g, beta, state):
    """The reference's validation (gated_delta.py:57-79): raises ValueError."""

    if q.ndim != 3 or k.shape != q.shape or v.ndim != 3:
        raise ValueError("q/k must have matching (L, key_heads, key_dim) shapes; v must be 3-D")
    length, key_heads, key_dim = q.shape
    _, value_heads, value_dim = v.shape
    if min(length, key_heads, key_dim, value_heads, value_dim) <= 0:
        raise ValueError("gated_delta_scan requires nonempty sequence and head dimensions")
    if v.shape[0] != length or value_heads % key_heads:
        raise ValueError("v must match q's sequence length and have a multiple of its head count")
    if g.shape != (length, value_heads) or beta.shape != g.shape:
        raise ValueError("g and beta must have shape (L, value_heads)")
    if state.shape != (value_heads, value_dim, key_dim):
        raise ValueError("state must have shape (value_heads, value_dim, key_dim)")


def gated_delta_scan(q, k, v, g, beta, state, dtype=np.float64):
    check_scan_shapes(*(np.asarray(t) for t in (q, k, v, g, beta, state)))
    return gated_delta_scan_ops(q, k, v, g, beta, state, dtype=dtype)


def gated_delta_update(q, k, v, a, b, A_log, dt_bias, state=None, cu_seqlens=None,
                       act=None, dtype=np.float64):
    """Batched/varlen gated-delta update with the gates computed inside.

    Batch-first shapes as the reference's upstream cross-check calls it
    (tests/test_qwen3_5_gated_delta.py:59-69): q/k ``(B, L, Hk, Dk)``,
    v ``(B, L, Hv, Dv)``, a/b ``(B, L, Hv)``, state ``(B, Hv, Dv, Dk)``.
    With ``cu_seqlens`` (length N+1) the token axis is packed: q ``(T, Hk, Dk)``
    etc. and state ``(N, Hv, Dv, Dk)``. Each sequence is an independent run of
    ``gated_delta_scan_ops`` (the reference has no batch axis)."""

    g = forget_gate(a, A_log, dt_bias, dtype)
    beta = beta_gate(b, act, dtype)
    if cu_seqlens is None:
        B, L, _, Dk = q.shape
        Hv, Dv = v.shape[-2:]
        if state is None:
            state = np.zeros((B, Hv, Dv, Dk), dtype)
        ys, states = [], []
        for i in range(B):
            y, s = gated_delta_scan_ops(q[i], k[i], v[i], g[i], beta[i], state[i], dtype)
            ys.append(y)
            states.append(s)
        return np.stack(ys), np.stack(states)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    n = len(cu) - 1
    Dk = q.shape[-1]
    Hv, Dv = v.shape[-2:]
    if state is None:
        state = np.zeros((n, Hv, Dv, Dk), dtype)
    y = np.zeros(v.shape, dtype)
    states = []
    for i in range(n):
        s0, s1 = cu[i], cu[i + 1]
        if s1 > s0:
            yi, si = gated_delta_scan_ops(q[s0:s1], k[s0:s1], v[s0:s1], g[s0:s1],
                                          beta[s0:s1], state[i], dtype)
            y[s0:s1] = yi
        else:
            si = np.asarray(state[i], dtype)
        states.append(si)
    return y, np.stack(states)


# --------------------------------------------------------------------------
# the layer's front-end and epilogue
# --------------------------------------------------------------------------


def convolve(qkv, conv_state, weight, act=None, dtype=np.float64):
    """Depthwise causal conv + SiLU + state roll (linear_attention.py:61-79).

    ``qkv (L, C)``, ``conv_state (K-1, C)``, ``weight (C, K)`` (the
    reference's ``(C, K, 1)`` squeezed). MLX's conv1d is a cross-correlation,
    so output row t is ``sum_j weight[c, j] * in[t + j, c]`` over
    ``in = concat(conv_state, qkv)``; the last tap meets the current token.
    Returns ``(silu(out) (L, C), new_state (K-1, C))``."""

    qkv = act_round(qkv, act, dtype)
    conv_in = np.concatenate([act_round(conv_state, act, dtype), qkv], axis=0)
    w = act_round(np.asarray(weight, dtype=dtype).reshape(weight.shape[0], -1), act, dtype)
    K = w.shape[1]
    L = qkv.shape[0]
    out = np.zeros((L, qkv.shape[1]), dtype)
    for j in range(K):
        out += w[:, j][None, :] * conv_in[j:j + L]
    out = act_round(out, act, dtype)
    tail_start = conv_in.shape[0] - (K - 1)
    return act_round(silu(out), act, dtype), conv_in[tail_start:]


def qk_scale(q, k, act=None, dtype=np.float64):
    """``q = Dk^-1 * rms_norm(q, eps=1e-6)``, ``k = Dk^-1/2 * rms_norm(k, eps=1e-6)``
    (linear_attention.py:109-113). In a bf16 graph the Python scalar joins as a
    bf16 constant and the product is rounded again."""

    Dk = q.shape[-1]
    inv = Dk ** -0.5
    sq, sk = act_round(inv * inv, act, dtype), act_round(inv, act, dtype)
    qn = act_round(rms_norm(q, None, EPS_QK), act, dtype)
    kn = act_round(rms_norm(k, None, EPS_QK), act, dtype)
    return act_round(sq * qn, act, dtype), act_round(sk * kn, act, dtype)


def gated_rms_norm(x, gate, weight, eps, act=None, dtype=np.float64):
    """``silu(gate) * rms_norm(x, weight)`` with the product in float and the
    result in x's dtype (linear_attention.py:22-32)."""

    normed = act_round(rms_norm(np.asarray(x, dtype), np.asarray(weight, dtype), eps), act, dtype)
    return act_round(silu(np.asarray(gate, dtype)) * normed, act, dtype)


def linear_attention_core(qkv, z, a, b, conv_state, ssm_state, conv_weight, A_log, dt_bias,
                          norm_weight, dims, eps=1e-6, act=None, dtype=np.float64):
    """The layer between the input projections and out_proj
    (linear_attention.py:103-124) for one sequence.

    ``qkv (L, C)``, ``z (L, Hv, Dv)``, ``a, b (L, Hv)``. ``dims`` is
    ``(Hk, Hv, Dk, Dv)``. Returns ``(out (L, Hv*Dv), new_conv_state, new_ssm_state)``."""

    Hk, Hv, Dk, Dv = dims
    L = qkv.shape[0]
    conv_out, new_conv = convolve(qkv, conv_state, conv_weight, act, dtype)
    key_dim = Hk * Dk
    q = conv_out[:, :key_dim].reshape(L, Hk, Dk)
    k = conv_out[:, key_dim:2 * key_dim].reshape(L, Hk, Dk)
    v = conv_out[:, 2 * key_dim:].reshape(L, Hv, Dv)
    q, k = qk_scale(q, k, act, dtype)
    g = forget_gate(a, A_log, dt_bias, dtype)
    beta = beta_gate(b, act, dtype)
    y, new_ssm = gated_delta_scan_ops(q, k, v, g, beta, ssm_state, dtype)
    y = act_round(y, act, dtype)  # y.astype(z.dtype)
    out = gated_rms_norm(y, z, norm_weight, eps, act, dtype)
    return out.reshape(L, Hv * Dv), new_conv, new_ssm


def linear_attention(x, weights, conv_state, ssm_state, dims, eps=1e-6, act=None,
                     dtype=np.float64):
    """Whole layer with dense projections (linear_attention.py:81-127).

    ``weights`` holds ``in_proj_qkv, in_proj_z, in_proj_a, in_proj_b,
    out_proj`` as ``(out, in)`` matrices (``x @ W.T``, moe_block.py:44-46) plus
    ``conv1d_weight, A_log, dt_bias, norm_weight``."""

    squeeze = np.ndim(x) == 1
    rows = np.asarray(x, dtype)[None, :] if squeeze else np.asarray(x, dtype)
    Hk, Hv, Dk, Dv = dims
    L = rows.shape[0]
    proj = lambda name: act_round(rows @ np.asarray(weights[name], dtype).T, act, dtype)
    qkv = proj("in_proj_qkv")
    z = proj("in_proj_z").reshape(L, Hv, Dv)
    a = proj("in_proj_a")
    b = proj("in_proj_b")
    out, new_conv, new_ssm = linear_attention_core(
        qkv, z, a, b, conv_state, ssm_state, weights["conv1d_weight"], weights["A_log"],
        weights["dt_bias"], weights["norm_weight"], dims, eps, act, dtype)
    out = act_round(out @ np.asarray(weights["out_proj"], dtype).T, act, dtype)
    return (out[0] if squeeze else out), new_conv, new_ssm


# --------------------------------------------------------------------------
# the reference test's seeded inputs and float64 check
# --------------------------------------------------------------------------


def metal_test_inputs(length, key_dim=128, value_dim=17, key_heads=2, value_heads=4):
    """Seeded inputs of tests/test_gated_delta_metal.py:10-23 (rng seed 42):
    q, k unit-normalised with q also divided by sqrt(key_dim); g ~ U(0.98, 1)
    with value head 0 at g = 1; beta ~ U(0, 1); state ~ 0.1 N(0, 1).
    Returned as float32 arrays ``(q, k, v, g, beta, state)``."""

    rng = np.random.default_rng(42)
    q = rng.normal(size=(length, key_heads, key_dim))
    k = rng.normal(size=q.shape)
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * key_dim ** 0.5
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(length, value_heads, value_dim))
    g = rng.uniform(0.98, 1, size=(length, value_heads))
    g[:, 0] = 1
    beta = rng.uniform(0, 1, size=g.shape)
    state = rng.normal(size=(value_heads, value_dim, key_dim)) * 0.1
    return [a.astype(np.float32) for a in (q, k, v, g, beta, state)]


def metal_test_reference(inputs):
    """The reference test's own float64 recurrence (tests/test_gated_delta_metal.py:26-39),
    written with einsum rather than broadcast-and-sum."""

    q, k, v, g, beta, state = [np.array(a).astype(np.float64) for a in inputs]
    repeat = v.shape[1] // q.shape[1]
    q, k = np.repeat(q, repeat, axis=1), np.repeat(k, repeat, axis=1)
    output = []
    for t in range(len(q)):
        state *= g[t, :, None, None]
        read = np.einsum("hvk,hk->hv", state, k[t])
        correction = (v[t] - read) * beta[t, :, None]
        state += np.einsum("hv,hk->hvk", correction, k[t])
        output.append(np.einsum("hvk,hk->hv", state, q[t]))
    return np.stack(output), state
