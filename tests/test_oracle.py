"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is independent of the formula it tests: the reference test's own
float64 einsum recurrence and seeded inputs, an index-loop brute force,
closed forms that fix the answer, the chunked WY form (a different
algorithm), split/carry invariants, torch's CPU library routines for the
front-end pieces, and the C restatement.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import chunked_ref, cref
from oracle import gated_delta_ref as R
from tests.golden.make_golden import (LONG_LENGTH, METAL_SHAPES, fixture_name,
                                      inputs_digest)
from tests.helpers import assert_bf16_out_close, layer_inputs, layer_params, max_rel

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------------------
# golden vectors of the reference's scan test
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("shape", METAL_SHAPES + [(LONG_LENGTH,)])
def test_oracle_reproduces_golden_fixture(shape):
    inputs = R.metal_test_inputs(*shape)
    fx = np.load(os.path.join(GOLDEN, fixture_name(shape)))
    assert str(fx["digest"]) == inputs_digest(inputs), "numpy's seeded generator drifted"
    y, state = R.gated_delta_scan(*inputs)
    np.testing.assert_allclose(y, fx["y"], rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(state, fx["state"], rtol=1e-6, atol=1e-9)


def test_reference_inputs_have_the_documented_properties():
    q, k, v, g, beta, state = R.metal_test_inputs(33, key_dim=64)
    np.testing.assert_allclose(np.linalg.norm(k, axis=-1), 1, rtol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(q, axis=-1), 64 ** -0.5, rtol=1e-6)
    assert (g[:, 0] == 1).all() and (g >= 0.98).all() and (g <= 1).all()
    assert (beta >= 0).all() and (beta <= 1).all()


# ---------------------------------------------------------------------------
# the recurrence: brute force, closed forms, invariants
# ---------------------------------------------------------------------------


def _brute_force_scan(q, k, v, g, beta, state):
    """Scalar index loops, value head h reading key head h // (Hv / Hk)."""

    L, Hk, Dk = q.shape
    Hv, Dv = v.shape[1:]
    S = [[[float(state[h, i, j]) for j in range(Dk)] for i in range(Dv)] for h in range(Hv)]
    y = np.zeros((L, Hv, Dv))
    for t in range(L):
        for h in range(Hv):
            hk = h // (Hv // Hk)
            for i in range(Dv):
                row = S[h][i]
                for j in range(Dk):
                    row[j] *= float(g[t, h])
                read = sum(row[j] * float(k[t, hk, j]) for j in range(Dk))
                delta = (float(v[t, h, i]) - read) * float(beta[t, h])
                for j in range(Dk):
                    row[j] += float(k[t, hk, j]) * delta
                y[t, h, i] = sum(row[j] * float(q[t, hk, j]) for j in range(Dk))
    return y, np.array(S)


def _small_inputs(seed, L, Hk=2, Hv=6, Dk=16, Dv=8):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s)
    a, b = f(L, Hv), f(L, Hv)
    A_log, dt_bias = f(Hv), f(Hv)
    g = R.forget_gate(a, A_log, dt_bias)
    beta = R.sigmoid(b)
    return f(L, Hk, Dk), f(L, Hk, Dk), f(L, Hv, Dv), g, beta, f(Hv, Dv, Dk) * 0.1


@pytest.mark.parametrize("seed", range(4))
def test_scan_matches_index_loop_brute_force(seed):
    inputs = _small_inputs(seed, L=5)
    y, s = R.gated_delta_scan(*inputs)
    yb, sb = _brute_force_scan(*inputs)
    np.testing.assert_allclose(y, yb, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s, sb, rtol=1e-12, atol=1e-12)


def test_gqa_is_repeat_not_tile():
    # Key head 1 is zero: with repeat (hv // r) value heads 3..5 see it, with
    # tiling (hv % Hk) the odd heads would.
    q, k, v, g, beta, state = _small_inputs(7, L=1)
    q[:, 1] = 0
    y, _ = R.gated_delta_scan(q, k, v, g, beta, state)
    assert np.all(y[0, 3:] == 0)
    assert np.all(np.abs(y[0, :3]).max(axis=-1) > 0)


def test_identity_when_no_decay_and_no_write():
    q, k, v, g, beta, state = _small_inputs(1, L=3)
    g[:] = 1
    beta[:] = 0
    y, s = R.gated_delta_scan(q, k, v, g, beta, state)
    np.testing.assert_array_equal(s, state)
    qh = np.repeat(q, 3, axis=1)
    np.testing.assert_allclose(y, np.einsum("hij,thj->thi", state, qh), rtol=1e-12)


def test_full_write_overwrites_the_key_direction():
    # beta = 1 with unit k: after the step S k = v exactly (delta rule).
    q, k, v, g, beta, state = _small_inputs(2, L=1)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    beta[:] = 1
    _, s = R.gated_delta_scan(q, k, v, g, beta, state)
    kh = np.repeat(k, 3, axis=1)[0]
    np.testing.assert_allclose(np.einsum("hij,hj->hi", s, kh), v[0], rtol=1e-10, atol=1e-12)


def test_zero_gate_resets_the_state():
    q, k, v, g, beta, state = _small_inputs(3, L=1)
    g[:] = 0
    _, s = R.gated_delta_scan(q, k, v, g, beta, state)
    kh = np.repeat(k, 3, axis=1)[0]
    expected = beta[0][:, None, None] * v[0][:, :, None] * kh[:, None, :]
    np.testing.assert_allclose(s, expected, rtol=1e-12, atol=1e-14)


def test_split_carry_equals_one_scan():
    inputs = _small_inputs(4, L=9)
    y, s = R.gated_delta_scan(*inputs)
    state = inputs[-1]
    ys = []
    for lo, hi in [(0, 2), (2, 3), (3, 9)]:
        yi, state = R.gated_delta_scan(*(a[lo:hi] for a in inputs[:-1]), state)
        ys.append(yi)
    np.testing.assert_allclose(np.concatenate(ys), y, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(state, s, rtol=1e-12, atol=1e-14)


def test_single_step_equals_scan_of_one():
    q, k, v, g, beta, state = _small_inputs(5, L=1)
    y, s = R.gated_delta_scan(q, k, v, g, beta, state)
    ys, ss = R.gated_delta_step(np.repeat(q[0], 3, 0), np.repeat(k[0], 3, 0), v[0], g[0],
                                beta[0], state)
    np.testing.assert_allclose(ys, y[0], rtol=1e-14)
    np.testing.assert_allclose(ss, s, rtol=1e-14)


def test_scan_does_not_modify_its_input_state():
    inputs = _small_inputs(6, L=4)
    before = inputs[-1].copy()
    R.gated_delta_scan(*inputs)
    np.testing.assert_array_equal(inputs[-1], before)


@pytest.mark.parametrize("bad", ["k", "v", "g", "beta", "state", "heads", "empty"])
def test_invalid_shapes_raise(bad):
    q, k, v, g, beta, state = R.metal_test_inputs(5)
    if bad == "k":
        k = k[:1]
    elif bad == "v":
        v = v[:1]
    elif bad == "g":
        g = g[:1]
    elif bad == "beta":
        beta = beta[:1]
    elif bad == "state":
        state = state[:1]
    elif bad == "heads":
        q = np.repeat(q[:, :1], 3, axis=1)
        k = q
    else:
        q, k, v, g, beta = (a[:0] for a in (q, k, v, g, beta))
    with pytest.raises(ValueError):
        R.gated_delta_scan(q, k, v, g, beta, state)


# ---------------------------------------------------------------------------
# the chunked form (an independent algorithm for the same recurrence)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("chunk", [1, 3, 8, 64])
def test_chunked_form_equals_sequential(chunk):
    q, k, v, g, beta, state = R.metal_test_inputs(150, key_dim=32, value_dim=12, key_heads=2,
                                                  value_heads=4)
    y, s = R.gated_delta_scan(q, k, v, g, beta, state)
    yc, sc = chunked_ref.chunked_scan(q, k, v, g, beta, state, chunk=chunk)
    np.testing.assert_allclose(yc, y, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(sc, s, rtol=1e-9, atol=1e-12)


def test_chunked_form_survives_vanishing_gates():
    # Large decays underflow g to 0 inside a chunk: the log-space form must
    # still agree with the sequential recurrence (which zeroes the state).
    inputs = list(_small_inputs(8, L=70, Hv=4, Dk=16, Dv=8))
    inputs[3][10:20] = 0.0
    inputs[3][30] = 1e-30
    y, s = R.gated_delta_scan(*inputs)
    yc, sc = chunked_ref.chunked_scan(*inputs, chunk=64)
    np.testing.assert_allclose(yc, y, rtol=1e-8, atol=1e-12)
    np.testing.assert_allclose(sc, s, rtol=1e-8, atol=1e-12)


# ---------------------------------------------------------------------------
# front-end and gated norm: library cross-checks and closed forms
# ---------------------------------------------------------------------------


def test_gates_closed_forms():
    assert R.softplus(np.array(0.0)) == pytest.approx(math.log(2))
    assert R.softplus(np.array(50.0)) == pytest.approx(50.0)
    assert R.sigmoid(np.array(0.0)) == 0.5
    x = np.linspace(-30, 30, 101)
    np.testing.assert_allclose(R.softplus(x), torch.nn.functional.softplus(
        torch.tensor(x), threshold=1e9).numpy(), rtol=1e-12)
    np.testing.assert_allclose(R.sigmoid(x), torch.sigmoid(torch.tensor(x)).numpy(), rtol=1e-12)
    np.testing.assert_allclose(R.silu(x), torch.nn.functional.silu(torch.tensor(x)).numpy(),
                               rtol=1e-12)
    rng = np.random.default_rng(3)
    a, A_log, dt = rng.standard_normal((4, 6)), rng.standard_normal(6), rng.standard_normal(6)
    g = R.forget_gate(a, A_log, dt)
    assert (g > 0).all() and (g <= 1).all()
    np.testing.assert_allclose(np.log(g), -np.exp(A_log) * np.log1p(np.exp(a + dt)), rtol=1e-12)


def test_convolve_matches_torch_conv1d():
    rng = np.random.default_rng(0)
    L, C, K = 7, 24, 4
    qkv, state, w = rng.standard_normal((L, C)), rng.standard_normal((K - 1, C)), rng.standard_normal((C, K))
    out, new_state = R.convolve(qkv, state, w)
    x = torch.tensor(np.concatenate([state, qkv]).T[None])  # (1, C, L+K-1)
    ref = torch.nn.functional.conv1d(x, torch.tensor(w)[:, None, :], groups=C)[0].T
    np.testing.assert_allclose(out, torch.nn.functional.silu(ref).numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_array_equal(new_state, qkv[-(K - 1):])


def test_convolve_short_input_keeps_old_state_rows():
    rng = np.random.default_rng(1)
    qkv, state, w = rng.standard_normal((1, 5)), rng.standard_normal((3, 5)), rng.standard_normal((5, 4))
    _, new_state = R.convolve(qkv, state, w)
    np.testing.assert_array_equal(new_state, np.concatenate([state[1:], qkv]))
    # a delta kernel on the last tap reproduces silu(current token)
    w = np.zeros((5, 4))
    w[:, 3] = 1
    out, _ = R.convolve(qkv, state, w)
    np.testing.assert_allclose(out, R.silu(qkv), rtol=1e-15)


def test_qk_scale_norms_and_rms_norm():
    rng = np.random.default_rng(2)
    q, k = rng.standard_normal((3, 2, 128)), rng.standard_normal((3, 2, 128))
    qs, ks = R.qk_scale(q, k)
    np.testing.assert_allclose(np.linalg.norm(qs, axis=-1), 128 ** -0.5, rtol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(ks, axis=-1), 1.0, rtol=1e-6)
    x, w = rng.standard_normal((4, 16)), rng.standard_normal(16)
    ref = torch.nn.functional.rms_norm(torch.tensor(x), (16,), torch.tensor(w), eps=1e-6)
    np.testing.assert_allclose(R.rms_norm(x, w, 1e-6), ref.numpy(), rtol=1e-12)


def test_gated_rms_norm_closed_form():
    c = np.full((2, 8), 3.0)
    w = np.linspace(0.5, 1.5, 8)
    z = np.full((2, 8), 40.0)  # silu(40) = 40 to 1e-16
    out = R.gated_rms_norm(c, z, w, eps=0.0)
    np.testing.assert_allclose(out, 40.0 * np.broadcast_to(w, (2, 8)), rtol=1e-12)


def test_bf16_rounding_is_round_to_nearest_even():
    one = np.float32(1.0)
    assert R.bf16_round(one + np.float32(2 ** -8))[()] == 1.0  # tie -> even
    assert R.bf16_round(one + np.float32(3 * 2 ** -8))[()] == np.float32(1 + 2 ** -6)  # tie -> even
    assert R.bf16_round(one + np.float32(2 ** -8 + 2 ** -12))[()] == np.float32(1 + 2 ** -7)
    x = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    ref = torch.tensor(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(R.bf16_round(x), ref)


def _bf16_exact(v: float) -> float:
    """Round-to-nearest-even to 8 significant bits by exact rationals."""
    from fractions import Fraction

    f = Fraction(v)
    if f == 0:
        return 0.0
    sign = -1 if f < 0 else 1
    f = abs(f)
    e = 0
    while f >= 2:
        f /= 2
        e += 1
    while f < 1:
        f *= 2
        e -= 1
    scaled = f * 128  # 8 significant bits: [128, 256)
    n = int(scaled)
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return float(sign * Fraction(n, 128) * Fraction(2) ** e)


def test_bf16_rounding_of_float64_is_one_rounding():
    """Float64 values just above or below a bf16 tie (closer to it than a
    float32 ulp, where rounding through float32 first would land on the tie
    and go to even) round to the side they lie on; random float64 values
    agree with exact rational rounding."""

    rng = np.random.default_rng(3)
    for base in (1.0, 1.5, -3.25, 0.0078125, 1232.0):  # bf16 values
        ulp = 2.0 ** (np.floor(np.log2(abs(base))) - 7)
        tie = base + np.copysign(ulp / 2, base)  # between base and the next bf16 away from zero
        for nudge, expect in ((2 ** -40, base + np.copysign(ulp, base)), (-(2 ** -40), base)):
            x = np.float64(tie + np.sign(base) * abs(tie) * nudge)
            assert float(R.bf16_round(x).reshape(-1)[0]) == expect, (base, nudge)
            assert _bf16_exact(float(x)) == expect
    x = rng.standard_normal(2000) * np.exp(rng.uniform(-20, 20, 2000))
    got = R.bf16_round(x)
    assert got.dtype == np.float32
    assert [float(v) for v in got] == [_bf16_exact(float(v)) for v in x]


def test_bf16_rounding_of_float64_below_the_normal_range():
    """Below 2^-126 bfloat16 holds multiples of 2^-133 (its subnormals):
    float64 values there, and across the boundary, round like torch's
    float32 -> bfloat16 conversion of the same (float32-exact) values, in the
    NumPy and the C oracle alike; sigmoid(-88.5) is one such beta."""

    rng = np.random.default_rng(11)
    x32 = np.concatenate([
        (rng.uniform(-1, 1, 3000) * 2.0 ** -126).astype(np.float32),
        (rng.uniform(0.9, 1.1, 1000) * 2.0 ** -126).astype(np.float32),
        (np.arange(-600, 600) * 2.0 ** -134).astype(np.float32),  # every tie of the range
    ])
    want = torch.from_numpy(x32).to(torch.bfloat16).float().numpy()
    x = x32.astype(np.float64)
    np.testing.assert_array_equal(R.bf16_round(x), want)
    np.testing.assert_array_equal(cref.bf16_of_double(x), want)
    beta = R.beta_gate(np.array([-88.5], np.float32), "bf16")
    assert 0 < beta[0] < 2.0 ** -126 and float(beta[0] / 2.0 ** -133).is_integer()


# ---------------------------------------------------------------------------
# the C restatement (timed CPU comparator) agrees with the NumPy oracle
# ---------------------------------------------------------------------------


def test_c_scan_matches_numpy_oracle():
    q, k, v, g, beta, state = R.metal_test_inputs(17, 128, 128, 16, 32)
    y, s = R.metal_test_reference([q, k, v, g, beta, state])
    yc, sc = cref.scan(q[None], k[None], v[None], g[None], beta[None], state[None])
    np.testing.assert_allclose(yc[0], y, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(sc[0], s, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("act_bf16", [False, True])
@pytest.mark.parametrize("with_z", [False, True])
def test_c_decode_step_matches_numpy_layer_core(act_bf16, with_z):
    rng = np.random.default_rng(11)
    dims = (2, 4, 128, 128)
    B = 3
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, dims)
    qkv, z, a, b = layer_inputs(rng, dims, L=1, act_bf16=act_bf16, B=B)
    C = qkv.shape[-1]
    conv = (rng.standard_normal((B, 3, C))).astype(np.float32)
    if act_bf16:
        conv = R.bf16_round(conv)
    state = (rng.standard_normal((B, 4, 128, 128)) * 0.05).astype(np.float32)
    act = "bf16" if act_bf16 else None
    out_c, conv_c, state_c = cref.decode_step(qkv[:, 0], conv, conv_w, a[:, 0], b[:, 0], A_log,
                                              dt_bias, state, z[:, 0] if with_z else None,
                                              norm_w, 1e-6, dims, act_bf16)
    for i in range(B):
        o, nc, ns = R.linear_attention_core(qkv[i], z[i], a[i], b[i], conv[i], state[i], conv_w,
                                            A_log, dt_bias, norm_w, dims, 1e-6, act)
        assert max_rel(state_c[i], ns) < 1e-5
        np.testing.assert_allclose(conv_c[i], nc, rtol=0, atol=0)
        if with_z:
            tol = 2e-2 if act_bf16 else 1e-4
            np.testing.assert_allclose(out_c[i].reshape(-1), o.reshape(-1), atol=tol)


def test_c_decode_rounds_like_the_float64_oracle_at_hv64():
    """Three chained decode steps of 16 sequences at Hk=16, Hv=64 with bf16
    activations (about 200 000 values rounded to bf16 per step): the C
    restatement's front-end (conv, SiLU, q/k scaling, sigmoid(b), gated
    norm) evaluates each rounded value in double and rounds once, so its
    state stays within 1e-6 of the float64 oracle's. On these inputs the
    same restatement with a float32 front-end (its earlier form) is up to
    3e-4 apart from it: a float32 error decides some values that lie within
    a float32 ulp of a bf16 tie."""

    B, Hk, Hv, D = 16, 16, 64, 128
    rng = np.random.default_rng(33)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, (Hk, Hv, D, D))
    C = 2 * Hk * D + Hv * D
    conv = R.bf16_round(rng.standard_normal((B, 3, C)))
    state = (rng.standard_normal((B, Hv, D, D)) * 0.05).astype(np.float32)
    conv64, state64 = conv.astype(np.float64), state.astype(np.float64)
    for step in range(3):
        qkv, z, a, b = layer_inputs(rng, (Hk, Hv, D, D), L=1, act_bf16=True, B=B)
        out_c, conv, state = cref.decode_step(qkv[:, 0], conv, conv_w, a[:, 0], b[:, 0], A_log,
                                              dt_bias, state, z[:, 0], norm_w, 1e-6,
                                              (Hk, Hv, D, D), True)
        nxt = [R.linear_attention_core(qkv[i], z[i], a[i], b[i], conv64[i], state64[i], conv_w,
                                       A_log, dt_bias, norm_w, (Hk, Hv, D, D), 1e-6, "bf16")
               for i in range(B)]
        conv64 = np.stack([n[1] for n in nxt])
        state64 = np.stack([n[2] for n in nxt])
        np.testing.assert_array_equal(conv, conv64)
        assert max_rel(state, state64) < 1e-6, step
        assert_bf16_out_close(out_c.reshape(B, -1), np.stack([n[0] for n in nxt]).reshape(B, -1))


# ---------------------------------------------------------------------------
# layer-level invariants on the oracle
# ---------------------------------------------------------------------------


def test_layer_stepwise_equals_batched_and_state_size_is_constant():
    rng = np.random.default_rng(101)
    dims = (2, 4, 32, 32)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, dims)
    qkv, z, a, b = layer_inputs(rng, dims, L=5, act_bf16=False)
    C = qkv.shape[-1]
    conv0, ssm0 = np.zeros((3, C)), np.zeros((4, 32, 32))
    out, conv_b, ssm_b = R.linear_attention_core(qkv, z, a, b, conv0, ssm0, conv_w, A_log,
                                                 dt_bias, norm_w, dims)
    conv, ssm, outs = conv0, ssm0, []
    for t in range(5):
        o, conv, ssm = R.linear_attention_core(qkv[t:t + 1], z[t:t + 1], a[t:t + 1],
                                               b[t:t + 1], conv, ssm, conv_w, A_log, dt_bias,
                                               norm_w, dims)
        assert conv.shape == conv0.shape and ssm.shape == ssm0.shape
        outs.append(o)
    np.testing.assert_allclose(np.concatenate(outs), out, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(ssm, ssm_b, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(conv, conv_b, rtol=0, atol=0)
