"""GPU parity of the sequential scans against the golden fixtures and the
oracle (the reference's tests/test_gated_delta_metal.py and
tests/test_qwen3_5_gated_delta.py, restated for this library)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from mlx_lean_moe_amd import gated_delta
from oracle import gated_delta_ref as R
from tests.golden.make_golden import LONG_LENGTH, METAL_SHAPES, fixture_name
from tests.helpers import max_rel

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _to(dev, arrays, dtype=torch.float32):
    return [torch.tensor(np.asarray(a, np.float32), dtype=dtype, device=dev) for a in arrays]


@pytest.fixture
def forbid_reference_kernel(monkeypatch):
    real = gated_delta._lib.call

    def guarded(name, *args):
        assert name != "gdn_scan_reference", "supported inputs must use the optimised scan"
        return real(name, *args)

    monkeypatch.setattr(gated_delta._lib, "call", guarded)


@pytest.mark.parametrize("shape", METAL_SHAPES)
@pytest.mark.parametrize("strided", [False, True])
def test_kernel_matches_float64_reference_and_preserves_input_state(
        gpu, shape, strided, forbid_reference_kernel):
    inputs = _to(gpu, R.metal_test_inputs(*shape))
    if strided:
        inputs = [torch.stack([a, a], dim=-1)[..., 0] for a in inputs]
        assert not inputs[0].is_contiguous()
    fx = np.load(os.path.join(GOLDEN, fixture_name(shape)))
    initial_state = inputs[-1].clone()
    y, state = gdn.gated_delta_scan(*inputs)
    assert y.dtype == state.dtype == torch.float32
    np.testing.assert_allclose(y.cpu().numpy(), fx["y"], rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(state.cpu().numpy(), fx["state"], rtol=2e-5, atol=2e-6)
    assert torch.equal(inputs[-1], initial_state)


def test_long_scan_and_prefill_then_decode_preserve_carried_state(gpu):
    inputs = _to(gpu, R.metal_test_inputs(LONG_LENGTH))
    fx = np.load(os.path.join(GOLDEN, fixture_name((LONG_LENGTH,))))
    whole_y, whole_state = gdn.gated_delta_scan(*inputs)
    state = inputs[-1]
    outputs = []
    bounds = [0, 1, 128, 383, 1024, 1920, *range(1921, 2049)]
    for start, end in zip(bounds, bounds[1:]):
        y, state = gdn.gated_delta_scan(*(a[start:end] for a in inputs[:-1]), state)
        outputs.append(y)
    split_y = torch.cat(outputs)
    for actual in (whole_y, split_y):
        np.testing.assert_allclose(actual.cpu().numpy(), fx["y"], rtol=2e-5, atol=2e-6)
    for actual in (whole_state, state):
        np.testing.assert_allclose(actual.cpu().numpy(), fx["state"], rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("case", ["float16", "bfloat16", "mixed", "small_head", "disabled"])
def test_other_dtypes_and_shapes_keep_the_ops_promotion_and_results(gpu, case):
    inputs = _to(gpu, R.metal_test_inputs(5, key_dim=16 if case == "small_head" else 128))
    if case in ("float16", "bfloat16"):
        inputs = [a.to(getattr(torch, case)) for a in inputs]
    elif case == "mixed":
        inputs[2] = inputs[2].to(torch.float16)
    actual = gdn.gated_delta_scan(*inputs, use_kernel=case != "disabled")
    reference_kernel = gdn.gated_delta_scan(*inputs, use_kernel=False)
    expected = R.gated_delta_scan(*[a.float().cpu().numpy() for a in inputs])
    for got, ref, want in zip(actual, reference_kernel, expected):
        assert got.dtype == ref.dtype == gated_delta._promote(*inputs)
        tol = 2e-2 if got.dtype != torch.float32 else 2e-5
        np.testing.assert_allclose(got.float().cpu().numpy(), want, rtol=tol, atol=tol)
        np.testing.assert_allclose(got.float().cpu().numpy(), ref.float().cpu().numpy(),
                                   rtol=tol, atol=tol)


def _seeded_update_inputs(seed, B, L, Hk=2, Hv=6, Dk=16, Dv=8, dtype=torch.float32, dev="cuda"):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    arrays = dict(q=f(B, L, Hk, Dk), k=f(B, L, Hk, Dk), v=f(B, L, Hv, Dv), a=f(B, L, Hv),
                  b=f(B, L, Hv), A_log=f(Hv), dt_bias=f(Hv))
    t = {n: torch.tensor(x, device=dev) for n, x in arrays.items()}
    for n in ("q", "k", "v", "a", "b"):
        t[n] = t[n].to(dtype)
    return arrays, t


@pytest.mark.parametrize("seq_len", [1, 5])
def test_update_matches_oracle(gpu, seq_len):
    arrays, t = _seeded_update_inputs(0, B=3, L=seq_len, dev=gpu)
    y, state = gdn.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"],
                                      t["dt_bias"])
    ye, se = R.gated_delta_update(arrays["q"], arrays["k"], arrays["v"], arrays["a"],
                                  arrays["b"], arrays["A_log"], arrays["dt_bias"])
    np.testing.assert_allclose(y.cpu().numpy(), ye, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(state.cpu().numpy(), se, rtol=1e-4, atol=1e-5)


def test_scan_continues_from_a_carried_state(gpu):
    arrays, t = _seeded_update_inputs(1, B=1, L=5, dev=gpu)
    g = gdn.forget_gate(t["a"][0], t["A_log"], t["dt_bias"])
    beta = torch.sigmoid(t["b"][0])
    q, k, v = t["q"][0], t["k"][0], t["v"][0]
    zero = torch.zeros(6, 8, 16, device=gpu)
    whole_y, whole_state = gdn.gated_delta_scan(q, k, v, g, beta, zero)
    first_y, mid = gdn.gated_delta_scan(q[:2], k[:2], v[:2], g[:2], beta[:2], zero)
    second_y, final = gdn.gated_delta_scan(q[2:], k[2:], v[2:], g[2:], beta[2:], mid)
    torch.testing.assert_close(torch.cat([first_y, second_y]), whole_y, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(final, whole_state, rtol=1e-5, atol=1e-6)


def test_single_step_matches_the_scan_of_one(gpu):
    arrays, t = _seeded_update_inputs(2, B=1, L=1, dev=gpu)
    g = gdn.forget_gate(t["a"][0], t["A_log"], t["dt_bias"])
    beta = torch.sigmoid(t["b"][0])
    state = torch.zeros(6, 8, 16, device=gpu)
    scan_y, scan_state = gdn.gated_delta_scan(t["q"][0], t["k"][0], t["v"][0], g, beta, state)
    rep = lambda x: x[0].repeat_interleave(3, dim=0)
    step_y, step_state = gdn.gated_delta_step(rep(t["q"][0]), rep(t["k"][0]), t["v"][0][0], g[0],
                                              beta[0], state)
    torch.testing.assert_close(scan_y[0], step_y, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(scan_state, step_state, rtol=1e-6, atol=1e-7)


def test_forget_gate_and_beta_match_oracle(gpu):
    arrays, t = _seeded_update_inputs(3, B=2, L=4, dev=gpu)
    g = gdn.forget_gate(t["a"], t["A_log"], t["dt_bias"])
    assert g.dtype == torch.float32
    assert bool((g > 0).all()) and bool((g <= 1).all())
    np.testing.assert_allclose(g.cpu().numpy(), R.forget_gate(arrays["a"], arrays["A_log"],
                                                               arrays["dt_bias"]), rtol=1e-5)
    bb = t["b"].to(torch.bfloat16)
    beta = gdn.beta_gate(bb)
    assert beta.dtype == torch.bfloat16
    np.testing.assert_array_equal(beta.float().cpu().numpy(),
                                  R.beta_gate(bb.float().cpu().numpy(), "bf16"))


def test_beta_of_every_bf16_input_is_the_rounded_exact_sigmoid(gpu):
    """All 65 536 bfloat16 bit patterns (NaNs aside) through the gates
    kernel: each beta is sigmoid(b) evaluated in float64 and rounded once to
    bfloat16, including the inputs whose float32 sigmoid lands near a
    bfloat16 rounding boundary (the kernel re-evaluates those in double)."""

    bits = np.arange(1 << 16, dtype=np.uint32)
    b = (bits << 16).view(np.float32)
    b = b[np.isfinite(b)]
    bb = torch.from_numpy(b).to(gpu).to(torch.bfloat16).reshape(-1, 4)
    got = gdn.beta_gate(bb).float().cpu().numpy().reshape(-1)
    # (b < -87.3 gives bfloat16 subnormals, multiples of 2^-133)
    np.testing.assert_array_equal(got, R.beta_gate(b, "bf16"))
    # the sweep does reach the boundary cases: some float32 sigmoids fall
    # within 16 float ulps of a bfloat16 midpoint
    f32 = (1.0 / (1.0 + np.exp(-b.astype(np.float32)))).astype(np.float32)
    low = f32.view(np.uint32) & 0xFFFF
    assert int((np.abs(low.astype(np.int64) - 0x8000) <= 16).sum()) > 0


def test_varlen_update_matches_per_sequence_oracle(gpu):
    rng = np.random.default_rng(5)
    lens = [3, 0, 1, 17, 8]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T, Hk, Hv, D = int(cu[-1]), 2, 4, 32
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    q, k, v, a, b = f(T, Hk, D), f(T, Hk, D), f(T, Hv, D), f(T, Hv), f(T, Hv)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    A_log, dt = f(Hv), f(Hv)
    s0 = f(len(lens), Hv, D, D) * 0.05
    dev = lambda x: torch.tensor(x, device=gpu)
    y, s = gdn.gated_delta_update(dev(q), dev(k), dev(v), dev(a), dev(b), dev(A_log), dev(dt),
                                  dev(s0), cu_seqlens=cu)
    ye, se = R.gated_delta_update(q, k, v, a, b, A_log, dt, s0, cu_seqlens=cu)
    np.testing.assert_allclose(y.cpu().numpy(), ye, rtol=1e-4, atol=1e-5)
    assert max_rel(s.cpu().numpy(), se) < 1e-5
    np.testing.assert_array_equal(s[1].cpu().numpy(), s0[1])  # empty run keeps its state


def test_optimised_scan_matches_reference_kernel_at_production_shape(gpu):
    rng = np.random.default_rng(9)
    L, Hk, Hv, D = 40, 16, 32, 128
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    q, k = f(L, Hk, D), f(L, Hk, D)
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * D ** 0.5
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    t = _to(gpu, [q, k, f(L, Hv, D), rng.uniform(0.5, 1, (L, Hv)), rng.uniform(0, 1, (L, Hv)),
                  f(Hv, D, D) * 0.05])
    y1, s1 = gdn.gated_delta_scan(*t)
    y2, s2 = gdn.gated_delta_scan(*t, use_kernel=False)
    assert max_rel(y1.cpu().numpy(), y2.cpu().numpy()) < 1e-5
    assert max_rel(s1.cpu().numpy(), s2.cpu().numpy()) < 1e-5
