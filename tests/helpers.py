"""Shared helpers for the tests (seeded inputs, tolerance checks)."""

from __future__ import annotations

import numpy as np

from oracle.gated_delta_ref import bf16_round


def max_rel(actual, expected) -> float:
    """max |a - e| / max |e| (the normalised max error used for states)."""

    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    scale = np.abs(expected).max()
    return float(np.abs(actual - expected).max() / (scale if scale > 0 else 1.0))


def layer_inputs(rng, dims, L, act_bf16: bool, B: int | None = None):
    """Pre-conv qkv, z, a, b for L tokens (bf16-representable when act_bf16)."""

    Hk, Hv, Dk, Dv = dims
    C = 2 * Hk * Dk + Hv * Dv
    lead = (L,) if B is None else (B, L)
    rnd = bf16_round if act_bf16 else (lambda x: np.asarray(x, np.float32))
    qkv = rnd(rng.standard_normal(lead + (C,)))
    z = rnd(rng.standard_normal(lead + (Hv, Dv)))
    a = rnd(rng.standard_normal(lead + (Hv,)))
    b = rnd(rng.standard_normal(lead + (Hv,)))
    return qkv, z, a, b


def layer_params(rng, dims, K=4):
    Hk, Hv, Dk, Dv = dims
    C = 2 * Hk * Dk + Hv * Dv
    conv_w = (rng.standard_normal((C, K)) * 0.2).astype(np.float32)
    A_log = rng.uniform(0, np.log(16), Hv).astype(np.float32)
    dt_bias = rng.uniform(-1, 1, Hv).astype(np.float32)
    norm_w = rng.uniform(0.5, 1.5, Dv).astype(np.float32)
    return conv_w, A_log, dt_bias, norm_w


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bfloat16 values at |x| (8 significant bits)."""

    ax = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def assert_bf16_out_close(got, ref, atol: float = 2e-2) -> None:
    """The bf16 output bar: |got - ref| <= 2e-2, or two bf16 ulps of the
    value where those are larger. A gated-norm output passes through three
    bf16 roundings (y, the normalised value, the gated product), so a
    one-ulp flip of y, which a different float32 summation order produces
    near a rounding boundary, moves the output by up to two of its ulps;
    from |value| >= 2.56 an ulp is >= 2^-6 and two exceed 2e-2."""

    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    tol = np.maximum(atol, 2 * bf16_ulp(ref))
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} values outside max(2e-2, 2 ulp); "
                           f"worst {err.max():.3g} at |ref| {np.abs(ref).flat[err.argmax()]:.3g}")


def assert_within_bf16_ulps(got, ref, ulps: int = 1) -> None:
    """|got - ref| <= `ulps` bf16 ulps of the larger magnitude: values that
    the two sides round to bf16 from float32 and float64 arithmetic, where a
    value within a float32 ulp of a tie may go either way."""

    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    tol = ulps * bf16_ulp(np.maximum(np.abs(got), np.abs(ref)))
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} values beyond {ulps} bf16 ulp; "
                           f"worst {err.max():.3g} at |ref| {np.abs(ref).flat[err.argmax()]:.3g}")


def device_halves(half, arrivals):
    """The conv halves a decode step reads from a pool's bits and arrival
    counters: the bit XOR bit 16 of the counter."""
    return (half ^ (arrivals >> 16)) & 1


def counters_settled(arrivals) -> bool:
    """Between steps the counters' bits below 16 are zero (every workgroup
    of every step added its share)."""
    return not bool((arrivals & 0xFFFF).any())
