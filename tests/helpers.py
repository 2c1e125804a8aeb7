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
