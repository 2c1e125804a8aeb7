"""Bit-level checks of the kernels' storage conversions: a float32 value
stored as bf16 / f16 must round exactly as the oracle's round-to-nearest-even
(ties, denormals, large magnitudes included).

The plain scan kernel with Dk = 1, q = 1, k = 0, g = 1, beta = 0 returns its
input state row as y, so storing y in a 16-bit dtype exercises exactly the
kernels' float32 -> storage conversion."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from oracle.gated_delta_ref import bf16_round, f16_round

pytestmark = pytest.mark.gpu


def _values() -> np.ndarray:
    rng = np.random.default_rng(0)
    one = np.float32(1)
    specials = [0.0, -0.0, one + 2 ** -8, one + 3 * 2 ** -8, one + 2 ** -8 + 2 ** -20,
                -(one + 2 ** -8), 1e-40, -3e-39, 1.1754944e-38, 3.0e38, 65504.0, 6e-5, 1e-7]
    x = np.concatenate([np.array(specials, np.float32),
                        rng.standard_normal(4000).astype(np.float32),
                        (rng.standard_normal(2000) * 1e-30).astype(np.float32),
                        (rng.standard_normal(2000) * 1e4).astype(np.float32)])
    return x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_storage_rounding_matches_oracle(gpu, dtype):
    x = _values()
    if dtype == torch.float16:
        x = x[np.abs(x) < 65504]
    n = x.size
    state = torch.tensor(x, device=gpu).reshape(1, n, 1)
    q = torch.ones(1, 1, 1, device=gpu)
    k = torch.zeros(1, 1, 1, device=gpu)
    v = torch.zeros(1, 1, n, device=gpu)
    g = torch.ones(1, 1, device=gpu)
    beta = torch.zeros(1, 1, device=gpu)
    y = torch.empty(1, 1, n, dtype=dtype, device=gpu)
    out_state = torch.empty_like(state)
    from mlx_lean_moe_amd import gated_delta

    gated_delta._launch_scan("gdn_scan_reference", q, k, v, g, beta, state, out_state, y, None,
                             1, 1, 1, 1, 1, n, gpu)
    got = y.float().cpu().numpy().reshape(-1)
    want = bf16_round(x) if dtype == torch.bfloat16 else f16_round(x)
    np.testing.assert_array_equal(got, want)
    torch.testing.assert_close(out_state, state, rtol=0, atol=0)
