"""GPU parity of the chunked MFMA prefill against the sequential recurrence.

Tolerances are the ones the path is specified to: outputs within 2e-2
max-abs (bf16 inputs) and the final state within 1e-3 relative (max-abs error
over max-abs value) of the float64 / float32 sequential oracle on identical
inputs; against this library's own sequential GPU scan on the same device
inputs the agreement is tighter (1e-4 relative state)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from mlx_lean_moe_amd import gated_delta
from oracle import cref
from oracle import gated_delta_ref as R
from tests.helpers import max_rel

pytestmark = pytest.mark.gpu

Y_ATOL = 2e-2
STATE_REL = 1e-3


def _cfg_inputs(seed, T, Hk, Hv, d=128, state_scale=0.0, N=1):
    """Seeded inputs of the chunked-prefill workload: q, k, v bf16 ~N(0,1)
    with q/k L2-normalised (q also / sqrt(d)); a, b bf16 ~N(0,1);
    A_log ~U(0, ln 16), dt_bias ~U(-1, 1); state ~N(0, scale)."""

    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, Hk, d))
    k = rng.standard_normal((T, Hk, d))
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * d ** 0.5
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q, k = R.bf16_round(q), R.bf16_round(k)
    v = R.bf16_round(rng.standard_normal((T, Hv, d)))
    a = R.bf16_round(rng.standard_normal((T, Hv)))
    b = R.bf16_round(rng.standard_normal((T, Hv)))
    A_log = rng.uniform(0, np.log(16), Hv).astype(np.float32)
    dt_bias = rng.uniform(-1, 1, Hv).astype(np.float32)
    state = (rng.standard_normal((N, Hv, d, d)) * state_scale).astype(np.float32)
    return q, k, v, a, b, A_log, dt_bias, state


def _dev(gpu, arrays, bf16_names=("q", "k", "v", "a", "b")):
    names = ("q", "k", "v", "a", "b", "A_log", "dt_bias", "state")
    out = {}
    for n, x in zip(names, arrays):
        t = torch.tensor(np.asarray(x, np.float32), device=gpu)
        out[n] = t.to(torch.bfloat16) if n in bf16_names else t
    return out


def _prefill(t, cu=None, y_dtype=torch.float32, zero_state=False):
    """Direct launch of the chunked prefill (gate_mode 0), whatever the run
    lengths; ``zero_state`` passes a null initial-state pointer."""

    q, k, v = t["q"], t["k"], t["v"]
    T, Hk, D = q.shape
    Hv = v.shape[1]
    N = t["state"].shape[0]
    dev = q.device
    y = torch.empty(T, Hv, D, dtype=y_dtype, device=dev)
    s_out = torch.empty_like(t["state"])
    cu_dev = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=dev)
    gated_delta._launch_prefill(q, k, v, t["a"], t["b"], t["A_log"], t["dt_bias"], 0,
                                None if zero_state else t["state"], s_out, y, cu_dev, N, T, Hk,
                                Hv, D, D, dev)
    return y, s_out


def _oracle(arrays, cu=None):
    q, k, v, a, b, A_log, dt_bias, state = arrays
    if cu is None:
        y, s = R.gated_delta_update(q[None], k[None], v[None], a[None], b[None], A_log, dt_bias,
                                    state, act="bf16")
        return y[0], s
    return R.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, cu_seqlens=cu, act="bf16")


@pytest.mark.parametrize("T", [64, 130, 200])
def test_prefill_matches_sequential_oracle(gpu, T):
    arrays = _cfg_inputs(0, T, Hk=2, Hv=4, state_scale=0.05)
    t = _dev(gpu, arrays)
    y, s = _prefill(t)
    ye, se = _oracle(arrays)
    assert np.abs(y.cpu().numpy() - ye).max() < Y_ATOL
    assert max_rel(y.cpu().numpy(), ye) < 1e-3
    assert max_rel(s.cpu().numpy(), se) < STATE_REL


def test_prefill_wide_gqa_group(gpu):
    # 12 value heads on one key head (more than the production 2:1 grouping)
    arrays = _cfg_inputs(6, 130, Hk=1, Hv=12, state_scale=0.05)
    t = _dev(gpu, arrays)
    y, s = _prefill(t)
    ye, se = _oracle(arrays)
    assert np.abs(y.cpu().numpy() - ye).max() < Y_ATOL
    assert max_rel(s.cpu().numpy(), se) < STATE_REL


def test_prefill_exact_zero_and_unit_gates(gpu):
    """Gates of exactly 0 (a state reset: log-gate clamped at -80) and exactly
    1 (no decay) mid-sequence, through gated_delta_scan's chunked path (fp32
    g and beta, bf16 q/k/v), against the float64 recurrence."""

    T, Hk, Hv, D = 200, 2, 4, 128
    q, k, v, g, beta, s0 = R.metal_test_inputs(T, key_dim=D, value_dim=D, key_heads=Hk,
                                               value_heads=Hv)
    q, k, v = (R.bf16_round(x) for x in (q, k, v))
    g = g.copy()
    g[70, 1] = 0.0
    g[130:140, :] = 0.0
    g[10:40, 2] = 1.0
    g[150:, 3] = 1.0
    dev = lambda x, dt=torch.float32: torch.tensor(x, device=gpu).to(dt)
    y, s = gdn.gated_delta_scan(dev(q, torch.bfloat16), dev(k, torch.bfloat16),
                                dev(v, torch.bfloat16), dev(g), dev(beta), dev(s0))
    ye, se = R.gated_delta_scan(q, k, v, g, beta, s0)
    assert np.abs(y.cpu().numpy() - ye).max() < Y_ATOL
    assert max_rel(y.cpu().numpy(), ye) < 1e-3
    assert max_rel(s.cpu().numpy(), se) < STATE_REL


def test_prefill_many_short_runs(gpu):
    # 64 packed runs of 1..100 tokens: chunk bookkeeping across many runs
    lens = np.random.default_rng(11).integers(1, 101, 64)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    arrays = _cfg_inputs(12, T, Hk=2, Hv=4, state_scale=0.05, N=len(lens))
    t = _dev(gpu, arrays)
    y, s = _prefill(t, cu=cu)
    ye, se = _oracle(arrays, cu=cu)
    assert np.abs(y.cpu().numpy() - ye).max() < Y_ATOL
    for i in range(len(lens)):
        assert max_rel(s[i].cpu().numpy(), se[i]) < STATE_REL, i


def test_prefill_matches_gpu_sequential_scan_slow_decay(gpu):
    # the reference scan test's decay regime (g in [0.98, 1], beta in [0, 1]):
    # long memory, the hardest case for the chunked state update
    T, Hk, Hv, D = 300, 2, 4, 128
    q, k, v, g, beta, s0 = R.metal_test_inputs(T, key_dim=D, value_dim=D, key_heads=Hk,
                                               value_heads=Hv)
    q, k, v = (R.bf16_round(x) for x in (q, k, v))
    dev = lambda x, dt=torch.float32: torch.tensor(x, device=gpu).to(dt)
    args = [dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16), dev(g),
            dev(beta), dev(s0)]
    y_chunk, s_chunk = gdn.gated_delta_scan(*args)  # bf16, L >= 64: chunked prefill
    y_seq, s_seq = gdn.gated_delta_scan(*args, use_kernel=False)
    ye, se = R.gated_delta_scan(q, k, v, g, beta, s0)
    assert max_rel(s_chunk.cpu().numpy(), se) < STATE_REL
    assert max_rel(s_chunk.cpu().numpy(), s_seq.cpu().numpy()) < STATE_REL
    assert np.abs(y_chunk.cpu().numpy() - ye).max() < Y_ATOL


def test_prefill_is_dispatched_for_long_bf16_runs(gpu, monkeypatch):
    arrays = _cfg_inputs(1, 128, Hk=2, Hv=4)
    t = _dev(gpu, arrays)
    seen = []
    real = gated_delta._lib.call
    monkeypatch.setattr(gated_delta._lib, "call", lambda name, *a: (seen.append(name), real(name, *a))[1])
    gdn.gated_delta_update(t["q"][None], t["k"][None], t["v"][None], t["a"][None], t["b"][None],
                           t["A_log"], t["dt_bias"], t["state"])
    assert seen == ["gdn_prefill_chunked"]


def test_prefill_varlen_with_ragged_and_empty_runs(gpu):
    lens = [64, 1, 0, 200, 63, 65, 129]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    arrays = _cfg_inputs(2, T, Hk=2, Hv=4, state_scale=0.05, N=len(lens))
    t = _dev(gpu, arrays)
    y, s = _prefill(t, cu=cu)
    ye, se = _oracle(arrays, cu=cu)
    assert np.abs(y.cpu().numpy() - ye).max() < Y_ATOL
    for i in range(len(lens)):
        assert max_rel(s[i].cpu().numpy(), se[i]) < STATE_REL, i
    np.testing.assert_array_equal(s[2].cpu().numpy(), arrays[-1][2])  # empty run


def test_prefill_split_carry_equals_one_call(gpu):
    arrays = _cfg_inputs(4, 256, Hk=2, Hv=4, state_scale=0.05)
    t = _dev(gpu, arrays)
    y, s = _prefill(t)
    first = {n: (x[:100] if n not in ("A_log", "dt_bias", "state") else x) for n, x in t.items()}
    y1, s1 = _prefill(first)
    second = {n: (x[100:] if n not in ("A_log", "dt_bias", "state") else x) for n, x in t.items()}
    second["state"] = s1
    y2, s2 = _prefill(second)
    assert np.abs(torch.cat([y1, y2]).cpu().numpy() - y.cpu().numpy()).max() < 1e-3
    assert max_rel(s2.cpu().numpy(), s.cpu().numpy()) < 1e-4


def test_prefill_sequential_reference_config(gpu):
    """B=1, T=128, Hk=16, Hv=32, d=128, zero state, seed 0 (the sequential
    reference configuration) against the float64 oracle."""

    arrays = _cfg_inputs(0, 128, Hk=16, Hv=32)
    t = _dev(gpu, arrays)
    y, s = gdn.gated_delta_update(t["q"][None], t["k"][None], t["v"][None], t["a"][None],
                                  t["b"][None], t["A_log"], t["dt_bias"], t["state"])
    ye, se = _oracle(arrays)
    assert np.abs(y[0].cpu().numpy() - ye).max() < Y_ATOL
    assert max_rel(s.cpu().numpy(), se) < STATE_REL


def test_prefill_full_size_against_c_oracle(gpu):
    """T=4096, Hk=16, Hv=32, chunk 64, zero initial state: output and final
    state against the token-by-token recurrence (C oracle, float32)."""

    T, Hk, Hv = 4096, 16, 32
    arrays = _cfg_inputs(0, T, Hk=Hk, Hv=Hv)
    q, k, v, a, b, A_log, dt_bias, state = arrays
    t = _dev(gpu, arrays)
    y, s = gdn.gated_delta_update(t["q"][None], t["k"][None], t["v"][None], t["a"][None],
                                  t["b"][None], t["A_log"], t["dt_bias"], t["state"])
    g = R.forget_gate(a, A_log, dt_bias).astype(np.float32)
    beta = R.beta_gate(b, "bf16").astype(np.float32)
    ye, se = cref.scan(q[None], k[None], v[None], g[None], beta[None], state)
    assert np.abs(y.cpu().numpy() - ye).max() < Y_ATOL
    assert max_rel(y.cpu().numpy(), ye) < 1e-3
    assert max_rel(s.cpu().numpy(), se) < STATE_REL
    # and against this library's sequential scan on the same device inputs
    y2, s2 = gdn.gated_delta_update(t["q"][None], t["k"][None], t["v"][None], t["a"][None],
                                    t["b"][None], t["A_log"], t["dt_bias"], t["state"],
                                    use_kernel=False)
    assert max_rel(s.cpu().numpy(), s2.cpu().numpy()) < 1e-4


@pytest.mark.parametrize("packed", [False, True])
def test_gates_as_column_slices_of_one_projection(gpu, packed):
    """a and b as column views of one (T, 2 Hv) projection output (the
    layer's a||b block): the chunked prefill reads them with their row
    stride, bit for bit the packed call; the scan path packs them."""

    T, Hv = 200, 4
    arrays = _cfg_inputs(9, T, Hk=2, Hv=Hv)
    t = _dev(gpu, arrays)
    ab = torch.cat([t["a"], t["b"]], dim=-1)
    a, b = ab[:, :Hv], ab[:, Hv:]
    assert a.stride() == (2 * Hv, 1)
    if packed:
        cu = [0, 70, 70, 200]
        state = torch.zeros(3, Hv, 128, 128, device=gpu)
        run = lambda a_, b_: gdn.gated_delta_update(t["q"], t["k"], t["v"], a_, b_, t["A_log"],
                                                    t["dt_bias"], state, cu_seqlens=cu)
    else:
        run = lambda a_, b_: gdn.gated_delta_update(t["q"][None], t["k"][None], t["v"][None],
                                                    a_[None], b_[None], t["A_log"], t["dt_bias"],
                                                    t["state"])
    y1, s1 = run(a, b)
    y2, s2 = run(a.contiguous(), b.contiguous())
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
    # the scan path (runs under 64 tokens) with the same views
    y3, s3 = gdn.gated_delta_update(t["q"][None, :20], t["k"][None, :20], t["v"][None, :20],
                                    a[None, :20], b[None, :20], t["A_log"], t["dt_bias"], t["state"])
    y4, s4 = gdn.gated_delta_update(t["q"][None, :20], t["k"][None, :20], t["v"][None, :20],
                                    a[None, :20].contiguous(), b[None, :20].contiguous(), t["A_log"],
                                    t["dt_bias"], t["state"])
    assert torch.equal(y3, y4) and torch.equal(s3, s4)


@pytest.mark.parametrize("T", [96, 20])  # the chunked kernel; the sequential scan
def test_update_y_dtype_is_the_rounded_float32_output(gpu, T):
    """gated_delta_update(..., y_dtype=bf16) gives y.to(bf16) bit for bit
    (what the layer's norm reads), the state unchanged."""

    arrays = _cfg_inputs(7, T, Hk=2, Hv=4)
    t = _dev(gpu, arrays)
    args = (t["q"][None], t["k"][None], t["v"][None], t["a"][None], t["b"][None], t["A_log"],
            t["dt_bias"], t["state"])
    y32, s32 = gdn.gated_delta_update(*args)
    y16, s16 = gdn.gated_delta_update(*args, y_dtype=torch.bfloat16)
    assert y32.dtype == torch.float32 and y16.dtype == torch.bfloat16
    assert torch.equal(y16, y32.to(torch.bfloat16))
    assert torch.equal(s16, s32)
    with pytest.raises(ValueError, match="y_dtype"):
        gdn.gated_delta_update(*args, y_dtype=torch.int32)


@pytest.mark.parametrize("T", [96, 20])
def test_update_writes_a_given_state_out(gpu, T):
    arrays = _cfg_inputs(11, T, Hk=2, Hv=4, state_scale=0.05)
    t = _dev(gpu, arrays)
    args = (t["q"][None], t["k"][None], t["v"][None], t["a"][None], t["b"][None], t["A_log"],
            t["dt_bias"], t["state"])
    y1, s1 = gdn.gated_delta_update(*args)
    out = torch.full_like(s1, float("nan"))
    y2, s2 = gdn.gated_delta_update(*args, state_out=out)
    assert s2 is out and torch.equal(s2, s1) and torch.equal(y2, y1)
    with pytest.raises(ValueError, match="overlap"):
        gdn.gated_delta_update(*args, state_out=t["state"])
    with pytest.raises(ValueError, match="state_out"):
        gdn.gated_delta_update(*args, state_out=out[..., :64])


def test_prefill_bf16_output_and_zero_state_pointer(gpu):
    arrays = _cfg_inputs(5, 96, Hk=2, Hv=4)  # zero initial state
    t = _dev(gpu, arrays)
    y32, s32 = _prefill(t)
    y16, s16 = _prefill(t, y_dtype=torch.bfloat16, zero_state=True)
    assert y16.dtype == torch.bfloat16
    np.testing.assert_array_equal(y16.float().cpu().numpy(), R.bf16_round(y32.cpu().numpy()))
    torch.testing.assert_close(s16, s32, rtol=0, atol=0)


def _f32_inputs(seed, T, Hk, Hv, d=128, state_scale=0.0, N=1):
    """The workload's inputs in float32, as the reference's layers carry
    activations: q/k L2-normalised (q also / sqrt(d)) but not bf16-rounded;
    v, a, b ~N(0, 1)."""

    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, Hk, d))
    k = rng.standard_normal((T, Hk, d))
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * d ** 0.5
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    f = lambda x: np.asarray(x, np.float32)
    v, a, b = rng.standard_normal((T, Hv, d)), rng.standard_normal((T, Hv)), rng.standard_normal((T, Hv))
    A_log = rng.uniform(0, np.log(16), Hv).astype(np.float32)
    dt_bias = rng.uniform(-1, 1, Hv).astype(np.float32)
    state = (rng.standard_normal((N, Hv, d, d)) * state_scale).astype(np.float32)
    return f(q), f(k), f(v), f(a), f(b), A_log, dt_bias, state


@pytest.mark.parametrize("lens", [[64], [200], [3, 63, 130, 0, 65, 130]])
def test_prefill_float32_inputs_match_float64_oracle(gpu, lens):
    """float32 q, k, v, a, b (the reference's activation dtype, not
    representable in bf16) take the chunked prefill, each value split into
    a bf16 high part and residual: y and state within 1e-4 relative of the
    float64 recurrence, with nonzero initial states and ragged packed runs."""

    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, N = int(cu[-1]), len(lens)
    arrays = _f32_inputs(20 + T, T, Hk=2, Hv=4, state_scale=0.05, N=N)
    t = _dev(gpu, arrays, bf16_names=())
    assert gated_delta._prefill_eligible(t["q"], t["k"], t["v"], 64)
    calls = []
    real = gated_delta._lib.call
    gated_delta._lib.call = lambda name, *a: (calls.append(name), real(name, *a))[1]
    try:
        y, s = gdn.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"],
                                      t["dt_bias"], t["state"], cu_seqlens=cu)
    finally:
        gated_delta._lib.call = real
    assert "gdn_prefill_chunked" in calls and y.dtype == torch.float32
    q, k, v, a, b, A_log, dt_bias, state = arrays
    ye, se = R.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, cu_seqlens=cu)
    assert max_rel(y.cpu().numpy(), ye) < 1e-4
    assert max_rel(s.cpu().numpy(), se) < 1e-4


@pytest.mark.parametrize("Hk,Hv", [(2, 6), (1, 4), (3, 3)])
def test_prefill_float32_head_groups(gpu, Hk, Hv):
    """float32 input with three, four and one value heads per key head: the
    chunk pass takes two value heads of a key head per workgroup where their
    count is even (one or two such pairs here) and one otherwise; y and state
    within 1e-4 relative of the float64 recurrence over ragged packed runs."""

    lens = [130, 0, 65, 7, 200]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, N = int(cu[-1]), len(lens)
    arrays = _f32_inputs(40 + Hk * Hv, T, Hk=Hk, Hv=Hv, state_scale=0.05, N=N)
    t = _dev(gpu, arrays, bf16_names=())
    calls = []
    real = gated_delta._lib.call
    gated_delta._lib.call = lambda name, *a: (calls.append(name), real(name, *a))[1]
    try:
        y, s = gdn.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"],
                                      t["dt_bias"], t["state"], cu_seqlens=cu)
    finally:
        gated_delta._lib.call = real
    assert "gdn_prefill_chunked" in calls
    q, k, v, a, b, A_log, dt_bias, state = arrays
    ye, se = R.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, cu_seqlens=cu)
    assert max_rel(y.cpu().numpy(), ye) < 1e-4
    assert max_rel(s.cpu().numpy(), se) < 1e-4


def test_prefill_float32_full_size_against_c_oracle(gpu):
    """T=4096, Hk=16, Hv=32, float32 inputs, zero initial state: y and final
    state within 1e-3 relative of the float32 token-by-token recurrence (C
    oracle); and within 1e-4 of this library's sequential scan."""

    T, Hk, Hv = 4096, 16, 32
    arrays = _f32_inputs(1, T, Hk=Hk, Hv=Hv)
    q, k, v, a, b, A_log, dt_bias, state = arrays
    t = _dev(gpu, arrays, bf16_names=())
    y, s = gdn.gated_delta_update(t["q"][None], t["k"][None], t["v"][None], t["a"][None],
                                  t["b"][None], t["A_log"], t["dt_bias"], t["state"])
    g = R.forget_gate(a, A_log, dt_bias).astype(np.float32)
    beta = R.beta_gate(b).astype(np.float32)
    ye, se = cref.scan(q[None], k[None], v[None], g[None], beta[None], state)
    assert max_rel(y.cpu().numpy(), ye) < 1e-3
    assert max_rel(s.cpu().numpy(), se) < STATE_REL
    y2, s2 = gdn.gated_delta_update(t["q"][None], t["k"][None], t["v"][None], t["a"][None],
                                    t["b"][None], t["A_log"], t["dt_bias"], t["state"],
                                    use_kernel=False)
    assert max_rel(s.cpu().numpy(), s2.cpu().numpy()) < 1e-4
    assert max_rel(y.cpu().numpy(), y2.cpu().numpy()) < 1e-4
