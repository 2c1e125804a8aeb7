"""Varlen packed prefill followed by decode continuation, on the GPU against
the oracle: 16 sequences with seeded lengths U[128, 8192] packed through
cu_seqlens, nonzero float32 initial states, then 128 decode steps per
sequence from the returned states; plus a layer-level version (conv
front-end, prefill, fused decode) at small sizes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from oracle import cref
from oracle import gated_delta_ref as R
from tests.helpers import assert_bf16_out_close, layer_inputs, layer_params, max_rel

pytestmark = pytest.mark.gpu

Y_ATOL = 2e-2
STATE_REL = 1e-3


def _tokens(rng, T, Hk, Hv, d=128):
    q = rng.standard_normal((T, Hk, d))
    k = rng.standard_normal((T, Hk, d))
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * d ** 0.5
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, Hv, d))
    a = rng.standard_normal((T, Hv))
    b = rng.standard_normal((T, Hv))
    return [R.bf16_round(x) for x in (q, k, v, a, b)]


def test_varlen_prefill_then_128_decode_steps(gpu):
    Hk, Hv, d = 16, 32, 128
    lens = np.random.default_rng(0).integers(128, 8193, 16)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, N = int(cu[-1]), len(lens)
    rng = np.random.default_rng(1)
    q, k, v, a, b = _tokens(rng, T, Hk, Hv)
    A_log = rng.uniform(0, np.log(16), Hv).astype(np.float32)
    dt_bias = rng.uniform(-1, 1, Hv).astype(np.float32)
    s0 = (rng.standard_normal((N, Hv, d, d)) * 0.05).astype(np.float32)
    bf = lambda x: torch.tensor(x, device=gpu).to(torch.bfloat16)
    f32 = lambda x: torch.tensor(x, device=gpu)

    y, s = gdn.gated_delta_update(bf(q), bf(k), bf(v), bf(a), bf(b), f32(A_log), f32(dt_bias),
                                  f32(s0), cu_seqlens=cu)
    g = R.forget_gate(a, A_log, dt_bias).astype(np.float32)
    beta = R.beta_gate(b, "bf16").astype(np.float32)
    y_np, s_np = y.cpu().numpy(), s.cpu().numpy()
    s_ref = np.empty_like(s0)
    for i in range(N):
        sl = slice(cu[i], cu[i + 1])
        ye, se = cref.scan(q[sl][None], k[sl][None], v[sl][None], g[sl][None], beta[sl][None],
                           s0[i:i + 1])
        assert np.abs(y_np[sl] - ye[0]).max() < Y_ATOL, i
        assert max_rel(y_np[sl], ye[0]) < 1e-3, i
        assert max_rel(s_np[i], se[0]) < STATE_REL, i
        s_ref[i] = se[0]

    # 128 decode steps of all 16 sequences from the returned states
    steps = 128
    qd, kd, vd, ad, bd = _tokens(rng, steps * N, Hk, Hv)
    state_dev, state_ref = s, s_ref
    for t in range(steps):
        sl = slice(t * N, (t + 1) * N)
        yt, state_dev = gdn.gated_delta_update(
            bf(qd[sl])[:, None], bf(kd[sl])[:, None], bf(vd[sl])[:, None], bf(ad[sl])[:, None],
            bf(bd[sl])[:, None], f32(A_log), f32(dt_bias), state_dev)
        gt = R.forget_gate(ad[sl], A_log, dt_bias).astype(np.float32)
        bt = R.beta_gate(bd[sl], "bf16").astype(np.float32)
        ye, state_ref = cref.scan(qd[sl][:, None], kd[sl][:, None], vd[sl][:, None],
                                  gt[:, None], bt[:, None], state_ref)
        if t % 32 == 31 or t == 0:
            assert np.abs(yt.cpu().numpy() - ye).max() < Y_ATOL, t
    for i in range(N):
        assert max_rel(state_dev[i].cpu().numpy(), state_ref[i]) < STATE_REL, i

    # the same continuation as the benchmark runs it: 128 fused decode steps
    # (conv + roll, q/k scaling, gates, recurrence, gated norm) of the 16
    # sequences from the prefill's states, state in place, conv state
    # alternating between two buffers, against the C oracle's decode step
    dims = gdn.LinearAttentionDims(Hk, Hv, d, d, 4)
    conv_w, _, _, norm_w = layer_params(rng, (Hk, Hv, d, d))
    conv_ref = R.bf16_round(rng.standard_normal((N, 3, dims.conv_dim))).astype(np.float32)
    conv_dev, conv_spare = bf(conv_ref), torch.empty(N, 3, dims.conv_dim, dtype=torch.bfloat16,
                                                      device=gpu)
    state_dev, state_ref = s.clone(), s_ref.copy()
    params = [f32(conv_w), f32(A_log), f32(dt_bias), f32(norm_w)]
    for t in range(steps):
        x_qkv, x_z, x_a, x_b = layer_inputs(rng, (Hk, Hv, d, d), L=1, act_bf16=True, B=N)
        out, _, _ = gdn.fused_decode_step(bf(x_qkv[:, 0]), bf(x_z[:, 0]), bf(x_a[:, 0]),
                                          bf(x_b[:, 0]), conv_dev, state_dev, *params, 1e-6, dims,
                                          conv_out=conv_spare, state_out=state_dev)
        conv_dev, conv_spare = conv_spare, conv_dev
        out_ref, conv_ref, state_ref = cref.decode_step(
            x_qkv[:, 0], conv_ref, conv_w, x_a[:, 0], x_b[:, 0], A_log, dt_bias, state_ref,
            x_z[:, 0], norm_w, 1e-6, (Hk, Hv, d, d), True, state_out=state_ref)
        assert_bf16_out_close(out.float().cpu().numpy(), out_ref)
        if t % 32 == 31 or t == 0:
            np.testing.assert_array_equal(conv_dev.float().cpu().numpy(), conv_ref)
    assert max_rel(state_dev.cpu().numpy(), state_ref) < STATE_REL


def test_layer_varlen_prefill_then_fused_decode(gpu):
    """Front-end + prefill for 4 packed prompts (one shorter than the conv
    kernel), then 8 fused decode steps from the returned conv and ssm states,
    against the oracle's layer core run per sequence."""

    dims = gdn.LinearAttentionDims(2, 4, 128, 128, 4)
    dt = (2, 4, 128, 128)
    rng = np.random.default_rng(7)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, dt)
    lens = [70, 2, 130, 64]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, N, C = int(cu[-1]), len(lens), dims.conv_dim
    qkv, z, a, b = layer_inputs(rng, dt, L=T, act_bf16=True)
    conv0 = R.bf16_round(rng.standard_normal((N, 3, C)))
    ssm0 = (rng.standard_normal((N, 4, 128, 128)) * 0.05).astype(np.float32)
    bf = lambda x: torch.tensor(np.asarray(x, np.float32), device=gpu).to(torch.bfloat16)
    f32 = lambda x: torch.tensor(np.asarray(x, np.float32), device=gpu)
    layer = gdn.Qwen3_5LinearAttention(dims, None, None, None, None, f32(conv_w)[:, :, None],
                                       f32(A_log), f32(dt_bias), f32(norm_w), None)
    out, conv, ssm = layer.core(bf(qkv), bf(z), bf(a), bf(b), bf(conv0), f32(ssm0), cu_seqlens=cu)
    conv_ref, ssm_ref = [], []
    for i in range(N):
        sl = slice(cu[i], cu[i + 1])
        o, nc, ns = R.linear_attention_core(qkv[sl], z[sl], a[sl], b[sl], conv0[i], ssm0[i],
                                            conv_w, A_log, dt_bias, norm_w, dt, 1e-6, "bf16")
        assert_bf16_out_close(out[sl].float().cpu().numpy(), o)
        np.testing.assert_array_equal(conv[i].float().cpu().numpy(), nc)
        assert max_rel(ssm[i].cpu().numpy(), ns) < STATE_REL, i
        conv_ref.append(nc)
        ssm_ref.append(ns)

    pool = gdn.RecurrentStatePool(N, 4, C, 4, 128, 128, dtype=torch.bfloat16, device=gpu)
    pool.conv_buf[:N].copy_(conv)  # every slot starts in the first half
    pool.ssm_state.copy_(ssm)
    slots = list(range(N))
    for _ in range(8):
        x_qkv, x_z, x_a, x_b = layer_inputs(rng, dt, L=1, act_bf16=True, B=N)
        o_dev, _, _ = gdn.fused_decode_step(bf(x_qkv[:, 0]), bf(x_z[:, 0]), bf(x_a[:, 0]),
                                            bf(x_b[:, 0]), pool.conv_buf, pool.ssm_state,
                                            layer.conv1d_weight, layer.A_log, layer.dt_bias,
                                            layer.norm_weight, 1e-6, dims, slots=slots,
                                            conv_half=pool.conv_half_dev)
        pool.advance(slots)
        for i in range(N):
            o, conv_ref[i], ssm_ref[i] = R.linear_attention_core(
                x_qkv[i], x_z[i], x_a[i], x_b[i], conv_ref[i], ssm_ref[i], conv_w, A_log,
                dt_bias, norm_w, dt, 1e-6, "bf16")
            assert_bf16_out_close(o_dev[i].float().cpu().numpy().reshape(-1), o.reshape(-1))
    for i in range(N):
        np.testing.assert_array_equal(pool.conv_state[i].float().cpu().numpy(), conv_ref[i])
        assert max_rel(pool.ssm_state[i].cpu().numpy(), ssm_ref[i]) < STATE_REL
