"""GPU parity of the fused decode kernel, the prefill front-end and the
gated RMSNorm against the oracle (seeded inputs, production head shape)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from oracle import cref
from oracle import gated_delta_ref as R
from tests.helpers import (assert_bf16_out_close, assert_within_bf16_ulps, layer_inputs,
                           layer_params, max_rel)

pytestmark = pytest.mark.gpu

DIMS_PROD = gdn.LinearAttentionDims(16, 32, 128, 128, 4)


def _dims_tuple(d):
    return (d.num_key_heads, d.num_value_heads, d.key_head_dim, d.value_head_dim)


def _t(x, dev, dtype=torch.float32):
    return torch.tensor(np.asarray(x, np.float32), device=dev).to(dtype)


def _decode_case(seed, dims, B, act_bf16):
    rng = np.random.default_rng(seed)
    dt = _dims_tuple(dims)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, dt)
    qkv, z, a, b = layer_inputs(rng, dt, L=1, act_bf16=act_bf16, B=B)
    conv = rng.standard_normal((B, 3, dims.conv_dim)).astype(np.float32)
    if act_bf16:
        conv = R.bf16_round(conv)
    state = (rng.standard_normal((B,) + (dims.num_value_heads, 128, 128)) * 0.05).astype(np.float32)
    return dict(qkv=qkv[:, 0], z=z[:, 0], a=a[:, 0], b=b[:, 0], conv=conv, state=state,
                conv_w=conv_w, A_log=A_log, dt_bias=dt_bias, norm_w=norm_w)


@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("with_z", [False, True])
def test_fused_decode_matches_oracle(gpu, act, with_z):
    dims = gdn.LinearAttentionDims(2, 4, 128, 128, 4)
    B = 3
    c = _decode_case(0, dims, B, act == "bf16")
    adt = torch.bfloat16 if act == "bf16" else torch.float32
    out, conv_out, state_out = gdn.fused_decode_step(
        _t(c["qkv"], gpu, adt), _t(c["z"], gpu, adt) if with_z else None, _t(c["a"], gpu, adt),
        _t(c["b"], gpu, adt), _t(c["conv"], gpu, adt), _t(c["state"], gpu), _t(c["conv_w"], gpu),
        _t(c["A_log"], gpu), _t(c["dt_bias"], gpu), _t(c["norm_w"], gpu), 1e-6, dims)
    oracle_act = "bf16" if act == "bf16" else None
    for i in range(B):
        ycore = R.linear_attention_core(c["qkv"][i:i + 1], c["z"][i:i + 1], c["a"][i:i + 1],
                                        c["b"][i:i + 1], c["conv"][i], c["state"][i],
                                        c["conv_w"], c["A_log"], c["dt_bias"], c["norm_w"],
                                        _dims_tuple(dims), 1e-6, oracle_act)
        o, nc, ns = ycore
        assert max_rel(state_out[i].cpu().numpy(), ns) < 1e-5
        np.testing.assert_array_equal(conv_out[i].float().cpu().numpy(), nc)
        if with_z and act == "bf16":
            assert_bf16_out_close(out[i].float().cpu().numpy().reshape(-1), o.reshape(-1))
        elif with_z:
            np.testing.assert_allclose(out[i].cpu().numpy().reshape(-1), o.reshape(-1),
                                       rtol=1e-4, atol=1e-4)
    if not with_z:
        # y itself: the recurrence output before the norm
        q, k, v = _frontend_oracle(c, dims, oracle_act)
        g = R.forget_gate(c["a"], c["A_log"], c["dt_bias"])
        beta = R.beta_gate(c["b"], oracle_act)
        for i in range(B):
            y, _ = R.gated_delta_scan_ops(q[i:i + 1], k[i:i + 1], v[i:i + 1], g[i:i + 1],
                                          beta[i:i + 1], c["state"][i])
            np.testing.assert_allclose(out[i].cpu().numpy(), y[0], rtol=1e-4, atol=1e-5)


def _frontend_oracle(c, dims, act):
    Hk, Hv, Dk, Dv = _dims_tuple(dims)
    qs, ks, vs = [], [], []
    for i in range(c["qkv"].shape[0]):
        out, _ = R.convolve(c["qkv"][i:i + 1], c["conv"][i], c["conv_w"], act)
        q = out[:, :Hk * Dk].reshape(1, Hk, Dk)
        k = out[:, Hk * Dk:2 * Hk * Dk].reshape(1, Hk, Dk)
        q, k = R.qk_scale(q, k, act)
        qs.append(q[0])
        ks.append(k[0])
        vs.append(out[0, 2 * Hk * Dk:].reshape(Hv, Dv))
    return np.stack(qs), np.stack(ks), np.stack(vs)


@pytest.mark.parametrize("with_z", [False, True])
def test_fused_decode_production_shape_matches_c_oracle_over_steps(gpu, with_z):
    """B=8 sequences, Hk=16/Hv=32, four chained decode steps with the state
    updated in place (the decode loop's own pattern) against the C oracle."""

    B = 8
    dims = DIMS_PROD
    c = _decode_case(1, dims, B, True)
    adt = torch.bfloat16
    rng = np.random.default_rng(2)
    state_dev = _t(c["state"], gpu)
    conv_dev = _t(c["conv"], gpu, adt)
    conv_spare = torch.empty_like(conv_dev)
    state_ref, conv_ref = c["state"].copy(), c["conv"].copy()
    params = [_t(c[n], gpu) for n in ("conv_w", "A_log", "dt_bias", "norm_w")]
    for step in range(4):
        qkv, z, a, b = layer_inputs(rng, _dims_tuple(dims), L=1, act_bf16=True, B=B)
        out, _, _ = gdn.fused_decode_step(
            _t(qkv[:, 0], gpu, adt), _t(z[:, 0], gpu, adt) if with_z else None,
            _t(a[:, 0], gpu, adt), _t(b[:, 0], gpu, adt), conv_dev, state_dev, *params, 1e-6,
            dims, conv_out=conv_spare, state_out=state_dev)
        conv_dev, conv_spare = conv_spare, conv_dev
        out_ref, conv_ref, state_ref = cref.decode_step(
            qkv[:, 0], conv_ref, c["conv_w"], a[:, 0], b[:, 0], c["A_log"], c["dt_bias"],
            state_ref, z[:, 0] if with_z else None, c["norm_w"], 1e-6, _dims_tuple(dims), True)
        if with_z:
            assert_bf16_out_close(out.float().cpu().numpy(), out_ref)
        else:
            np.testing.assert_allclose(out.cpu().numpy(), out_ref, atol=1e-4, rtol=1e-4)
        np.testing.assert_array_equal(conv_dev.float().cpu().numpy(), conv_ref)
    assert max_rel(state_dev.cpu().numpy(), state_ref) < 1e-4


def test_frontend_matches_oracle_varlen_with_short_runs(gpu):
    dims = gdn.LinearAttentionDims(2, 4, 32, 32, 4)
    rng = np.random.default_rng(4)
    lens = [1, 0, 2, 9, 5]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T, C = int(cu[-1]), dims.conv_dim
    qkv = R.bf16_round(rng.standard_normal((T, C)))
    conv = rng.standard_normal((len(lens), 3, C)).astype(np.float32)  # float32 state in
    w = (rng.standard_normal((C, 4)) * 0.2).astype(np.float32)
    q, k, v, new_conv = gdn.conv_frontend(_t(qkv, gpu, torch.bfloat16), _t(conv, gpu), _t(w, gpu),
                                          dims, torch.tensor(cu, device=gpu))
    assert new_conv.dtype == torch.bfloat16
    for i in range(len(lens)):
        s0, s1 = cu[i], cu[i + 1]
        out, nc = R.convolve(qkv[s0:s1], conv[i], w, "bf16")
        np.testing.assert_array_equal(new_conv[i].float().cpu().numpy(), nc)
        if s1 == s0:
            continue
        qe = out[:, :64].reshape(-1, 2, 32)
        ke = out[:, 64:128].reshape(-1, 2, 32)
        qe, ke = R.qk_scale(qe, ke, "bf16")
        np.testing.assert_allclose(q[s0:s1].float().cpu().numpy(), qe, atol=2e-3, rtol=1e-2)
        np.testing.assert_allclose(k[s0:s1].float().cpu().numpy(), ke, atol=2e-3, rtol=1e-2)
        # fp32 vs fp64 arithmetic may move the conv sum across a bf16 rounding
        # boundary; SiLU of the neighbouring value lands up to two ulps away
        assert_within_bf16_ulps(v[s0:s1].float().cpu().numpy(), out[:, 128:].reshape(-1, 4, 32), 2)


def _frontend_vs_oracle(gpu, dims, qkv, conv, w, cu, conv_dev_dtype, pass_cu=True):
    Hk, Hv, Dk = dims.num_key_heads, dims.num_value_heads, dims.key_head_dim
    q, k, v, new_conv = gdn.conv_frontend(_t(qkv, gpu, torch.bfloat16), _t(conv, gpu, conv_dev_dtype),
                                          _t(w, gpu), dims,
                                          torch.tensor(cu, device=gpu) if pass_cu else None)
    assert new_conv.dtype == torch.bfloat16
    qkd = Hk * Dk
    for i in range(len(cu) - 1):
        s0, s1 = cu[i], cu[i + 1]
        out, nc = R.convolve(qkv[s0:s1], conv[i], w, "bf16")
        np.testing.assert_array_equal(new_conv[i].float().cpu().numpy(), nc)
        if s1 == s0:
            continue
        qe, ke = R.qk_scale(out[:, :qkd].reshape(-1, Hk, Dk), out[:, qkd:2 * qkd].reshape(-1, Hk, Dk),
                            "bf16")
        np.testing.assert_allclose(q[s0:s1].float().cpu().numpy(), qe, atol=2e-3, rtol=1e-2)
        np.testing.assert_allclose(k[s0:s1].float().cpu().numpy(), ke, atol=2e-3, rtol=1e-2)
        assert_within_bf16_ulps(v[s0:s1].float().cpu().numpy(), out[:, 2 * qkd:].reshape(-1, Hv, 128), 2)


def test_frontend_every_bf16_value_silu_and_qk_scaling(gpu):
    """Every finite bf16 value through the tiled front-end: conv weights
    (0, 0, 0, 1) make the conv the identity, so the 4096 v channels of 16
    tokens carry all 65 280 finite bf16 values, and the q and k channels the
    same values again. SiLU (the float32 sequence every kernel shares) is
    within one bf16 ulp of silu(x) in float64 rounded once, equal in all but
    a few near a rounding boundary — except below about -88.7, where e^-x
    overflows float32 and the result is -0 for exact values under 2e-37 in
    magnitude. The q/k scaling of those SiLU values (the kernel's own v;
    rms_norm8, which the decode step shares) is within one bf16 ulp of the
    exact value rounded once for every row inside float32's range, and
    equal to it for all but a few of the rows its eps does not dominate."""

    dims = DIMS_PROD
    vals = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    vals = vals[np.isfinite(vals)]
    per_tok = dims.num_value_heads * 128
    T = -(-vals.size // per_tok)
    vv = np.zeros(T * per_tok, np.float32)
    vv[:vals.size] = vals
    vv = vv.reshape(T, per_tok)
    qkv = np.concatenate([vv, vv], axis=1)  # q | k (2 x 2048) and v (4096) the same values
    w = np.zeros((dims.conv_dim, 4), np.float32)
    w[:, 3] = 1.0
    conv = np.zeros((1, 3, dims.conv_dim), np.float32)
    q, k, v, _ = gdn.conv_frontend(_t(qkv, gpu, torch.bfloat16), _t(conv, gpu, torch.bfloat16), _t(w, gpu),
                                   dims)
    got_v = v.float().cpu().numpy().reshape(T, per_tok)
    exact = R.bf16_round(R.silu(vv.astype(np.float64)))
    tiny = (vv < -88.7) & (np.abs(exact) < 2e-37)
    assert (got_v[tiny] == 0).all()
    assert_within_bf16_ulps(got_v[~tiny], exact[~tiny], 1)
    assert (got_v[~tiny] != exact[~tiny]).sum() <= 16, int((got_v[~tiny] != exact[~tiny]).sum())
    half = dims.num_key_heads * 128
    pre_q = got_v[:, :half].reshape(T, -1, 128).astype(np.float64)
    pre_k = got_v[:, half:].reshape(T, -1, 128).astype(np.float64)
    with np.errstate(over="ignore"):
        qe, ke = R.qk_scale(pre_q, pre_k, "bf16")
    checked = 0
    for got, ref, pre in ((q, qe, pre_q), (k, ke, pre_k)):
        got = got.float().cpu().numpy()
        amax = np.abs(pre).max(axis=-1, keepdims=True)
        ms = (pre * pre).mean(axis=-1, keepdims=True)
        in_range = np.broadcast_to((amax < 1e18) & ((amax > 1e-18) | (amax == 0)), got.shape)
        assert_within_bf16_ulps(got[in_range], ref[in_range], 1)
        norm_rows = np.broadcast_to((amax < 1e18) & (ms > 1e-6 * 2.0 ** -20), got.shape)
        checked += int(norm_rows.sum())
        assert (got[norm_rows] != ref[norm_rows]).mean() < 1e-3
    assert checked > 10_000


@pytest.mark.parametrize("Hk,Hv", [(16, 32), (3, 6), (1, 1)])
def test_frontend_production_heads_ragged_runs_match_oracle(gpu, Hk, Hv):
    """The tiled front-end (128-wide heads, 4 taps, bf16): runs that are
    empty, shorter than the conv window, or cross the 16-token tiles, a
    float32 conv state in, and a partial last tile. Three key heads put k
    and v heads in one wave (the v lanes skip the norm); one of each leaves
    a wave's fourth group of lanes idle."""

    dims = gdn.LinearAttentionDims(Hk, Hv, 128, 128, 4)
    rng = np.random.default_rng(8 + Hk)
    lens = [0, 1, 2, 3, 16, 0, 37, 5, 70, 1]  # 135 tokens
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T, C = int(cu[-1]), dims.conv_dim
    qkv = R.bf16_round(rng.standard_normal((T, C)))
    conv = rng.standard_normal((len(lens), 3, C)).astype(np.float32)
    w = (rng.standard_normal((C, 4)) * 0.2).astype(np.float32)
    _frontend_vs_oracle(gpu, dims, qkv, conv, w, cu, torch.float32)


@pytest.mark.parametrize("dims", [gdn.LinearAttentionDims(2, 4, 32, 32, 4), DIMS_PROD])
def test_frontend_reads_qkv_as_a_column_view(gpu, dims):
    """qkv as the first columns of a stacked projection output, read with
    its row stride (general kernel for 32-wide heads, tiled for 128): bit
    for bit the packed qkv, with packed runs and a float32 conv state."""

    rng = np.random.default_rng(13)
    C = dims.conv_dim
    cu = torch.tensor([0, 5, 5, 40, 77], dtype=torch.int32, device=gpu)
    stacked = _t(R.bf16_round(rng.standard_normal((77, C + 40))), gpu, torch.bfloat16)
    qkv = stacked[:, :C]
    conv = _t(rng.standard_normal((4, 3, C)), gpu)
    w = _t(rng.standard_normal((C, 4)) * 0.2, gpu)
    a = gdn.conv_frontend(qkv, conv, w, dims, cu)
    b = gdn.conv_frontend(qkv.contiguous(), conv, w, dims, cu)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_frontend_writes_a_given_conv_out(gpu):
    rng = np.random.default_rng(10)
    C = DIMS_PROD.conv_dim
    qkv = _t(R.bf16_round(rng.standard_normal((40, C))), gpu, torch.bfloat16)
    conv = _t(rng.standard_normal((1, 3, C)), gpu, torch.bfloat16)
    w = _t(rng.standard_normal((C, 4)) * 0.2, gpu)
    q1, k1, v1, c1 = gdn.conv_frontend(qkv, conv, w, DIMS_PROD)
    out = torch.empty_like(c1)
    q2, k2, v2, c2 = gdn.conv_frontend(qkv, conv, w, DIMS_PROD, conv_out=out)
    assert c2 is out and torch.equal(c2, c1) and torch.equal(q2, q1) and torch.equal(v2, v1)
    with pytest.raises(ValueError, match="overlap"):
        gdn.conv_frontend(qkv, conv, w, DIMS_PROD, conv_out=conv)


@pytest.mark.parametrize("N,L", [(3, 45), (1, 2100), (2, 2050)])
def test_frontend_production_heads_equal_runs_match_oracle(gpu, N, L):
    """N equal runs without cu_seqlens (the batched layer), bf16 conv state;
    the token counts take the 4-, 8- and 16-token tiles (partial last tile)."""

    rng = np.random.default_rng(9 + L)
    cu = (np.arange(N + 1) * L).astype(np.int32)
    C = DIMS_PROD.conv_dim
    qkv = R.bf16_round(rng.standard_normal((N * L, C)))
    conv = R.bf16_round(rng.standard_normal((N, 3, C)))
    w = (rng.standard_normal((C, 4)) * 0.2).astype(np.float32)
    _frontend_vs_oracle(gpu, DIMS_PROD, qkv, conv, w, cu, torch.bfloat16, pass_cu=False)


@pytest.mark.parametrize("D,rows,x_dtype", [(128, 21, torch.float32), (128, 21, torch.bfloat16),
                                            (64, 13, torch.float32), (256, 7, torch.bfloat16)])
@pytest.mark.parametrize("misaligned", [False, True])
def test_gated_rms_norm_row_shapes_match_oracle(gpu, D, rows, x_dtype, misaligned):
    """bf16 gate and result: 16-byte rows take the vectorised kernel (8
    elements a lane, several rows a wave, the last wave part empty), a
    misaligned x the general one; both as the oracle."""

    rng = np.random.default_rng(D + rows)
    y = rng.standard_normal((rows, D)).astype(np.float32)
    if x_dtype == torch.bfloat16:
        y = R.bf16_round(y).astype(np.float32)
    z = R.bf16_round(rng.standard_normal((rows, D)))
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    x = _t(y, gpu, x_dtype)
    if misaligned:
        buf = torch.empty(rows * D + 1, dtype=x_dtype, device=gpu)
        buf[1:] = x.reshape(-1)
        x = buf[1:].view(rows, D)
    out = gdn.gated_rms_norm(x, _t(z, gpu, torch.bfloat16), _t(w, gpu), 1e-6, out_dtype=torch.bfloat16)
    expected = R.gated_rms_norm(R.act_round(y, "bf16"), z, w, 1e-6, "bf16")
    assert_bf16_out_close(out.float().cpu().numpy(), expected)


@pytest.mark.parametrize("zdt", [torch.bfloat16, torch.float32])
def test_gated_rms_norm_reads_a_column_view_of_z(gpu, zdt):
    """z as the (T, H, D) column view of a stacked projection output, read
    in place (bf16: the vectorised kernel; float32: the general one): bit
    for bit the packed z."""

    rng = np.random.default_rng(12)
    T, H, D = 37, 4, 128
    y = _t(rng.standard_normal((T, H, D)), gpu, torch.bfloat16)
    stacked = _t(R.bf16_round(rng.standard_normal((T, 8 + H * D + 24))), gpu, zdt)
    z = stacked[:, 8:8 + H * D].reshape(T, H, D)
    assert not z.is_contiguous() and z.stride() == (8 + H * D + 24, D, 1)
    w = _t(rng.uniform(0.5, 1.5, D), gpu)
    a = gdn.gated_rms_norm(y, z, w, 1e-6, out_dtype=torch.bfloat16)
    b = gdn.gated_rms_norm(y, z.contiguous(), w, 1e-6, out_dtype=torch.bfloat16)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_rms_norm_matches_oracle(gpu, dtype):
    rng = np.random.default_rng(6)
    y = rng.standard_normal((5, 4, 128)).astype(np.float32)
    z = R.bf16_round(rng.standard_normal((5, 4, 128)))
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    out = gdn.gated_rms_norm(_t(y, gpu), _t(z, gpu, dtype), _t(w, gpu), 1e-6, out_dtype=dtype)
    act = "bf16" if dtype == torch.bfloat16 else None
    expected = R.gated_rms_norm(R.act_round(y, act), z, w, 1e-6, act)
    assert out.dtype == dtype
    if act:
        assert_bf16_out_close(out.float().cpu().numpy(), expected)
    else:
        np.testing.assert_allclose(out.cpu().numpy(), expected, atol=1e-5, rtol=1e-5)
