"""GPU tests of the fused prefill (gdn_prefill_fused): the front-end computed
inside the chunked prefill's chunk pass must give the same bits as
gdn_frontend followed by gdn_prefill_chunked (each pinned to the oracle by
the front-end and prefill tests): y, the new conv state and the new ssm
state. Covered: one 4096-token prompt at the production head shape with qkv,
a and b read as column views of one stacked projection output; packed runs
with empty, one- and two-token runs (conv taps from the conv state, the new
conv state partly the old one), a float32 conv state; y in bf16 and float32;
the layer's prompt path, which takes the fused call."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn

pytestmark = pytest.mark.gpu

D = 128


def _case(gpu, seed, T, N, Hk, Hv, conv_dtype=torch.bfloat16):
    g = torch.Generator(device=gpu).manual_seed(seed)
    dims = gdn.LinearAttentionDims(Hk, Hv, D, D, 4)
    C = dims.conv_dim
    randn = lambda *s: torch.randn(*s, generator=g, device=gpu)
    # one stacked projection output: qkv | z | a | b columns, read as views
    width = C + Hv * D + 2 * Hv
    stacked = randn(T, width).to(torch.bfloat16)
    qkv = stacked[:, :C]
    a, b = stacked[:, C + Hv * D:C + Hv * D + Hv], stacked[:, C + Hv * D + Hv:]
    return dict(dims=dims, qkv=qkv, a=a, b=b,
                conv=randn(N, 3, C).to(conv_dtype), ssm=randn(N, Hv, D, D) * 0.05,
                w=randn(C, 4) * 0.2, A_log=torch.rand(Hv, generator=g, device=gpu) * 2.5,
                dt_bias=torch.rand(Hv, generator=g, device=gpu) - 0.5)


def _unfused(c, cu, y_dtype):
    """gdn_frontend's tiled kernel (which the fused pass shares its
    arithmetic with) on a contiguous copy of qkv: the stacked rows of an
    odd head count are not a multiple of 8 elements, which sends the view to
    the general front-end kernel (another summation order)."""

    d = c["dims"]
    q, k, v, conv = gdn.conv_frontend(c["qkv"].contiguous(), c["conv"], c["w"], d, cu)
    if cu is None:
        y, ssm = gdn.gated_delta_update(q[None], k[None], v[None], c["a"][None], c["b"][None],
                                        c["A_log"], c["dt_bias"], c["ssm"], y_dtype=y_dtype)
        y = y[0]
    else:
        y, ssm = gdn.gated_delta_update(q, k, v, c["a"], c["b"], c["A_log"], c["dt_bias"], c["ssm"],
                                        cu_seqlens=cu, y_dtype=y_dtype)
    return y, conv, ssm


@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_fused_prefill_equals_frontend_then_chunked_prefill_t4096(gpu, y_dtype):
    c = _case(gpu, 1, 4096, 1, 16, 32)
    assert gdn.fused_prefill_ok(c["qkv"], c["a"], c["b"], c["conv"], c["ssm"], c["dims"], 1)
    y, conv, ssm = gdn.prefill_fused(c["qkv"], c["a"], c["b"], c["conv"], c["ssm"], c["w"],
                                     c["A_log"], c["dt_bias"], c["dims"], y_dtype=y_dtype)
    y_ref, conv_ref, ssm_ref = _unfused(c, None, y_dtype)
    assert y.dtype == y_dtype and conv.dtype == torch.bfloat16
    assert torch.equal(conv, conv_ref)
    assert torch.equal(y, y_ref)
    assert torch.equal(ssm, ssm_ref)


@pytest.mark.parametrize("conv_dtype,Hk,Hv", [(torch.bfloat16, 2, 4), (torch.float32, 2, 4),
                                              (torch.bfloat16, 2, 8), (torch.float32, 1, 4),
                                              (torch.bfloat16, 3, 3)])
def test_fused_prefill_over_packed_runs_with_short_and_empty_ones(gpu, conv_dtype, Hk, Hv):
    """Two or four value heads per key head (one workgroup per key head) and
    one (one per value head)."""

    lens = [700, 0, 2, 130, 1, 64, 65, 300, 0, 3]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32), device=gpu)
    T, N = int(sum(lens)), len(lens)
    c = _case(gpu, 2, T, N, Hk, Hv, conv_dtype)
    assert gdn.fused_prefill_ok(c["qkv"], c["a"], c["b"], c["conv"], c["ssm"], c["dims"], N)
    y, conv, ssm = gdn.prefill_fused(c["qkv"], c["a"], c["b"], c["conv"], c["ssm"], c["w"],
                                     c["A_log"], c["dt_bias"], c["dims"], cu, y_dtype=torch.bfloat16)
    y_ref, conv_ref, ssm_ref = _unfused(c, cu, torch.bfloat16)
    assert torch.equal(conv, conv_ref)
    # empty runs keep their state (in bf16) and their conv state
    for r in (1, 8):
        assert torch.equal(conv[r], c["conv"][r].to(torch.bfloat16))
        assert torch.equal(ssm[r], c["ssm"][r])
    assert torch.equal(y, y_ref)
    assert torch.equal(ssm, ssm_ref)


def test_layer_prompt_path_takes_the_fused_call(gpu, monkeypatch):
    """The layer's core on a 512-token prompt (dense bf16 projections) runs
    gdn_prefill_fused, not gdn_frontend, and its output and states equal
    those of the unfused calls."""

    from mlx_lean_moe_amd import _lib, linear_attention

    c = _case(gpu, 3, 512, 1, 16, 32)
    d = c["dims"]
    g = torch.Generator(device=gpu).manual_seed(4)
    z = torch.randn(512, d.num_value_heads, D, generator=g, device=gpu).to(torch.bfloat16)
    norm_w = torch.rand(D, generator=g, device=gpu) + 0.5
    layer = gdn.Qwen3_5LinearAttention.__new__(gdn.Qwen3_5LinearAttention)
    layer.linear, layer.rms_norm_eps = d, 1e-6
    layer.conv1d_weight, layer.A_log, layer.dt_bias, layer.norm_weight = (c["w"], c["A_log"],
                                                                          c["dt_bias"], norm_w)
    called = []
    real = _lib.call

    def spy(name, *args):
        called.append(name)
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    out, conv, ssm = layer.core(c["qkv"], z, c["a"], c["b"], c["conv"], c["ssm"])
    monkeypatch.setattr(_lib, "call", real)
    assert "gdn_prefill_fused" in called and "gdn_frontend" not in called
    y_ref, conv_ref, ssm_ref = _unfused(c, None, z.dtype)
    out_ref = linear_attention.gated_rms_norm(y_ref, z, norm_w, 1e-6, out_dtype=z.dtype)
    assert torch.equal(out, out_ref.reshape(512, d.value_dim))
    assert torch.equal(conv, conv_ref) and torch.equal(ssm, ssm_ref)
