"""The whole layer on the GPU against the oracle's layer
(tests/test_qwen3_5_linear_attention.py restated: layer parity, stepwise
decode equals one batched pass, constant state size), on the unfused path
(small heads) and the fused decode path (production heads)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from oracle import gated_delta_ref as R

pytestmark = pytest.mark.gpu
HIDDEN = 128


def _build(seed, dims, dev, dtype=torch.float32):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    w = {
        "in_proj_qkv": f(dims.conv_dim, HIDDEN) * 0.05,
        "in_proj_z": f(dims.value_dim, HIDDEN) * 0.05,
        "in_proj_a": f(dims.num_value_heads, HIDDEN) * 0.05,
        "in_proj_b": f(dims.num_value_heads, HIDDEN) * 0.05,
        "out_proj": f(HIDDEN, dims.value_dim) * 0.05,
        "conv1d_weight": f(dims.conv_dim, dims.conv_kernel_dim, 1) * 0.2,
        "A_log": f(dims.num_value_heads),
        "dt_bias": f(dims.num_value_heads),
        "norm_weight": f(dims.value_head_dim) * 0.1 + 1.0,
    }
    t = {n: torch.tensor(x, device=dev) for n, x in w.items()}
    for n in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj"):
        t[n] = t[n].to(dtype)
    layer = gdn.Qwen3_5LinearAttention(dims, t["in_proj_qkv"], t["in_proj_z"], t["in_proj_a"],
                                       t["in_proj_b"], t["conv1d_weight"], t["A_log"],
                                       t["dt_bias"], t["norm_weight"], t["out_proj"])
    w["conv1d_weight"] = w["conv1d_weight"][..., 0]
    return layer, w


def _oracle_layer(x, w, dims, conv, ssm, act=None):
    d = (dims.num_key_heads, dims.num_value_heads, dims.key_head_dim, dims.value_head_dim)
    return R.linear_attention(x, w, conv, ssm, d, 1e-6, act)


DIMS_SMALL = gdn.LinearAttentionDims(2, 4, 32, 32, 4)
DIMS_PROD = gdn.LinearAttentionDims(2, 4, 128, 128, 4)


@pytest.mark.parametrize("dims", [DIMS_SMALL, DIMS_PROD], ids=["small", "prod_heads"])
@pytest.mark.parametrize("seq_len", [1, 6])
def test_layer_matches_oracle(gpu, dims, seq_len):
    layer, w = _build(0, dims, gpu)
    rng = np.random.default_rng(100)
    x = rng.standard_normal((seq_len, HIDDEN)).astype(np.float32)
    cache = layer.new_cache()
    got = layer(torch.tensor(x, device=gpu), cache)
    conv0 = np.zeros((dims.conv_kernel_dim - 1, dims.conv_dim))
    ssm0 = np.zeros((dims.num_value_heads, dims.value_head_dim, dims.key_head_dim))
    expected, conv, ssm = _oracle_layer(x, w, dims, conv0, ssm0)
    np.testing.assert_allclose(got.cpu().numpy(), expected, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(cache.conv_state.cpu().numpy(), conv, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cache.ssm_state.cpu().numpy(), ssm, rtol=1e-4, atol=1e-5)
    assert cache.size == seq_len


@pytest.mark.parametrize("dims", [DIMS_SMALL, DIMS_PROD], ids=["small", "prod_heads"])
def test_decoding_step_by_step_matches_one_batched_pass(gpu, dims):
    layer, _ = _build(1, dims, gpu)
    rng = np.random.default_rng(101)
    x = torch.tensor(rng.standard_normal((5, HIDDEN)).astype(np.float32), device=gpu)
    batched = layer(x, layer.new_cache())
    cache = layer.new_cache()
    stepwise = torch.stack([layer(x[t], cache) for t in range(5)])
    torch.testing.assert_close(batched, stepwise, rtol=1e-4, atol=1e-5)


def test_cache_state_is_constant_in_sequence_length(gpu):
    layer, _ = _build(2, DIMS_SMALL, gpu)
    rng = np.random.default_rng(102)
    cache = layer.new_cache()
    shapes = []
    for _ in range(4):
        x = torch.tensor(rng.standard_normal((3, HIDDEN)).astype(np.float32), device=gpu)
        layer(x, cache)
        conv, ssm = cache.state()
        shapes.append((tuple(conv.shape), tuple(ssm.shape)))
    assert len(set(shapes)) == 1
    assert cache.size == 12


def test_bf16_layer_matches_oracle_with_bf16_rounding(gpu):
    dims = DIMS_PROD
    layer, w = _build(3, dims, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(103)
    x = R.bf16_round(rng.standard_normal((7, HIDDEN)))
    cache = layer.new_cache()
    got = layer(torch.tensor(x, device=gpu).to(torch.bfloat16), cache)
    wq = dict(w)
    for n in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj"):
        wq[n] = R.bf16_round(w[n])
    conv0 = np.zeros((3, dims.conv_dim))
    ssm0 = np.zeros((dims.num_value_heads, 128, 128))
    expected, _, ssm = _oracle_layer(x, wq, dims, conv0, ssm0, act="bf16")
    np.testing.assert_allclose(got.float().cpu().numpy(), expected, atol=2e-2)
    rel = np.abs(cache.ssm_state.cpu().numpy() - ssm).max() / np.abs(ssm).max()
    assert rel < 2e-2  # projections run in bf16 BLAS on one side, float64 on the other


@pytest.mark.parametrize("seq_len", [1, 7, 130])
def test_bf16_layer_core_matches_oracle_on_its_own_projections(gpu, seq_len):
    """The layer between its projections at the north-star bars: the
    oracle's core (conv, q/k scaling, gates, recurrence, gated norm, with
    bf16 rounding) fed the GPU layer's own bf16 projection outputs, so the
    two sides differ only in the path itself. State within 1e-3 relative,
    conv state bit for bit, the core output and the layer output (out_proj
    of the core output, float64 on the oracle's side) within the bf16 bar.
    One token takes the fused decode kernel, 7 the sequential scan, 130 the
    chunked prefill."""

    from tests.helpers import assert_bf16_out_close, max_rel

    dims = DIMS_PROD
    layer, w = _build(3, dims, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(103 + seq_len)
    x = torch.tensor(R.bf16_round(rng.standard_normal((seq_len, HIDDEN))), device=gpu).to(torch.bfloat16)
    cache = layer.new_cache(torch.bfloat16)
    conv0, ssm0 = (t.float().cpu().numpy() for t in cache.state())
    got = layer(x, cache)
    qkv, z, a, b = (t.float().cpu().numpy() for t in layer._project(x))
    d = (dims.num_key_heads, dims.num_value_heads, dims.key_head_dim, dims.value_head_dim)
    core, conv, ssm = R.linear_attention_core(qkv, z.reshape(seq_len, dims.num_value_heads, -1),
                                              a, b, conv0, ssm0, w["conv1d_weight"], w["A_log"],
                                              w["dt_bias"], w["norm_weight"], d, 1e-6, "bf16")
    assert max_rel(cache.ssm_state.cpu().numpy(), ssm) < 1e-3
    np.testing.assert_array_equal(cache.conv_state.float().cpu().numpy(), conv)
    # the GPU's core output on the path the layer took (the fused decode
    # kernel for one token, the unfused core otherwise)
    proj = layer._project(x)
    conv_z, ssm_z = torch.zeros_like(cache.conv_state)[None], torch.zeros_like(cache.ssm_state)[None]
    if seq_len == 1:
        core_gpu = layer._decode_fused(*proj, conv_z, ssm_z, in_place=False)[0].reshape(1, -1)
    else:
        core_gpu = layer.core(*proj, conv_z, ssm_z)[0]
    assert_bf16_out_close(core_gpu.float().cpu().numpy(), core)
    expected = R.bf16_round(core_gpu.float().cpu().numpy().astype(np.float64)
                            @ R.bf16_round(w["out_proj"]).astype(np.float64).T)
    assert_bf16_out_close(got.float().cpu().numpy(), expected)


def test_decode_batch_matches_per_sequence_layer_calls(gpu):
    dims = DIMS_PROD
    layer, _ = _build(4, dims, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(104)
    B = 3
    pool = gdn.RecurrentStatePool(B, 4, dims.conv_dim, dims.num_value_heads, 128, 128,
                                  dtype=torch.bfloat16, device=gpu)
    caches = [layer.new_cache(torch.bfloat16) for _ in range(B)]
    prompts = [torch.tensor(rng.standard_normal((n, HIDDEN)), dtype=torch.bfloat16, device=gpu)
               for n in (2, 5, 1)]
    for i, p in enumerate(prompts):
        layer(p, caches[i])
        pool.load(i, caches[i])
    for _ in range(3):
        x = torch.tensor(rng.standard_normal((B, HIDDEN)), dtype=torch.bfloat16, device=gpu)
        out = layer.decode_batch(x, pool)
        ref = torch.stack([layer(x[i], caches[i]) for i in range(B)])
        torch.testing.assert_close(out.float(), ref.float(), rtol=0, atol=0)
    for i in range(B):
        torch.testing.assert_close(pool.ssm_state[i], caches[i].ssm_state, rtol=0, atol=0)
        torch.testing.assert_close(pool.conv_state[i], caches[i].conv_state, rtol=0, atol=0)


def test_launch_stream_is_the_current_stream(gpu):
    """Kernels go to torch's current stream of the tensors' device, also
    inside a stream context."""

    from mlx_lean_moe_amd import _lib

    side = torch.cuda.Stream(gpu)
    assert _lib.stream_ptr(gpu) == torch.cuda.current_stream(gpu).cuda_stream
    assert _lib.stream_ptr(torch.device("cuda")) == torch.cuda.current_stream().cuda_stream
    with torch.cuda.stream(side):
        assert _lib.stream_ptr(gpu) == side.cuda_stream
    assert _lib.stream_ptr(gpu) != side.cuda_stream
