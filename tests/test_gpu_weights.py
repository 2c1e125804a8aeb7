"""A gated-delta layer loaded from a checkpoint's shards (the reference's
names and dtypes, transformer.py:52-65) runs like the same layer built from
the decoded tensors directly, and its quantized projections match dense
weights from the oracle's dequantization."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from mlx_lean_moe_amd import weights as W
from oracle import quant_ref as Q
from tests.test_weights import PREFIX, write_checkpoint

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_loaded_layer_runs_like_the_decoded_tensors(gpu, tmp_path, act):
    # bf16 activations with every projection quantized; float32 activations
    # (the reference's: embeddings are read as float32) with a dense in_proj_b
    dense_b = act == "f32"
    adt = torch.bfloat16 if act == "bf16" else torch.float32
    bf, u32, cfg = write_checkpoint(tmp_path, Hk=2, Hv=4, d=128, hidden=256, bits=4, gs=64,
                                    dense_b=dense_b)
    layer = W.load_linear_attention(tmp_path, 0, device=gpu)
    dims = W.linear_dims_from_hf(cfg)
    assert layer.linear == dims
    q4 = gdn.QuantScheme(4, 64)

    def qw(name):
        return gdn.LinearWeights({"weight": torch.tensor(u32[f"{PREFIX}.{name}.weight"].view(np.int32), device=gpu),
                                  "scales": bf[f"{PREFIX}.{name}.scales"].to(gpu),
                                  "biases": bf[f"{PREFIX}.{name}.biases"].to(gpu)}, q4)

    f32 = lambda name: bf[f"{PREFIX}.{name}"].float().to(gpu)
    direct = gdn.Qwen3_5LinearAttention(dims, qw("in_proj_qkv"), qw("in_proj_z"), qw("in_proj_a"),
                                        gdn.LinearWeights(f32("in_proj_b.weight"), None)
                                        if dense_b else qw("in_proj_b"),
                                        f32("conv1d.weight"), f32("A_log"), f32("dt_bias"),
                                        f32("norm.weight"), qw("out_proj"))
    rng = np.random.default_rng(5)
    x = torch.tensor(rng.standard_normal((7, 256)), dtype=adt, device=gpu)
    c1, c2 = layer.new_cache(adt), direct.new_cache(adt)
    torch.testing.assert_close(layer(x[:5], c1), direct(x[:5], c2), rtol=0, atol=0)
    for t in (5, 6):
        torch.testing.assert_close(layer(x[t], c1), direct(x[t], c2), rtol=0, atol=0)
    torch.testing.assert_close(c1.ssm_state, c2.ssm_state, rtol=0, atol=0)
    # the decoder layer's residual, h = x + layer(x), fused into out_proj's
    # store: bit for bit the separate add (a prompt chunk and a decode step)
    for xs in (x[5:7], x[6]):
        h = layer(xs, c1, residual=xs)
        assert torch.equal(h, direct(xs, c2) + xs)

    # the loaded quantized projection equals x times the oracle's dense weights
    words = u32[f"{PREFIX}.in_proj_z.weight"]
    s = bf[f"{PREFIX}.in_proj_z.scales"].float().numpy()
    b = bf[f"{PREFIX}.in_proj_z.biases"].float().numpy()
    xr = x[:3].float().cpu().numpy().astype(np.float64)
    ref = Q.quantized_matmul(xr, words, s, b, 4, 64, w_round="f32")
    got = gdn.quantized_linear(x[:3], layer.in_proj_z).float().cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-2, atol=2e-2 * np.abs(ref).max())
