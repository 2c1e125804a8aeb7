"""Host-side behaviour of the quantized projections (no GPU): the scheme
validation of the reference's QuantScheme (config.py:17-33) and the checks
quantized_linear makes before any launch (moe_block.py:27-55)."""

from __future__ import annotations

import pytest
import torch

import mlx_lean_moe_amd as gdn
from mlx_lean_moe_amd import quant


@pytest.mark.parametrize("bits,gs,mode", [(4, 64, "affine"), (8, 32, "affine"), (2, 128, "affine"),
                                           (4, 32, "mxfp4"), (8, 32, "mxfp8"), (4, 16, "nvfp4")])
def test_quant_scheme_accepts_what_mlx_executes(bits, gs, mode):
    assert gdn.QuantScheme(bits, gs, mode).bits == bits


@pytest.mark.parametrize("bits,gs,mode", [(7, 64, "affine"), (4, 16, "affine"), (4, 64, "mxfp4"),
                                           (4, 32, "int4")])
def test_quant_scheme_rejects_combinations_mlx_cannot_execute(bits, gs, mode):
    with pytest.raises(ValueError):
        gdn.QuantScheme(bits, gs, mode)


def _qweights(N=8, K=128, bits=4, gs=64):
    return {"weight": torch.zeros(N, K * bits // 32, dtype=torch.int32),
            "scales": torch.ones(N, K // gs, dtype=torch.bfloat16),
            "biases": torch.zeros(N, K // gs, dtype=torch.bfloat16)}


def test_dense_weights_are_a_plain_matmul():
    x = torch.randn(3, 16)
    w = torch.randn(5, 16)
    torch.testing.assert_close(gdn.quantized_linear(x, w), x @ w.T)
    torch.testing.assert_close(gdn.quantized_linear(x, gdn.LinearWeights(w, None)), x @ w.T)


def test_quantized_weights_need_a_scheme():
    with pytest.raises(ValueError, match="require a quantization scheme"):
        gdn.quantized_linear(torch.randn(2, 128), _qweights())


def test_every_scheme_is_checked_before_any_launch():
    # 3-bit codes: 128 of them fill 12 words; 16 words of 4-bit codes hold no
    # whole number of 3-bit ones, 24 hold 256
    with pytest.raises(ValueError, match="no whole number"):
        gdn.quantized_linear(torch.randn(2, 128), _qweights(bits=4), gdn.QuantScheme(3, 64))
    with pytest.raises(ValueError, match="input width"):
        gdn.quantized_linear(torch.randn(2, 128), _qweights(K=256, bits=3), gdn.QuantScheme(3, 64))
    # the float schemes carry uint8 scales and no biases
    with pytest.raises(ValueError, match="no biases"):
        gdn.quantized_linear(torch.randn(2, 128), _qweights(), gdn.QuantScheme(4, 32, "mxfp4"))
    fp = _qweights(gs=32)
    del fp["biases"]
    with pytest.raises(ValueError, match="uint8"):
        gdn.quantized_linear(torch.randn(2, 128), fp, gdn.QuantScheme(4, 32, "mxfp4"))
    fp["scales"] = torch.zeros(fp["weight"].shape[0], 4, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="ROCm"):
        gdn.quantized_linear(torch.randn(2, 128), fp, gdn.QuantScheme(4, 32, "mxfp4"))


def test_shape_checks_before_any_launch():
    s = gdn.QuantScheme(4, 64)
    with pytest.raises(ValueError, match="input width"):
        gdn.quantized_linear(torch.randn(2, 64), _qweights(K=128), s)
    bad = _qweights()
    bad["scales"] = bad["scales"][:, :1]
    with pytest.raises(ValueError, match="scales and biases"):
        gdn.quantized_linear(torch.randn(2, 128), bad, s)
    nob = _qweights()
    del nob["biases"]
    with pytest.raises(ValueError, match="biases"):
        gdn.quantized_linear(torch.randn(2, 128), nob, s)


def test_cpu_tensors_raise_instead_of_falling_back():
    with pytest.raises(RuntimeError, match="ROCm"):
        gdn.quantized_linear(torch.randn(2, 128, dtype=torch.bfloat16), _qweights(),
                             gdn.QuantScheme(4, 64))


def test_concat_quantized_stacks_along_rows():
    a, b = _qweights(N=3), _qweights(N=5)
    c = quant.concat_quantized([a, b])
    assert tuple(c["weight"].shape) == (8, 16) and tuple(c["scales"].shape) == (8, 2)
