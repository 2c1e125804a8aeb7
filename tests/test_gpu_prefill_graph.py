"""PrefillGraph: a prompt chunk of the layer captured in a HIP graph. Every
replay, with unrelated eager work and synchronizations between replays,
equals the eager ``layer(x, cache)`` on a twin cache bit for bit (outputs
and both states), on the three prompt paths a chunk length selects."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from oracle import quant_ref as Q

pytestmark = pytest.mark.gpu

DIMS = gdn.LinearAttentionDims(16, 32, 128, 128, 4)
HIDDEN = 256


def _quantized_layer(seed, dev):
    rng = np.random.default_rng(seed)

    def qw(n, k):
        words, s, b = Q.quantize(rng.standard_normal((n, k)) * 0.05, 4, 64, sb="bf16")
        return {"weight": torch.tensor(words.view(np.int32), device=dev),
                "scales": torch.tensor(s, dtype=torch.float32, device=dev).to(torch.bfloat16),
                "biases": torch.tensor(b, dtype=torch.float32, device=dev).to(torch.bfloat16)}

    f = lambda *s: torch.tensor(rng.standard_normal(s).astype(np.float32), device=dev)
    d = DIMS
    return gdn.Qwen3_5LinearAttention(
        d, qw(d.conv_dim, HIDDEN), qw(d.value_dim, HIDDEN), qw(d.num_value_heads, HIDDEN),
        qw(d.num_value_heads, HIDDEN), f(d.conv_dim, 4, 1) * 0.2, f(d.num_value_heads),
        f(d.num_value_heads), f(d.value_head_dim) * 0.1 + 1.0, qw(HIDDEN, d.value_dim),
        quant=gdn.QuantScheme(4, 64))


def _x(rng, n, dev):
    return torch.tensor(rng.standard_normal((n, HIDDEN)), dtype=torch.float32, device=dev).to(torch.bfloat16)


# 512: dequantized weights on the vendor BLAS + chunked prefill; 96: the
# quantized kernels + chunked prefill; 40: the quantized kernels + the scan
@pytest.mark.parametrize("chunk", [512, 96, 40])
def test_prefill_graph_replays_equal_eager_chunks(gpu, chunk):
    layer = _quantized_layer(chunk, gpu)
    rng = np.random.default_rng(chunk + 1)
    xs = [_x(rng, chunk, gpu) for _ in range(3)]
    eager, graphed = layer.new_cache(), layer.new_cache()  # float32 conv state at first
    step = gdn.PrefillGraph(layer, xs[0])
    scratch = torch.randn(1 << 20, device=gpu)
    for x in xs:
        ref = layer(x, eager)
        out = step.step(graphed, x)
        assert torch.equal(out, ref)
        assert torch.equal(graphed.conv_state, eager.conv_state)
        assert torch.equal(graphed.ssm_state, eager.ssm_state)
        scratch.mul_(1.0001).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
    assert graphed.size == eager.size == 3 * chunk
    # the prompt's shorter last chunk, eager, on the graph-driven cache
    tail = _x(rng, 7, gpu)
    assert torch.equal(layer(tail, graphed), layer(tail, eager))
    assert torch.equal(graphed.ssm_state, eager.ssm_state)


def test_prefill_graph_with_a_residual_and_a_second_sequence(gpu):
    """The decoder layer's residual inside the captured chunk; a second
    sequence's cache on the same graph gets its own state copied in."""

    layer = _quantized_layer(5, gpu)
    rng = np.random.default_rng(6)
    chunk = 96
    step = gdn.PrefillGraph(layer, _x(rng, chunk, gpu), residual_example=_x(rng, chunk, gpu))
    caches = [[layer.new_cache(torch.bfloat16), layer.new_cache(torch.bfloat16)] for _ in range(2)]
    for rnd in range(2):
        for seq in (0, 1):
            x, r = _x(rng, chunk, gpu), _x(rng, chunk, gpu)
            eager, graphed = caches[seq]
            ref = layer(x, eager, residual=r)
            out = step.step(graphed, x, r)
            assert torch.equal(out, ref)
            assert torch.equal(graphed.ssm_state, eager.ssm_state)
            assert torch.equal(graphed.conv_state, eager.conv_state)
            # the other sequence's step overwrites the graph's buffers: keep copies
            caches[seq][1] = _detached(graphed)
            torch.cuda.synchronize()
    with pytest.raises(ValueError, match="residual"):
        gdn.PrefillGraph(layer, _x(rng, chunk, gpu)).step(layer.new_cache(), residual=_x(rng, chunk, gpu))
    with pytest.raises(ValueError, match="x must be"):
        step.step(layer.new_cache(), _x(rng, chunk + 1, gpu))


def _detached(cache):
    """A cache holding copies of ``cache``'s state (the graph's buffers
    change with the next sequence's step)."""

    out = gdn.RecurrentCache.__new__(gdn.RecurrentCache)
    out.conv_state, out.ssm_state, out.size = cache.conv_state.clone(), cache.ssm_state.clone(), cache.size
    return out


def test_kept_dense_weights_change_no_result(gpu):
    """keep_dense_weights: the prompt-sized products use the kept bf16
    copies instead of dequantizing per call; eager calls (dense and
    quantized-kernel sizes) and graph chunks are bit-identical."""

    plain, dense = _quantized_layer(21, gpu), _quantized_layer(21, gpu)
    dense.keep_dense_weights()
    assert dense._in_stacked.dense is not None and dense.out_proj.dense is not None
    rng = np.random.default_rng(22)
    c1, c2 = plain.new_cache(), dense.new_cache()
    for n in (600, 70, 1):
        x = _x(rng, n, gpu)
        assert torch.equal(plain(x if n > 1 else x[0], c1), dense(x if n > 1 else x[0], c2))
    assert torch.equal(c1.ssm_state, c2.ssm_state)
    step = gdn.PrefillGraph(dense, _x(rng, 512, gpu))
    for _ in range(2):
        x = _x(rng, 512, gpu)
        assert torch.equal(step.step(c2, x), plain(x, c1))
        torch.cuda.synchronize()
