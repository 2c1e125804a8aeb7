"""GPU parity of the affine-quantized projections against the oracle's
restatement of MLX's format: y = x @ dequantize(W).T (the reference test's
dense comparison, tests/test_qwen3_5_linear_attention.py:59-86)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from mlx_lean_moe_amd import _lib
from mlx_lean_moe_amd.quant import decode_kernel_takes, quantized_linear_split
from oracle import quant_ref as Q
from oracle import gated_delta_ref as R
from tests.helpers import assert_bf16_out_close, layer_inputs, layer_params

pytestmark = pytest.mark.gpu

_TORCH = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _weights(rng, N, K, bits, gs, sb):
    words, s, b = Q.quantize(rng.standard_normal((N, K)) * 0.05, bits, gs, sb=sb)
    return words, s, b


def _dev_weights(gpu, words, s, b, sb):
    return {"weight": torch.tensor(words.view(np.int32), device=gpu),
            "scales": torch.tensor(s, dtype=torch.float32, device=gpu).to(_TORCH[sb]),
            "biases": torch.tensor(b, dtype=torch.float32, device=gpu).to(_TORCH[sb])}


def _decode_kernel_takes(M, K, bits, gs, sb):
    return decode_kernel_takes(M, K, bits, gs, _TORCH[sb])


@pytest.mark.parametrize("M,N,K,bits,gs,sb", [
    (1, 40, 128, 4, 64, "bf16"),
    (7, 96, 256, 4, 32, "f16"),
    (64, 12352, 2048, 4, 64, "bf16"),   # the layer's stacked input projection at decode
    (33, 2048, 4096, 4, 64, "bf16"),    # out_proj at decode (value_dim 4096 -> hidden)
    (5, 70, 1024, 8, 32, "f16"),
    (200, 130, 512, 8, 128, "f32"),
    (300, 2048, 1024, 4, 64, "bf16"),   # large-M tiles, partial edge tiles
    (2, 78, 256, 4, 64, "bf16"),        # decode kernel: 4 groups per column, last block partial
    (3, 77, 256, 4, 64, "bf16"),        # scales span not whole 16-byte pieces: tiled kernel
    (16, 200, 1024, 4, 32, "f32"),      # decode kernel with float32 scales
    (64, 100, 4096, 8, 32, "f32"),      # scales exceed the decode kernel's LDS: tiled kernel
    (9, 64, 4096, 8, 128, "bf16"),      # 8-bit codes past the decode kernel's registers: tiled
    (1, 4096, 2048, 4, 64, "bf16"),     # decode kernel, one row
    (2, 78, 512, 4, 64, "bf16"),        # decode kernel, one step, last block partial
    (17, 130, 2048, 8, 64, "f16"),      # decode kernel, 8-bit codes, 64-k slices
    (48, 96, 1024, 4, 128, "f32"),      # decode kernel, two slices per group
    (600, 256, 512, 4, 64, "bf16"),     # quantized_linear: dequantize + BLAS; the ABI: tiled kernel
])
def test_quantized_matmul_matches_oracle(gpu, M, N, K, bits, gs, sb):
    rng = np.random.default_rng(M + N + K)
    words, s, b = _weights(rng, N, K, bits, gs, sb)
    x = R.bf16_round(rng.standard_normal((M, K)))
    # bf16 activations: the decode kernel applies scales and biases to float
    # partial sums (exact weights); the tiled kernels dequantize the weights
    # to bf16 whatever the scales' dtype (gdn_quantized_matmul's contract)
    exact = _decode_kernel_takes(M, K, bits, gs, sb)
    ref = Q.quantized_matmul(x, words, s, b, bits, gs, w_round="f32" if exact else "bf16")
    scheme = gdn.QuantScheme(bits, gs)
    W = _dev_weights(gpu, words, s, b, sb)
    xt = torch.tensor(x, dtype=torch.float32, device=gpu).to(torch.bfloat16)
    y = gdn.quantized_linear(xt, W, scheme)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (M, N)
    assert_bf16_out_close(y.float().cpu().numpy(), ref)
    # float32 output: the accumulation alone (no output rounding)
    y32 = torch.empty(M, N, device=gpu)
    _lib.call("gdn_quantized_matmul", _lib.ptr(xt), _lib.GDN_BF16, _lib.ptr(W["weight"]),
              _lib.ptr(W["scales"]), _lib.ptr(W["biases"]), _lib.dtype_code(W["scales"].dtype),
              _lib.ptr(y32), _lib.GDN_F32, None, M, N, K, bits, gs, None, 0, _lib.stream_ptr(xt.device))
    err = np.abs(y32.cpu().numpy() - ref).max()
    assert err <= 1e-5 * np.abs(ref).max() + 1e-6, err


@pytest.mark.parametrize("M,N,K,bits,gs,sb", [
    (1, 4096, 2048, 4, 64, "bf16"),     # one decode row, as the reference runs (float32 activations)
    (16, 200, 1024, 4, 32, "f32"),
    (17, 130, 2048, 8, 64, "f16"),      # 17-32 rows: 64-column workgroups
    (32, 78, 512, 4, 64, "bf16"),
])
def test_float32_activations_on_the_decode_kernel(gpu, M, N, K, bits, gs, sb):
    """float32 x (split into bf16 hi + lo, ~16 significant bits) against the
    exact weights: what mx.quantized_matmul computes for float32 x."""
    assert decode_kernel_takes(M, K, bits, gs, _TORCH[sb])
    rng = np.random.default_rng(M * 7 + N)
    words, s, b = _weights(rng, N, K, bits, gs, sb)
    x = rng.standard_normal((M, K)).astype(np.float32)
    ref = Q.quantized_matmul(x, words, s, b, bits, gs, w_round="f32")
    W = _dev_weights(gpu, words, s, b, sb)
    y = gdn.quantized_linear(torch.tensor(x, device=gpu), W, gdn.QuantScheme(bits, gs))
    assert y.dtype == torch.float32
    err = np.abs(y.cpu().numpy() - ref).max()
    assert err <= 1e-4 * np.abs(ref).max() + 1e-6, err
    # more than 32 float32 rows: the C entry declines, quantized_linear dequantizes
    assert _lib.load().gdn_quantized_matmul(
        None, _lib.GDN_F32, _lib.ptr(W["weight"]), _lib.ptr(W["scales"]), _lib.ptr(W["biases"]),
        _lib.dtype_code(W["scales"].dtype), None, _lib.GDN_F32, None, 33, N, K, bits, gs,
        None, 0, None) == _lib.GDN_EUNSUPPORTED


@pytest.mark.parametrize("N,K,gs,sb,x32", [
    (12352, 2048, 64, "bf16", False),   # the stacked input projection, one sequence
    (12352, 2048, 64, "bf16", True),
    (2048, 4096, 64, "bf16", False),    # out_proj: two rounds of lane chunks
    (2047, 4096, 128, "bf16", True),    # odd N: the last wave's second column is idle
    (777, 1024, 32, "f16", False),      # half the lanes hold a chunk
    (130, 512, 128, "f32", True),       # a quarter of them; f32 scales
])
def test_one_row_runs_the_matrix_vector_kernel_exactly(gpu, N, K, gs, sb, x32):
    """One row of x and 4-bit codes (a single sequence's decode step) take
    the matrix-vector kernel: products against the exact weights s q + b,
    accumulated in float (bf16 x as bf16 pairs against 1 + q / 16; float32
    x in float32), within 1e-5 of the float64 product."""

    assert _decode_kernel_takes(1, K, 4, gs, sb)
    assert _lib.load().gdn_quantized_matmul_workspace_size(
        _lib.GDN_F32 if x32 else _lib.GDN_BF16, _lib.dtype_code(_TORCH[sb]), 1, N, K, 4, gs) == 0
    rng = np.random.default_rng(N + K)
    words, s, b = _weights(rng, N, K, 4, gs, sb)
    x = rng.standard_normal((1, K)).astype(np.float32)
    if not x32:
        x = R.bf16_round(x)
    ref = Q.quantized_matmul(x, words, s, b, 4, gs, w_round="f32")
    W = _dev_weights(gpu, words, s, b, sb)
    xt = torch.tensor(x, device=gpu).to(torch.float32 if x32 else torch.bfloat16)
    y = torch.empty(1, N, device=gpu)
    _lib.call("gdn_quantized_matmul", _lib.ptr(xt), _lib.dtype_code(xt.dtype), _lib.ptr(W["weight"]),
              _lib.ptr(W["scales"]), _lib.ptr(W["biases"]), _lib.dtype_code(W["scales"].dtype),
              _lib.ptr(y), _lib.GDN_F32, None, 1, N, K, 4, gs, None, 0, _lib.stream_ptr(gpu))
    err = np.abs(y.cpu().numpy() - ref).max()
    assert err <= 1e-5 * np.abs(ref).max() + 1e-6, err
    # a 1-D x through quantized_linear gives the same bits in x's dtype
    y1 = gdn.quantized_linear(xt[0], W, gdn.QuantScheme(4, gs))
    assert tuple(y1.shape) == (N,)
    np.testing.assert_array_equal(y1.float().cpu().numpy(), y[0].to(xt.dtype).float().cpu().numpy())


@pytest.mark.parametrize("M,N,K,bits,gs,sb,x32,splits", [
    (64, 8192, 2048, 8, 64, "bf16", False, 2),   # 128 column tiles of 64
    (16, 2048, 4096, 4, 64, "bf16", False, 4),   # out_proj at 16 rows: 64 tiles of 32
    (1, 1000, 2048, 8, 32, "f16", False, 8),     # ragged last tile
    (40, 100, 2048, 8, 64, "f32", False, 4),
    (5, 300, 1024, 4, 32, "bf16", True, 4),      # float32 x
])
def test_split_k_matches_the_unsplit_kernel_and_the_oracle(gpu, M, N, K, bits, gs, sb, x32, splits):
    """Few column tiles: with the workspace the decode kernel splits K over
    workgroups (float32 partial blocks, added in a fixed order). Both the
    split and the unsplit result meet the oracle's bound, they agree to
    float32 rounding, and two split runs agree bit for bit."""

    rng = np.random.default_rng(M * 31 + N)
    words, s, b = _weights(rng, N, K, bits, gs, sb)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if not x32:
        x = R.bf16_round(x)
    ref = Q.quantized_matmul(x, words, s, b, bits, gs, w_round="f32")
    W = _dev_weights(gpu, words, s, b, sb)
    xdt = torch.float32 if x32 else torch.bfloat16
    xt = torch.tensor(x, device=gpu).to(xdt)
    lib = _lib.load()
    ws_bytes = lib.gdn_quantized_matmul_workspace_size(_lib.dtype_code(xdt), _lib.dtype_code(_TORCH[sb]),
                                                       M, N, K, bits, gs)
    assert ws_bytes == splits * M * N * 4
    ws = torch.full((ws_bytes // 4,), float("nan"), device=gpu)  # every partial is written
    outs = []
    for w_ptr, w_len in ((None, 0), (_lib.ptr(ws), ws_bytes), (_lib.ptr(ws), ws_bytes),
                         (_lib.ptr(ws), ws_bytes // 2)):
        y = torch.empty(M, N, device=gpu)
        _lib.call("gdn_quantized_matmul", _lib.ptr(xt), _lib.dtype_code(xdt), _lib.ptr(W["weight"]),
                  _lib.ptr(W["scales"]), _lib.ptr(W["biases"]), _lib.dtype_code(W["scales"].dtype),
                  _lib.ptr(y), _lib.GDN_F32, None, M, N, K, bits, gs, w_ptr, w_len, _lib.stream_ptr(gpu))
        outs.append(y.cpu().numpy())
    tol = (1e-4 if x32 else 1e-5) * np.abs(ref).max() + 1e-6
    for y in outs:
        assert np.abs(y - ref).max() <= tol
    assert np.array_equal(outs[1], outs[2])
    assert np.abs(outs[1] - outs[0]).max() <= 1e-5 * np.abs(ref).max() + 1e-6
    # through quantized_linear (its own workspace), in x's dtype
    y = gdn.quantized_linear(xt, W, gdn.QuantScheme(bits, gs))
    np.testing.assert_array_equal(y.float().cpu().numpy(), torch.tensor(outs[1]).to(xdt).float().numpy())


@pytest.mark.parametrize("M,N,K,sb", [
    (64, 2048, 4096, "bf16"),   # the layer's out_proj: 64 column tiles x 4 row blocks
    (40, 2048, 4096, "f16"),    # ragged last row block (8 rows)
    (17, 100, 4096, "f32"),     # one row in the second block; ragged last column tile
])
def test_row_blocks_match_the_oracle_in_one_launch(gpu, M, N, K, sb):
    """17-64 rows of 4-bit group-64 codes with few column tiles run as
    16-row blocks of the 16-row kernel in one launch: no workspace is asked
    for or used (the same bits with and without one), every row block
    meets the oracle's bound, and the residual is added in the store as the
    unfused add of two bf16 arrays."""

    bits, gs = 4, 64
    rng = np.random.default_rng(M * 7 + N)
    words, s, b = _weights(rng, N, K, bits, gs, sb)
    x = R.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    ref = Q.quantized_matmul(x, words, s, b, bits, gs, w_round="f32")
    W = _dev_weights(gpu, words, s, b, sb)
    xt = torch.tensor(x, device=gpu).to(torch.bfloat16)
    lib = _lib.load()
    assert lib.gdn_quantized_matmul_workspace_size(_lib.GDN_BF16, _lib.dtype_code(_TORCH[sb]), M, N, K,
                                                   bits, gs) == 0
    ws = torch.full((1 << 20,), float("nan"), device=gpu)
    outs = []
    for w_ptr, w_len in ((None, 0), (_lib.ptr(ws), 4 << 20)):
        y = torch.empty(M, N, device=gpu)
        _lib.call("gdn_quantized_matmul", _lib.ptr(xt), _lib.GDN_BF16, _lib.ptr(W["weight"]),
                  _lib.ptr(W["scales"]), _lib.ptr(W["biases"]), _lib.dtype_code(W["scales"].dtype),
                  _lib.ptr(y), _lib.GDN_F32, None, M, N, K, bits, gs, w_ptr, w_len, _lib.stream_ptr(gpu))
        outs.append(y.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    assert torch.isnan(ws).all()  # untouched
    tol = 1e-5 * np.abs(ref).max() + 1e-6
    for r0 in range(0, M, 16):
        assert np.abs(outs[0][r0:r0 + 16] - ref[r0:r0 + 16]).max() <= tol, r0
    # bf16 y with a residual: the product rounded, then the sum rounded
    res = torch.randn(M, N, device=gpu).to(torch.bfloat16)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    _lib.call("gdn_quantized_matmul", _lib.ptr(xt), _lib.GDN_BF16, _lib.ptr(W["weight"]),
              _lib.ptr(W["scales"]), _lib.ptr(W["biases"]), _lib.dtype_code(W["scales"].dtype),
              _lib.ptr(y), _lib.GDN_BF16, _lib.ptr(res), M, N, K, bits, gs, None, 0, _lib.stream_ptr(gpu))
    unfused = (torch.tensor(outs[0], device=gpu).to(torch.bfloat16) + res).cpu()
    assert torch.equal(y.cpu(), unfused)


@pytest.mark.parametrize("bits,gs,sb,out", [(4, 64, "bf16", "bf16"), (8, 32, "f16", "f32"),
                                             (4, 128, "f32", "f32")])
def test_dequantize_is_bit_exact(gpu, bits, gs, sb, out):
    rng = np.random.default_rng(bits * gs)
    words, s, b = _weights(rng, 33, 256, bits, gs, sb)
    W = _dev_weights(gpu, words, s, b, sb)
    dense = gdn.dequantize(W, gdn.QuantScheme(bits, gs), _TORCH[out])
    np.testing.assert_array_equal(dense.float().cpu().numpy(),
                                  Q.dequantize(words, s, b, bits, gs, out=out))


def test_non_bf16_activations_use_dense_weights(gpu):
    rng = np.random.default_rng(4)
    words, s, b = _weights(rng, 48, 128, 4, 64, "bf16")
    W = _dev_weights(gpu, words, s, b, "bf16")
    x = rng.standard_normal((5, 128)).astype(np.float32)
    y = gdn.quantized_linear(torch.tensor(x, device=gpu), W, gdn.QuantScheme(4, 64))
    assert y.dtype == torch.float32
    ref = x.astype(np.float64) @ Q.dequantize(words, s, b, 4, 64, out="f32").T
    assert np.abs(y.cpu().numpy() - ref).max() < 1e-4


@pytest.mark.parametrize("M", [64, 600, 2100])
def test_stacked_projection_blocks_match_the_oracle(gpu, M):
    """quantized_linear_split: one quantized launch split into column views
    below 512 rows, one dequantized product split into views below 2048,
    a GEMM per block (packed) from 2048 rows on; either way each block is
    x @ W_block.T."""

    from mlx_lean_moe_amd.quant import concat_quantized, quantized_linear_split

    rng = np.random.default_rng(M)
    sizes, K = [96, 64, 16], 512
    parts = [_weights(rng, n, K, 4, 64, "bf16") for n in sizes]
    stacked = gdn.LinearWeights(concat_quantized([_dev_weights(gpu, *p, "bf16") for p in parts]),
                                gdn.QuantScheme(4, 64))
    x = R.bf16_round(rng.standard_normal((M, K)))
    xt = torch.tensor(x, dtype=torch.float32, device=gpu).to(torch.bfloat16)
    blocks = quantized_linear_split(xt, stacked, sizes)
    exact = _decode_kernel_takes(M, K, 4, 64, "bf16")
    for blk, (words, s, b), n in zip(blocks, parts, sizes):
        assert tuple(blk.shape) == (M, n) and blk.dtype == torch.bfloat16
        assert blk.is_contiguous() == (M >= 2048)
        ref = Q.quantized_matmul(x, words, s, b, 4, 64, w_round="f32" if exact else "bf16")
        assert_bf16_out_close(blk.float().cpu().numpy(), ref)


@pytest.mark.parametrize("T", [70, 600])
def test_layer_with_quantized_projections_matches_dense_weights(gpu, T):
    """The reference's layer test setup: quantized projections against the
    same layer on the dequantized dense weights, decode and prefill (600
    prompt tokens: the stacked input projection as one GEMM per block)."""

    dims = gdn.LinearAttentionDims(2, 4, 128, 128, 4)
    dt = (2, 4, 128, 128)
    H = 256
    rng = np.random.default_rng(21)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, dt)
    scheme = gdn.QuantScheme(4, 64)
    shapes = {"qkv": dims.conv_dim, "z": dims.value_dim, "a": 4, "b": 4}
    quant, dense = {}, {}
    for name, n in shapes.items():
        words, s, b = _weights(rng, n, H, 4, 64, "bf16")
        quant[name] = _dev_weights(gpu, words, s, b, "bf16")
        dense[name] = torch.tensor(Q.dequantize(words, s, b, 4, 64), dtype=torch.float32,
                                   device=gpu).to(torch.bfloat16)
    words, s, b = _weights(rng, H, dims.value_dim, 4, 64, "bf16")
    quant["out"] = _dev_weights(gpu, words, s, b, "bf16")
    dense["out"] = torch.tensor(Q.dequantize(words, s, b, 4, 64), dtype=torch.float32,
                                device=gpu).to(torch.bfloat16)
    f32 = lambda x: torch.tensor(np.asarray(x, np.float32), device=gpu)
    common = (f32(conv_w)[:, :, None], f32(A_log), f32(dt_bias), f32(norm_w))

    def make(w, q):
        return gdn.Qwen3_5LinearAttention(dims, w["qkv"], w["z"], w["a"], w["b"], common[0],
                                          common[1], common[2], common[3], w["out"], quant=q)

    lq, ld = make(quant, scheme), make(dense, None)
    assert lq._in_stacked is not None  # one launch for the four input projections
    x = torch.tensor(R.bf16_round(rng.standard_normal((T, H))), dtype=torch.float32,
                     device=gpu).to(torch.bfloat16)
    cq, cd = lq.new_cache(torch.bfloat16), ld.new_cache(torch.bfloat16)
    oq, od = lq(x, cq), ld(x, cd)
    assert_bf16_out_close(oq.float().cpu().numpy(), od.float().cpu().numpy().astype(np.float64))
    for t in range(3):
        xt = x[t]
        oq, od = lq(xt, cq), ld(xt, cd)
        assert_bf16_out_close(oq.float().cpu().numpy(), od.float().cpu().numpy().astype(np.float64))


@pytest.mark.parametrize("M,N,K,gs,dt", [
    (1, 2048, 4096, 64, "bf16"),      # the one-row matrix-vector kernel
    (16, 2048, 4096, 64, "bf16"),     # decode kernel, K split (sum kernel stores)
    (32, 12352, 2048, 64, "f32"),     # decode kernel, float32 x and result
    (100, 300, 512, 64, "bf16"),      # tiled kernel
    (600, 256, 512, 64, "bf16"),      # quantized_linear: dequantize + BLAS, then the add
])
def test_residual_is_the_unfused_add(gpu, M, N, K, gs, dt):
    """residual + x W^T, the product rounded to the result dtype first: bit
    for bit the unfused add of the two arrays (the decoder layer's
    h = rows + attention(...))."""

    rng = np.random.default_rng(M + 3 * N)
    words, s, b = _weights(rng, N, K, 4, gs, "bf16")
    W = _dev_weights(gpu, words, s, b, "bf16")
    xdt = _TORCH[dt]
    x = torch.tensor(rng.standard_normal((M, K)), dtype=torch.float32, device=gpu).to(xdt)
    r = torch.tensor(rng.standard_normal((M, N)), dtype=torch.float32, device=gpu).to(xdt)
    scheme = gdn.QuantScheme(4, gs)
    want = gdn.quantized_linear(x, W, scheme) + r
    got = gdn.quantized_linear(x, W, scheme, residual=r)
    assert torch.equal(got, want)
    if M < 512 and dt == "bf16":
        # through the C ABI, residual aliasing y: y = x W^T + y
        y = r.clone()
        nb = _lib.load().gdn_quantized_matmul_workspace_size(_lib.GDN_BF16, _lib.GDN_BF16, M, N, K, 4, gs)
        ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=gpu)
        _lib.call("gdn_quantized_matmul", _lib.ptr(x), _lib.GDN_BF16, _lib.ptr(W["weight"]),
                  _lib.ptr(W["scales"]), _lib.ptr(W["biases"]), _lib.GDN_BF16, _lib.ptr(y), _lib.GDN_BF16,
                  _lib.ptr(y), M, N, K, 4, gs, _lib.ptr(ws), nb, _lib.stream_ptr(gpu))
        assert torch.equal(y, want)
    with pytest.raises(ValueError, match="residual"):
        gdn.quantized_linear(x, W, scheme, residual=r[:, :-1])


@pytest.mark.parametrize("bits,gs,sb,out", [(2, 64, "bf16", "bf16"), (3, 32, "bf16", "f32"),
                                             (5, 128, "f16", "f16"), (6, 32, "f32", "bf16"),
                                             (6, 64, "bf16", "f32")])
def test_dequantize_every_affine_width_is_bit_exact(gpu, bits, gs, sb, out):
    """2-, 3-, 5- and 6-bit codes (the 3/5/6-bit ones straddle word
    boundaries) against the oracle: s * q + b in float32, one rounding."""

    rng = np.random.default_rng(bits * 1000 + gs)
    words, s, b = _weights(rng, 33, 256, bits, gs, sb)
    W = _dev_weights(gpu, words, s, b, sb)
    dense = gdn.dequantize(W, gdn.QuantScheme(bits, gs), _TORCH[out])
    np.testing.assert_array_equal(dense.float().cpu().numpy(),
                                  Q.dequantize(words, s, b, bits, gs, out=out))


def _fp_weights(rng, gpu, N, K, mode, gs):
    bits = 8 if mode == "mxfp8" else 4
    q = rng.integers(0, 2 ** bits, (N, K))
    if mode == "mxfp8":
        q[(q & 0x7F) == 0x7F] = 0x7E  # no NaN codes
    if mode == "nvfp4":
        scales = rng.integers(0x08, 0x7F, (N, K // gs))  # positive e4m3, none NaN
    else:
        scales = rng.integers(110, 140, (N, K // gs))
    W = {"weight": torch.tensor(Q.pack(q, bits).view(np.int32), device=gpu),
         "scales": torch.tensor(scales.astype(np.uint8), device=gpu)}
    return W, Q.dequantize_fp(Q.pack(q, bits), scales, mode, gs)


@pytest.mark.parametrize("mode,gs,K", [("mxfp4", 32, 256), ("mxfp8", 32, 256), ("nvfp4", 16, 256),
                                        ("nvfp4", 16, 240)])
def test_dequantize_float_schemes_is_bit_exact(gpu, mode, gs, K):
    """mxfp4, mxfp8 and nvfp4 codes (nvfp4 with a row of 240: a 16-code
    tail) against the oracle: value times scale, exact in bf16 and float32."""

    rng = np.random.default_rng(K + gs + len(mode))
    W, ref = _fp_weights(rng, gpu, 37, K, mode, gs)
    scheme = gdn.QuantScheme(8 if mode == "mxfp8" else 4, gs, mode)
    for dt in (torch.bfloat16, torch.float32):
        dense = gdn.dequantize(W, scheme, dt)
        np.testing.assert_array_equal(dense.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M", [1, 64, 600])
@pytest.mark.parametrize("scheme", [(3, 64, "affine"), (6, 32, "affine"), (2, 128, "affine"),
                                    (4, 32, "mxfp4"), (8, 32, "mxfp8"), (4, 16, "nvfp4")])
def test_quantized_linear_every_scheme_matches_oracle(gpu, scheme, M, monkeypatch):
    """The schemes outside gdn_quantized_matmul's kernels through
    quantized_linear, bf16 x, with and without the residual, against x @ W.T
    in float64. Up to 64 rows gdn_quantized_matmul_scheme multiplies the
    packed codes (nothing is dequantized; the exact weights s * q + b, float32
    sums: within the output's bf16 rounding); above, the weights are
    dequantized to bf16 for the vendor BLAS."""

    bits, gs, mode = scheme
    rng = np.random.default_rng(bits + gs + M)
    N, K = 96, 512
    if mode == "affine":
        words, s, b = _weights(rng, N, K, bits, gs, "bf16")
        W = _dev_weights(gpu, words, s, b, "bf16")
        # the exact weights (decode sizes) or the bf16 ones the BLAS multiplies
        w = Q.dequantize(words, s, b, bits, gs, out="f32" if M <= 64 else "bf16")
    else:
        W, w = _fp_weights(rng, gpu, N, K, mode, gs)  # exact in bf16
    calls = []
    call = _lib.call
    monkeypatch.setattr(_lib, "call", lambda name, *a: (calls.append(name), call(name, *a))[1])
    x = R.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xt = torch.tensor(x, device=gpu).to(torch.bfloat16)
    q = gdn.QuantScheme(bits, gs, mode)
    y = gdn.quantized_linear(xt, gdn.LinearWeights(W, q))
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert y.dtype == torch.bfloat16 and y.shape == (M, N)
    err = np.abs(y.float().cpu().numpy() - ref)
    if M <= 64:
        assert calls == ["gdn_quantized_matmul_scheme"], calls
        assert (err <= 2.0 ** -8 * np.abs(ref) + 1e-4 * np.abs(ref).max()).all(), err.max()
    else:
        assert "gdn_dequantize" in calls
        assert err.max() <= 1e-2 * np.abs(ref).max()
    r = torch.randn(M, N, device=gpu).to(torch.bfloat16)
    yr = gdn.quantized_linear(xt, gdn.LinearWeights(W, q), residual=r)
    assert torch.equal(yr, y + r)
    parts = quantized_linear_split(xt, gdn.LinearWeights(W, q), [40, 56])
    assert torch.equal(torch.cat(parts, dim=-1), y)


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("scheme,N,K", [((5, 32, "affine"), 200, 480), ((3, 128, "affine"), 70, 768),
                                        ((8, 64, "affine"), 64, 256), ((4, 32, "affine"), 33, 2048),
                                        ((2, 32, "affine"), 96, 352), ((3, 32, "affine"), 80, 224),
                                        ((3, 64, "affine"), 65, 2560), ((5, 64, "affine"), 40, 640),
                                        ((6, 64, "affine"), 48, 192), ((2, 64, "affine"), 17, 4096),
                                        ((6, 128, "affine"), 64, 1024), ((8, 128, "affine"), 96, 512),
                                        ((4, 16, "nvfp4"), 130, 288), ((4, 32, "mxfp4"), 64, 1056),
                                        ((8, 32, "mxfp8"), 129, 320), ((4, 16, "nvfp4"), 24, 4096),
                                        ((8, 32, "mxfp8"), 2048, 1024)])
def test_scheme_matmul_shapes_and_outputs(gpu, scheme, N, K, M):
    """gdn_quantized_matmul_scheme through the C ABI at ragged sizes: every
    row-tile kernel (1-16 rows, 17-64 rows), each code width with runs of
    1, 2 and 4 MFMA blocks per lane (group sizes 32, 64, 128: runs starting
    on a word and runs shifted into place), K split over workgroups (long K,
    few columns), column counts that leave a block part-empty, and the output
    in bfloat16, float16 and float32 with the residual aliasing y; against
    the exact weights in float64 (float32 output: float32 sums)."""

    bits, gs, mode = scheme
    rng = np.random.default_rng(M * 7 + N + K)
    if mode == "affine":
        words, s, b = _weights(rng, N, K, bits, gs, "f16" if bits == 5 else "bf16")
        W = _dev_weights(gpu, words, s, b, "f16" if bits == 5 else "bf16")
        w = Q.dequantize(words, s, b, bits, gs, out="f32")
        sb = _lib.dtype_code(W["scales"].dtype)
    else:
        W, w = _fp_weights(rng, gpu, N, K, mode, gs)
        sb = 0
    x = R.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xt = torch.tensor(x, device=gpu).to(torch.bfloat16)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    mode_code = {"affine": 0, "mxfp4": 1, "mxfp8": 2, "nvfp4": 3}[mode]
    nb = _lib.load().gdn_quantized_matmul_scheme_workspace_size(M, N, K)
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=gpu)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        if dt == torch.float16 and np.abs(ref).max() > 3e4:
            continue  # beyond float16's range (the float formats' large scales)
        r = torch.randn(M, N, device=gpu).to(dt)
        y = r.clone()
        _lib.call("gdn_quantized_matmul_scheme", _lib.ptr(xt), _lib.ptr(W["weight"]), _lib.ptr(W["scales"]),
                  _lib.ptr(W.get("biases")), sb, _lib.ptr(y), _lib.dtype_code(dt), _lib.ptr(y), M, N, K,
                  bits, gs, mode_code, _lib.ptr(ws), nb, _lib.stream_ptr(gpu))
        got = (y.double() - r.double()).cpu().numpy()
        rel = 2.0 ** -20 if dt == torch.float32 else 2.0 ** -7
        assert (np.abs(got - ref) <= rel * (np.abs(ref) + np.abs(r.double().cpu().numpy()))
                + 1e-5 * np.abs(ref).max()).all(), (dt, np.abs(got - ref).max())


@pytest.mark.parametrize("mode,gs,M", [("mxfp4", 32, 1), ("mxfp4", 32, 40), ("mxfp8", 32, 1), ("nvfp4", 16, 64)])
def test_scheme_matmul_special_scale_codes(gpu, mode, gs, M):
    """Scale codes at the ends of their formats through
    gdn_quantized_matmul_scheme: e8m0 255 (NaN) and e4m3 0x7F (NaN) make
    their column NaN, as x times a NaN weight does in the oracle; e8m0 0
    (2^-127) and 1 (2^-126) give their groups weights of at most 6 * 2^-126
    or 448 * 2^-126, whose products vanish beside the other groups'; mxfp8's
    NaN weight codes (0x7F, 0xFF) make their column NaN."""

    rng = np.random.default_rng(17 + M)
    N, K = 64, 256
    bits = 8 if mode == "mxfp8" else 4
    q = rng.integers(0, 2 ** bits, (N, K))
    if mode == "mxfp8":
        q[(q & 0x7F) == 0x7F] = 0x7E
        q[9, 100] = 0x7F
        q[10, 3] = 0xFF
    if mode == "nvfp4":
        scales = rng.integers(0x20, 0x40, (N, K // gs))
        scales[3, 2], scales[4, 0] = 0x7F, 0xFF  # NaN
        scales[5, 1], scales[6, 7] = 0x00, 0x01  # zero, the smallest subnormal
    else:
        scales = rng.integers(120, 130, (N, K // gs))
        scales[3, 2] = 255  # NaN
        scales[5, 1], scales[6, 7] = 0, 1
    scales = scales.astype(np.uint8)
    words = Q.pack(q, bits)
    w = Q.dequantize_fp(words, scales, mode, gs)
    x = R.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    with np.errstate(invalid="ignore", over="ignore"):
        ref = x.astype(np.float64) @ w.T
    xt = torch.tensor(x, device=gpu).to(torch.bfloat16)
    y = torch.empty(M, N, dtype=torch.float32, device=gpu)
    wt = torch.tensor(words.view(np.int32), device=gpu)
    st = torch.tensor(scales, device=gpu)
    mode_code = {"mxfp4": 1, "mxfp8": 2, "nvfp4": 3}[mode]
    _lib.call("gdn_quantized_matmul_scheme", _lib.ptr(xt), _lib.ptr(wt), _lib.ptr(st), None, 0, _lib.ptr(y),
              _lib.GDN_F32, None, M, N, K, bits, gs, mode_code, None, 0, _lib.stream_ptr(gpu))
    got = y.cpu().numpy()
    nan_cols = np.isnan(ref).any(axis=0)
    assert nan_cols.sum() >= (3 if mode == "mxfp8" else 1)
    assert np.isnan(got[:, nan_cols]).all()
    ok = ~nan_cols
    err = np.abs(got[:, ok] - ref[:, ok])
    assert (err <= 2.0 ** -20 * np.abs(ref[:, ok]) + 1e-5 * np.abs(ref[:, ok]).max()).all(), err.max()
