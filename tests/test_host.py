"""Host-side behaviour of the Python surface without a GPU: shape errors are
ValueError before any kernel call (as tests/test_gated_delta_metal.py:137-156
requires of the reference), and CPU tensors are refused loudly."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from mlx_lean_moe_amd import _lib, gated_delta
from oracle.gated_delta_ref import metal_test_inputs


@pytest.fixture
def no_launch(monkeypatch):
    def unexpected(*args):
        pytest.fail("a kernel was reached")

    monkeypatch.setattr(_lib, "call", unexpected)


def _inputs(n=5):
    return [torch.tensor(a) for a in metal_test_inputs(n)]


@pytest.mark.parametrize("invalid", ["k", "v", "g", "beta", "state", "heads", "empty"])
def test_invalid_shapes_are_rejected_before_kernel_dispatch(invalid, no_launch):
    inputs = _inputs()
    index = {"k": 1, "v": 2, "g": 3, "beta": 4, "state": 5}
    if invalid in index:
        inputs[index[invalid]] = inputs[index[invalid]][:1]
    elif invalid == "heads":
        inputs[0] = inputs[0][:, :1].repeat_interleave(3, dim=1)
        inputs[1] = inputs[0]
    else:
        inputs = [a[:0] for a in inputs[:-1]] + inputs[-1:]
    with pytest.raises(ValueError):
        gdn.gated_delta_scan(*inputs)


def test_cpu_tensors_are_refused(no_launch):
    with pytest.raises(RuntimeError, match="ROCm"):
        gdn.gated_delta_scan(*_inputs())


@pytest.mark.parametrize("bad", ["a_shape", "A_log", "heads", "state", "cu_order", "cu_end"])
def test_update_shape_errors(bad, no_launch):
    q = torch.zeros(2, 3, 2, 16)
    k, v = q.clone(), torch.zeros(2, 3, 4, 8)
    a = b = torch.zeros(2, 3, 4)
    A_log = dt = torch.zeros(4)
    state = None
    cu = None
    if bad == "a_shape":
        a = torch.zeros(2, 3, 5)
    elif bad == "A_log":
        A_log = torch.zeros(3)
    elif bad == "heads":
        v = torch.zeros(2, 3, 3, 8)
        a = b = torch.zeros(2, 3, 3)
        A_log = dt = torch.zeros(3)
    elif bad == "state":
        state = torch.zeros(2, 4, 8, 8)
    else:
        q, k, v = q[0], k[0], v[0]
        a = b = a[0]
        cu = [0, 2, 1, 3] if bad == "cu_order" else [0, 2]
    with pytest.raises(ValueError):
        gdn.gated_delta_update(q, k, v, a, b, A_log, dt, state, cu_seqlens=cu)


def test_layer_rejects_bad_rank(no_launch):
    dims = gdn.LinearAttentionDims(2, 4, 32, 32, 4)
    C = dims.conv_dim
    layer = gdn.Qwen3_5LinearAttention(
        dims, torch.zeros(C, 16), torch.zeros(128, 16), torch.zeros(4, 16), torch.zeros(4, 16),
        torch.zeros(C, 4, 1), torch.zeros(4), torch.zeros(4), torch.ones(32), torch.zeros(16, 128))
    with pytest.raises(ValueError):
        layer(torch.zeros(2, 2, 16), None)


def test_dims_mirror_the_reference_dataclass():
    d = gdn.QWEN3_5_LINEAR
    assert (d.key_dim, d.value_dim, d.conv_dim) == (2048, 4096, 8192)


def test_promotion_matches_reference_ops_dtypes():
    f32, bf16, f16 = torch.float32, torch.bfloat16, torch.float16
    t = lambda dt: torch.zeros(1, dtype=dt)
    assert gated_delta._promote(t(bf16), t(bf16), t(f16)) == f32
    assert gated_delta._promote(t(bf16), t(bf16)) == bf16
    assert gated_delta._promote(t(bf16), t(f32)) == f32


def test_decode_slots_are_checked_on_the_host():
    from mlx_lean_moe_amd.linear_attention import check_slots

    assert check_slots([3, 0, 2], 3, 4) == [3, 0, 2]
    assert check_slots(torch.tensor([1, 0], dtype=torch.int32), 2, 2) == [1, 0]
    for bad, msg in (([0, 0], "distinct"), ([0, 4], r"\[0, 4\)"), ([-1, 0], r"\[0, 4\)"),
                     ([0], "expected 2")):
        with pytest.raises(ValueError, match=msg):
            check_slots(bad, 2, 4)
    with pytest.raises(ValueError, match="one-dimensional"):
        check_slots(torch.zeros(2, 1, dtype=torch.int64), 2, 4)
    with pytest.raises(ValueError, match="integers"):
        check_slots(torch.zeros(2), 2, 4)


def test_row_views_are_read_in_place_and_other_layouts_copied():
    """The decode step reads qkv, z, a and b at a row stride: column slices
    of one stacked projection output go in as they are (their row stride
    reported), anything whose rows are not packed is copied."""
    from mlx_lean_moe_amd.linear_attention import _rows

    stacked = torch.arange(5 * 40, dtype=torch.float32).reshape(5, 40)
    qkv, z, a = stacked[:, :24], stacked[:, 24:32].reshape(5, 2, 4), stacked[:, 32:36]
    for t, width in ((qkv, 24), (z, 8), (a, 4)):
        got, stride = _rows(t)
        assert got.data_ptr() == t.data_ptr() and stride == 40
        assert got.stride(0) == 40 and got[0].numel() == width
    packed, stride = _rows(torch.zeros(3, 6))
    assert stride == 6
    # a column view with a non-unit inner stride, or overlapping rows, is copied
    for t in (stacked[:, ::2], torch.zeros(1, 8).expand(4, 8)):
        got, stride = _rows(t)
        assert got.is_contiguous() and stride == t.shape[1] and torch.equal(got, t)
    one, stride = _rows(stacked[2:3, :7])
    assert one.data_ptr() == stacked[2:3, :7].data_ptr() and stride == 7


def test_conv_half_bits_and_residuals_are_checked_on_the_host():
    from mlx_lean_moe_amd.linear_attention import check_half_bits
    from mlx_lean_moe_amd.quant import _check_residual

    assert check_half_bits([0, 1, 1], 3) == [0, 1, 1]
    for bad in ([0, 2, 1], [0, 1], [-1, 0, 0]):
        with pytest.raises(ValueError, match="bits"):
            check_half_bits(bad, 3)
    _check_residual(torch.zeros(2, 5, dtype=torch.bfloat16), (2, 5), torch.bfloat16)
    for r in (torch.zeros(2, 4, dtype=torch.bfloat16), torch.zeros(2, 5)):
        with pytest.raises(ValueError, match="residual"):
            _check_residual(r, (2, 5), torch.bfloat16)


def test_stacked_projection_block_sizes_must_cover_the_rows(no_launch):
    from mlx_lean_moe_amd.quant import quantized_linear_split

    w = gdn.LinearWeights({"weight": torch.zeros(10, 16, dtype=torch.int32),
                           "scales": torch.ones(10, 2, dtype=torch.bfloat16),
                           "biases": torch.zeros(10, 2, dtype=torch.bfloat16)}, gdn.QuantScheme(4, 64))
    with pytest.raises(ValueError, match="do not add up"):
        quantized_linear_split(torch.zeros(3, 128, dtype=torch.bfloat16), w, [4, 5])


def test_dense_path_choice_follows_the_measured_crossovers():
    from mlx_lean_moe_amd.quant import _dense_rows

    assert not _dense_rows(64, 2048, 4096)       # decode sizes: quantized kernels
    assert _dense_rows(65, 2048, 4096)           # out_proj above 64 rows: dense
    assert not _dense_rows(300, 12352, 2048)     # the stacked input projection: tiled kernel
    assert _dense_rows(512, 12352, 2048)         # prefill sizes: dense for every shape
    assert _dense_rows(200, 12352, 4096)         # deep weights
    assert _dense_rows(100, 300, 512)            # narrow weights


def test_pool_host_bookkeeping_flips_bits_and_sizes():
    """The pool's host copies of the half bits and sizes (NumPy views of its
    torch tensors): a decode of some slots flips exactly their bits and adds
    one token; tokens=-1 undoes it."""

    pool = gdn.RecurrentStatePool.__new__(gdn.RecurrentStatePool)
    pool.conv_half = torch.zeros(6, dtype=torch.int64)
    pool.size = torch.zeros(6, dtype=torch.int64)
    pool._half_np, pool._size_np = pool.conv_half.numpy(), pool.size.numpy()
    idx = np.array([4, 1])
    pool.flip_host(idx)
    assert pool.conv_half.tolist() == [0, 1, 0, 0, 1, 0] and pool.size.tolist() == [0, 1, 0, 0, 1, 0]
    pool.flip_host(np.array([1, 2]))
    assert pool.conv_half.tolist() == [0, 0, 1, 0, 1, 0] and pool.size.tolist() == [0, 2, 1, 0, 1, 0]
    pool.flip_host(np.array([1, 2]), tokens=-1)
    assert pool.conv_half.tolist() == [0, 1, 0, 0, 1, 0] and pool.size.tolist() == [0, 1, 0, 0, 1, 0]
    # once a step has flipped halves through the arrival counters, flipping
    # the bits alone (gdn_pool_advance) is refused: it would read them wrong
    pool._counted = False
    pool.advance([3], device_flipped=True)
    assert pool.conv_half.tolist() == [0, 1, 0, 1, 1, 0]
    with pytest.raises(ValueError, match="conv_arrivals"):
        pool.advance([3])
    assert pool.conv_half.tolist() == [0, 1, 0, 1, 1, 0]


@pytest.mark.parametrize("bad", ["short", "long", "start", "end", "order", "uneven"])
def test_malformed_run_offsets_raise_before_any_launch(bad, no_launch, monkeypatch):
    """The front-end and the layer's core check cu_seqlens on the host
    before their first launch: N+1 offsets for N conv states, from 0 to
    the token count, non-decreasing; without offsets the tokens must split
    evenly. (The device check is bypassed so the CPU tensors reach the
    offset checks.)"""
    from types import SimpleNamespace

    from mlx_lean_moe_amd import linear_attention as LA

    monkeypatch.setattr(LA, "_require_device", lambda *t: torch.device("cpu"))
    dims = gdn.LinearAttentionDims(2, 4, 32, 32, 4)
    T, N, C = 10, 3, dims.conv_dim
    cu = {"short": [0, 4, 10], "long": [0, 2, 4, 6, 10], "start": [1, 2, 4, 10],
          "end": [0, 2, 4, 11], "order": [0, 5, 4, 10], "uneven": None}[bad]
    qkv = torch.zeros(T, C, dtype=torch.bfloat16)
    conv = torch.zeros(N, 3, C, dtype=torch.bfloat16)
    w = torch.zeros(C, 4)
    with pytest.raises(ValueError, match="cu_seqlens|equal runs"):
        LA.conv_frontend(qkv, conv, w, dims, None if cu is None else torch.tensor(cu, dtype=torch.int32))
    if cu is None:
        return
    layer = SimpleNamespace(linear=dims, conv1d_weight=w)
    z = torch.zeros(T, 4, 32, dtype=torch.bfloat16)
    ab = torch.zeros(T, 4, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="cu_seqlens"):
        LA.Qwen3_5LinearAttention.core(layer, qkv, z, ab, ab, conv, torch.zeros(N, 4, 32, 32),
                                       cu_seqlens=cu)
