"""GPU parity of the fused decode kernel at the two benchmarked decode sizes,
against the C oracle (gdn_ref.c):

* B=256 sequences, Hk=16 key heads, Hv=64 value heads (GQA 4:1), d=128,
  conv channels C = 12288, z gate and gated RMSNorm fused, float32 state
  ~N(0, 0.05) (1 GiB), bf16 activations: one full step; four chained
  in-place steps at B=16; a pooled run with the conv half bits and arrival
  counters;
* B=64, Hk=16, Hv=32 (GQA 2:1), no gate: 256 chained in-place steps, as
  the decode loop runs them.

Bars: the bf16 output within max(2e-2, one bf16 ulp), the state within
1e-3 of the oracle's largest value (relative), the rolled conv state bit
for bit. Large states are compared on the device (a host float64 copy of
1 GiB of state would need 2 GiB more per operand)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from oracle import cref
from tests.helpers import assert_bf16_out_close, counters_settled, device_halves, layer_params

pytestmark = pytest.mark.gpu

D = 128


def _bf16(x) -> np.ndarray:
    """Round float32 to bfloat16 and back (round to nearest even)."""

    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).bfloat16().float().numpy()


def _inputs(rng, B, Hk, Hv, with_z):
    C = 2 * Hk * D + Hv * D
    f = lambda *s: rng.standard_normal(s, dtype=np.float32)
    return dict(qkv=_bf16(f(B, C)), z=_bf16(f(B, Hv, D)) if with_z else None,
                a=_bf16(f(B, Hv)), b=_bf16(f(B, Hv)))


def _dev(x, gpu, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu).to(dtype)


def _state_rel_err(got: torch.Tensor, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| over the whole state, computed on the
    device one sequence block at a time."""

    worst, scale = 0.0, 0.0
    n = got.shape[0]
    step = max(1, n // 8)
    for i in range(0, n, step):
        r = torch.from_numpy(ref[i:i + step]).to(got.device)
        worst = max(worst, (got[i:i + step] - r).abs().max().item())
        scale = max(scale, r.abs().max().item())
    return worst / scale


def _params(seed, Hk, Hv):
    rng = np.random.default_rng(seed)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, (Hk, Hv, D, D))
    return rng, conv_w, A_log, dt_bias, norm_w


def test_decode_b256_hv64_full_step_matches_c_oracle(gpu):
    """One step of the whole B=256, Hv=64 batch with the gated norm: every
    one of the 16 384 workgroups, every key head's conv roll taken by the
    first of its four value heads."""

    B, Hk, Hv = 256, 16, 64
    dims = gdn.LinearAttentionDims(Hk, Hv, D, D, 4)
    rng, conv_w, A_log, dt_bias, norm_w = _params(31, Hk, Hv)
    x = _inputs(rng, B, Hk, Hv, True)
    conv = _bf16(rng.standard_normal((B, 3, dims.conv_dim), dtype=np.float32))
    state = rng.standard_normal((B, Hv, D, D), dtype=np.float32) * np.float32(0.05)
    bf = torch.bfloat16
    state_dev = _dev(state, gpu)
    out, conv_out, state_out = gdn.fused_decode_step(
        _dev(x["qkv"], gpu, bf), _dev(x["z"], gpu, bf), _dev(x["a"], gpu, bf),
        _dev(x["b"], gpu, bf), _dev(conv, gpu, bf), state_dev, _dev(conv_w, gpu),
        _dev(A_log, gpu), _dev(dt_bias, gpu), _dev(norm_w, gpu), 1e-6, dims, state_out=state_dev)
    out_ref, conv_ref, state_ref = cref.decode_step(
        x["qkv"], conv, conv_w, x["a"], x["b"], A_log, dt_bias, state, x["z"], norm_w, 1e-6,
        (Hk, Hv, D, D), True, state_out=state)  # the oracle also updates in place
    assert out.dtype == bf and out.shape == (B, Hv, D)
    assert_bf16_out_close(out.float().cpu().numpy(), out_ref)
    np.testing.assert_array_equal(conv_out.float().cpu().numpy(), conv_ref)
    assert _state_rel_err(state_out, state_ref) < 1e-3


def test_decode_hv64_chained_in_place_steps_match_c_oracle(gpu):
    """Four chained steps at B=16, Hv=64: the state updated in place, the
    conv state rolled into the other of two buffers each step, as the decode
    loop runs."""

    B, Hk, Hv = 16, 16, 64
    dims = gdn.LinearAttentionDims(Hk, Hv, D, D, 4)
    rng, conv_w, A_log, dt_bias, norm_w = _params(32, Hk, Hv)
    conv_ref = _bf16(rng.standard_normal((B, 3, dims.conv_dim), dtype=np.float32))
    state_ref = rng.standard_normal((B, Hv, D, D), dtype=np.float32) * np.float32(0.05)
    bf = torch.bfloat16
    state_dev, conv_dev = _dev(state_ref, gpu), _dev(conv_ref, gpu, bf)
    conv_spare = torch.empty_like(conv_dev)
    params = [_dev(p, gpu) for p in (conv_w, A_log, dt_bias, norm_w)]
    for step in range(4):
        x = _inputs(rng, B, Hk, Hv, True)
        out, _, _ = gdn.fused_decode_step(
            _dev(x["qkv"], gpu, bf), _dev(x["z"], gpu, bf), _dev(x["a"], gpu, bf),
            _dev(x["b"], gpu, bf), conv_dev, state_dev, *params, 1e-6, dims,
            conv_out=conv_spare, state_out=state_dev)
        conv_dev, conv_spare = conv_spare, conv_dev
        out_ref, conv_ref, state_ref = cref.decode_step(
            x["qkv"], conv_ref, conv_w, x["a"], x["b"], A_log, dt_bias, state_ref, x["z"], norm_w,
            1e-6, (Hk, Hv, D, D), True)
        assert_bf16_out_close(out.float().cpu().numpy(), out_ref)
        np.testing.assert_array_equal(conv_dev.float().cpu().numpy(), conv_ref)
        assert _state_rel_err(state_dev, state_ref) < 1e-3, step


def test_decode_hv64_pool_with_half_bits_and_arrivals_matches_c_oracle(gpu):
    """B=16 of a 40-slot pool at Hv=64: the conv state in the pool's two
    halves, the kernel flipping each decoded slot's bit once its 64 value
    heads have arrived. Three steps, each against the oracle on the gathered
    sequences; undecoded slots keep their state and bits, counters return to
    zero."""

    P, Hk, Hv = 40, 16, 64
    slots = [37, 0, 5, 12, 39, 21, 8, 30, 3, 17, 26, 14, 33, 1, 9, 22]
    B = len(slots)
    dims = gdn.LinearAttentionDims(Hk, Hv, D, D, 4)
    rng, conv_w, A_log, dt_bias, norm_w = _params(33, Hk, Hv)
    conv0 = _bf16(rng.standard_normal((P, 3, dims.conv_dim), dtype=np.float32))
    state0 = rng.standard_normal((P, Hv, D, D), dtype=np.float32) * np.float32(0.05)
    bits0 = rng.integers(0, 2, P).astype(np.int32)
    conv_buf = torch.zeros((2 * P, 3, dims.conv_dim), dtype=torch.bfloat16, device=gpu)
    for s in range(P):
        conv_buf[s + P * int(bits0[s])] = _dev(conv0[s], gpu, torch.bfloat16)
    state_dev = _dev(state0, gpu)
    half = torch.from_numpy(bits0).to(gpu)
    arrivals = torch.zeros(P, dtype=torch.int32, device=gpu)
    idx = np.array(slots)
    conv_ref, state_ref = conv0[idx].copy(), state0[idx].copy()
    untouched = np.setdiff1d(np.arange(P), idx)
    params = [_dev(p, gpu) for p in (conv_w, A_log, dt_bias, norm_w)]
    bf = torch.bfloat16
    slot_t = torch.tensor(slots, dtype=torch.int32, device=gpu)
    for step in range(3):
        x = _inputs(rng, B, Hk, Hv, True)
        out, _, _ = gdn.fused_decode_step(
            _dev(x["qkv"], gpu, bf), _dev(x["z"], gpu, bf), _dev(x["a"], gpu, bf),
            _dev(x["b"], gpu, bf), conv_buf, state_dev, *params, 1e-6, dims, slots=slot_t,
            conv_half=half, conv_arrivals=arrivals)
        out_ref, conv_ref, state_ref = cref.decode_step(
            x["qkv"], conv_ref, conv_w, x["a"], x["b"], A_log, dt_bias, state_ref, x["z"], norm_w,
            1e-6, (Hk, Hv, D, D), True)
        assert_bf16_out_close(out.float().cpu().numpy(), out_ref)
        bits = device_halves(half, arrivals).cpu().numpy()
        expect_bits = bits0.copy()
        expect_bits[idx] ^= (step + 1) & 1
        np.testing.assert_array_equal(bits, expect_bits)
        assert counters_settled(arrivals)
        rows = torch.from_numpy(idx + P * bits[idx]).to(gpu)
        np.testing.assert_array_equal(conv_buf[rows].float().cpu().numpy(), conv_ref)
        assert _state_rel_err(state_dev[torch.from_numpy(idx).to(gpu)], state_ref) < 1e-3, step
    keep = torch.from_numpy(untouched).to(gpu)
    assert torch.equal(state_dev[keep], _dev(state0[untouched], gpu))
    np.testing.assert_array_equal(device_halves(half, arrivals).cpu().numpy()[untouched], bits0[untouched])


def test_decode_b64_hv32_256_chained_steps_match_c_oracle(gpu):
    """The B=64, Hv=32 decode benchmark's pattern at its full length: 256
    steps, state in place, conv state alternating between two buffers,
    output y in bf16 (no gate); every step's y and conv state checked, the
    state after steps 1, 64 and 256."""

    B, Hk, Hv, steps = 64, 16, 32, 256
    dims = gdn.LinearAttentionDims(Hk, Hv, D, D, 4)
    rng, conv_w, A_log, dt_bias, _ = _params(34, Hk, Hv)
    conv_ref = _bf16(rng.standard_normal((B, 3, dims.conv_dim), dtype=np.float32))
    state_ref = rng.standard_normal((B, Hv, D, D), dtype=np.float32) * np.float32(0.05)
    bf = torch.bfloat16
    state_dev, conv_dev = _dev(state_ref, gpu), _dev(conv_ref, gpu, bf)
    conv_spare = torch.empty_like(conv_dev)
    params = [_dev(p, gpu) for p in (conv_w, A_log, dt_bias)]
    for step in range(steps):
        x = _inputs(rng, B, Hk, Hv, False)
        out, _, _ = gdn.fused_decode_step(
            _dev(x["qkv"], gpu, bf), None, _dev(x["a"], gpu, bf), _dev(x["b"], gpu, bf),
            conv_dev, state_dev, *params, None, 1e-6, dims, conv_out=conv_spare,
            state_out=state_dev, y_dtype=bf)
        conv_dev, conv_spare = conv_spare, conv_dev
        out_ref, conv_ref, state_ref = cref.decode_step(
            x["qkv"], conv_ref, conv_w, x["a"], x["b"], A_log, dt_bias, state_ref, None, None,
            1e-6, (Hk, Hv, D, D), True, state_out=state_ref)
        assert out.dtype == bf
        got = out.float().cpu().numpy()
        assert_bf16_out_close(got, out_ref)
        # y is small here (|y| ~ 0.1): also within 1 % of its largest value
        assert np.abs(got - out_ref).max() <= 1e-2 * np.abs(out_ref).max(), step
        np.testing.assert_array_equal(conv_dev.float().cpu().numpy(), conv_ref)
        if step in (0, 63, steps - 1):
            assert _state_rel_err(state_dev, state_ref) < 1e-3, step
