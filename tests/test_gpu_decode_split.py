"""GPU tests of the fused decode's row split. With few sequences (B * Hv up
to 128) a step without the gated norm shares each value head among several
workgroups, each reading, updating and storing its share of the 128 state
rows: 8 at B=1, 4 at B=2 and 2 at B=4 for Hv=32. A batch of 16 (B * Hv =
512) runs one 256-thread workgroup per head, and decoding the same
sequences in it gives the reference bits: the split launches must
reproduce output, conv state and ssm state bit for bit, with the state
updated in place. Steps with the gated norm keep one workgroup per head at
every B (a split reading the whole tile would race with the other splits'
in-place rows), of 512 threads up to 256 heads (two row blocks); the same
comparison covers them. Also checked against the C oracle (gdn_ref.c) at B=1
and B=4 over chained steps, and on a slot pool whose conv half bits the
kernel flips (each slot's bit once per step, counted over all the
workgroups of its heads). From 2048 (sequence, head) pairs a step without
the norm runs two workgroups per head again (B=64 at Hv=32): checked the
same way against one workgroup per head, directly and through a pool."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from oracle import cref
from tests.helpers import assert_bf16_out_close, counters_settled, device_halves, layer_params, max_rel

pytestmark = pytest.mark.gpu

D = 128
HK, HV = 16, 32
DIMS = gdn.LinearAttentionDims(HK, HV, D, D, 4)
DT = (HK, HV, D, D)


def _bf16(x) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).bfloat16().float().numpy()


def _case(seed, B, bf16: bool):
    rng = np.random.default_rng(seed)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, DT)
    f = lambda *s: rng.standard_normal(s, dtype=np.float32)
    rnd = _bf16 if bf16 else (lambda x: x)
    return dict(conv_w=conv_w, A_log=A_log, dt_bias=dt_bias, norm_w=norm_w,
                conv=rnd(f(B, 3, DIMS.conv_dim)), state=f(B, HV, D, D) * np.float32(0.05),
                steps=[dict(qkv=rnd(f(B, DIMS.conv_dim)), z=rnd(f(B, HV, D)), a=rnd(f(B, HV)),
                            b=rnd(f(B, HV))) for _ in range(4)])


def _dev(x, gpu, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu).to(dtype)


def _params(c, gpu):
    return [_dev(c[k], gpu) for k in ("conv_w", "A_log", "dt_bias", "norm_w")]


def _step(x, rows, conv, state, params, gpu, adt, with_z, **kw):
    """One fused decode step of the sequences ``rows`` (state in place)."""

    return gdn.fused_decode_step(
        _dev(x["qkv"][rows], gpu, adt), _dev(x["z"][rows], gpu, adt) if with_z else None,
        _dev(x["a"][rows], gpu, adt), _dev(x["b"][rows], gpu, adt), conv, state, *params[:3],
        params[3] if with_z else None, 1e-6, DIMS, state_out=state, **kw)


@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("with_z", [True, False])
def test_split_launches_match_one_workgroup_per_head_bit_for_bit(gpu, act, with_z):
    """Sequences 0..B-1 decoded alone (B = 1, 2, 4, 8; without the norm
    split 8, 4, 2, 1; with it, 512-thread workgroups) against the same
    sequences inside the batch of 16 (one 256-thread workgroup per head),
    over four chained in-place steps: output, rolled conv state and ssm
    state identical."""

    bf16 = act == "bf16"
    adt = torch.bfloat16 if bf16 else torch.float32
    c = _case(40 + bf16 + 2 * with_z, 16, bf16)
    params = _params(c, gpu)
    ref_state, ref_conv = _dev(c["state"], gpu), _dev(c["conv"], gpu, adt)
    runs = {B: (_dev(c["state"][:B], gpu), _dev(c["conv"][:B], gpu, adt)) for B in (1, 2, 4, 8)}
    for step, x in enumerate(c["steps"]):
        ref_out, ref_conv, _ = _step(x, slice(0, 16), ref_conv, ref_state, params, gpu, adt, with_z)
        for B, (state, conv) in runs.items():
            out, conv_new, _ = _step(x, slice(0, B), conv, state, params, gpu, adt, with_z)
            runs[B] = (state, conv_new)
            assert torch.equal(out, ref_out[:B]), (B, step)
            assert torch.equal(conv_new, ref_conv[:B]), (B, step)
            assert torch.equal(state, ref_state[:B]), (B, step)


@pytest.mark.parametrize("with_z", [False, True])
@pytest.mark.parametrize("B", [1, 4])
def test_split_decode_matches_c_oracle(gpu, B, with_z):
    """B=1 and B=4 (bf16) over four chained in-place steps against the C
    oracle: the output (gated norm, or y of the split launches, both in
    bf16) within max(2e-2, two bf16 ulps), conv state bit for bit, ssm state
    within 1e-5 of its largest value."""

    c = _case(50 + B + 10 * with_z, B, True)
    params = _params(c, gpu)
    state, conv = _dev(c["state"], gpu), _dev(c["conv"], gpu, torch.bfloat16)
    ref_state, ref_conv = c["state"].copy(), c["conv"].copy()
    for step, x in enumerate(c["steps"]):
        out, conv, _ = _step(x, slice(0, B), conv, state, params, gpu, torch.bfloat16, with_z,
                             y_dtype=torch.bfloat16)
        out_ref, ref_conv, ref_state = cref.decode_step(
            x["qkv"], ref_conv, c["conv_w"], x["a"], x["b"], c["A_log"], c["dt_bias"], ref_state,
            x["z"] if with_z else None, c["norm_w"] if with_z else None, 1e-6, DT, True)
        assert out.dtype == torch.bfloat16
        assert_bf16_out_close(out.float().cpu().numpy(), out_ref)
        np.testing.assert_array_equal(conv.float().cpu().numpy(), ref_conv)
        assert max_rel(state.cpu().numpy(), ref_state) < 1e-5, step


def test_split_decode_on_a_pool_flips_each_slot_once_per_step(gpu):
    """One slot (B=1, split 8) of a 4-slot pool, then slots 3 and 0 (B=2,
    split 4), without the norm: the conv state in the pool's two halves, the
    kernel flipping a decoded slot's bit once all its Hv * split workgroups
    have read it. Each step's y matches the oracle; the arrival counters end
    at zero."""

    P = 4
    c = _case(60, P, True)
    params = _params(c, gpu)
    bits0 = np.array([0, 1, 1, 0], np.int32)
    conv_buf = torch.zeros((2 * P, 3, DIMS.conv_dim), dtype=torch.bfloat16, device=gpu)
    for s in range(P):
        conv_buf[s + P * int(bits0[s])] = _dev(c["conv"][s], gpu, torch.bfloat16)
    state = _dev(c["state"], gpu)
    half = torch.from_numpy(bits0.copy()).to(gpu)
    arrivals = torch.zeros(P, dtype=torch.int32, device=gpu)
    ref_conv, ref_state = c["conv"].copy(), c["state"].copy()
    flips = np.zeros(P, np.int32)
    for step, slots in enumerate([[2], [2], [3, 0], [3, 0]]):
        x = c["steps"][step]
        idx = np.array(slots)
        rows = slice(0, len(slots))
        out, _, _ = gdn.fused_decode_step(
            _dev(x["qkv"][rows], gpu, torch.bfloat16), None,
            _dev(x["a"][rows], gpu, torch.bfloat16), _dev(x["b"][rows], gpu, torch.bfloat16),
            conv_buf, state, *params[:3], None, 1e-6, DIMS,
            slots=torch.tensor(slots, dtype=torch.int32, device=gpu), conv_half=half,
            conv_arrivals=arrivals, y_dtype=torch.bfloat16)
        out_ref, nc, ns = cref.decode_step(
            x["qkv"][rows], ref_conv[idx], c["conv_w"], x["a"][rows], x["b"][rows], c["A_log"],
            c["dt_bias"], ref_state[idx], None, None, 1e-6, DT, True)
        ref_conv[idx], ref_state[idx] = nc, ns
        flips[idx] ^= 1
        assert_bf16_out_close(out.float().cpu().numpy(), out_ref)
        bits = device_halves(half, arrivals).cpu().numpy()
        np.testing.assert_array_equal(bits, bits0 ^ flips)
        assert counters_settled(arrivals)
        cur = torch.from_numpy(np.arange(P) + P * bits).to(gpu)
        np.testing.assert_array_equal(conv_buf[cur].float().cpu().numpy(), ref_conv)
        assert max_rel(state.cpu().numpy(), ref_state) < 1e-5, step


@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_pair_split_at_many_heads_matches_one_workgroup_per_head(gpu, act):
    """B=64 (B * Hv = 2048 heads): a step without the gated norm gives each
    head two workgroups. Over three chained in-place steps its output equals
    sequences 0-7 decoded alone (256 heads, one workgroup each), and its conv
    and ssm state equal the same steps taken with the gated norm (one
    workgroup per head at every B), bit for bit. Then the same steps through
    a 64-slot pool in reverse slot order, the kernel flipping each slot's conv
    half once per step (2 * Hv shares of 2^16 per slot): the same outputs and
    states, and the counters' bits below 16 back at zero."""

    bf16 = act == "bf16"
    B, adt = 64, torch.bfloat16 if bf16 else torch.float32
    c = _case(70 + bf16, B, bf16)
    params = _params(c, gpu)
    st_split, cv_split = _dev(c["state"], gpu), _dev(c["conv"], gpu, adt)
    st_norm, cv_norm = _dev(c["state"], gpu), _dev(c["conv"], gpu, adt)
    st8, cv8 = _dev(c["state"][:8], gpu), _dev(c["conv"][:8], gpu, adt)
    outs = []
    for step, x in enumerate(c["steps"][:3]):
        out, cv_split, _ = _step(x, slice(0, B), cv_split, st_split, params, gpu, adt, False,
                                 y_dtype=torch.bfloat16)
        _, cv_norm, _ = _step(x, slice(0, B), cv_norm, st_norm, params, gpu, adt, True)
        out8, cv8, _ = _step(x, slice(0, 8), cv8, st8, params, gpu, adt, False, y_dtype=torch.bfloat16)
        outs.append(out)
        assert torch.equal(out[:8], out8), step
        assert torch.equal(cv_split, cv_norm), step
        assert torch.equal(st_split, st_norm), step

    # sequence i in slot P - 1 - i of a pool of P = B slots
    P = B
    slot_of = np.arange(P)[::-1].copy()
    bits0 = (np.arange(P) % 3 == 0).astype(np.int32)
    conv_buf = torch.zeros((2 * P, 3, DIMS.conv_dim), dtype=adt, device=gpu)
    pool = torch.empty((P, HV, D, D), dtype=torch.float32, device=gpu)
    for i in range(B):
        sl = int(slot_of[i])
        conv_buf[sl + P * int(bits0[sl])] = _dev(c["conv"][i], gpu, adt)
        pool[sl] = _dev(c["state"][i], gpu)
    half = torch.from_numpy(bits0.copy()).to(gpu)
    arrivals = torch.zeros(P, dtype=torch.int32, device=gpu)
    slots = torch.from_numpy(slot_of.astype(np.int32)).to(gpu)
    for step, x in enumerate(c["steps"][:3]):
        out, _, _ = gdn.fused_decode_step(
            _dev(x["qkv"], gpu, adt), None, _dev(x["a"], gpu, adt), _dev(x["b"], gpu, adt),
            conv_buf, pool, *params[:3], None, 1e-6, DIMS, slots=slots, conv_half=half,
            conv_arrivals=arrivals, y_dtype=torch.bfloat16)
        assert torch.equal(out, outs[step]), step
        np.testing.assert_array_equal(device_halves(half, arrivals).cpu().numpy(), bits0 ^ ((step + 1) & 1))
        assert counters_settled(arrivals)
    cur = torch.from_numpy(slot_of + P * device_halves(half, arrivals).cpu().numpy()[slot_of]).to(gpu)
    assert torch.equal(conv_buf[cur], cv_norm)
    assert torch.equal(pool[torch.from_numpy(slot_of).to(gpu)], st_norm)
