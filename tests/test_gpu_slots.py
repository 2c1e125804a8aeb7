"""Decode of active sequences at arbitrary slots of a device state pool
(the pool with slot indices): the fused kernel on slots equals the same
kernel on the gathered sequences, leaves every other slot untouched, and the
layer's pooled decode after a chunked prefill (the transformer's prefill
loop, transformer.py:283-304, at layer level) equals per-sequence calls."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_lean_moe_amd as gdn
from mlx_lean_moe_amd import _lib
from tests.helpers import counters_settled, device_halves, layer_inputs, layer_params
from tests.test_gpu_layer import HIDDEN, _build

pytestmark = pytest.mark.gpu

DIMS = gdn.LinearAttentionDims(2, 4, 128, 128, 4)


def _pool_case(seed, P, B, adt, dev):
    rng = np.random.default_rng(seed)
    dt = (DIMS.num_key_heads, DIMS.num_value_heads, 128, 128)
    conv_w, A_log, dt_bias, norm_w = layer_params(rng, dt)
    qkv, z, a, b = layer_inputs(rng, dt, L=1, act_bf16=adt == torch.bfloat16, B=B)
    t = lambda x, dtype=torch.float32: torch.tensor(np.asarray(x, np.float32), device=dev).to(dtype)
    conv = t(rng.standard_normal((P, 3, DIMS.conv_dim)), adt)
    state = t(rng.standard_normal((P, DIMS.num_value_heads, 128, 128)) * 0.05)
    return dict(qkv=t(qkv[:, 0], adt), z=t(z[:, 0], adt), a=t(a[:, 0], adt), b=t(b[:, 0], adt),
                conv=conv, state=state, conv_w=t(conv_w), A_log=t(A_log), dt_bias=t(dt_bias),
                norm_w=t(norm_w))


@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("with_z", [False, True])
def test_slot_decode_equals_decode_of_gathered_sequences(gpu, act, with_z):
    adt = torch.bfloat16 if act == "bf16" else torch.float32
    P, slots = 7, [5, 0, 3]
    c = _pool_case(11, P, len(slots), adt, gpu)
    z = c["z"] if with_z else None
    idx = torch.tensor(slots, device=gpu)
    conv_g, state_g = c["conv"][idx].clone(), c["state"][idx].clone()
    ref_out, ref_conv, ref_state = gdn.fused_decode_step(
        c["qkv"], z, c["a"], c["b"], conv_g, state_g, c["conv_w"], c["A_log"], c["dt_bias"],
        c["norm_w"], 1e-6, DIMS, state_out=state_g)
    before = c["state"].clone()
    conv_before = c["conv"].clone()
    out, conv_out, state_out = gdn.fused_decode_step(
        c["qkv"], z, c["a"], c["b"], c["conv"], c["state"], c["conv_w"], c["A_log"],
        c["dt_bias"], c["norm_w"], 1e-6, DIMS, slots=slots)
    assert state_out is c["state"]
    assert torch.equal(out, ref_out)
    assert torch.equal(conv_out, ref_conv)
    assert torch.equal(c["state"][idx], ref_state)
    others = torch.tensor([i for i in range(P) if i not in slots], device=gpu)
    assert torch.equal(c["state"][others], before[others])
    assert torch.equal(c["conv"], conv_before)  # the pool's conv rows are the caller's to update


def test_conv_half_rolls_into_the_other_half_without_a_copy(gpu):
    """Conv state in the two halves of one array, each slot's half given by
    the pool's bits: a row reads its slot's current row and writes the
    other; untouched rows keep their bytes, and the bits are not changed."""

    P, slots = 6, [4, 1]
    c = _pool_case(13, P, len(slots), torch.bfloat16, gpu)
    buf = torch.cat([c["conv"], torch.zeros_like(c["conv"])])  # slot s in row s (half 0)
    buf[P + 1] = c["conv"][1]  # slot 1 currently in half 1: row 7 (row 1 is stale)
    buf[1].fill_(3.0)
    bits = [0, 1, 0, 1, 0, 0]
    half = torch.tensor(bits, dtype=torch.int32, device=gpu)
    idx = torch.tensor(slots, device=gpu)
    ref_out, ref_conv, ref_state = gdn.fused_decode_step(
        c["qkv"], c["z"], c["a"], c["b"], c["conv"][idx].clone(), c["state"][idx].clone(),
        c["conv_w"], c["A_log"], c["dt_bias"], c["norm_w"], 1e-6, DIMS)
    before = buf.clone()
    out, conv_out, _ = gdn.fused_decode_step(
        c["qkv"], c["z"], c["a"], c["b"], buf, c["state"], c["conv_w"], c["A_log"], c["dt_bias"],
        c["norm_w"], 1e-6, DIMS, slots=slots, conv_half=half)
    assert conv_out is buf
    assert torch.equal(out, ref_out)
    written = {4 + P: ref_conv[0], 1: ref_conv[1]}  # slot 4: half 0 -> 1; slot 1: half 1 -> 0
    for r in range(2 * P):
        assert torch.equal(buf[r], written[r] if r in written else before[r]), r
    assert torch.equal(c["state"][idx], ref_state)
    assert half.tolist() == bits
    # with the arrival counters the kernel flips the decoded slots' halves
    # (2^16 added to their counters, bit 16 the parity; the bits are only
    # read), and a second step reads the halves the first one wrote
    half[4] = 1  # the step above left slot 4 in half 1 and slot 1 in half 0
    half[1] = 0
    arrivals = torch.zeros(P, dtype=torch.int32, device=gpu)
    state2 = c["state"].clone()
    out2, _, _ = gdn.fused_decode_step(
        c["qkv"], c["z"], c["a"], c["b"], buf, state2, c["conv_w"], c["A_log"], c["dt_bias"],
        c["norm_w"], 1e-6, DIMS, slots=slots, conv_half=half, conv_arrivals=arrivals)
    assert half.tolist() != bits and device_halves(half, arrivals).tolist() == bits
    assert arrivals.tolist() == [65536 if i in (4, 1) else 0 for i in range(P)]
    ref2 = gdn.fused_decode_step(c["qkv"], c["z"], c["a"], c["b"], ref_conv.clone(), ref_state.clone(),
                                 c["conv_w"], c["A_log"], c["dt_bias"], c["norm_w"], 1e-6, DIMS)
    assert torch.equal(out2, ref2[0])
    assert torch.equal(buf[4], ref2[1][0]) and torch.equal(buf[1 + P], ref2[1][1])
    with pytest.raises(ValueError, match="conv_arrivals"):
        gdn.fused_decode_step(c["qkv"], c["z"], c["a"], c["b"], buf, c["state"], c["conv_w"],
                              c["A_log"], c["dt_bias"], c["norm_w"], 1e-6, DIMS, slots=slots,
                              conv_half=bits, conv_arrivals=arrivals)
    for bad, conv_out in (([0, 2, 0, 0, 0, 0], None), ([0, 1], None), (bits, buf.clone())):
        with pytest.raises(ValueError):
            gdn.fused_decode_step(c["qkv"], c["z"], c["a"], c["b"], buf, c["state"], c["conv_w"],
                                  c["A_log"], c["dt_bias"], c["norm_w"], 1e-6, DIMS, slots=slots,
                                  conv_half=bad, conv_out=conv_out)
    with pytest.raises(ValueError, match="needs slots"):
        gdn.fused_decode_step(c["qkv"], c["z"], c["a"], c["b"], buf[:2], c["state"][:2],
                              c["conv_w"], c["A_log"], c["dt_bias"], c["norm_w"], 1e-6, DIMS,
                              conv_half=bits[:2])


def test_arrival_counters_carry_across_the_sign_and_wrap(gpu):
    """The counters' bit 16 keeps flipping once per step where a count
    crosses 2^31 (int32 sign) and wraps at 2^32: two chained steps read and
    write the halves the shares select, as the dense reference steps do."""

    P, slots = 4, [1, 2]
    c = _pool_case(17, P, len(slots), torch.bfloat16, gpu)
    # bits 0; counters with bit 16 set: both slots currently in half 1
    half = torch.zeros(P, dtype=torch.int32, device=gpu)
    arrivals = torch.tensor([0, 0x7FFF0000, -0x10000, 0], dtype=torch.int32, device=gpu)
    buf = torch.zeros((2 * P,) + tuple(c["conv"].shape[1:]), dtype=c["conv"].dtype, device=gpu)
    for s_ in slots:
        buf[P + s_] = c["conv"][s_]
    idx = torch.tensor(slots, device=gpu)
    conv_g, state_g = c["conv"][idx].clone(), c["state"][idx].clone()
    state = c["state"].clone()
    for step in range(2):
        ref_out, conv_g, state_g = gdn.fused_decode_step(
            c["qkv"], c["z"], c["a"], c["b"], conv_g, state_g, c["conv_w"], c["A_log"], c["dt_bias"],
            c["norm_w"], 1e-6, DIMS)
        out, _, _ = gdn.fused_decode_step(
            c["qkv"], c["z"], c["a"], c["b"], buf, state, c["conv_w"], c["A_log"], c["dt_bias"],
            c["norm_w"], 1e-6, DIMS, slots=slots, conv_half=half, conv_arrivals=arrivals)
        assert torch.equal(out, ref_out), step
        now = device_halves(half, arrivals).tolist()
        assert now == [0, step % 2, step % 2, 0], (step, now)
        for i, s_ in enumerate(slots):
            assert torch.equal(buf[s_ + P * now[s_]], conv_g[i]), (step, s_)
        assert torch.equal(state[idx], state_g)
    assert arrivals.tolist() == [0, 0x7FFF0000 + 2 * 0x10000 - 2 ** 32, 0x10000, 0]
    assert half.tolist() == [0] * P


def test_pool_advance_flips_the_bits_of_the_decoded_slots(gpu):
    pool = gdn.RecurrentStatePool(300, 4, DIMS.conv_dim, DIMS.num_value_heads, 128, 128,
                                  dtype=torch.bfloat16, device=gpu)
    rng = np.random.default_rng(5)
    want = np.zeros(300, np.int64)
    for n in (3, 257, 300, 1):  # more slots than one workgroup holds, and all of them
        slots = rng.permutation(300)[:n].tolist()
        pool.advance(slots)
        want[slots] ^= 1
        assert pool.conv_half.tolist() == want.tolist()
        assert pool.conv_half_dev.cpu().tolist() == want.tolist()


@pytest.mark.parametrize("with_z", [False, True])
def test_row_strided_inputs_are_read_in_place(gpu, with_z):
    """qkv, z, a and b as column slices of one stacked (B, C + Hv Dv + 2 Hv)
    array (the stacked projection's output) give the same bits as packed
    copies."""

    P, slots = 5, [3, 0, 4]
    c = _pool_case(14, P, len(slots), torch.bfloat16, gpu)
    B = len(slots)
    stacked = torch.cat([c["qkv"], c["z"].reshape(B, -1), c["a"], c["b"], c["a"][:, :3]], 1)
    qkv, z, a, b = torch.split(stacked, [DIMS.conv_dim, DIMS.value_dim, DIMS.num_value_heads,
                                         DIMS.num_value_heads, 3], 1)[:4]
    z = z.reshape(B, DIMS.num_value_heads, 128)
    assert not qkv.is_contiguous() and not z.is_contiguous() and not a.is_contiguous()
    state = c["state"].clone()
    conv = c["conv"]
    res = []
    for args, st in (((c["qkv"], c["z"], c["a"], c["b"]), c["state"]), ((qkv, z, a, b), state)):
        res.append(gdn.fused_decode_step(args[0], args[1] if with_z else None, args[2], args[3], conv,
                                         st, c["conv_w"], c["A_log"], c["dt_bias"], c["norm_w"],
                                         1e-6, DIMS, slots=slots))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    assert torch.equal(c["state"], state)


def test_slot_outside_pool_touches_no_state(gpu):
    """The C ABI's own guard (the Python layer rejects such slots first): a
    row whose slot lies outside the pool writes NaN and leaves the state."""

    P, B = 4, 2
    c = _pool_case(12, P, B, torch.bfloat16, gpu)
    before = c["state"].clone()
    slots = torch.tensor([P, 1], dtype=torch.int32, device=gpu)
    conv_out = torch.empty(B, 3, DIMS.conv_dim, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(B, DIMS.num_value_heads, 128, dtype=torch.float32, device=gpu)
    _lib.call("gdn_decode_step", _lib.ptr(c["qkv"]), _lib.ptr(c["conv"]), _lib.ptr(conv_out),
              _lib.ptr(c["conv_w"].reshape(DIMS.conv_dim, 4).contiguous()), _lib.ptr(c["a"]),
              _lib.ptr(c["b"]), _lib.ptr(c["A_log"]), _lib.ptr(c["dt_bias"]), _lib.ptr(c["state"]),
              _lib.ptr(c["state"]), None, None, 1e-6, _lib.ptr(out), _lib.GDN_F32, B, 2, 4, 128,
              128, 4, _lib.GDN_BF16, _lib.ptr(slots), P, None, None, None, _lib.stream_ptr(gpu))
    torch.cuda.synchronize()
    assert torch.isnan(out[0]).all() and torch.isfinite(out[1]).all()
    assert torch.equal(c["state"][0], before[0]) and torch.equal(c["state"][2:], before[2:])
    assert not torch.equal(c["state"][1], before[1])


def test_pooled_decode_after_chunked_prefill_matches_per_sequence_calls(gpu):
    layer, _ = _build(6, DIMS, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(106)
    P = 6
    pool = gdn.RecurrentStatePool(P, 4, DIMS.conv_dim, DIMS.num_value_heads, 128, 128,
                                  dtype=torch.bfloat16, device=gpu)
    slots = [4, 1, 2]
    prompts = [torch.tensor(rng.standard_normal((n, HIDDEN)), dtype=torch.bfloat16, device=gpu)
               for n in (9, 5, 1)]
    caches = [layer.new_cache(torch.bfloat16) for _ in slots]
    for slot, p, cache in zip(slots, prompts, caches):
        # prefill in chunks of 4 tokens, carrying the cache, then copy it into
        # the pool; the cache itself goes on as the per-sequence reference
        for start in range(0, p.shape[0], 4):
            layer(p[start:start + 4], cache)
        pool.load(slot, cache)
    for step in range(3):
        active = slots if step != 1 else [2, 4]  # a step where one sequence sits out
        x = torch.tensor(rng.standard_normal((len(active), HIDDEN)), dtype=torch.bfloat16,
                         device=gpu)
        out = layer.decode_batch(x, pool, slots=active)
        ref = torch.stack([layer(x[i], caches[slots.index(s)]) for i, s in enumerate(active)])
        torch.testing.assert_close(out.float(), ref.float(), rtol=0, atol=0)
        # the decode kernel flipped the decoded slots' halves itself (its
        # counters' bit 16) and left the counters' low bits at zero
        assert pool.device_halves().cpu().tolist() == pool.conv_half.tolist()
        assert counters_settled(pool.conv_arrivals)
    for slot, cache in zip(slots, caches):
        torch.testing.assert_close(pool.ssm_state[slot], cache.ssm_state, rtol=0, atol=0)
        torch.testing.assert_close(pool.conv_state[slot], cache.conv_state, rtol=0, atol=0)
        assert int(pool.size[slot]) == cache.size
    for free in (0, 3, 5):
        assert not pool.ssm_state[free].any() and not pool.conv_state[free].any()


def test_pooled_decode_with_non_power_of_two_heads(gpu):
    """Hv = 6 value heads: the kernel cannot split a step's 2^16 into equal
    shares, so decode_batch leaves the counters alone and flips the bits
    with gdn_pool_advance; the steps still equal per-sequence calls."""

    dims = gdn.LinearAttentionDims(2, 6, 128, 128, 4)
    layer, _ = _build(9, dims, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(109)
    pool = gdn.RecurrentStatePool(4, 4, dims.conv_dim, dims.num_value_heads, 128, 128,
                                  dtype=torch.bfloat16, device=gpu)
    slots = [3, 0]
    caches = [layer.new_cache(torch.bfloat16) for _ in slots]
    for slot, cache in zip(slots, caches):
        layer(torch.tensor(rng.standard_normal((3, HIDDEN)), dtype=torch.bfloat16, device=gpu), cache)
        pool.load(slot, cache)
    for _ in range(3):
        x = torch.tensor(rng.standard_normal((2, HIDDEN)), dtype=torch.bfloat16, device=gpu)
        out = layer.decode_batch(x, pool, slots=slots)
        ref = torch.stack([layer(x[i], caches[i]) for i in range(2)])
        torch.testing.assert_close(out.float(), ref.float(), rtol=0, atol=0)
        assert pool.conv_half_dev.cpu().tolist() == pool.conv_half.tolist()
        assert not pool.conv_arrivals.any()
    for slot, cache in zip(slots, caches):
        torch.testing.assert_close(pool.conv_state[slot], cache.conv_state, rtol=0, atol=0)
        torch.testing.assert_close(pool.ssm_state[slot], cache.ssm_state, rtol=0, atol=0)


def test_decode_graph_replays_equal_eager_decode(gpu):
    """A captured decode step replayed several times, with other eager GPU
    work and synchronizations between replays, equals eager decode_batch on
    a twin pool at every step (outputs and both states)."""

    layer, _ = _build(7, DIMS, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(107)
    P, slots = 6, [5, 2, 3]
    pools = [gdn.RecurrentStatePool(P, 4, DIMS.conv_dim, DIMS.num_value_heads, 128, 128,
                                    dtype=torch.bfloat16, device=gpu) for _ in range(2)]
    for i, p in enumerate((rng.standard_normal((4, HIDDEN)), rng.standard_normal((2, HIDDEN)),
                           rng.standard_normal((7, HIDDEN)))):
        cache = layer.new_cache(torch.bfloat16)
        layer(torch.tensor(p, dtype=torch.bfloat16, device=gpu), cache)
        for pool in pools:
            pool.load(slots[i], cache)
    eager, graphed = pools
    xs = [torch.tensor(rng.standard_normal((3, HIDDEN)), dtype=torch.bfloat16, device=gpu)
          for _ in range(4)]
    step = gdn.DecodeGraph(layer, graphed, slots, xs[0])
    scratch = torch.randn(1 << 20, device=gpu)
    for x in xs:
        ref = layer.decode_batch(x, eager, slots=slots)
        out = step.step(x)
        torch.testing.assert_close(out.float(), ref.float(), rtol=0, atol=0)
        scratch.mul_(1.0001).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
    torch.testing.assert_close(graphed.ssm_state, eager.ssm_state, rtol=0, atol=0)
    torch.testing.assert_close(graphed.conv_state, eager.conv_state, rtol=0, atol=0)
    assert torch.equal(graphed.size, eager.size) and torch.equal(graphed.conv_half, eager.conv_half)
    assert torch.equal(graphed.device_halves(), eager.device_halves())
    assert graphed.device_halves().cpu().tolist() == graphed.conv_half.tolist()
    assert counters_settled(graphed.conv_arrivals)


def test_decode_graph_outlives_the_pools_slot_cache(gpu):
    """The pool keeps at most 64 slot arrays and drops them all when a 65th
    set arrives; a captured step holds its own, so after 65 other slot sets
    have decoded eagerly (and new device memory has been allocated over
    whatever was freed) its replay still decodes its own slots, equal to
    eager decode_batch on a twin pool."""

    layer, _ = _build(8, DIMS, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(108)
    P, slots = 70, [4, 1, 66]
    pools = [gdn.RecurrentStatePool(P, 4, DIMS.conv_dim, DIMS.num_value_heads, 128, 128,
                                    dtype=torch.bfloat16, device=gpu) for _ in range(2)]
    init = torch.tensor(rng.standard_normal((P, DIMS.num_value_heads, 128, 128)) * 0.05,
                        dtype=torch.float32, device=gpu)
    for pool in pools:
        pool.ssm_state.copy_(init)
    eager, graphed = pools
    mk = lambda n: torch.tensor(rng.standard_normal((n, HIDDEN)), dtype=torch.bfloat16, device=gpu)
    step = gdn.DecodeGraph(layer, graphed, slots, mk(3))
    # 65 other single-slot sets through the graphed pool's cache (their
    # slots differ from the graph's, so its slots' states are untouched)
    others = [s for s in range(P) if s not in slots][:65]
    for s in others:
        x1 = mk(1)
        layer.decode_batch(x1, graphed, slots=[s])
        layer.decode_batch(x1, eager, slots=[s])
    assert len(graphed._slot_sets) < 64
    filler = [torch.full((3,), 1 << 20, dtype=torch.int32, device=gpu) for _ in range(256)]
    for _ in range(2):
        x = mk(3)
        ref = layer.decode_batch(x, eager, slots=slots)
        out = step.step(x)
        torch.testing.assert_close(out.float(), ref.float(), rtol=0, atol=0)
    torch.testing.assert_close(graphed.ssm_state, eager.ssm_state, rtol=0, atol=0)
    torch.testing.assert_close(graphed.conv_state, eager.conv_state, rtol=0, atol=0)
    del filler


def test_decode_graph_with_a_residual(gpu):
    """The decoder layer's residual inside the captured step: each replay
    equals eager decode_batch(..., residual=) on a twin pool."""

    layer, _ = _build(8, DIMS, gpu, dtype=torch.bfloat16)
    rng = np.random.default_rng(108)
    P, slots = 4, [3, 1]
    pools = [gdn.RecurrentStatePool(P, 4, DIMS.conv_dim, DIMS.num_value_heads, 128, 128,
                                    dtype=torch.bfloat16, device=gpu) for _ in range(2)]
    for i, n in enumerate((3, 6)):
        cache = layer.new_cache(torch.bfloat16)
        layer(torch.tensor(rng.standard_normal((n, HIDDEN)), dtype=torch.bfloat16, device=gpu), cache)
        for pool in pools:
            pool.load(slots[i], cache)
    eager, graphed = pools
    mk = lambda: torch.tensor(rng.standard_normal((2, HIDDEN)), dtype=torch.bfloat16, device=gpu)
    step = gdn.DecodeGraph(layer, graphed, slots, mk(), residual_example=mk())
    for _ in range(3):
        x, r = mk(), mk()
        ref = layer.decode_batch(x, eager, slots=slots, residual=r)
        out = step.step(x, r)
        assert torch.equal(out, ref)
        torch.cuda.synchronize()
    torch.testing.assert_close(graphed.ssm_state, eager.ssm_state, rtol=0, atol=0)
    with pytest.raises(ValueError, match="without a residual"):
        gdn.DecodeGraph(layer, graphed, [0], mk()[:1]).step(residual=mk()[:1])


_FRESH_PROCESS_GRAPH = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
import mlx_lean_moe_amd as gdn
from tests.test_gpu_layer import HIDDEN, _build
from tests.test_gpu_slots import DIMS

dev = torch.device("cuda:0")
print("fresh process: DecodeGraph before any other GPU work", flush=True)
layer, _ = _build(9, DIMS, dev, dtype=torch.bfloat16)
rng = np.random.default_rng(109)
slots = [2, 0]
pools = [gdn.RecurrentStatePool(3, 4, DIMS.conv_dim, DIMS.num_value_heads, 128, 128,
                                dtype=torch.bfloat16, device=dev) for _ in range(2)]
mk = lambda: torch.tensor(rng.standard_normal((2, HIDDEN)), dtype=torch.bfloat16, device=dev)
step = gdn.DecodeGraph(layer, pools[1], slots, mk())
for _ in range(2):
    x = mk()
    ref = layer.decode_batch(x, pools[0], slots=slots)
    assert torch.equal(step.step(x), ref)
assert torch.equal(pools[1].ssm_state, pools[0].ssm_state)
assert not pools[0].ssm_state[1].any()
print("OK", flush=True)
"""


def test_decode_graph_captured_first_in_a_fresh_process(gpu, tmp_path):
    """A DecodeGraph built before any other GPU work of its process (so
    that the vendor BLAS is first used by the step being captured) replays
    equal to eager decode_batch on a twin pool. Run in a child process: the
    parent's earlier tests have set the libraries up already."""

    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "fresh_graph.py"
    script.write_text(_FRESH_PROCESS_GRAPH)
    proc = subprocess.run([sys.executable, "-u", str(script), root], cwd=root, capture_output=True,
                          text=True, timeout=240)
    assert proc.returncode == 0 and proc.stdout.strip().endswith("OK"), (
        f"child exited {proc.returncode}\nstdout:\n{proc.stdout[-2000:]}\nstderr:\n{proc.stderr[-2000:]}")
