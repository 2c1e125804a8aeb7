"""Benchmark of the gated-delta path on one MI355X.

Default workload (the headline line): batched single-token decode, B=256
sequences, Hk=16 key heads, Hv=64 value heads, d=128, K=4 conv taps, bf16
activations, float32 recurrent state (1 GiB), the z gate and gated RMSNorm
fused; one step = one fused decode launch (conv + SiLU + roll, q/k scaling,
gates, recurrence, gated norm) for all 256 sequences. The state rotates
through four buffers: step s reads buffer s % 4 and writes (s + 2) % 4, so
no step reads what the step before it wrote, and the working set (4 GiB)
exceeds the 256 MB Infinity Cache: the bandwidth figure is HBM's.

Also measured in the same run (reported under "also"):
  decode_b64:   B=64, Hv=32, no gate (128 MiB state, four rotating buffers
                as above: 512 MiB)
  decode_b1:    one sequence (the reference's own decode), Hv=32, with and
                without the gated norm; 64 steps per HIP graph, as the
                launch itself takes longer than the step
  prefill:      B=1, T=4096 chunked prefill (bf16 MFMA), with its roofline
                and CPU baseline
  prefill_f32:  the same with float32 q/k/v/a/b
  prefill_varlen: 16 packed runs of U[128, 8192] tokens (67,128 in all)
  decode_slots: B=64 active sequences at random slots of a 256-sequence pool
  layer_decode: the whole layer's decode step with 4-bit projections, B=64
  of 256 slots, from HIP graphs
  (--workload layer_decode: the same alone, with its parts,
  --batch B active sequences, 64 by default)
  layer_prefill: the whole layer over a 4096-token prompt, 4-bit
  projections (--workload layer_prefill: the same alone)
  qlinear_schemes (alone only): gdn_quantized_matmul_scheme for affine
  2/3/5/6-bit, mxfp4, mxfp8 and nvfp4 codes on the layer's two projection
  shapes at one and 64 rows, weights read from HBM
  decode_sizes (alone only): the decode kernel without the gated norm at
  Hk=16, Hv=32 over B = 1 .. 256, and the headline configuration: kernel
  time and fraction of HBM at each size

python bench.py [--steps K] [--warmup W] [--batch B]
                [--workload decode|decode_b64|decode_b1|decode_slots|decode_sizes|layer_decode|
                            layer_prefill|prefill|prefill_f32|prefill_varlen|qlinear|
                            qlinear_schemes|copy]
(--workload decode_large is the default decode workload under its older name.)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import mlx_lean_moe_amd as gdn  # noqa: E402
from mlx_lean_moe_amd import gated_delta  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "gated-delta tokens/s at 1 GPU; decode HBM GB/s %peak; prefill MFMA util %"


def decode_bytes(B, Hk, Hv, d, K, with_z):
    """Algorithmic HBM bytes of one decode step (per-token terms x B plus the
    per-step parameters)."""

    C = 2 * Hk * d + Hv * d
    per_token = 8 * Hv * d * d + 4 * (K - 1) * C + 2 * C + 4 * Hv + 2 * Hv * d
    per_step = C * K * 4 + 8 * Hv
    if with_z:
        per_token += 2 * Hv * d
        per_step += 4 * d
    return per_token, per_step, B * per_token + per_step


class DecodeWorkload:
    """Synthetic decode inputs resident in HBM, with rotating state buffers."""

    def __init__(self, dev, B, Hk, Hv, with_z, seed=0, n_state=4, n_inputs=8):
        d, K = 128, 4
        self.dims = gdn.LinearAttentionDims(Hk, Hv, d, d, K)
        C = self.dims.conv_dim
        g = torch.Generator(device=dev).manual_seed(seed)
        bf = torch.bfloat16
        randn = lambda *s: torch.randn(*s, generator=g, device=dev)
        self.qkv = [randn(B, C).to(bf) for _ in range(n_inputs)]
        self.a = [randn(B, Hv).to(bf) for _ in range(n_inputs)]
        self.b = [randn(B, Hv).to(bf) for _ in range(n_inputs)]
        self.z = [randn(B, Hv, d).to(bf) for _ in range(n_inputs)] if with_z else None
        self.states = [randn(B, Hv, d, d) * 0.05 for _ in range(n_state)]
        self.convs = [randn(B, K - 1, C).to(bf) for _ in range(2)]
        self.conv_w = randn(C, K) * 0.2
        self.A_log = torch.rand(Hv, generator=g, device=dev) * float(np.log(16))
        self.dt_bias = torch.rand(Hv, generator=g, device=dev) * 2 - 1
        self.norm_w = torch.rand(d, generator=g, device=dev) + 0.5
        self.B, self.with_z = B, with_z
        self.out = torch.empty(B, Hv, d, dtype=bf, device=dev)
        _, _, self.bytes_per_step = decode_bytes(B, Hk, Hv, d, K, with_z)
        self.args = self._bind()

    def _bind(self, stream=None):
        """Pre-resolved C-ABI argument tuples, one per step phase, so the
        timed loop is a bare sequence of launches (on `stream`, by default
        the current one)."""

        from mlx_lean_moe_amd import _lib

        d = self.dims
        lib = _lib.load()
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        n_s, n_i = len(self.states), len(self.qkv)
        phases = []
        # step s reads state buffer s % n_s and writes (s + 2) % n_s: the
        # buffer a step reads was last written two steps earlier
        for s in range(np.lcm(np.lcm(n_s, n_i), 2)):
            phases.append((
                self.qkv[s % n_i].data_ptr(), self.convs[s % 2].data_ptr(),
                self.convs[(s + 1) % 2].data_ptr(), self.conv_w.data_ptr(),
                self.a[s % n_i].data_ptr(), self.b[s % n_i].data_ptr(), self.A_log.data_ptr(),
                self.dt_bias.data_ptr(), self.states[s % n_s].data_ptr(),
                self.states[(s + 2) % n_s].data_ptr(),
                self.z[s % n_i].data_ptr() if self.with_z else None,
                self.norm_w.data_ptr() if self.with_z else None, 1e-6, self.out.data_ptr(),
                _lib.GDN_BF16, self.B, d.num_key_heads, d.num_value_heads, 128, 128, 4,
                _lib.GDN_BF16, None, 0, None, None, None, stream))
        self._fn = lib.gdn_decode_step
        return phases

    def step(self, s):
        rc = self._fn(*self.args[s % len(self.args)])
        if rc != 0:
            raise RuntimeError(f"gdn_decode_step failed with {rc}")


def time_steps(step, steps, warmup):
    """Total time of `steps` back-to-back steps (one event pair on the launch
    stream around the timed region) and, as a cross-check, the mean time of
    one step timed alone (an event pair around each step, which adds the
    events' own overhead of ~2 us per step)."""

    stream = torch.cuda.current_stream()
    for s in range(warmup):
        step(s)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for s in range(steps):
        step(warmup + s)
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(steps)]
    for s, (e0, e1) in enumerate(pairs):
        e0.record(stream)
        step(warmup + steps + s)
        e1.record(stream)
    torch.cuda.synchronize()
    launch_ms = float(np.mean([e0.elapsed_time(e1) for e0, e1 in pairs]))
    return total_ms, launch_ms


class SlotDecodeWorkload:
    """B active sequences decoding out of a device pool of P = 4 B state
    slots (the pool with slot indices): step s takes the next of four
    disjoint random slot sets, so the 512 MB of state the steps touch exceed
    the Infinity Cache. A step is one fused kernel launch on those slots:
    state tiles updated in place at the slots, conv state read from each
    slot's current half of a two-half buffer and rolled into the other."""

    def __init__(self, dev, B, Hk, Hv, seed=0, n_inputs=8):
        d, K = 128, 4
        self.dims = gdn.LinearAttentionDims(Hk, Hv, d, d, K)
        C = self.dims.conv_dim
        P = 4 * B
        g = torch.Generator(device=dev).manual_seed(seed)
        bf = torch.bfloat16
        randn = lambda *s: torch.randn(*s, generator=g, device=dev)
        self.qkv = [randn(B, C).to(bf) for _ in range(n_inputs)]
        self.a = [randn(B, Hv).to(bf) for _ in range(n_inputs)]
        self.b = [randn(B, Hv).to(bf) for _ in range(n_inputs)]
        self.state = randn(P, Hv, d, d) * 0.05
        self.conv = randn(2 * P, K - 1, C).to(bf)  # two halves
        self.conv_w = randn(C, K) * 0.2
        self.A_log = torch.rand(Hv, generator=g, device=dev) * float(np.log(16))
        self.dt_bias = torch.rand(Hv, generator=g, device=dev) * 2 - 1
        self.out = torch.empty(B, Hv, d, dtype=bf, device=dev)
        perm = torch.randperm(P, generator=torch.Generator().manual_seed(seed))
        sets = [perm[i * B:(i + 1) * B] for i in range(4)]
        # a slot set's k-th visit reads half k % 2 and writes the other (the
        # pool's half bits all 0, then all 1); 8 phases (two visits of each
        # set) close the cycle
        self.halves = [torch.full((P,), h, dtype=torch.int32, device=dev) for h in (0, 1)]
        phases = [(sets[ph % 4].to(torch.int32).to(dev), self.halves[(ph // 4) % 2])
                  for ph in range(8)]
        self.phases = phases
        self.B, self.P = B, P
        _, _, self.bytes_per_step = decode_bytes(B, Hk, Hv, d, K, False)
        from mlx_lean_moe_amd import _lib

        self._fn = _lib.load().gdn_decode_step
        stream = torch.cuda.current_stream().cuda_stream
        self.args = [(self.qkv[ph % n_inputs].data_ptr(), self.conv.data_ptr(), self.conv.data_ptr(),
                      self.conv_w.data_ptr(), self.a[ph % n_inputs].data_ptr(),
                      self.b[ph % n_inputs].data_ptr(), self.A_log.data_ptr(),
                      self.dt_bias.data_ptr(), self.state.data_ptr(), self.state.data_ptr(), None,
                      None, 1e-6, self.out.data_ptr(), _lib.GDN_BF16, B, Hk, Hv, d, d, K,
                      _lib.GDN_BF16, sl.data_ptr(), P, half.data_ptr(), None, None, stream)
                     for ph, (sl, half) in enumerate(phases)]

    def step(self, s):
        rc = self._fn(*self.args[s % len(self.args)])
        if rc != 0:
            raise RuntimeError(f"gdn_decode_step failed with {rc}")


def quantized_layer(dev, hidden=2048, seed=0):
    """The gated-delta layer (Hk=16, Hv=32, d=128) with random 4-bit group-64
    projections (qkv|z|a|b in, out_proj out) and random conv, gate and norm
    parameters; returns (layer, generator, randn)."""

    d = gdn.QWEN3_5_LINEAR
    q = gdn.QuantScheme(4, 64)
    g = torch.Generator(device=dev).manual_seed(seed)

    def qweights(n, k):
        return gdn.LinearWeights({
            "weight": torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), generator=g, device=dev,
                                    dtype=torch.int32),
            "scales": (torch.rand(n, k // 64, generator=g, device=dev) * 0.004 + 0.001).to(torch.bfloat16),
            "biases": ((torch.rand(n, k // 64, generator=g, device=dev) - 0.5) * 0.05).to(torch.bfloat16)}, q)

    rnd = lambda *s_: torch.randn(*s_, generator=g, device=dev)
    layer = gdn.Qwen3_5LinearAttention(
        d, qweights(d.conv_dim, hidden), qweights(d.value_dim, hidden),
        qweights(d.num_value_heads, hidden), qweights(d.num_value_heads, hidden),
        rnd(d.conv_dim, 4, 1) * 0.2, torch.rand(d.num_value_heads, generator=g, device=dev) * 2.7,
        rnd(d.num_value_heads), torch.rand(d.value_head_dim, generator=g, device=dev) + 0.5,
        qweights(hidden, d.value_dim))
    return layer, g, rnd


def bench_layer_stack_decode(dev, B, layers, steps, warmup, hidden=2048):
    """`layers` gated-delta layers (each with its own 4-bit weights and a
    pool of 4 B slots) decoding B sequences, chained through the decoder's
    residual (h = h + layer(h)), all captured in one HIP graph: the per-layer
    cost of a decode step when the host's launch work is amortised over the
    stack, as in a whole-model graph."""

    d = gdn.QWEN3_5_LINEAR
    P = 4 * B
    stack, pools = [], []
    for i in range(layers):
        layer, g, rnd = quantized_layer(dev, hidden, seed=100 + i)
        pool = gdn.RecurrentStatePool(P, 4, d.conv_dim, d.num_value_heads, 128, 128,
                                      dtype=torch.bfloat16, device=dev)
        pool.ssm_state.normal_(0, 0.05, generator=g)
        stack.append(layer)
        pools.append(pool)
    slots = list(range(B))
    x = torch.randn(B, hidden, device=dev).to(torch.bfloat16)

    def run():
        h = x
        for layer, pool in zip(stack, pools):
            h = layer.decode_batch(h, pool, slots=slots, residual=h)
        return h

    for _ in range(max(warmup, 1)):
        run()
    torch.cuda.synchronize()
    for pool in pools:  # the slot arrays exist before capture
        pool.device_slots(slots)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        run()
    gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    step_us = e0.elapsed_time(e1) * 1e3 / steps
    return {"workload": f"{layers} gated-delta layers decoding B={B} (each of 4 B slots, 4-bit "
                        f"projections, hidden {hidden}) chained through the residual, one HIP graph",
            "layers": layers, "step_us": step_us, "per_layer_us": step_us / layers,
            "tokens_per_s": B / (step_us * 1e-6)}


def bench_layer_decode(dev, B, steps, warmup, hidden=2048):
    """The whole gated-delta layer (Hk=16, Hv=32, d=128) decoding B active
    sequences out of a pool of 4 B slots, 4-bit group-64 projections
    (stacked qkv|z|a|b in, out_proj out) with bf16 activations: one
    decode_batch call per step, slot sets rotating as in decode_slots. Also
    times its three launches alone (input projection, fused decode,
    out_proj) so the per-part figures add up."""

    d = gdn.QWEN3_5_LINEAR
    layer, g, rnd = quantized_layer(dev, hidden)
    P = 4 * B
    pool = gdn.RecurrentStatePool(P, 4, d.conv_dim, d.num_value_heads, 128, 128,
                                  dtype=torch.bfloat16, device=dev)
    pool.ssm_state.normal_(0, 0.05, generator=g)
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(0)).tolist()
    sets = [perm[i * B:(i + 1) * B] for i in range(4)]
    xs = [rnd(B, hidden).to(torch.bfloat16) for _ in range(4)]
    total_ms, _ = time_steps(lambda s_: layer.decode_batch(xs[s_ % 4], pool, slots=sets[s_ % 4]),
                             steps, warmup)
    # the same steps replayed from HIP graphs (one per slot set)
    graphs = [gdn.DecodeGraph(layer, pool, sets[i], xs[i]) for i in range(4)]
    graph_ms, _ = time_steps(lambda s_: graphs[s_ % 4].step(), steps, warmup)
    # the two projections alone, 20 calls a graph (device time, not the
    # host's launch rate)
    x = xs[0]
    o = rnd(B, d.value_dim).to(torch.bfloat16)

    def graph_us(fn, reps=20, replays=20):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(reps):
                fn()
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * replays)

    in_us = graph_us(lambda: layer._project(x))
    out_us = graph_us(lambda: gdn.quantized_linear(o, layer.out_proj))
    ms = total_ms / steps
    return {"workload": f"gated-delta layer decode, B={B} active of {P} slots, hidden {hidden}, "
                        f"4-bit group-64 projections, bf16 activations",
            "tokens_per_s": B / (ms * 1e-3), "step_us": ms * 1e3,
            "graph_step_us": graph_ms / steps * 1e3,
            "graph_tokens_per_s": B / (graph_ms / steps * 1e-3),
            "input_projection_us": in_us, "out_proj_us": out_us}


def bench_layer_prefill(dev, T, steps, warmup, hidden=2048, chunk=512):
    """The whole gated-delta layer (Hk=16, Hv=32, d=128, 4-bit group-64
    projections, bf16 activations) over a T-token prompt: one layer(x, cache)
    call per step, the cache carried from step to step. Also times its
    three parts alone (input projections, everything between them, out_proj),
    and a prompt prefilled in `chunk`-token pieces, eager and from a
    PrefillGraph."""

    d = gdn.QWEN3_5_LINEAR
    layer, g, rnd = quantized_layer(dev, hidden)
    cache = layer.new_cache()
    xs = [rnd(T, hidden).to(torch.bfloat16) for _ in range(2)]
    total_ms, _ = time_steps(lambda s_: layer(xs[s_ % 2], cache), steps, warmup)
    x = xs[0]
    qkv, z, a, b = layer._project(x)
    conv, ssm = cache.state()
    o = rnd(T, d.value_dim).to(torch.bfloat16)
    in_ms, _ = time_steps(lambda s_: layer._project(x), steps, warmup)
    core_ms, _ = time_steps(lambda s_: layer.core(qkv, z, a, b, conv[None], ssm[None]), steps, warmup)
    out_ms, _ = time_steps(lambda s_: gdn.quantized_linear(o, layer.out_proj), steps, warmup)
    xc = [rnd(chunk, hidden).to(torch.bfloat16) for _ in range(2)]
    ce, cg = layer.new_cache(), layer.new_cache()
    chunk_eager_ms, _ = time_steps(lambda s_: layer(xc[s_ % 2], ce), steps, warmup)
    pg = gdn.PrefillGraph(layer, xc[0])
    chunk_graph_ms, _ = time_steps(lambda s_: pg.step(cg, xc[s_ % 2]), steps, warmup)
    # the same with the projections' bf16 dequantization kept
    layer.keep_dense_weights()
    pgd, cd = gdn.PrefillGraph(layer, xc[0]), layer.new_cache()
    chunk_dense_ms, _ = time_steps(lambda s_: pgd.step(cd, xc[s_ % 2]), steps, warmup)
    ms = total_ms / steps
    proj_flops = 2 * T * hidden * (d.conv_dim + d.value_dim + 2 * d.num_value_heads + d.value_dim)
    return {"workload": f"gated-delta layer prefill, T={T}, hidden {hidden}, 4-bit group-64 "
                        f"projections, bf16 activations",
            "tokens_per_s": T / (ms * 1e-3), "step_us": ms * 1e3,
            "input_projection_us": in_ms / steps * 1e3, "core_us": core_ms / steps * 1e3,
            "out_proj_us": out_ms / steps * 1e3, "projection_flops": proj_flops,
            "chunk": chunk, "chunk_eager_us": chunk_eager_ms / steps * 1e3,
            "chunk_graph_us": chunk_graph_ms / steps * 1e3,
            "chunk_graph_tokens_per_s": chunk / (chunk_graph_ms / steps * 1e-3),
            "chunk_graph_dense_us": chunk_dense_ms / steps * 1e3}


def bench_decode_slots(dev, B, Hk, Hv, steps, warmup):
    w = SlotDecodeWorkload(dev, B, Hk, Hv)
    total_ms, _ = time_steps(w.step, steps, warmup)
    ms = total_ms / steps  # one launch per step
    gbs = w.bytes_per_step / (ms * 1e-3) / 1e9
    return {
        "workload": f"decode of B={B} active sequences at random slots of a pool of {w.P} "
                    f"(Hk={Hk} Hv={Hv} d=128), four rotating slot sets",
        "tokens_per_s": B * steps / (total_ms * 1e-3),
        "kernel_us": ms * 1e3,
        "hbm_gbs": gbs,
        "hbm_frac": gbs / HBM_PEAK_GBS,
        "bytes_per_step": w.bytes_per_step,
    }


def bench_decode(dev, B, Hk, Hv, with_z, steps, warmup):
    w = DecodeWorkload(dev, B, Hk, Hv, with_z)
    total_ms, isolated_ms = time_steps(w.step, steps, warmup)
    ms = total_ms / steps  # one launch per step
    achieved = w.bytes_per_step / (ms * 1e-3) / 1e9
    return {
        "tokens_per_s": B * steps / (total_ms * 1e-3),
        "ms_per_step": ms,
        "kernel_us": ms * 1e3,
        "isolated_launch_us": isolated_ms * 1e3,
        "bytes_per_step": w.bytes_per_step,
        "hbm_gbs": achieved,
        "hbm_frac": achieved / HBM_PEAK_GBS,
    }


def bench_decode_graph(dev, B, Hk, Hv, with_z, replays=20, per_graph=64):
    """Decode steps at sizes where one launch takes less time than issuing
    it (a single sequence): `per_graph` steps captured in one HIP graph,
    `replays` replays timed by one event pair; per-step time is the graph's
    time over its steps (kernel time plus the graph's own gap between
    launches)."""

    w = DecodeWorkload(dev, B, Hk, Hv, with_z)
    fn = w._fn
    for s in range(8):
        w.step(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        args = w._bind(torch.cuda.current_stream().cuda_stream)
        for s in range(per_graph):
            if fn(*args[s % len(args)]) != 0:
                raise RuntimeError("gdn_decode_step failed during capture")
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * per_graph)
    gbs = w.bytes_per_step / (us * 1e-6) / 1e9
    return {
        "workload": f"decode B={B} Hk={Hk} Hv={Hv} d=128 K=4, fused conv roll"
                    + (" + gated RMSNorm" if with_z else ""),
        "step_us": us, "tokens_per_s": B / (us * 1e-6), "hbm_gbs": gbs,
        "hbm_frac": gbs / HBM_PEAK_GBS, "bytes_per_step": w.bytes_per_step,
        "timing": f"{per_graph} steps per HIP graph, {replays} replays",
    }


def prefill_flops(T, Hv, d=128, chunk=64):
    """Algorithmic flops of the chunked prefill: the GEMMs K K^T, Q K^T,
    T(beta K), T(beta V), (Q K^T o M) U', W S, Q S and K^T U' per token
    (the triangular solve excluded)."""

    return T * Hv * (10 * chunk * d + 6 * d * d)


class PrefillWorkload:
    """Synthetic chunked-prefill inputs resident in HBM: N runs of L tokens
    (or packed runs of the given lengths, through cu_seqlens), q/k/v and a/b
    in `dtype` (bf16, or float32 as the reference's layers carry them; q, k
    L2-normalised), initial state zero (or ~N(0, 0.05) with packed runs); y
    in bf16."""

    def __init__(self, dev, N, L, Hk, Hv, seed=0, lens=None, dtype=torch.bfloat16):
        d = 128
        g = torch.Generator(device=dev).manual_seed(seed)
        bf = dtype
        if lens is not None:
            N = len(lens)
            cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
            self.cu = torch.tensor(cu, device=dev)
            T = int(cu[-1])
        else:
            self.cu = None
            T = N * L
        randn = lambda *s: torch.randn(*s, generator=g, device=dev)
        q = randn(T, Hk, d)
        k = randn(T, Hk, d)
        self.q = (q / q.norm(dim=-1, keepdim=True) / d ** 0.5).to(bf)
        self.k = (k / k.norm(dim=-1, keepdim=True)).to(bf)
        self.v = randn(T, Hv, d).to(bf)
        self.a = randn(T, Hv).to(bf)
        self.b = randn(T, Hv).to(bf)
        self.A_log = torch.rand(Hv, generator=g, device=dev) * float(np.log(16))
        self.dt_bias = torch.rand(Hv, generator=g, device=dev) * 2 - 1
        self.state_out = torch.empty(N, Hv, d, d, device=dev)
        self.state_in = (randn(N, Hv, d, d) * 0.05 if lens is not None else None)
        self.y = torch.empty(T, Hv, d, dtype=torch.bfloat16, device=dev)
        nbytes = gated_delta.prefill_workspace_bytes(N, T, Hk, Hv, d, d)
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        self.T, self.flops = T, prefill_flops(T, Hv)
        # algorithmic HBM bytes of one call: q, k, v, a, b (and the initial
        # states) read once, y and the final states written once
        es = torch.finfo(dtype).bits // 8
        self.bytes = (T * (2 * Hk * d + Hv * d + 2 * Hv) * es + T * Hv * d * 2
                      + N * Hv * d * d * 4 * (1 if self.state_in is None else 2))
        from mlx_lean_moe_amd import _lib

        self._fn = _lib.load().gdn_prefill_chunked
        self._args = (self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                      _lib.dtype_code(dtype), self.a.data_ptr(),
                      self.b.data_ptr(), _lib.dtype_code(dtype), Hv, self.A_log.data_ptr(),
                      self.dt_bias.data_ptr(), 0,
                      None if self.state_in is None else self.state_in.data_ptr(),
                      self.state_out.data_ptr(), self.y.data_ptr(), _lib.GDN_BF16,
                      None if self.cu is None else self.cu.data_ptr(), N, T, Hk, Hv, d, d,
                      self.ws.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)

    def step(self, s):
        rc = self._fn(*self._args)
        if rc != 0:
            raise RuntimeError(f"gdn_prefill_chunked failed with {rc}")


class QLinearWorkload:
    """The layer's stacked input projection (qkv | z | a | b: 2048 -> 12352)
    as a 4-bit affine (group 64, bf16 scales/biases) quantized matmul of M
    bf16 rows; random codes, scales ~U(0.001, 0.01), biases ~U(-0.05, 0.05).
    With `rotate` the packed weights, scales and biases cycle through enough
    copies (over 320 MB) that every launch reads them from HBM rather than
    the 256 MB Infinity Cache, as a decode step does after the other layers'
    weights have passed through it."""

    def __init__(self, dev, M, N=12352, K=2048, bits=4, group_size=64, seed=0, rotate=True):
        g = torch.Generator(device=dev).manual_seed(seed)
        self.x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        wbytes = N * K * bits // 8 + 2 * N * (K // group_size) * 2
        self.copies = -(-320_000_000 // wbytes) if rotate else 1
        self.weights = []
        for _ in range(self.copies):
            w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K * bits // 32), generator=g,
                              device=dev, dtype=torch.int32)
            sc = (torch.rand(N, K // group_size, generator=g, device=dev) * 0.009
                  + 0.001).to(torch.bfloat16)
            bi = ((torch.rand(N, K // group_size, generator=g, device=dev) - 0.5)
                  * 0.1).to(torch.bfloat16)
            self.weights.append((w, sc, bi))
        self.y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        self.M, self.N, self.K = M, N, K
        self.flops = 2 * M * N * K
        self.bytes = wbytes + M * K * 2 + M * N * 2
        from mlx_lean_moe_amd import _lib

        self._fn = _lib.load().gdn_quantized_matmul
        stream = torch.cuda.current_stream().cuda_stream
        ws_bytes = int(_lib.load().gdn_quantized_matmul_workspace_size(
            _lib.GDN_BF16, _lib.GDN_BF16, M, N, K, bits, group_size))
        self.ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        self._args = [(self.x.data_ptr(), _lib.GDN_BF16, w.data_ptr(), sc.data_ptr(),
                       bi.data_ptr(), _lib.GDN_BF16, self.y.data_ptr(), _lib.GDN_BF16, None, M, N, K,
                       bits, group_size, self.ws.data_ptr(), ws_bytes, stream)
                      for w, sc, bi in self.weights]

    def step(self, s):
        rc = self._fn(*self._args[s % self.copies])
        if rc != 0:
            raise RuntimeError(f"gdn_quantized_matmul failed with {rc}")


class SchemeWorkload:
    """A decode-size projection of M bf16 rows with the codes of one of the
    schemes gdn_quantized_matmul_scheme multiplies directly (affine 2-8 bits,
    mxfp4, mxfp8, nvfp4): random codes; affine scales and biases as in
    QLinearWorkload, e8m0 scale codes for 2^-10 .. 2^-4 (mx formats), e4m3
    scale codes (nvfp4). The weights cycle through over 320 MB of copies, so
    every launch reads them from HBM."""

    MODES = {"affine": 0, "mxfp4": 1, "mxfp8": 2, "nvfp4": 3}

    def __init__(self, dev, M, N, K, bits, group_size, mode, seed=0):
        from mlx_lean_moe_amd import _lib

        g = torch.Generator(device=dev).manual_seed(seed)
        self.x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        affine = mode == "affine"
        groups = N * (K // group_size)
        wbytes = N * K * bits // 8 + (4 * groups if affine else groups)
        self.copies = -(-320_000_000 // wbytes)
        self.weights = []
        for _ in range(self.copies):
            w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K * bits // 32), generator=g,
                              device=dev, dtype=torch.int32)
            if affine:
                sc = (torch.rand(N, K // group_size, generator=g, device=dev) * 0.009
                      + 0.001).to(torch.bfloat16)
                bi = ((torch.rand(N, K // group_size, generator=g, device=dev) - 0.5)
                      * 0.1).to(torch.bfloat16)
            else:
                lo, hi = (0x20, 0x40) if mode == "nvfp4" else (117, 124)
                sc = torch.randint(lo, hi, (N, K // group_size), generator=g, device=dev,
                                   dtype=torch.uint8)
                bi = None
            self.weights.append((w, sc, bi))
        self.y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        self.bytes = wbytes + M * K * 2 + M * N * 2
        self.weight_bytes = wbytes
        lib = _lib.load()
        self._fn = lib.gdn_quantized_matmul_scheme
        ws_bytes = int(lib.gdn_quantized_matmul_scheme_workspace_size(M, N, K))
        self.ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        stream = torch.cuda.current_stream().cuda_stream
        self._args = [(self.x.data_ptr(), w.data_ptr(), sc.data_ptr(),
                       None if bi is None else bi.data_ptr(), _lib.GDN_BF16 if affine else 0,
                       self.y.data_ptr(), _lib.GDN_BF16, None, M, N, K, bits, group_size,
                       self.MODES[mode], self.ws.data_ptr(), ws_bytes, stream)
                      for w, sc, bi in self.weights]

    def step(self, s):
        rc = self._fn(*self._args[s % self.copies])
        if rc != 0:
            raise RuntimeError(f"gdn_quantized_matmul_scheme failed with {rc}")


# the layer's stacked input projection and out_proj, each scheme at one and
# 64 rows
SCHEME_CASES = [(bits, gs, mode) for bits, gs, mode in
                [(3, 64, "affine"), (5, 64, "affine"), (6, 64, "affine"), (2, 64, "affine"),
                 (4, 32, "mxfp4"), (8, 32, "mxfp8"), (4, 16, "nvfp4")]]
SCHEME_SHAPES = [(12352, 2048), (2048, 4096)]


def bench_schemes(dev, steps, warmup):
    out = []
    for N, K in SCHEME_SHAPES:
        for bits, gs, mode in SCHEME_CASES:
            for M in (1, 64):
                w = SchemeWorkload(dev, M, N, K, bits, gs, mode)
                total_ms, isolated_ms = time_steps(w.step, steps, warmup)
                us = total_ms / steps * 1e3
                out.append({"N": N, "K": K, "M": M, "scheme": f"{mode} {bits}-bit group {gs}",
                            "call_us": us, "isolated_call_us": isolated_ms * 1e3,
                            "weight_bytes": w.weight_bytes, "bytes_per_call": w.bytes,
                            "hbm_gbs": w.bytes / us / 1e3,
                            "hbm_frac": w.bytes / us / 1e3 / HBM_PEAK_GBS})
                print(f"# N={N} K={K} M={M} {mode} {bits}/{gs}: {us:.2f} us", file=sys.stderr,
                      flush=True)
                del w
    return out


def bench_qlinear(dev, M, steps, warmup, rotate=True, layer_path=False):
    w = QLinearWorkload(dev, M, rotate=rotate)
    total_ms, isolated_ms = time_steps(w.step, steps, warmup)
    ms = total_ms / steps
    r = {"kernel_us": ms * 1e3, "isolated_launch_us": isolated_ms * 1e3,
         "hbm_gbs": w.bytes / (ms * 1e-3) / 1e9, "tflops": w.flops / (ms * 1e-3) / 1e12,
         "bytes_per_launch": w.bytes, "flops_per_launch": w.flops,
         "tokens_per_s": M / (ms * 1e-3)}
    if layer_path:
        # what the layer runs at this size: quantized_linear (dequantize to
        # bf16 + vendor BLAS from 512 rows on)
        wt, sc, bi = w.weights[0]
        tensors, q = {"weight": wt, "scales": sc, "biases": bi}, gdn.QuantScheme(4, 64)
        lm, _ = time_steps(lambda s: gdn.quantized_linear(w.x, tensors, q), steps, warmup)
        r["layer_path_us"] = lm / steps * 1e3
        r["layer_path_tflops"] = w.flops / (lm / steps * 1e-3) / 1e12
    return r


VARLEN_LENS = np.random.default_rng(0).integers(128, 8193, 16)  # 16 runs, 67,128 tokens


def bench_prefill(dev, N, L, Hk, Hv, steps, warmup, lens=None, dtype=torch.bfloat16,
                  compare_scan=False):
    w = PrefillWorkload(dev, N, L, Hk, Hv, lens=lens, dtype=dtype)
    total_ms, isolated_ms = time_steps(w.step, steps, warmup)
    call_ms = total_ms / steps  # one gdn_prefill_chunked call per step
    tflops = w.flops / (call_ms * 1e-3) / 1e12
    extra = {} if lens is None else {"continuation": bench_continuation(dev, w, Hk, Hv)}
    if compare_scan:
        extra["sequential_scan_us"] = scan_call_us(w, Hk, Hv, max(steps // 4, 2))
    return {
        **extra,
        "tokens_per_s": w.T * steps / (total_ms * 1e-3),
        "ms_per_step": call_ms,
        "call_us": call_ms * 1e3,
        "isolated_call_us": isolated_ms * 1e3,
        "flops_per_call": w.flops,
        "bytes_per_call": w.bytes,
        "tflops": tflops,
        "mfma_frac": tflops / BF16_PEAK_TFLOPS,
    }


def scan_call_us(w, Hk, Hv, steps):
    """The same workload through the sequential register-resident scan
    (gdn_scan, the reference's Metal-kernel form), gates precomputed: the
    path float32 activations took before the chunked prefill took them."""

    d = 128
    g, beta = gated_delta._gates(w.a, w.b, w.A_log, w.dt_bias)
    state_in = (w.state_in if w.state_in is not None
                else torch.zeros_like(w.state_out))
    y = torch.empty(w.T, Hv, d, dtype=torch.float32, device=w.q.device)
    cu = w.cu
    N = state_in.shape[0]

    def step(_):
        gated_delta._launch_scan("gdn_scan", w.q, w.k, w.v, g, beta, state_in, w.state_out, y,
                                 cu, N, w.T, Hk, Hv, d, d, w.q.device)

    total_ms, _ = time_steps(step, steps, 1)
    return total_ms / steps * 1e3


def bench_continuation(dev, w, Hk, Hv, steps=128, warmup=8):
    """The packed prefill's sequences decoding `steps` tokens each from its
    final states: one fused decode launch (conv roll, gated RMSNorm) per
    token for all of them, the states updated in place and two conv-state
    buffers alternating."""

    d = gdn.LinearAttentionDims(Hk, Hv, 128, 128, 4)
    B, C = w.state_out.shape[0], d.conv_dim
    g = torch.Generator(device=dev).manual_seed(1)
    bf = torch.bfloat16
    rnd = lambda *s_: torch.randn(*s_, generator=g, device=dev)
    state = w.state_out.clone()
    convs = [rnd(B, 3, C).to(bf), torch.empty(B, 3, C, dtype=bf, device=dev)]
    n_in = 8
    qkv = [rnd(B, C).to(bf) for _ in range(n_in)]
    z = [rnd(B, Hv, 128).to(bf) for _ in range(n_in)]
    a = [rnd(B, Hv).to(bf) for _ in range(n_in)]
    b = [rnd(B, Hv).to(bf) for _ in range(n_in)]
    conv_w = rnd(C, 4) * 0.2
    norm_w = torch.rand(128, generator=g, device=dev) + 0.5

    def step(s_):
        i = s_ % n_in
        gdn.fused_decode_step(qkv[i], z[i], a[i], b[i], convs[s_ % 2], state, conv_w, w.A_log,
                              w.dt_bias, norm_w, 1e-6, d, conv_out=convs[(s_ + 1) % 2],
                              state_out=state)

    # eight steps a HIP graph (the conv buffers back at their start), replayed
    # steps / 8 times: device time, not Python's launch rate
    for s_ in range(warmup):
        step(s_)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for s_ in range(8):
            step(s_)
    gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps // 8):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (steps // 8 * 8)
    _, _, nbytes = decode_bytes(B, Hk, Hv, 128, 4, True)
    return {"workload": f"{steps} decode steps of the {B} sequences from the packed prefill's "
                        f"states (fused decode in place, from HIP graphs; the "
                        f"{B * Hv * 128 * 128 * 4 >> 20} MiB of state stay in the 256 MB Infinity "
                        f"Cache)",
            "tokens_per_s": B / (ms * 1e-3), "step_us": ms * 1e3,
            "gbs": nbytes / (ms * 1e-3) / 1e9}


def cpu_baseline_prefill(Hk, Hv, budget_s=10.0):
    """The C restatement of the reference's sequential recurrence
    (gated_delta.py:93-109; float32, OpenMP over value heads) timed on the
    host over a bounded number of tokens of the same prefill workload."""

    from oracle import cref

    rng = np.random.default_rng(0)
    d, L = 128, 64
    q = rng.standard_normal((1, L, Hk, d)).astype(np.float32) * 0.01
    k = rng.standard_normal((1, L, Hk, d)).astype(np.float32) * 0.09
    v = rng.standard_normal((1, L, Hv, d)).astype(np.float32)
    g = rng.uniform(0.3, 0.9, (1, L, Hv)).astype(np.float32)
    beta = rng.uniform(0, 1, (1, L, Hv)).astype(np.float32)
    state = np.zeros((1, Hv, d, d), np.float32)
    cref.scan(q, k, v, g, beta, state)
    tokens, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        _, state = cref.scan(q, k, v, g, beta, state)
        tokens += L
    dt = time.perf_counter() - t0
    threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    return {
        "value": tokens / dt,
        "unit": "tokens/s",
        "cores": min(threads, len(os.sched_getaffinity(0))),
        "kind": "port",
        "sample": f"{tokens} tokens ({tokens // L} runs of {L}) of the T=4096 Hk={Hk} Hv={Hv} "
                  f"prefill recurrence, {dt:.1f} s, float32 C/OpenMP restatement",
    }


def cpu_baseline_decode(B, Hk, Hv, with_z, budget_s=10.0):
    """The C restatement of the reference's decode path (fused front-end +
    recurrence [+ gated RMSNorm], float32, OpenMP over (sequence, head))
    timed on the host on a bounded number of steps of the same workload."""

    from oracle import cref

    rng = np.random.default_rng(0)
    d, K = 128, 4
    C = 2 * Hk * d + Hv * d
    conv_w = (rng.standard_normal((C, K)) * 0.2).astype(np.float32)
    A_log = rng.uniform(0, np.log(16), Hv).astype(np.float32)
    dt_bias = rng.uniform(-1, 1, Hv).astype(np.float32)
    norm_w = rng.uniform(0.5, 1.5, d).astype(np.float32) if with_z else None
    state = rng.standard_normal((B, Hv, d, d), dtype=np.float32) * np.float32(0.05)
    conv = rng.standard_normal((B, K - 1, C), dtype=np.float32)
    qkv = rng.standard_normal((B, C), dtype=np.float32)
    a = rng.standard_normal((B, Hv), dtype=np.float32)
    b = rng.standard_normal((B, Hv), dtype=np.float32)
    z = rng.standard_normal((B, Hv, d), dtype=np.float32) if with_z else None
    cref.decode_step(qkv, conv, conv_w, a, b, A_log, dt_bias, state, z, norm_w, 1e-6,
                     (Hk, Hv, d, d), True, state_out=state)
    steps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        _, conv, _ = cref.decode_step(qkv, conv, conv_w, a, b, A_log, dt_bias, state, z, norm_w,
                                      1e-6, (Hk, Hv, d, d), True, state_out=state)
        steps += 1
    dt = time.perf_counter() - t0
    threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    return {
        "value": B * steps / dt,
        "unit": "tokens/s",
        "cores": min(threads, len(os.sched_getaffinity(0))),
        "kind": "port",
        "sample": f"{steps} fused decode steps of the B={B}, Hv={Hv} workload "
                  f"{'with the gated RMSNorm ' if with_z else ''}({B * steps} tokens, {dt:.1f} s), "
                  f"float32 C/OpenMP restatement",
    }


def cpu_baseline_qlinear(M=64, N=12352, K=2048, bits=4, group_size=64, budget_s=10.0):
    """The oracle's restatement of the quantized projection (dequantize the
    MLX-packed codes, then x @ W.T; what mx.quantized_matmul computes on the
    reference's CPU path, model/moe_block.py:44-55) timed on the host over a
    bounded number of calls of the same M=64 workload."""

    from oracle import quant_ref as Q

    rng = np.random.default_rng(0)
    words = rng.integers(0, 2 ** 32, (N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    scales = rng.uniform(0.001, 0.01, (N, K // group_size))
    biases = rng.uniform(-0.05, 0.05, (N, K // group_size))
    x = rng.standard_normal((M, K))
    Q.quantized_matmul(x, words, scales, biases, bits, group_size, w_round="f32")
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        Q.quantized_matmul(x, words, scales, biases, bits, group_size, w_round="f32")
        calls += 1
    dt = time.perf_counter() - t0
    threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    return {
        "value": M * calls / dt,
        "unit": "tokens/s",
        "cores": min(threads, len(os.sched_getaffinity(0))),
        "kind": "port",
        "sample": f"{calls} calls of the M={M} N={N} K={K} 4-bit projection ({M * calls} tokens, "
                  f"{dt:.1f} s), NumPy float64 dequantize + BLAS matmul",
    }


def load_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""

    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


DECODE_WORKLOADS = {
    False: "decode B=256 Hk=16 Hv=64 d=128 K=4, fused conv roll + gated RMSNorm",
    True: "decode B=64 Hk=16 Hv=32 d=128 K=4, fused conv roll",
}


def decode_roofline(r, small):
    return {
        "bound": "hbm",
        "achieved": r["hbm_gbs"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": r["hbm_frac"],
        "traffic": load_traffic(f"gdn_decode_step_{'b64_hv32' if small else 'b256_hv64'}_traffic.json"),
        "kernel": "gdn_decode_step",
        "kernel_us": r["kernel_us"],
        "isolated_launch_us": r["isolated_launch_us"],
        "algorithmic_bytes_per_launch": r["bytes_per_step"],
    }


def prefill_roofline(r):
    intensity = r["flops_per_call"] / r["bytes_per_call"]
    attainable = min(BF16_PEAK_TFLOPS, intensity * HBM_PEAK_GBS / 1e3)
    return {
        "bound": "mfma",
        "achieved": r["tflops"],
        "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": r["mfma_frac"],
        "traffic": load_traffic("gdn_prefill_chunked_t4096_traffic.json"),
        "kernel": "gdn_prefill_chunked (one call: all its launches)",
        "kernel_us": r["call_us"],
        "isolated_launch_us": r["isolated_call_us"],
        "algorithmic_flops_per_launch": r["flops_per_call"],
        # below the ridge point the attainable rate is the HBM roofline
        # I * 8 TB/s (I = algorithmic flops per algorithmic byte)
        "algorithmic_bytes_per_launch": r["bytes_per_call"],
        "intensity_flop_per_byte": intensity,
        "attainable": attainable,
        "frac_of_attainable": r["tflops"] / attainable,
    }


def bench_also(dev, cpu=True):
    """The secondary workloads of the default run."""

    sm = bench_decode(dev, 64, 16, 32, False, steps=64, warmup=8)
    d1 = bench_decode_graph(dev, 1, 16, 32, True)
    d1n = bench_decode_graph(dev, 1, 16, 32, False)
    # ~0.1-2 ms per call: enough steps that the clocks have settled (20
    # steps after 3 read ~8 % slower than 256 after 20)
    pf = bench_prefill(dev, 1, 4096, 16, 32, steps=100, warmup=20)
    pv = bench_prefill(dev, 0, 0, 16, 32, steps=20, warmup=4, lens=VARLEN_LENS)
    p32 = bench_prefill(dev, 1, 4096, 16, 32, steps=100, warmup=20, dtype=torch.float32,
                        compare_scan=True)
    sl = bench_decode_slots(dev, 64, 16, 32, steps=64, warmup=8)
    ld = bench_layer_decode(dev, 64, steps=64, warmup=8)
    lp = bench_layer_prefill(dev, 4096, steps=50, warmup=10)
    return {
        "decode_b64": {
            "workload": DECODE_WORKLOADS[True], "tokens_per_s": sm["tokens_per_s"],
            "roofline": decode_roofline(sm, True),
            **({"cpu_baseline": cpu_baseline_decode(64, 16, 32, False, budget_s=5.0)} if cpu else {})},
        "decode_b1": d1,
        "decode_b1_no_norm": d1n,
        "prefill": {
            "workload": "chunked prefill B=1 T=4096 Hk=16 Hv=32 d=128 chunk 64, bf16 MFMA",
            "tokens_per_s": pf["tokens_per_s"], "call_us": pf["call_us"],
            "roofline": prefill_roofline(pf),
            **({"cpu_baseline": cpu_baseline_prefill(16, 32, budget_s=10.0)} if cpu else {})},
        "prefill_f32": {
            "workload": "chunked prefill B=1 T=4096 Hk=16 Hv=32 d=128 chunk 64, float32 q/k/v/a/b "
                        "(bf16 hi + lo on MFMA)",
            "tokens_per_s": p32["tokens_per_s"], "call_us": p32["call_us"],
            "tflops": p32["tflops"], "mfma_frac": p32["mfma_frac"],
            "sequential_scan_us": p32["sequential_scan_us"]},
        "prefill_varlen": {
            "workload": "packed prefill of 16 runs U[128, 8192] (67,128 tokens) Hk=16 "
                        "Hv=32, nonzero initial states",
            "tokens_per_s": pv["tokens_per_s"], "call_us": pv["call_us"],
            "tflops": pv["tflops"], "mfma_frac": pv["mfma_frac"],
            "continuation": pv["continuation"]},
        "decode_slots": sl,
        "layer_decode": {
            "workload": ld["workload"] + ", HIP-graph steps",
            "tokens_per_s": ld["graph_tokens_per_s"], "step_us": ld["graph_step_us"],
            "input_projection_us": ld["input_projection_us"],
            "out_proj_us": ld["out_proj_us"]},
        "layer_prefill": {
            "workload": lp["workload"], "tokens_per_s": lp["tokens_per_s"],
            "step_us": lp["step_us"], "input_projection_us": lp["input_projection_us"],
            "core_us": lp["core_us"], "out_proj_us": lp["out_proj_us"],
            "chunk512_eager_us": lp["chunk_eager_us"],
            "chunk512_graph_us": lp["chunk_graph_us"]},
    }


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "decode_large", "decode_b64", "decode_b1", "decode_slots", "decode_sizes",
                             "layer_decode",
                             "layer_prefill", "prefill_f32",
                             "prefill", "prefill_varlen", "qlinear", "qlinear_schemes", "copy"])
    ap.add_argument("--layers", type=int, default=1,
                    help="layer_decode: also time this many layers chained in one graph")
    ap.add_argument("--batch", type=int, default=64,
                    help="active sequences of the layer_decode workload (pool of 4x as many slots)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-also", action="store_true", help="skip the secondary workloads")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the gated-delta path needs no collective and this "
              "build runs on a single MI355X (see the sharding notes); use --gpus 1",
              file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.workload == "decode_sizes":
        # the HBM fraction the decode kernel reaches as the batch grows (one
        # launch per step, state in four rotating buffers)
        sizes = {}
        for B in (1, 8, 32, 64, 128, 256):
            r = bench_decode(dev, B, 16, 32, False, steps=max(args.steps, 64), warmup=max(args.warmup, 8))
            sizes[f"B={B} Hv=32"] = {"kernel_us": r["kernel_us"], "hbm_frac": r["hbm_frac"],
                                     "bytes_per_step": r["bytes_per_step"]}
        r = bench_decode(dev, 256, 16, 64, True, steps=max(args.steps, 64), warmup=max(args.warmup, 8))
        sizes["B=256 Hv=64 + gated norm"] = {"kernel_us": r["kernel_us"], "hbm_frac": r["hbm_frac"],
                                             "bytes_per_step": r["bytes_per_step"]}
        print(json.dumps({"workload": "gdn_decode_step over batch sizes (Hk=16, fused conv roll)",
                          "sizes": sizes}))
        return 0

    if args.workload == "copy":
        # Plain 1 GiB device copy: the HBM read+write ceiling a copy reaches,
        # and the known byte counts that scale rocprofv3's FETCH/WRITE_SIZE.
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).normal_()
        dst = torch.empty_like(src)
        n = max(args.steps, 1)
        total_ms, _ = time_steps(lambda s: dst.copy_(src), n, max(args.warmup, 1))
        copy_ms = total_ms / n
        nbytes = 2 * src.numel() * 4
        print(json.dumps({"workload": "copy 1 GiB float32 (torch copy_)", "bytes_read": nbytes // 2,
                          "bytes_written": nbytes // 2, "launches": n,
                          "copy_us": copy_ms * 1e3,
                          "gbs": nbytes / (copy_ms * 1e-3) / 1e9}))
        return 0

    if args.workload in ("decode", "decode_large", "decode_b64"):
        small = args.workload == "decode_b64"
        B, Hk, Hv, with_z = (64, 16, 32, False) if small else (256, 16, 64, True)
        r = bench_decode(dev, B, Hk, Hv, with_z, args.steps, args.warmup)
        line = {
            "metric": METRIC,
            "value": r["tokens_per_s"],
            "unit": "tokens/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": r["ms_per_step"],
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic",
            "config": {
                "workload": DECODE_WORKLOADS[small],
                "batch": B, "tokens_per_step": B, "key_heads": Hk, "value_heads": Hv,
                "head_dim": 128, "state": "float32, 4 buffers: step s reads s % 4, writes (s + 2) % 4",
            },
            "roofline": decode_roofline(r, small),
        }
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = cpu_baseline_decode(B, Hk, Hv, with_z, budget_s=10.0)
        if not args.no_also and not small:
            line["also"] = bench_also(dev, cpu=not args.no_cpu_baseline)
        print(json.dumps(line))
        return 0

    if args.workload == "decode_b1":
        print(json.dumps({"decode_b1": bench_decode_graph(dev, 1, 16, 32, True),
                          "decode_b1_no_norm": bench_decode_graph(dev, 1, 16, 32, False)}))
        return 0

    if args.workload == "layer_decode":
        r = bench_layer_decode(dev, args.batch, args.steps, args.warmup)
        stack = (bench_layer_stack_decode(dev, args.batch, args.layers, args.steps, args.warmup)
                 if args.layers > 1 else None)
        print(json.dumps({"metric": "gated-delta layer decode tokens/s (projections included)",
                          "value": r["graph_tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["graph_step_us"] * 1e-3, "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic", "config": {"workload": r["workload"] + ", HIP-graph steps"},
                          "eager_step_us": r["step_us"],
                          "parts_us": {"input_projection": r["input_projection_us"],
                                       "out_proj": r["out_proj_us"],
                                       "note": "each part alone, 20 calls a HIP graph"},
                          **({"stack": stack} if stack else {})}))
        return 0

    if args.workload == "layer_prefill":
        r = bench_layer_prefill(dev, 4096, args.steps, args.warmup)
        print(json.dumps({"metric": "gated-delta layer prefill tokens/s (projections included)",
                          "value": r["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["step_us"] * 1e-3, "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic", "config": {"workload": r["workload"]},
                          "parts_us": {"input_projection": r["input_projection_us"],
                                       "core": r["core_us"], "out_proj": r["out_proj_us"]},
                          "chunked": {"chunk": r["chunk"], "eager_step_us": r["chunk_eager_us"],
                                      "graph_step_us": r["chunk_graph_us"],
                                      "graph_dense_weights_step_us": r["chunk_graph_dense_us"],
                                      "graph_tokens_per_s": r["chunk_graph_tokens_per_s"]}}))
        return 0

    if args.workload == "decode_slots":
        r = bench_decode_slots(dev, 64, 16, 32, args.steps, args.warmup)
        print(json.dumps({"metric": METRIC, "value": r["tokens_per_s"], "unit": "tokens/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["kernel_us"] * 1e-3, "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic", "config": {"workload": r["workload"]},
                          "roofline": {"bound": "hbm", "achieved": r["hbm_gbs"],
                                       "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                       "frac": r["hbm_frac"], "traffic": None,
                                       "kernel": "gdn_decode_step (slots, conv half bits)",
                                       "kernel_us": r["kernel_us"],
                                       "algorithmic_bytes_per_launch": r["bytes_per_step"]}}))
        return 0

    if args.workload == "qlinear":
        dec = bench_qlinear(dev, 64, args.steps, args.warmup)
        pre = (None if args.no_also else
               bench_qlinear(dev, 4096, max(args.steps // 4, 5), args.warmup, rotate=False,
                             layer_path=True))
        print(json.dumps({
            "metric": "4-bit affine quantized input projection (hidden 2048 -> qkv|z|a|b 12352)",
            "value": dec["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": dec["kernel_us"] * 1e-3,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic",
            "config": {"workload": "gdn_quantized_matmul M=64 (decode) N=12352 K=2048, "
                                   "4-bit group 64, bf16 scales/biases"},
            "roofline": {"bound": "hbm", "achieved": dec["hbm_gbs"], "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": dec["hbm_gbs"] / HBM_PEAK_GBS,
                         "traffic": load_traffic("gdn_quantized_matmul_m64_n12352_k2048_traffic.json"),
                         "kernel": "gdn_quantized_matmul", "kernel_us": dec["kernel_us"],
                         "isolated_launch_us": dec["isolated_launch_us"],
                         "algorithmic_bytes_per_launch": dec["bytes_per_launch"]},
            **({} if args.no_cpu_baseline else {"cpu_baseline": cpu_baseline_qlinear()}),
            "also": {} if pre is None else {"prefill_m4096": {
                "kernel_us": pre["kernel_us"], "tflops": pre["tflops"],
                "mfma_frac": pre["tflops"] / BF16_PEAK_TFLOPS,
                "flops_per_launch": pre["flops_per_launch"],
                "layer_path_us": pre["layer_path_us"],
                "layer_path_mfma_frac": pre["layer_path_tflops"] / BF16_PEAK_TFLOPS}}}))
        return 0

    if args.workload == "qlinear_schemes":
        cases = bench_schemes(dev, args.steps, args.warmup)
        head = cases[0 if cases[0]["M"] == 64 else 1]
        print(json.dumps({
            "metric": "decode-size quantized projections of every scheme (no dequantization)",
            "value": 64 / (head["call_us"] * 1e-6), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["call_us"] * 1e-3,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic",
            "config": {"workload": "gdn_quantized_matmul_scheme at N=12352 K=2048 and N=2048 "
                                   "K=4096, M=1 and 64; value: M=64 N=12352 " + head["scheme"]},
            "roofline": {"bound": "hbm", "achieved": head["hbm_gbs"], "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": head["hbm_frac"], "traffic": None,
                         "kernel": "gdn_quantized_matmul_scheme", "kernel_us": head["call_us"],
                         "algorithmic_bytes_per_launch": head["bytes_per_call"]},
            "cases": cases}))
        return 0

    if args.workload in ("prefill", "prefill_varlen", "prefill_f32"):
        varlen = args.workload == "prefill_varlen"
        f32 = args.workload == "prefill_f32"
        r = bench_prefill(dev, 1, 4096, 16, 32, args.steps, args.warmup,
                          lens=VARLEN_LENS if varlen else None,
                          dtype=torch.float32 if f32 else torch.bfloat16, compare_scan=f32)
        print(json.dumps({"metric": METRIC, "value": r["tokens_per_s"], "unit": "tokens/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["ms_per_step"], "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic",
                          "config": {"workload": (
                              "packed prefill of 16 runs U[128, 8192] (67,128 tokens) Hk=16 Hv=32 "
                              "d=128 chunk 64" if varlen else
                              "chunked prefill B=1 T=4096 Hk=16 Hv=32 d=128 chunk 64" +
                              (", float32 q/k/v/a/b" if f32 else ""))},
                          "roofline": ({**prefill_roofline(r), "traffic": None} if varlen
                                       else prefill_roofline(r)),
                          **({} if args.no_cpu_baseline or varlen or f32 else
                             {"cpu_baseline": cpu_baseline_prefill(16, 32, budget_s=10.0)}),
                          **({"continuation": r["continuation"]} if varlen else {}),
                          **({"sequential_scan_us": r["sequential_scan_us"]} if f32 else {})}))
        return 0

    raise SystemExit(f"unknown workload {args.workload}")


if __name__ == "__main__":
    sys.exit(main())
