"""gdn_quantized_matmul_noalloc, the quantized matmul that allocates
nothing: its split-K partials live in the library's static per-GPU scratch.
On the GPU, through the C ABI, it gives the same bits as
gdn_quantized_matmul with a full caller workspace, on two calls in a row
(the second smaller, over the scratch the first one left behind); on the
host, every decode-kernel shape needs at most the scratch it holds."""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from mlx_lean_moe_amd import _lib

SCRATCH_BYTES = 4 << 20


def test_every_decode_shape_fits_the_scratch():
    """The workspace the full split takes, over decode-kernel shapes (rows
    1-64, the layer's projection widths and depths, both bit widths and all
    group sizes), never exceeds the 4 MiB scratch; 64 rows of 8192 columns
    in 8-bit codes take all of it (2 splits of 128 column tiles), and
    out_proj's shape in 4-bit codes none (16-row blocks, no split)."""

    lib = _lib.load()
    worst = 0
    for M, N, K, bits, gs, sb in itertools.product(
            (1, 2, 16, 17, 32, 33, 64), (64, 256, 1024, 2048, 4096, 8192, 12352),
            (512, 1024, 2048, 4096, 8192), (4, 8), (32, 64, 128), (_lib.GDN_BF16, _lib.GDN_F32)):
        for xd in (_lib.GDN_BF16, _lib.GDN_F32):
            need = lib.gdn_quantized_matmul_workspace_size(xd, sb, M, N, K, bits, gs)
            assert 0 <= need <= SCRATCH_BYTES, (M, N, K, bits, gs, sb, xd, need)
            worst = max(worst, need)
    assert worst == SCRATCH_BYTES
    assert lib.gdn_quantized_matmul_workspace_size(_lib.GDN_BF16, _lib.GDN_BF16, 64, 8192, 2048,
                                                   8, 64) == SCRATCH_BYTES
    assert lib.gdn_quantized_matmul_workspace_size(_lib.GDN_BF16, _lib.GDN_BF16, 64, 2048, 4096,
                                                   4, 64) == 0


def _case(dev, M, N, K, bits, gs, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K * bits // 32), generator=g, device=dev,
                          dtype=torch.int32)
    scales = (torch.rand(N, K // gs, generator=g, device=dev) * 0.004 + 0.001).to(torch.bfloat16)
    biases = ((torch.rand(N, K // gs, generator=g, device=dev) - 0.5) * 0.05).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    residual = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
    return x, words, scales, biases, residual


def _run(lib, fn, dev, x, words, scales, biases, residual, M, N, K, bits, gs, workspace=None):
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = [x.data_ptr(), _lib.GDN_BF16, words.data_ptr(), scales.data_ptr(), biases.data_ptr(),
            _lib.GDN_BF16, y.data_ptr(), _lib.GDN_BF16,
            None if residual is None else residual.data_ptr(), M, N, K, bits, gs]
    if fn == "gdn_quantized_matmul":
        args += [None if workspace is None else workspace.data_ptr(),
                 0 if workspace is None else workspace.numel()]
    rc = getattr(lib, fn)(*args, stream)
    assert rc == 0, lib.gdn_last_error().decode()
    return y


@pytest.mark.gpu
def test_noalloc_matches_the_workspace_entry_point_on_two_calls(gpu):
    """Two calls in a row, each against gdn_quantized_matmul with a full
    workspace (same split, so the same bits): 64 rows of 8192 columns in
    8-bit codes (2 splits, the whole scratch) with a residual, then a smaller call
    (16 rows of a 1024 x 2048 projection, fewer and smaller partial
    blocks) that reads none of what the first left in the scratch; and a
    one-row call (no split, no scratch)."""

    lib = _lib.load()
    shapes = [(64, 8192, 2048, 8, 64, True), (16, 1024, 2048, 4, 64, False),
              (1, 2048, 4096, 8, 32, False)]
    for i, (M, N, K, bits, gs, with_res) in enumerate(shapes):
        print(f"noalloc case {i}: M={M} N={N} K={K} bits={bits} group={gs}", flush=True)
        x, words, scales, biases, residual = _case(gpu, M, N, K, bits, gs, seed=40 + i)
        residual = residual if with_res else None
        need = lib.gdn_quantized_matmul_workspace_size(_lib.GDN_BF16, _lib.GDN_BF16, M, N, K, bits, gs)
        assert need <= SCRATCH_BYTES
        if i == 0:
            assert need == SCRATCH_BYTES
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=gpu)
        ref = _run(lib, "gdn_quantized_matmul", gpu, x, words, scales, biases, residual, M, N, K,
                   bits, gs, ws if need else None)
        got = _run(lib, "gdn_quantized_matmul_noalloc", gpu, x, words, scales, biases, residual, M,
                   N, K, bits, gs)
        torch.cuda.synchronize()
        assert not torch.isnan(ref.float()).any()
        assert torch.equal(got, ref), i
    # an invalid call is refused before any launch
    rc = lib.gdn_quantized_matmul_noalloc(None, _lib.GDN_BF16, None, None, None, _lib.GDN_BF16, None,
                                          _lib.GDN_BF16, None, 4, 64, 64, 4, 64, None)
    assert rc == _lib.GDN_EINVAL


@pytest.mark.gpu
def test_noalloc_captured_in_a_graph_replays_the_workspace_entry_points_bits(gpu):
    """A noalloc call captured in a HIP graph (torch.cuda.graph), after one
    eager call on the device (the first call looks up the scratch's address,
    which is not a call to make inside a capture): three replays, each after
    eager work that leaves other partial blocks in the scratch, give
    gdn_quantized_matmul's bits with a full workspace, on 64 rows of 8192
    columns in 8-bit codes (2 splits, the whole scratch) with a residual."""

    lib = _lib.load()
    M, N, K, bits, gs = 64, 8192, 2048, 8, 64
    x, words, scales, biases, residual = _case(gpu, M, N, K, bits, gs, seed=77)
    need = lib.gdn_quantized_matmul_workspace_size(_lib.GDN_BF16, _lib.GDN_BF16, M, N, K, bits, gs)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    ref = _run(lib, "gdn_quantized_matmul", gpu, x, words, scales, biases, residual, M, N, K, bits, gs, ws)
    # the eager call that sets the device up, outside any capture
    first = _run(lib, "gdn_quantized_matmul_noalloc", gpu, x, words, scales, biases, residual, M, N, K,
                 bits, gs)
    torch.cuda.synchronize()
    assert torch.equal(first, ref)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.gdn_quantized_matmul_noalloc(
            x.data_ptr(), _lib.GDN_BF16, words.data_ptr(), scales.data_ptr(), biases.data_ptr(),
            _lib.GDN_BF16, y.data_ptr(), _lib.GDN_BF16, residual.data_ptr(), M, N, K, bits, gs,
            torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.gdn_last_error().decode()
    other = _case(gpu, 16, 1024, 2048, 4, 64, seed=78)
    for i in range(3):
        print(f"noalloc graph replay {i}", flush=True)
        y.fill_(float("nan"))
        _run(lib, "gdn_quantized_matmul_noalloc", gpu, *other[:4], None, 16, 1024, 2048, 4, 64)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), i


@pytest.mark.gpu
def test_noalloc_calls_from_two_streams_take_the_scratch_in_turn(gpu):
    """Calls on two streams, each enqueued right after the other's, both
    using the whole scratch (64 rows of 8192 columns in 8-bit codes, 2
    splits): the second stream waits on the GPU for the first one's call,
    so every result has gdn_quantized_matmul's bits with a workspace of its
    own. Five rounds, alternating which stream goes first."""

    lib = _lib.load()
    M, N, K, bits, gs = 64, 8192, 2048, 8, 64
    need = lib.gdn_quantized_matmul_workspace_size(_lib.GDN_BF16, _lib.GDN_BF16, M, N, K, bits, gs)
    assert need == SCRATCH_BYTES
    cases = [_case(gpu, M, N, K, bits, gs, seed=90 + j) for j in range(2)]
    refs = []
    for x, words, scales, biases, residual in cases:
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        refs.append(_run(lib, "gdn_quantized_matmul", gpu, x, words, scales, biases, residual, M, N, K,
                         bits, gs, ws))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    for r in range(5):
        print(f"noalloc two-stream round {r}", flush=True)
        order = (0, 1) if r % 2 == 0 else (1, 0)
        got = {}
        for j in order:
            with torch.cuda.stream(streams[j]):
                x, words, scales, biases, residual = cases[j]
                got[j] = _run(lib, "gdn_quantized_matmul_noalloc", gpu, x, words, scales, biases, residual,
                              M, N, K, bits, gs)
        torch.cuda.synchronize()
        for j in (0, 1):
            assert torch.equal(got[j], refs[j]), (r, j)
