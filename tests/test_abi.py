"""The C-ABI library loads, exports every symbol include/gdn.h declares, and
rejects invalid arguments before launching anything (no GPU needed)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from mlx_lean_moe_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions() -> list[str]:
    text = open(os.path.join(ROOT, "include", "gdn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s+\**\s*(gdn_[a-z_0-9]+)\s*\(", text, flags=re.M)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.EXPORTED), "ctypes signatures out of sync with gdn.h"


def test_abi_version_and_single_hip_runtime():
    lib = _lib.load()
    assert lib.gdn_abi_version() == _lib.ABI_VERSION
    assert len(_lib._hip_runtimes_mapped()) == 1


def _err(lib) -> str:
    return lib.gdn_last_error().decode()


def test_invalid_arguments_return_einval_without_launching():
    lib = _lib.load()
    # bad head ratio
    rc = lib.gdn_scan(None, None, 0, None, 0, None, 0, None, 0, None, None, 0, None, 0, None, 1,
                      4, 3, 4, 32, 8, None)
    assert rc == _lib.GDN_EINVAL and "multiple" in _err(lib)
    # bad dtype code
    rc = lib.gdn_gates(None, None, 7, None, None, None, None, 0, 4, 2, None)
    assert rc == _lib.GDN_EINVAL
    # T not divisible by N without cu_seqlens
    rc = lib.gdn_scan_reference(None, None, 0, None, 0, None, 0, None, 0, ctypes.c_void_p(16),
                                ctypes.c_void_p(16), 0, None, 0, None, 3, 4, 1, 1, 32, 8, None)
    assert rc == _lib.GDN_EINVAL and "divisible" in _err(lib)
    # the fused decode kernel is specialised for Dk = Dv = 128
    rc = lib.gdn_decode_step(*([None] * 12), 1e-6, None, 0, 1, 2, 4, 64, 64, 4, 1, None, 0, None,
                             None, None, None)
    assert rc == _lib.GDN_EUNSUPPORTED
    # row strides below a row's width, and conv_half with two conv arrays
    fake = [ctypes.c_void_p(1 << (20 + i)) for i in range(12)]
    C = 2 * 1 * 128 + 2 * 128
    slots = ctypes.c_void_p(1 << 40)
    for strides, conv_out, what in (((C - 1, 256, 2, 2), fake[1], "row stride 0"),
                                    ((C, 256, 2, 1), fake[1], "row stride 3"),
                                    ((C, 256, 2, 2), fake[2], "one array")):
        rc = lib.gdn_decode_step(fake[0], fake[1], conv_out, *fake[3:12], 1e-6, fake[11], 0, 1, 1, 2,
                                 128, 128, 4, 1, slots, 4, slots, (ctypes.c_int64 * 4)(*strides), None,
                                 None)
        assert rc == _lib.GDN_EINVAL and what in _err(lib), (what, _err(lib))
    # the kernel flips the halves through conv_arrivals only where the step's
    # 2^16 splits evenly over the row's workgroups: a power-of-two Hv
    rc = lib.gdn_decode_step(fake[0], fake[1], fake[1], *fake[3:12], 1e-6, fake[11], 0, 1, 2, 6, 128, 128,
                             4, 1, slots, 4, slots, None, slots, None)
    assert rc == _lib.GDN_EUNSUPPORTED and "power-of-two" in _err(lib), _err(lib)
    # a gate row stride below Hv
    rc = lib.gdn_prefill_chunked(*fake[:3], 1, *fake[3:5], 1, 3, *fake[5:7], 0, None, fake[7], fake[8], 0,
                                 None, 1, 64, 2, 4, 128, 128, fake[9], 1 << 30, None)
    assert rc == _lib.GDN_EINVAL and "gate_stride" in _err(lib), _err(lib)
    # overlapping conv state buffers are rejected
    p = ctypes.c_void_p(4096)
    rc = lib.gdn_frontend(p, 128, p, p, 1, p, None, 1, 1, p, p, p, 1, 2, 32, 32, 4, 1, None)
    assert rc == _lib.GDN_EINVAL and "overlaps" in _err(lib)
    # a qkv row stride below conv_dim
    rc = lib.gdn_frontend(p, 127, p, ctypes.c_void_p(1 << 30), 1, p, None, 1, 1, p, p, p, 1, 2, 32, 32,
                          4, 1, None)
    assert rc == _lib.GDN_EINVAL and "qkv_stride" in _err(lib)


def test_empty_work_is_a_no_op():
    lib = _lib.load()
    assert lib.gdn_gates(None, None, 0, None, None, None, None, 0, 0, 4, None) == 0
    assert lib.gdn_gated_rmsnorm(None, 0, None, 0, 8, 1, None, 1e-6, None, 0, 0, 8, None) == 0
    # a z layout that does not fit the rows
    p = ctypes.c_void_p(4096)
    assert lib.gdn_gated_rmsnorm(p, 0, p, 0, 8, 3, p, 1e-6, p, 0, 4, 8, None) == _lib.GDN_EINVAL
    assert lib.gdn_gated_rmsnorm(p, 0, p, 0, 15, 2, p, 1e-6, p, 0, 4, 8, None) == _lib.GDN_EINVAL


def test_quantized_matmul_workspace_size():
    """K is split only where the decode kernel runs few column tiles: 8-bit
    codes of 64 rows over 2048 columns (32 tiles of 64) take 4 splits of
    float32 (M, N) blocks; out_proj's shape in 4-bit group-64 codes at
    17-64 rows runs as 16-row blocks with no split (none), one 16-row block
    splits 4 ways, and the stacked input projection (N = 12352) does not
    split; shapes the decode kernel does not take need none, and neither
    does one row of 4-bit codes (the matrix-vector kernel)."""

    lib = _lib.load()
    size = lambda *a: lib.gdn_quantized_matmul_workspace_size(*a)
    bf, f32 = _lib.GDN_BF16, _lib.GDN_F32
    assert size(bf, bf, 64, 2048, 2048, 8, 64) == 4 * 64 * 2048 * 4  # 32 tiles, 4 steps
    assert size(bf, bf, 64, 8192, 2048, 8, 64) == 2 * 64 * 8192 * 4  # 128 tiles: 2 splits
    assert size(bf, bf, 64, 2048, 4096, 4, 64) == 0                # 4 row blocks of 16
    assert size(bf, bf, 17, 2048, 4096, 4, 64) == 0                # 2 row blocks
    assert size(bf, bf, 16, 2048, 4096, 4, 64) == 4 * 16 * 2048 * 4  # one block: split
    assert size(bf, bf, 2, 2048, 4096, 4, 64) == 4 * 2 * 2048 * 4  # 64 tiles of 32 columns
    assert size(bf, bf, 1, 2048, 4096, 4, 64) == 0                 # one row: matrix-vector kernel
    assert size(bf, bf, 1, 2048, 2048, 8, 64) == 4 * 2048 * 4      # (not for 8-bit codes)
    assert size(bf, bf, 64, 12352, 2048, 4, 64) == 0
    assert size(f32, bf, 5, 300, 1024, 4, 32) == 4 * 5 * 300 * 4  # 4 steps: at most 4 splits
    assert size(bf, bf, 65, 2048, 4096, 4, 64) == 0                # tiled kernel
    assert size(f32, bf, 33, 2048, 4096, 4, 64) == 0               # float32 x beyond 32 rows
    assert size(bf, bf, 64, 2048, 4160, 4, 64) == 0                # not whole steps
    # a misaligned workspace is refused before anything runs
    p = ctypes.c_void_p(1 << 30)
    rc = lib.gdn_quantized_matmul(p, bf, p, p, p, bf, ctypes.c_void_p(1 << 31), bf, None, 1, 64, 512, 4,
                                  64, ctypes.c_void_p((1 << 32) + 8), 1024, None)
    assert rc == _lib.GDN_EINVAL and "workspace" in _err(lib)


def test_fused_prefill_workspace_and_argument_checks():
    """gdn_prefill_fused's workspace is the chunked prefill's plus bf16 q, k
    and v, and every argument it cannot take is refused before a launch."""

    lib = _lib.load()
    N, T, Hk, Hv = 1, 4096, 16, 32
    base = lib.gdn_prefill_workspace_size(N, T, Hk, Hv, 128, 128)
    fused = lib.gdn_prefill_fused_workspace_size(N, T, Hk, Hv, 128, 128)
    assert fused >= base + T * (2 * Hk + Hv) * 128 * 2
    assert fused - base - T * (2 * Hk + Hv) * 128 * 2 < 256
    assert lib.gdn_prefill_fused_workspace_size(N, T, Hk, Hv, 64, 128) == _lib.GDN_EUNSUPPORTED
    C = (2 * Hk + Hv) * 128
    P = lambda i: ctypes.c_void_p((1 << 32) + (i << 28))  # distinct, aligned, never dereferenced

    def call(**over):
        args = dict(qkv=P(0), qs=C, cs_in=P(1), cs_out=P(2), cdt=_lib.GDN_BF16, w=P(3), K=4, a=P(4),
                    b=P(5), gdt=_lib.GDN_BF16, gs=Hv, A_log=P(6), dt=P(7), s_in=P(8), s_out=P(9),
                    y=P(10), ydt=_lib.GDN_BF16, cu=None, N=N, T=T, Hk=Hk, Hv=Hv, Dk=128, Dv=128,
                    ws=P(11), wsb=fused)
        args.update(over)
        return lib.gdn_prefill_fused(*args.values(), None)

    assert call(K=3) == _lib.GDN_EUNSUPPORTED
    assert call(cdt=_lib.GDN_F16) == _lib.GDN_EUNSUPPORTED
    assert call(qs=C + 4) == _lib.GDN_EINVAL and "qkv_stride" in _err(lib)
    assert call(qs=C - 8) == _lib.GDN_EINVAL and "qkv_stride" in _err(lib)
    assert call(wsb=fused - 1) == _lib.GDN_EINVAL and "workspace" in _err(lib)
    assert call(cs_out=ctypes.c_void_p((1 << 32) + (1 << 28) + 16)) == _lib.GDN_EINVAL
    assert "overlaps" in _err(lib)
    assert call(s_out=P(8)) == _lib.GDN_EINVAL and "alias" in _err(lib)
    assert call(qkv=ctypes.c_void_p((1 << 32) + 8)) == _lib.GDN_EINVAL and "aligned" in _err(lib)
    assert call(gs=Hv - 1) == _lib.GDN_EINVAL and "gate_stride" in _err(lib)
    assert call(N=2, T=T + 1) == _lib.GDN_EINVAL and "divisible" in _err(lib)


def test_scheme_matmul_argument_checks():
    """gdn_quantized_matmul_scheme refuses what it does not multiply before
    anything runs: schemes MLX does not define, more than 64 rows, K that is
    no multiple of 32 or of the group, misaligned operands; no rows is a
    no-op."""

    lib = _lib.load()
    bf = _lib.GDN_BF16
    p, y = ctypes.c_void_p(1 << 30), ctypes.c_void_p(1 << 31)

    def call(M=1, N=64, K=512, bits=3, gs=64, mode=0, x=p, sb=bf):
        return lib.gdn_quantized_matmul_scheme(x, p, p, p, sb, y, bf, None, M, N, K, bits, gs, mode, None, 0,
                                               None)

    for bits, gs, mode in [(7, 64, 0), (3, 16, 0), (4, 16, 1), (8, 16, 2), (4, 32, 3), (4, 32, 9)]:
        assert call(bits=bits, gs=gs, mode=mode) == _lib.GDN_EINVAL and "scheme" in _err(lib)
    assert call(M=65) == _lib.GDN_EINVAL and "64 rows" in _err(lib)
    assert call(K=496, bits=4, gs=16, mode=3) == _lib.GDN_EINVAL and "multiple" in _err(lib)
    assert call(K=480, gs=64) == _lib.GDN_EINVAL and "multiple" in _err(lib)
    assert call(x=ctypes.c_void_p((1 << 30) + 8)) == _lib.GDN_EINVAL and "aligned" in _err(lib)
    assert call(sb=7) == _lib.GDN_EINVAL and "scales dtype" in _err(lib)
    assert call(M=0) == 0
    # K is split where the column tiles are few: out_proj (N = 2048: 64
    # tiles of 32 columns) 4 ways, the stacked input projection (193 tiles
    # of 64 columns) not at all
    size = lib.gdn_quantized_matmul_scheme_workspace_size
    assert size(64, 2048, 4096) == 4 * 64 * 2048 * 4
    assert size(1, 12352, 2048) == 0
    assert size(1, 96, 512) == 0               # 16 blocks of 32 k: too few to split
    assert size(1, 96, 2048) == 4 * 96 * 4     # 64 blocks: 4 splits of 16
    assert size(65, 2048, 4096) == 0 and size(1, 2048, 4080) == 0
