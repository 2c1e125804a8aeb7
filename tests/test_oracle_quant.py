"""Pins the oracle's restatement of MLX's affine quantized format (packing
order and dequantization) with closed forms and an independent scalar loop;
CPU only."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quant_ref as Q
from oracle.gated_delta_ref import bf16_round


def test_unpack_fixed_words_least_significant_first():
    np.testing.assert_array_equal(Q.unpack(np.array([[0x76543210]], np.uint32), 4)[0],
                                  np.arange(8))
    np.testing.assert_array_equal(Q.unpack(np.array([[0xFEDCBA98]], np.uint32), 4)[0],
                                  np.arange(8, 16))
    np.testing.assert_array_equal(Q.unpack(np.array([[0x04030201, 0xFF00807F]], np.uint32), 8)[0],
                                  [1, 2, 3, 4, 0x7F, 0x80, 0x00, 0xFF])


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_unpack_round_trip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 2 ** bits, (5, 64))
    w = Q.pack(q, bits)
    assert w.dtype == np.uint32 and w.shape == (5, 64 * bits // 32)
    np.testing.assert_array_equal(Q.unpack(w, bits), q)


def test_dequantize_extreme_codes():
    bits, gs = 4, 32
    s = bf16_round(np.array([[0.5, -0.25]]))
    b = bf16_round(np.array([[-1.0, 2.0]]))
    zeros = Q.pack(np.zeros((1, 64), np.int64), bits)
    full = Q.pack(np.full((1, 64), 15, np.int64), bits)
    np.testing.assert_array_equal(Q.dequantize(zeros, s, b, bits, gs)[0],
                                  np.repeat(b[0], gs))
    np.testing.assert_array_equal(Q.dequantize(full, s, b, bits, gs)[0],
                                  np.repeat(15 * s[0] + b[0], gs))


def test_dequantize_matches_scalar_bit_extraction():
    # an independent scalar loop over Python ints
    bits, gs, N, K = 4, 32, 3, 64
    rng = np.random.default_rng(5)
    words = rng.integers(0, 2 ** 32, (N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = bf16_round(rng.uniform(0.01, 0.1, (N, K // gs)))
    b = bf16_round(rng.uniform(-1, 1, (N, K // gs)))
    got = Q.dequantize(words, s, b, bits, gs, out="f32")
    for n in range(N):
        for k in range(K):
            word = int(words[n, k // 8])
            code = (word >> (4 * (k % 8))) & 0xF
            want = float(np.float32(s[n, k // gs] * code + b[n, k // gs]))
            assert got[n, k] == want, (n, k)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_error_within_half_step(bits):
    rng = np.random.default_rng(9)
    w = rng.standard_normal((4, 128))
    words, s, b = Q.quantize(w, bits, 64, sb="f32")
    deq = Q.dequantize(words, s, b, bits, 64, out="f32")
    step = np.repeat(s, 64, axis=1)
    assert np.all(np.abs(deq - w) <= step * 0.5 + 1e-6)


def test_quantized_matmul_is_x_times_dequantized_weights():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 64))
    words, s, b = Q.quantize(rng.standard_normal((3, 64)), 4, 32)
    y = Q.quantized_matmul(x, words, s, b, 4, 32)
    deq = Q.dequantize(words, s, b, 4, 32)
    for m in range(2):
        for n in range(3):
            assert abs(y[m, n] - sum(x[m, k] * deq[n, k] for k in range(64))) < 1e-12


def _word_layout_pack(q, bits):
    """4-, 2- and 8-bit packing by words: code k at bit bits * (k % per) of
    word k // per (per = 32 / bits)."""

    per = 32 // bits
    N, K = q.shape
    out = np.zeros((N, K // per), np.uint64)
    for k in range(K):
        out[:, k // per] |= q[:, k].astype(np.uint64) << np.uint64(bits * (k % per))
    return out.astype(np.uint32)


def _byte_group_pack(q, bits):
    """3-, 5- and 6-bit packing as MLX's byte groups: pack_factor codes
    (8, 8, 4) into bytes_per_pack bytes (3, 5, 3), least significant code
    first, each group's integer written little-endian."""

    factor, nbytes = {3: (8, 3), 5: (8, 5), 6: (4, 3)}[bits]
    rows = []
    for row in q:
        out = bytearray()
        for i in range(0, len(row), factor):
            v = sum(int(c) << (bits * j) for j, c in enumerate(row[i:i + factor]))
            out += v.to_bytes(nbytes, "little")
        rows.append(np.frombuffer(bytes(out), "<u4").astype(np.uint32))
    return np.stack(rows)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_packing_of_every_affine_width(bits):
    """One bit stream for every width: 2/4/8-bit codes by words, 3/5/6-bit
    codes by MLX's byte groups (constructed independently), round trips,
    extreme codes and the reference's packed-width rule (K * bits / 32
    words, expert_loader.py's "expected packed width")."""

    rng = np.random.default_rng(100 + bits)
    q = rng.integers(0, 2 ** bits, (4, 128))
    q[0] = 2 ** bits - 1
    q[1] = 0
    w = Q.pack(q, bits)
    assert w.shape == (4, 128 * bits // 32)
    ref = _word_layout_pack(q, bits) if bits in (2, 4, 8) else _byte_group_pack(q, bits)
    np.testing.assert_array_equal(w, ref)
    np.testing.assert_array_equal(Q.unpack(w, bits), q)
    assert (w[0] == 0xFFFFFFFF).all() and (w[1] == 0).all()


def test_three_bit_codes_fixed_words():
    # codes 1..7, 0 repeated: each group of 8 is the 24-bit 0x1F58D1 (bytes D1 58 1F)
    q = np.array([[1, 2, 3, 4, 5, 6, 7, 0] * 4])
    np.testing.assert_array_equal(Q.pack(q, 3)[0], [0xD11F58D1, 0x58D11F58, 0x1F58D11F])


def test_e4m3_and_e8m0_codes_match_torch_float8():
    torch = pytest.importorskip("torch")
    codes = np.arange(256)
    as8 = torch.from_numpy(codes.astype(np.uint8))
    for mine, dt in ((Q.e4m3_value, torch.float8_e4m3fn), (Q.e8m0_value, torch.float8_e8m0fnu)):
        ref = as8.view(dt).double().numpy()
        got = mine(codes)
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
        np.testing.assert_array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])


def test_e2m1_codes_are_their_e4m3_reencoding():
    """Each fp4 code re-encoded in fp8's fields (the same sign, the exponent
    re-biased from 1 to 7, the mantissa bit on top of three) decodes to the
    same value through torch; and the OCP table's magnitudes."""

    torch = pytest.importorskip("torch")
    c = np.arange(16)
    s, e, m = c >> 3, (c >> 1) & 3, c & 1
    # exponent 0: 0 or 0.5 (= 2^-1: e4m3 exponent field 6, mantissa 0)
    fp8 = np.where(e > 0, (s << 7) | ((e - 1 + 7) << 3) | (m << 2), np.where(m == 1, (s << 7) | (6 << 3), s << 7))
    ref = torch.from_numpy(fp8.astype(np.uint8)).view(torch.float8_e4m3fn).double().numpy()
    np.testing.assert_array_equal(Q.e2m1_value(c), ref)
    np.testing.assert_array_equal(np.abs(Q.e2m1_value(c[:8])), [0, 0.5, 1, 1.5, 2, 3, 4, 6])


@pytest.mark.parametrize("mode,gs", [("mxfp4", 32), ("mxfp8", 32), ("nvfp4", 16)])
def test_float_scheme_is_code_value_times_group_scale(mode, gs):
    bits = 8 if mode == "mxfp8" else 4
    rng = np.random.default_rng(len(mode) + gs)
    q = rng.integers(0, 2 ** bits, (3, 64))
    scales = rng.integers(120, 135, (3, 64 // gs)) if mode != "nvfp4" else rng.integers(0x30, 0x50, (3, 4))
    w = Q.dequantize_fp(Q.pack(q, bits), scales, mode, gs)
    value = Q.e4m3_value if mode == "mxfp8" else Q.e2m1_value
    scale = Q.e4m3_value if mode == "nvfp4" else Q.e8m0_value
    for n in range(3):
        for k in range(64):
            assert w[n, k] == value(q[n, k]) * scale(scales[n, k // gs]) or np.isnan(w[n, k])
    finite = w[np.isfinite(w)]
    np.testing.assert_array_equal(bf16_round(finite), finite)  # exact in bf16
