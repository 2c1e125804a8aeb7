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
