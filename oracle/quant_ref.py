"""CPU restatement of the reference's affine-quantized projections.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker, never as a product code path.

The reference runs its projections as ``mx.quantized_matmul(x, weight,
scales, biases, group_size, bits, mode="affine")`` (``model/moe_block.py:44-55``,
called from ``model/qwen3_5/linear_attention.py:96-101,125``) on weights that
``mx.quantize`` packed; its tests build dense reference weights with
``mx.dequantize`` (``tests/test_qwen3_5_linear_attention.py:59-70``). MLX
(pinned 0.32.2) is not installed here, so its published affine format is
restated:

* ``weight`` is uint32 ``(N, K * bits / 32)``; element ``k`` of row ``n`` is
  the ``bits``-wide field at bit ``bits * k`` of the row's little-endian bit
  stream (bytes in address order, least significant bit first). For 2, 4 and
  8 bits that is bit ``bits * (k % (32 // bits))`` of word ``k // (32 //
  bits)``; MLX packs 3-, 5- and 6-bit codes into groups of 3, 5 and 3 bytes
  (8, 8 and 4 codes, least significant first), which is the same stream;
* affine: ``w[n, k] = scales[n, g] * q[n, k] + biases[n, g]`` with ``g = k //
  group_size``; ``mx.dequantize`` returns it in the scales' dtype;
* mxfp4 / mxfp8 / nvfp4 (the OCP microscaling formats): ``w`` is the code's
  e2m1 (fp4) or e4m3 (fp8) value times its group's uint8 scale, e8m0
  (``2**(s - 127)``) for mxfp4 / mxfp8 (groups of 32), e4m3 for nvfp4
  (groups of 16); no biases.

``quantize`` (the test-data generator) follows the affine min/max scheme:
``scale = (max - min) / (2**bits - 1)``, ``bias = min``, ``q = round((w -
bias) / scale)``. MLX's own ``quantize`` may choose scale and bias
differently; nothing here depends on it, only on ``dequantize``.

Parity unpinned against MLX itself (not importable): the bit layouts and
the dequantization formulas are restated from MLX's published formats and
pinned in ``tests/test_oracle_quant.py`` by closed forms (hand-packed words
of 2- to 8-bit codes, round trips, extreme codes), the e4m3 and e8m0 codes
against torch's float8 dtypes (all 256 each), and e2m1 against e4m3 (each fp4
value re-encoded in fp8's fields).
"""

from __future__ import annotations

import numpy as np

from .gated_delta_ref import bf16_round


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """Integer codes ``(N, K)`` in ``[0, 2**bits)`` -> uint32 words
    ``(N, K * bits / 32)``: code k at bit ``bits * k`` of the row's
    little-endian bit stream."""

    N, K = q.shape
    if K * bits % 32:
        raise ValueError("K * bits must fill whole words")
    q = np.asarray(q, dtype=np.uint64)
    stream = ((q[:, :, None] >> np.arange(bits, dtype=np.uint64)) & np.uint64(1)).astype(np.uint8)
    packed = np.packbits(stream.reshape(N, K * bits), axis=-1, bitorder="little")
    return np.ascontiguousarray(packed).view("<u4").astype(np.uint32)


def unpack(words: np.ndarray, bits: int) -> np.ndarray:
    """uint32 words ``(N, W)`` -> integer codes ``(N, W * 32 / bits)``."""

    words = np.ascontiguousarray(np.asarray(words, dtype=np.uint32).astype("<u4"))
    N, W = words.shape
    stream = np.unpackbits(words.view(np.uint8), axis=-1, bitorder="little")
    fields = stream.reshape(N, W * 32 // bits, bits).astype(np.int64)
    return (fields << np.arange(bits, dtype=np.int64)).sum(axis=-1)


def e2m1_value(codes) -> np.ndarray:
    """OCP fp4 (E2M1): sign, a 2-bit exponent of bias 1 and a 1-bit
    mantissa; exponent 0 holds 0 and 0.5 (so the magnitudes are 0, 0.5, 1,
    1.5, 2, 3, 4, 6)."""

    c = np.asarray(codes, dtype=np.int64)
    e, m = (c >> 1) & 3, c & 1
    mag = np.where(e == 0, 0.5 * m, np.ldexp(1.0 + 0.5 * m, e - 1))
    return np.where(c & 8, -mag, mag)


def e4m3_value(codes) -> np.ndarray:
    """OCP fp8 E4M3 (the "fn" variant): sign, a 4-bit exponent of bias 7, a
    3-bit mantissa; exponent 0 subnormal (m * 2**-9); 0x7F and 0xFF NaN, no
    infinities."""

    c = np.asarray(codes, dtype=np.int64)
    e, m = (c >> 3) & 15, c & 7
    mag = np.where(e == 0, np.ldexp(m.astype(np.float64), -9), np.ldexp(1.0 + m / 8.0, e - 7))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(c & 0x80, -mag, mag)


def e8m0_value(codes) -> np.ndarray:
    """OCP E8M0 scale: 2**(c - 127); 255 is NaN."""

    c = np.asarray(codes, dtype=np.int64)
    return np.where(c == 255, np.nan, np.ldexp(1.0, c - 127))


_FP_MODES = {"mxfp4": (4, e2m1_value, e8m0_value), "mxfp8": (8, e4m3_value, e8m0_value),
             "nvfp4": (4, e2m1_value, e4m3_value)}


def dequantize_fp(words: np.ndarray, scales: np.ndarray, mode: str, group_size: int) -> np.ndarray:
    """Dense ``(N, K)`` float64 weights of an mxfp4 / mxfp8 / nvfp4
    projection: each code's value times its group's scale (exact in float32
    and bfloat16)."""

    bits, value, scale = _FP_MODES[mode]
    v = value(unpack(words, bits))
    return v * np.repeat(scale(np.asarray(scales)), group_size, axis=1)


def dequantize(words: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int,
               group_size: int, out: str = "bf16") -> np.ndarray:
    """Dense ``(N, K)`` float64 weights ``scales * q + biases`` rounded once
    to float32 (a fused multiply-add), then to ``out`` ("bf16", "f16" or
    "f32") like mx.dequantize's result in the scales' dtype."""

    q = unpack(words, bits).astype(np.float64)
    s = np.repeat(scales.astype(np.float64), group_size, axis=1)
    b = np.repeat(biases.astype(np.float64), group_size, axis=1)
    w = (s * q + b).astype(np.float32).astype(np.float64)
    if out == "bf16":
        return bf16_round(w)
    if out == "f16":
        return w.astype(np.float16).astype(np.float64)
    return w


def quantize(w: np.ndarray, bits: int, group_size: int, sb: str = "bf16"):
    """Affine min/max quantization of dense ``(N, K)`` weights: returns
    ``(words, scales, biases)`` with scales/biases rounded to ``sb``."""

    N, K = w.shape
    g = w.reshape(N, K // group_size, group_size).astype(np.float64)
    lo, hi = g.min(axis=-1), g.max(axis=-1)
    scale = np.maximum((hi - lo) / (2 ** bits - 1), 1e-8)
    rnd = bf16_round if sb == "bf16" else (lambda x: x.astype(np.float16).astype(np.float64)
                                           if sb == "f16" else x.astype(np.float32).astype(np.float64))
    scale, bias = rnd(scale), rnd(lo)
    q = np.clip(np.rint((g - bias[..., None]) / scale[..., None]), 0, 2 ** bits - 1)
    return pack(q.reshape(N, K).astype(np.int64), bits), scale, bias


def quantized_matmul(x: np.ndarray, words, scales, biases, bits: int, group_size: int,
                     w_round: str = "bf16") -> np.ndarray:
    """``x @ dequantize(W).T`` in float64 (the reference test's dense
    comparison: model/moe_block.py:44-55 against mx.dequantize weights)."""

    w = dequantize(words, scales, biases, bits, group_size, w_round)
    return x.astype(np.float64) @ w.T
