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
  the ``bits``-wide field at bit ``bits * (k % (32 // bits))`` of word
  ``k // (32 // bits)``, least significant first;
* ``w[n, k] = scales[n, g] * q[n, k] + biases[n, g]`` with ``g = k //
  group_size``; ``mx.dequantize`` returns it in the scales' dtype.

``quantize`` (the test-data generator) follows the affine min/max scheme:
``scale = (max - min) / (2**bits - 1)``, ``bias = min``, ``q = round((w -
bias) / scale)``. MLX's own ``quantize`` may choose scale and bias
differently; nothing here depends on it, only on ``dequantize``.

Parity unpinned against MLX itself (not importable): the bit layout and the
dequantization formula are restated from MLX's published format and pinned
here by closed forms (fixed words, round trips, extreme codes) in
``tests/test_oracle_quant.py``.
"""

from __future__ import annotations

import numpy as np

from .gated_delta_ref import bf16_round


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """Integer codes ``(N, K)`` in ``[0, 2**bits)`` -> uint32 words
    ``(N, K * bits / 32)``, least significant element first."""

    per = 32 // bits
    N, K = q.shape
    if K % per:
        raise ValueError("K must fill whole words")
    q = q.astype(np.uint64).reshape(N, K // per, per)
    shifts = (np.arange(per, dtype=np.uint64) * bits)[None, None, :]
    return (q << shifts).sum(axis=-1).astype(np.uint32)


def unpack(words: np.ndarray, bits: int) -> np.ndarray:
    """uint32 words ``(N, W)`` -> integer codes ``(N, W * 32 / bits)``."""

    per = 32 // bits
    w = words.astype(np.uint64)[:, :, None]
    shifts = (np.arange(per, dtype=np.uint64) * bits)[None, None, :]
    q = (w >> shifts) & np.uint64((1 << bits) - 1)
    return q.reshape(words.shape[0], -1).astype(np.int64)


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
