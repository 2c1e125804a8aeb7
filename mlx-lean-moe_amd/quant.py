"""Quantized linear projections (MLX's packings) for the layer's input and
output projections.

Mirrors ``mlx_lean_moe.config.QuantScheme`` (``config.py:10-33``) and
``mlx_lean_moe.model.moe_block.{LinearWeights, quantized_linear}``
(``model/moe_block.py:13-55``): a projection is either a dense ``(N, K)``
matrix or a dict ``{"weight", "scales"[, "biases"]}`` with ``weight`` uint32
``(N, K * bits / 32)`` (MLX's packing: element k at bit ``bits * k`` of the
row's little-endian bit stream) and per-group ``scales`` ``(N, K /
group_size)``. Affine schemes (2-8 bits): ``w = scales * q + biases``;
mxfp4 / mxfp8 / nvfp4: ``w`` = the e2m1 / e4m3 code's value times a uint8
scale (e8m0, e4m3 for nvfp4), no biases. Affine 4- and 8-bit projections of
bf16 activations run on ``gdn_quantized_matmul``; the other schemes and
activation dtypes dequantize on the GPU (``gdn_dequantize``) and multiply on
the vendor BLAS. Dense projections are ``x @ W.T``.
"""

from __future__ import annotations

import functools

from dataclasses import dataclass

import torch

from . import _lib

_SUPPORTED = {
    "affine": ({2, 3, 4, 5, 6, 8}, {32, 64, 128}),
    "mxfp4": ({4}, {32}),
    "mxfp8": ({8}, {32}),
    "nvfp4": ({4}, {16}),
}
# the mode codes of gdn_dequantize
_MODES = {"affine": 0, "mxfp4": 1, "mxfp8": 2, "nvfp4": 3}
# the affine widths the quantized matmul kernels take (the other schemes
# dequantize, then multiply on the vendor BLAS)
_KERNEL_BITS = {4, 8}
# From this many rows on, quantized_linear dequantizes the weights to bf16
# once and multiplies on the vendor BLAS (measured at hidden 2048 -> 12352:
# 73 vs 103 us at 1024 rows, 242 vs 336 us at 4096; even at 512 rows);
# below it gdn_quantized_matmul's kernels run directly, see _dense_rows.
_BLAS_ROWS = 512
# quantized_linear_split multiplies per block from this many rows on (one
# product of the stacked 2048 -> 12352 weight: 32.7 us at 512 rows against
# 45.9 us per block, 53.9 against 62.1 at 1024, even at 2048, 246 against
# 159 at 4096)
_SPLIT_ROWS = 2048


def _dense_rows(rows: int, N: int, K: int) -> bool:
    """Whether ``rows`` bf16 rows times a quantized ``(N, K)`` weight run on
    dequantized weights and the vendor BLAS rather than the quantized
    kernels. Above 64 rows the quantized tiled kernel takes 128 x 128 tiles
    with no K split, so a narrow or deep weight leaves the GPU idle: for
    4096 -> 2048 (out_proj) it takes 73-76 us from 65 to 1024 rows against
    23-34 us dense; for 2048 -> 12352 it wins up to ~400 rows (41-44 us
    against 45-57 us, device time from graphs)."""

    if rows >= _BLAS_ROWS:
        return True
    return rows > 64 and (N < 4096 or K >= 4096)


@dataclass(frozen=True)
class QuantScheme:
    """Bit width, group size and packing mode of a quantized projection;
    construction rejects the combinations MLX does not define (the checks
    of config.py:17-33)."""

    bits: int
    group_size: int
    mode: str = "affine"

    def __post_init__(self) -> None:
        if self.mode not in _SUPPORTED:
            raise ValueError(f"unsupported quantization mode {self.mode!r}")
        bits, groups = _SUPPORTED[self.mode]
        if self.bits not in bits or self.group_size not in groups:
            raise ValueError(f"unsupported {self.mode} quantization with bits={self.bits}, "
                             f"group_size={self.group_size}")


@dataclass(frozen=True)
class LinearWeights:
    """One projection's weights as read: a dense matrix (``quant`` None) or
    the packed codes with their per-group scales and biases under
    ``quant`` (the reference's type, moe_block.py:13-20).

    ``dense``, for quantized weights, optionally holds their bf16
    dequantization (``dequantize(tensors, quant, bfloat16)``, see
    :meth:`with_dense`): the prefill-sized products, which multiply on
    exactly those values, then skip converting the weights on every call, at
    the cost of keeping the copy (2 bytes per weight)."""

    tensors: object
    quant: QuantScheme | None
    dense: torch.Tensor | None = None

    def with_dense(self) -> "LinearWeights":
        """These weights with their bf16 dequantization kept alongside."""

        if self.quant is None:
            return self
        return LinearWeights(self.tensors, self.quant, dequantize(self.tensors, self.quant, torch.bfloat16))


def _on_kernels(quant: QuantScheme) -> bool:
    """Whether ``gdn_quantized_matmul`` multiplies by these codes directly."""

    return quant.mode == "affine" and quant.bits in _KERNEL_BITS


def _scheme_kernel_takes(x: torch.Tensor, rows: int, K: int, quant: QuantScheme) -> bool:
    """Whether gdn_quantized_matmul_scheme multiplies a scheme outside
    ``_on_kernels`` directly from its codes: bf16 ``x`` of at most 64 rows,
    ``K`` a multiple of 32 and at most 128 affine groups (256 of the float
    formats) per row, the scales its workgroups hold (decode sizes)."""

    groups = K // quant.group_size
    return (x.dtype == torch.bfloat16 and rows <= 64 and K % 32 == 0
            and groups <= (128 if quant.mode == "affine" else 256))


def _check_quantized(tensors: dict, quant: QuantScheme, K: int | None):
    w, scales = tensors["weight"], tensors["scales"]
    biases = tensors.get("biases")
    affine = quant.mode == "affine"
    if affine and biases is None:
        raise ValueError("affine quantized weights need biases")
    if not affine and biases is not None:
        raise ValueError(f"{quant.mode} weights carry no biases")
    if w.dtype not in (torch.int32, torch.uint32) or w.dim() != 2:
        raise ValueError("quantized weight must be a 2-D 32-bit integer tensor")
    N, words = w.shape
    if words * 32 % quant.bits:
        raise ValueError(f"{words} words per row hold no whole number of {quant.bits}-bit codes")
    k = words * 32 // quant.bits
    if K is not None and K != k:
        raise ValueError(f"input width {K} does not match the weight's {k}")
    if k % quant.group_size:
        raise ValueError(f"a row of {k} codes holds no whole number of groups of {quant.group_size}")
    if tuple(scales.shape) != (N, k // quant.group_size) or (affine and scales.shape != biases.shape):
        raise ValueError(f"scales{' and biases' if affine else ''} must have shape "
                         f"{(N, k // quant.group_size)}")
    if affine and scales.dtype != biases.dtype:
        raise ValueError("scales and biases must share a dtype")
    if not affine and scales.dtype != torch.uint8:
        raise ValueError(f"{quant.mode} scales are uint8 codes, got {scales.dtype}")
    return w, scales, biases, N, k


def _c(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def dequantize(tensors: dict, quant: QuantScheme, dtype: torch.dtype | None = None):
    """Dense ``(N, K)`` weights of a quantized projection, in ``dtype``
    (default: the scales' dtype for affine schemes, bf16 for the float
    ones), computed on the GPU (mx.dequantize's counterpart)."""

    w, scales, biases, N, K = _check_quantized(tensors, quant, None)
    if w.device.type != "cuda":
        raise RuntimeError(f"quantized weights must be on a ROCm device, got {w.device}")
    if dtype is None:
        dtype = scales.dtype if quant.mode == "affine" else torch.bfloat16
    out = torch.empty((N, K), dtype=dtype, device=w.device)
    w, scales = _c(w), _c(scales)
    if w.data_ptr() % 16:
        w = w.clone()
    biases = _c(biases) if biases is not None else None
    sb_dtype = _lib.dtype_code(scales.dtype) if quant.mode == "affine" else 0
    _lib.call("gdn_dequantize", _lib.ptr(w), _lib.ptr(scales), _lib.ptr(biases), sb_dtype,
              _lib.ptr(out), _lib.dtype_code(out.dtype), N, K, quant.bits, quant.group_size,
              _MODES[quant.mode], _lib.stream_ptr(w.device))
    return out


def decode_kernel_takes(M: int, K: int, bits: int, group_size: int, sb_dtype: torch.dtype) -> bool:
    """Whether gdn_quantized_matmul runs this shape on its decode kernel
    (the rule of decode_kernel_fits in gdn_qlinear.hip, for aligned
    operands): up to 64 rows, K in whole steps of 8 quantization slices (32
    k for group 32, else 64) with at most 16 steps and the packed words of a
    thread's share in 64 registers, K / group_size <= 64 and whole 16-byte
    pieces of scales per column. That kernel multiplies by the exact weights
    scale * q + bias; the tiled kernels by the weights rounded to bf16."""

    if M > 64:
        return False
    step = 8 * (32 if group_size == 32 else 64)
    ks, gpr = K // step, K // group_size
    return (K % step == 0 and ks in (1, 2, 4, 8, 16) and ks * step * bits // 256 <= 64
            and gpr <= 64 and gpr % (4 if sb_dtype == torch.float32 else 8) == 0)


def quantized_linear(x: torch.Tensor, tensors, quant: QuantScheme | None = None, *,
                     residual: torch.Tensor | None = None) -> torch.Tensor:
    """Linear projection for self-describing, legacy quantized, or dense
    weights (moe_block.py:27-55): ``x @ W.T`` over the last axis of ``x``.
    Quantized weights give ``x``'s dtype; dense ones the promotion of ``x``'s
    and ``W``'s dtypes, as MLX's matmul does (a checkpoint's bf16 dense
    weights are read widened to float32).

    ``residual`` (the result's shape and dtype) is added to the product
    rounded to that dtype, as the decoder layer's ``h = x + attention(...)``
    (transformer.py:110-112) adds two arrays of it; on the quantized
    kernels the add is part of the store."""

    dense = None
    if isinstance(tensors, LinearWeights):
        quant, dense = tensors.quant, tensors.dense
        tensors = tensors.tensors

    def with_residual(out: torch.Tensor) -> torch.Tensor:
        if residual is None:
            return out
        _check_residual(residual, out.shape, out.dtype)
        return out + residual

    if isinstance(tensors, torch.Tensor):
        dt = torch.promote_types(x.dtype, tensors.dtype)
        return with_residual(x.to(dt) @ tensors.to(dt).T)
    if quant is None:
        raise ValueError("quantized linear weights require a quantization scheme")
    w, scales, biases, N, K = _check_quantized(tensors, quant, x.shape[-1])
    if x.device.type != "cuda":
        raise RuntimeError(f"quantized projections run on ROCm devices only; got {x.device}")
    lead = x.shape[:-1]
    rows = x.reshape(-1, K).shape[0]
    if not _on_kernels(quant):
        if _scheme_kernel_takes(x, rows, K, quant):
            return _scheme_matmul(x, w, scales, biases, quant, N, K, residual)
        # above decode sizes: their exact weights in x's dtype (bf16 for
        # the float schemes is exact), then the vendor BLAS
        wd = dense if dense is not None else dequantize(tensors, quant, x.dtype)
        return with_residual(x @ wd.to(x.dtype).T)
    x_f32 = (x.dtype == torch.float32 and rows <= 32
             and decode_kernel_takes(rows, K, quant.bits, quant.group_size, scales.dtype))
    if x.dtype != torch.bfloat16 and not x_f32:
        return with_residual(x @ dequantize(tensors, quant, x.dtype).T)
    x2 = _c(x.reshape(-1, K))
    if _dense_rows(x2.shape[0], N, K):
        # the same bf16-rounded weights as the tiled kernel (gdn_dequantize),
        # one transient copy, and the vendor BLAS for the GEMM itself
        wd = dense if dense is not None else dequantize(tensors, quant, torch.bfloat16)
        return with_residual((x2 @ wd.T).reshape(*lead, N))
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    r = _residual_rows(residual, x, lead, M, N)
    w, scales, biases = _c(w), _c(scales), _c(biases)
    ws_bytes = workspace_bytes(x2.dtype, scales.dtype, M, N, K, quant.bits, quant.group_size)
    # a transient from the caching allocator (graph-capture safe); the split
    # kernels overwrite what they read
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.call("gdn_quantized_matmul", _lib.ptr(x2), _lib.dtype_code(x2.dtype), _lib.ptr(w), _lib.ptr(scales),
              _lib.ptr(biases), _lib.dtype_code(scales.dtype), _lib.ptr(y),
              _lib.dtype_code(y.dtype), _lib.ptr(r), M, N, K, quant.bits, quant.group_size, _lib.ptr(ws),
              ws_bytes, _lib.stream_ptr(x.device))
    return y.reshape(*lead, N)


def _residual_rows(residual, x: torch.Tensor, lead, M: int, N: int):
    """The residual as ``(M, N)`` rows for a kernel's fused add (None
    without one), after checking its shape, dtype and device."""

    if residual is None:
        return None
    _check_residual(residual, (*lead, N), x.dtype)
    if residual.device != x.device:
        raise ValueError("residual must be on the projection's device")
    return _c(residual.reshape(M, N))


def _scheme_matmul(x, w, scales, biases, quant: QuantScheme, N: int, K: int, residual):
    """``x @ W.T`` (+ residual) for affine 2/3/5/6-bit, mxfp4, mxfp8 and
    nvfp4 codes at decode sizes (gdn_quantized_matmul_scheme): the packed
    codes are multiplied where they lie, with float32 per-group sums, so a
    call reads the weight at its packed size."""

    lead = x.shape[:-1]
    x2 = _c(x.reshape(-1, K))
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    r = _residual_rows(residual, x, lead, M, N)
    w, scales = _c(w), _c(scales)
    if w.data_ptr() % 16:
        w = w.clone()
    affine = quant.mode == "affine"
    biases = _c(biases) if affine else None
    ws_bytes = scheme_workspace_bytes(M, N, K)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.call("gdn_quantized_matmul_scheme", _lib.ptr(x2), _lib.ptr(w), _lib.ptr(scales), _lib.ptr(biases),
              _lib.dtype_code(scales.dtype) if affine else 0, _lib.ptr(y), _lib.dtype_code(y.dtype),
              _lib.ptr(r), M, N, K, quant.bits, quant.group_size, _MODES[quant.mode], _lib.ptr(ws), ws_bytes,
              _lib.stream_ptr(x.device))
    return y.reshape(*lead, N)


def quantized_linear_split(x: torch.Tensor, weights: LinearWeights, sizes) -> list[torch.Tensor]:
    """``x @ W.T`` for a quantized ``W`` stacked from projections that share
    ``x`` (:func:`concat_quantized`), returned as the column blocks ``sizes``
    (which sum to ``W``'s rows): what :func:`quantized_linear` of each
    projection would give, in one launch where that pays.

    Where the dense path runs (bf16 ``x``, :func:`_dense_rows`: prefill
    sizes) ``W`` is dequantized once (or its kept copy used); from
    ``_SPLIT_ROWS`` rows on each block is its own GEMM on the vendor BLAS
    with a packed output: for hidden 2048 -> 8192|4096|64 at 4096 rows the
    blocks take 159 us together against 246 us for one 12352-column product
    (the library tiles that N poorly at that size), while below 2048 rows the
    one product is faster and the blocks are column views of it, as they are
    of the one quantized launch at decode sizes."""

    tensors, quant = weights.tensors, weights.quant
    sizes = [int(n) for n in sizes]
    if sum(sizes) != tensors["weight"].shape[0]:
        raise ValueError(f"block sizes {sizes} do not add up to the {tensors['weight'].shape[0]} "
                         f"stacked rows")
    K = x.shape[-1]
    rows = x.reshape(-1, K).shape[0]
    if (x.dtype == torch.bfloat16 and x.device.type == "cuda"
            and (_dense_rows(rows, tensors["weight"].shape[0], K)
                 or not (_on_kernels(quant) or _scheme_kernel_takes(x, rows, K, quant)))):
        _check_quantized(tensors, quant, K)
        lead = x.shape[:-1]
        x2 = _c(x.reshape(-1, K))
        wd = weights.dense if weights.dense is not None else dequantize(tensors, quant, torch.bfloat16)
        if rows < _SPLIT_ROWS:
            # one product; the blocks are column views of it
            return list(torch.split((x2 @ wd.T).reshape(*lead, -1), sizes, dim=-1))
        return [(x2 @ blk.T).reshape(*lead, blk.shape[0]) for blk in torch.split(wd, sizes)]
    return list(torch.split(quantized_linear(x, weights), sizes, dim=-1))


def _check_residual(residual: torch.Tensor, shape, dtype: torch.dtype) -> None:
    if tuple(residual.shape) != tuple(shape) or residual.dtype != dtype:
        raise ValueError(f"residual must be {tuple(shape)} {dtype}, got {tuple(residual.shape)} "
                         f"{residual.dtype}")


@functools.lru_cache(maxsize=256)
def scheme_workspace_bytes(M: int, N: int, K: int) -> int:
    """Workspace gdn_quantized_matmul_scheme splits K with (0: none)."""

    return int(_lib.load().gdn_quantized_matmul_scheme_workspace_size(M, N, K))


@functools.lru_cache(maxsize=256)
def workspace_bytes(x_dtype: torch.dtype, sb_dtype: torch.dtype, M: int, N: int, K: int, bits: int,
                    group_size: int) -> int:
    """Workspace gdn_quantized_matmul splits K with for these sizes (0: none)."""

    return int(_lib.load().gdn_quantized_matmul_workspace_size(
        _lib.dtype_code(x_dtype), _lib.dtype_code(sb_dtype), M, N, K, bits, group_size))


def concat_quantized(parts: list[dict]) -> dict:
    """Stacks quantized projections that share an input (same K, scheme and
    scales dtype) along N, so that one launch computes all of them."""

    keys = [k for k in ("weight", "scales", "biases") if k in parts[0]]
    return {key: torch.cat([p[key] for p in parts], dim=0) for key in keys}
