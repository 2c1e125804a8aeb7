"""Loading the gated-delta layer's weights from an MLX checkpoint's
safetensors shards, in the on-disk format the reference reads.

The reference indexes a checkpoint's shards by byte range
(``weights/safetensors_index.py``), reads single tensors with ``os.pread``
(``weights/expert_loader.py:164-180``), decodes them
(``expert_loader.py:53-85``: BF16 is widened exactly to float32, except the
quantization ``scales``/``biases``, which keep their stored bf16 width),
checks each projection's packed layout (``expert_loader.py:95-141``) and
reads it as dense or quantized weights (``expert_loader.py:144-161``); the
decoder layer pulls the linear-attention tensors by name
(``model/qwen3_5/transformer.py:52-65``) and the HF config supplies the shapes
and quantization (``model/qwen3_5/config.py:70-107,141-215``). This module restates
that format for torch tensors: the host side decodes into CPU tensors, which
``load_linear_attention`` moves to the device.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Iterator, NamedTuple

import torch

from .config import LinearAttentionDims
from .quant import LinearWeights, QuantScheme


class TensorSpan(NamedTuple):
    """One tensor inside a shard file: the safetensors dtype tag ("BF16",
    "F32", "U32", ...), its shape, and the absolute byte range
    ``[begin, end)`` of its data in that file."""

    shard: str
    dtype: str
    shape: tuple[int, ...]
    begin: int
    end: int

    @property
    def nbytes(self) -> int:
        return self.end - self.begin


def _read_header(path: Path) -> Iterator[tuple[str, str, tuple[int, ...], int, int]]:
    """The entries of one safetensors file: a little-endian u64 header
    length, that many bytes of JSON, then the data, which each entry's
    ``data_offsets`` address relative to the data's first byte."""

    with path.open("rb") as f:
        size = int.from_bytes(f.read(8), "little")
        entries = json.loads(f.read(size))
    base = 8 + size
    for key, meta in entries.items():
        if key != "__metadata__":
            lo, hi = meta["data_offsets"]
            yield key, meta["dtype"], tuple(meta["shape"]), base + lo, base + hi


def _shard_files(model_dir: Path) -> list[str]:
    """Shard file names of a checkpoint: the ones the HF sharding index
    ``model.safetensors.index.json`` maps tensors to, else the lone
    ``model.safetensors``."""

    sharded = model_dir / "model.safetensors.index.json"
    if sharded.is_file():
        mapping = json.loads(sharded.read_text())["weight_map"]
        return sorted(set(mapping.values()))
    if (model_dir / "model.safetensors").is_file():
        return ["model.safetensors"]
    raise FileNotFoundError(f"{model_dir} holds neither a sharding index "
                            f"(model.safetensors.index.json) nor model.safetensors")


def build_index(model_dir: str | Path) -> dict[str, TensorSpan]:
    """Tensor name -> :class:`TensorSpan` over every shard of a checkpoint."""

    model_dir = Path(model_dir)
    return {key: TensorSpan(shard, dtype, shape, lo, hi)
            for shard in _shard_files(model_dir)
            for key, dtype, shape, lo, hi in _read_header(model_dir / shard)}


# safetensors dtype -> the torch dtype holding the same bytes (unsigned
# integers as the signed type of their width: the packed U32 weights are
# handed to the kernels as raw words)
_TORCH_DTYPES = {
    "F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
    "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8,
    "U64": torch.int64, "U32": torch.int32, "U16": torch.int16, "U8": torch.uint8,
    "BOOL": torch.bool,
}


def is_quant_metadata(name: str) -> bool:
    """Whether a tensor is a quantized projection's per-group ``scales`` or
    ``biases``: those are handed to the matmul at their stored width. Every
    other bf16 tensor on this path (conv kernel, ``A_log``, ``dt_bias``,
    norm weight) feeds float32 arithmetic and is widened on read
    (expert_loader.py:53-59)."""

    return name.split(".")[-1] in ("scales", "biases")


def decode_tensor(raw: bytes, dtype: str, shape: tuple[int, ...], *,
                  stored_width: bool = False) -> torch.Tensor:
    """Raw little-endian bytes -> a CPU tensor (expert_loader.py:62-85):
    BF16 widens exactly to float32 (a bf16 value is the top half of its
    float32) unless ``stored_width``; other dtypes keep theirs."""

    torch_dtype = _TORCH_DTYPES.get(dtype)
    if torch_dtype is None:
        raise ValueError(f"unsupported safetensors dtype: {dtype!r}")
    buf = bytearray(raw)  # writable, so torch owns an ordinary tensor
    if dtype == "BF16":
        bits = torch.frombuffer(buf, dtype=torch.int16) if buf else torch.empty(0, dtype=torch.int16)
        if stored_width:
            return bits.view(torch.bfloat16).reshape(shape)
        return (bits.to(torch.int32) << 16).view(torch.float32).reshape(shape)
    if not buf:
        return torch.empty(shape, dtype=torch_dtype)
    return torch.frombuffer(buf, dtype=torch_dtype).reshape(shape)


class CheckpointReader:
    """Whole-tensor reads out of a checkpoint's shards by name
    (expert_loader.py:164-180): one ``os.pread`` per tensor, one descriptor
    per shard."""

    def __init__(self, model_dir: str | Path, index: dict[str, TensorSpan] | None = None):
        self.model_dir = Path(model_dir)
        self.index = index if index is not None else build_index(self.model_dir)
        self._fds: dict[str, int] = {}

    def _fd(self, shard: str) -> int:
        fd = self._fds.get(shard)
        if fd is None:
            fd = self._fds[shard] = os.open(str(self.model_dir / shard), os.O_RDONLY)
        return fd

    def read_tensor(self, name: str) -> torch.Tensor:
        span = self.index[name]
        raw = os.pread(self._fd(span.shard), span.nbytes, span.begin)
        if len(raw) != span.nbytes:
            raise ValueError(f"{name}: shard {span.shard} is truncated")
        return decode_tensor(raw, span.dtype, span.shape, stored_width=is_quant_metadata(name))

    def read_fields(self, name: str, fields) -> dict[str, torch.Tensor]:
        """``{field: tensor}`` for each ``name.field`` the checkpoint holds."""

        return {f: self.read_tensor(f"{name}.{f}") for f in fields if f"{name}.{f}" in self.index}

    def close(self) -> None:
        for fd in self._fds.values():
            os.close(fd)
        self._fds.clear()

    def __enter__(self) -> "CheckpointReader":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


class LayoutError(ValueError):
    """A projection's tensors in a checkpoint do not fit together under its
    quantization scheme."""


def projection_is_quantized(index: dict[str, TensorSpan], name: str, scheme: QuantScheme) -> bool:
    """Whether projection ``name`` is stored quantized (``name.scales``, and
    ``name.biases`` where the scheme has them, beside the packed
    ``name.weight``) or as a plain matrix (``name.weight`` alone).

    A missing weight raises ``KeyError``. Otherwise every inconsistency is
    collected and reported together in one :class:`LayoutError`: biases
    stored without scales; an affine scheme without biases; biases beside
    the codes of a float scheme (mxfp4, mxfp8, nvfp4), which has none; biases
    not shaped like the scales; weight and scales disagreeing in their leading
    (row) dimensions; a packed row width other than the scale groups'
    ``groups * group_size * bits / 32`` words. These are the conditions the
    reference's loader enforces (expert_loader.py:95-141) with one more:
    that loader only shape-checks biases stored beside float-scheme codes
    and hands them to the matmul, whose float modes have no bias term; here
    such a checkpoint is refused when it is read."""

    weight = index.get(f"{name}.weight")
    scales = index.get(f"{name}.scales")
    biases = index.get(f"{name}.biases")
    if weight is None:
        raise KeyError(f"{name}.weight is not in the checkpoint")
    if scales is None and biases is None:
        return False
    problems = []
    if scales is None:
        problems.append("per-group biases are stored without the scales they pair with")
    else:
        if biases is None and scheme.mode == "affine":
            problems.append("the affine scheme dequantizes with per-group biases; none are stored")
        if biases is not None and scheme.mode != "affine":
            problems.append(f"the {scheme.mode} scheme has no biases; some are stored")
        elif biases is not None and biases.shape != scales.shape:
            problems.append(f"biases {biases.shape} and scales {scales.shape} differ in shape")
        if weight.shape[:-1] != scales.shape[:-1]:
            problems.append(f"weight {weight.shape} and scales {scales.shape} differ in their "
                            f"leading dimensions")
        words = scales.shape[-1] * scheme.group_size * scheme.bits // 32
        if weight.shape[-1] != words:
            problems.append(f"{scales.shape[-1]} groups of {scheme.group_size} {scheme.bits}-bit "
                            f"codes pack into {words} words a row; weight {weight.shape} has "
                            f"{weight.shape[-1]}")
    if problems:
        raise LayoutError(f"{name}: " + "; ".join(problems))
    return True


def read_projection(reader: CheckpointReader, name: str, scheme: QuantScheme) -> LinearWeights:
    """Projection ``name`` as a plain matrix (``quant`` None) or as its
    quantized fields under ``scheme`` (expert_loader.py:144-161)."""

    if projection_is_quantized(reader.index, name, scheme):
        return LinearWeights(reader.read_fields(name, ("weight", "scales", "biases")), scheme)
    return LinearWeights(reader.read_tensor(f"{name}.weight"), None)


@dataclass(frozen=True)
class QuantConfig:
    """A checkpoint's quantization: the default scheme and exact
    per-projection overrides (config.py:70-77)."""

    default: QuantScheme
    overrides: tuple[tuple[str, QuantScheme], ...] = ()

    def quant_for(self, name: str, fallback: QuantScheme | None = None) -> QuantScheme:
        for tensor_name, scheme in self.overrides:
            if tensor_name == name:
                return scheme
        return fallback or self.default


def quant_config_from_hf(hf_config: dict) -> QuantConfig:
    """The ``quantization`` (or ``quantization_config``) block of an HF
    config: top-level bits/group_size/mode (defaults 4, 64, affine) and
    nested per-tensor dicts as overrides (config.py:80-107,172-173)."""

    quant = hf_config.get("quantization") or hf_config.get("quantization_config") or {}
    default = QuantScheme(int(quant.get("bits", 4)), int(quant.get("group_size", 64)),
                          str(quant.get("mode", "affine")))
    overrides = []
    for name, value in quant.items():
        if isinstance(value, dict):
            base = name.removesuffix(".weight").removesuffix(".scales").removesuffix(".biases")
            overrides.append((base, QuantScheme(int(value.get("bits", default.bits)),
                                                int(value.get("group_size", default.group_size)),
                                                str(value.get("mode", default.mode)))))
    return QuantConfig(default, tuple(overrides))


def linear_dims_from_hf(hf_config: dict) -> LinearAttentionDims:
    """The gated-delta shape from an HF config (its ``text_config`` when
    nested; config.py:141,187-193)."""

    text = hf_config.get("text_config", hf_config)
    return LinearAttentionDims(int(text["linear_num_key_heads"]), int(text["linear_num_value_heads"]),
                               int(text["linear_key_head_dim"]), int(text["linear_value_head_dim"]),
                               int(text["linear_conv_kernel_dim"]))


_PROJECTIONS = ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj")


def _to_device(w: LinearWeights, device) -> LinearWeights:
    if isinstance(w.tensors, dict):
        return LinearWeights({k: v.to(device) for k, v in w.tensors.items()}, w.quant)
    return LinearWeights(w.tensors.to(device), w.quant)


def load_linear_attention(model_dir: str | Path, layer_index: int, *, device="cuda",
                          hf_config: dict | None = None,
                          tensor_prefix: str = "language_model.model"):
    """The gated-delta layer ``layer_index`` of a checkpoint
    (transformer.py:52-65): projections with their own schemes (stored-width
    scales and biases), ``conv1d.weight (C, K, 1)``, ``A_log``, ``dt_bias``
    and ``norm.weight`` widened to float32, on ``device``."""

    from .linear_attention import Qwen3_5LinearAttention

    model_dir = Path(model_dir)
    if hf_config is None:
        hf_config = json.loads((model_dir / "config.json").read_text())
    dims = linear_dims_from_hf(hf_config)
    quant = quant_config_from_hf(hf_config)
    eps = float(hf_config.get("text_config", hf_config).get("rms_norm_eps", 1e-6))
    prefix = f"{tensor_prefix}.layers.{layer_index}.linear_attn"
    with CheckpointReader(model_dir) as reader:
        proj = {p: _to_device(read_projection(reader, f"{prefix}.{p}", quant.quant_for(f"{prefix}.{p}")),
                              device) for p in _PROJECTIONS}
        conv = reader.read_tensor(f"{prefix}.conv1d.weight")
        A_log = reader.read_tensor(f"{prefix}.A_log")
        dt_bias = reader.read_tensor(f"{prefix}.dt_bias")
        norm = reader.read_tensor(f"{prefix}.norm.weight")
    if tuple(conv.shape) != (dims.conv_dim, dims.conv_kernel_dim, 1):
        raise ValueError(f"{prefix}.conv1d.weight has shape {tuple(conv.shape)}, expected "
                         f"{(dims.conv_dim, dims.conv_kernel_dim, 1)}")
    f32 = lambda t: t.to(device=device, dtype=torch.float32)
    return Qwen3_5LinearAttention(dims, proj["in_proj_qkv"], proj["in_proj_z"], proj["in_proj_a"],
                                  proj["in_proj_b"], f32(conv), f32(A_log), f32(dt_bias), f32(norm),
                                  proj["out_proj"], rms_norm_eps=eps)
