"""Loading the gated-delta layer's weights from an MLX checkpoint's
safetensors shards, in the on-disk format the reference reads.

The reference indexes a checkpoint's shards by byte range
(``weights/safetensors_index.py``), reads single tensors with ``os.pread``
(``weights/expert_loader.py:164-180``), decodes them
(``expert_loader.py:53-85``: BF16 is widened exactly to float32, except the
quantization ``scales``/``biases``, which keep their stored bf16 width),
validates each projection's packed layout (``expert_loader.py:95-141``) and
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
import struct
from dataclasses import dataclass
from pathlib import Path

import torch

from .config import LinearAttentionDims
from .quant import LinearWeights, QuantScheme

_INDEX_FILENAME = "model.safetensors.index.json"
_SINGLE_FILENAME = "model.safetensors"


@dataclass(frozen=True)
class TensorLocation:
    """Where one tensor's raw bytes live (safetensors_index.py:18-24)."""

    shard: str  # file name, relative to the checkpoint directory
    dtype: str  # safetensors dtype string: "BF16", "F32", "U32", ...
    shape: tuple[int, ...]
    offset: int  # absolute byte offset in the shard
    length: int  # byte length of the raw data


def _shard_header(path: Path) -> tuple[dict, int]:
    with path.open("rb") as f:
        (header_len,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(header_len))
    return header, 8 + header_len


def _shards(model_dir: Path) -> list[str]:
    index_json = model_dir / _INDEX_FILENAME
    if index_json.exists():
        return sorted(set(json.loads(index_json.read_text())["weight_map"].values()))
    if (model_dir / _SINGLE_FILENAME).exists():
        return [_SINGLE_FILENAME]
    raise FileNotFoundError(f"no {_INDEX_FILENAME} or {_SINGLE_FILENAME} found under {model_dir}")


def build_index(model_dir: str | Path) -> dict[str, TensorLocation]:
    """Tensor name -> location over every shard of a checkpoint (the shards
    an index file names, or the single ``model.safetensors``)."""

    model_dir = Path(model_dir)
    index: dict[str, TensorLocation] = {}
    for shard in _shards(model_dir):
        header, data_start = _shard_header(model_dir / shard)
        for name, meta in header.items():
            if name == "__metadata__":
                continue
            start, end = meta["data_offsets"]
            index[name] = TensorLocation(shard, meta["dtype"], tuple(meta["shape"]),
                                         data_start + start, end - start)
    return index


# safetensors dtype -> the torch dtype holding the same bytes (unsigned
# integers as the signed type of their width: the packed U32 weights are
# handed to the kernels as raw words)
_TORCH_DTYPES = {
    "F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
    "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8,
    "U64": torch.int64, "U32": torch.int32, "U16": torch.int16, "U8": torch.uint8,
    "BOOL": torch.bool,
}
# Fields kept at their stored width: the quantization metadata. Norm weights,
# A_log, dt_bias and the conv kernel are bf16 on disk too and feed float32
# arithmetic, so they widen (expert_loader.py:53-59).
_STORED_WIDTH_FIELDS = ("scales", "biases")


def keeps_stored_width(name: str) -> bool:
    return name.rpartition(".")[2] in _STORED_WIDTH_FIELDS


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

    def __init__(self, model_dir: str | Path, index: dict[str, TensorLocation] | None = None):
        self.model_dir = Path(model_dir)
        self.index = index if index is not None else build_index(self.model_dir)
        self._fds: dict[str, int] = {}

    def _fd(self, shard: str) -> int:
        fd = self._fds.get(shard)
        if fd is None:
            fd = self._fds[shard] = os.open(str(self.model_dir / shard), os.O_RDONLY)
        return fd

    def read_tensor(self, name: str) -> torch.Tensor:
        loc = self.index[name]
        raw = os.pread(self._fd(loc.shard), loc.length, loc.offset)
        if len(raw) != loc.length:
            raise ValueError(f"{name}: shard {loc.shard} is truncated")
        return decode_tensor(raw, loc.dtype, loc.shape, stored_width=keeps_stored_width(name))

    def close(self) -> None:
        for fd in self._fds.values():
            os.close(fd)
        self._fds.clear()

    def __enter__(self) -> "CheckpointReader":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def validate_linear_layout(index: dict[str, TensorLocation], name: str, quant: QuantScheme) -> bool:
    """Check a projection's fields and packed shape; return whether it is
    quantized (expert_loader.py:95-141, same conditions)."""

    weight_name, scale_name, bias_name = f"{name}.weight", f"{name}.scales", f"{name}.biases"
    if weight_name not in index:
        raise KeyError(f"no weight tensor for {name}")
    has_scales, has_biases = scale_name in index, bias_name in index
    if not has_scales:
        if has_biases:
            raise ValueError(f"{name} has biases but no scales")
        return False
    if quant.mode == "affine" and not has_biases:
        raise ValueError(f"affine-quantized {name} has no biases")
    weight, scales = index[weight_name], index[scale_name]
    if weight.shape[:-1] != scales.shape[:-1]:
        raise ValueError(f"{name} weight shape {weight.shape} is incompatible with scales shape "
                         f"{scales.shape}")
    if has_biases and index[bias_name].shape != scales.shape:
        raise ValueError(f"{name} biases shape {index[bias_name].shape} does not match scales "
                         f"shape {scales.shape}")
    packed = scales.shape[-1] * quant.group_size * quant.bits // 32
    if weight.shape[-1] != packed:
        raise ValueError(f"{name} weight shape {weight.shape} does not match bits={quant.bits}, "
                         f"group_size={quant.group_size}; expected packed width {packed}")
    return True


def read_linear(reader: CheckpointReader, name: str, quant: QuantScheme) -> LinearWeights:
    """A projection as dense weights (``quant`` None) or its quantized fields
    (expert_loader.py:144-161)."""

    if not validate_linear_layout(reader.index, name, quant):
        return LinearWeights(reader.read_tensor(f"{name}.weight"), None)
    fields = [f for f in ("weight", "scales", "biases") if f"{name}.{f}" in reader.index]
    return LinearWeights({f: reader.read_tensor(f"{name}.{f}") for f in fields}, quant)


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
        proj = {p: _to_device(read_linear(reader, f"{prefix}.{p}", quant.quant_for(f"{prefix}.{p}")),
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
