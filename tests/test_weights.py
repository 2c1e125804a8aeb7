"""The checkpoint reader (mlx-lean-moe_amd/weights.py) against safetensors'
own loader and the reference's on-disk rules: bf16 widened exactly to
float32 except stored-width scales/biases (weights/expert_loader.py:53-85),
the projection layout checks (expert_loader.py:95-141), the shard index
(weights/safetensors_index.py) and the HF config's shapes and quantization
(model/qwen3_5/config.py:70-107,141-193)."""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file as save_numpy
from safetensors.torch import load_file as load_torch
from safetensors.torch import save_file as save_torch

from mlx_lean_moe_amd import weights as W
from mlx_lean_moe_amd.quant import QuantScheme

PREFIX = "language_model.model.layers.0.linear_attn"
HIDDEN = 64


def _quantized(rng, out_dim, in_dim, bits=4, gs=32):
    return {"weight": rng.integers(0, 2 ** 32, (out_dim, in_dim * bits // 32), dtype=np.uint64)
            .astype(np.uint32),
            "scales": torch.tensor(rng.uniform(0.001, 0.01, (out_dim, in_dim // gs))).to(torch.bfloat16),
            "biases": torch.tensor(rng.uniform(-0.05, 0.05, (out_dim, in_dim // gs))).to(torch.bfloat16)}


def write_checkpoint(path, *, Hk=1, Hv=2, d=32, K=4, hidden=HIDDEN, bits=4, gs=32, seed=0,
                     dense_b=False):
    """A two-shard checkpoint of one gated-delta layer in the reference's
    names and dtypes: packed U32 codes in one shard, bf16 everything else in
    the other, with a model.safetensors.index.json."""

    rng = np.random.default_rng(seed)
    conv_dim, value_dim = 2 * Hk * d + Hv * d, Hv * d
    bf = {}
    u32 = {}
    for name, out_dim, in_dim in (("in_proj_qkv", conv_dim, hidden), ("in_proj_z", value_dim, hidden),
                                  ("in_proj_a", Hv, hidden), ("in_proj_b", Hv, hidden),
                                  ("out_proj", hidden, value_dim)):
        if name == "in_proj_b" and dense_b:
            bf[f"{PREFIX}.{name}.weight"] = torch.tensor(rng.standard_normal((out_dim, in_dim)) * 0.05).to(torch.bfloat16)
            continue
        q = _quantized(rng, out_dim, in_dim, bits, gs)
        u32[f"{PREFIX}.{name}.weight"] = q["weight"]
        bf[f"{PREFIX}.{name}.scales"] = q["scales"]
        bf[f"{PREFIX}.{name}.biases"] = q["biases"]
    bf[f"{PREFIX}.conv1d.weight"] = torch.tensor(rng.standard_normal((conv_dim, K, 1)) * 0.2).to(torch.bfloat16)
    bf[f"{PREFIX}.A_log"] = torch.tensor(rng.uniform(0, np.log(16), Hv)).to(torch.bfloat16)
    bf[f"{PREFIX}.dt_bias"] = torch.tensor(rng.uniform(-1, 1, Hv)).to(torch.bfloat16)
    bf[f"{PREFIX}.norm.weight"] = torch.tensor(rng.uniform(0.5, 1.5, d)).to(torch.bfloat16)
    save_torch(bf, str(path / "model-00001-of-00002.safetensors"))
    save_numpy(u32, str(path / "model-00002-of-00002.safetensors"))
    weight_map = {n: "model-00001-of-00002.safetensors" for n in bf}
    weight_map.update({n: "model-00002-of-00002.safetensors" for n in u32})
    (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    config = {"model_type": "qwen3_5_moe",
              "text_config": {"linear_num_key_heads": Hk, "linear_num_value_heads": Hv,
                              "linear_key_head_dim": d, "linear_value_head_dim": d,
                              "linear_conv_kernel_dim": K, "rms_norm_eps": 1e-6,
                              "hidden_size": hidden},
              "quantization": {"bits": bits, "group_size": gs, "mode": "affine"}}
    (path / "config.json").write_text(json.dumps(config))
    return bf, u32, config


def test_index_and_reads_match_the_safetensors_loader(tmp_path):
    bf, u32, _ = write_checkpoint(tmp_path)
    index = W.build_index(tmp_path)
    assert set(index) == set(bf) | set(u32)
    lib = {}
    for shard in ("model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"):
        lib.update(load_torch(str(tmp_path / shard)))
    with W.CheckpointReader(tmp_path) as reader:
        for name, loc in index.items():
            got, want = reader.read_tensor(name), lib[name]
            assert tuple(got.shape) == tuple(want.shape) == loc.shape
            if loc.dtype == "BF16" and W.is_quant_metadata(name):
                assert got.dtype == torch.bfloat16
                assert torch.equal(got.view(torch.int16), want.view(torch.int16))
            elif loc.dtype == "BF16":
                assert got.dtype == torch.float32
                assert torch.equal(got, want.float())  # widening is exact
            else:
                assert loc.dtype == "U32" and got.dtype == torch.int32
                assert np.array_equal(got.numpy().view(np.uint32), u32[name])


def test_bf16_widening_of_special_values():
    bits = [0x3F80, 0xC000, 0x7F80, 0xFF80, 0x0001, 0x8000, 0x7F7F]
    raw = struct.pack("<7H", *bits)
    got = W.decode_tensor(raw, "BF16", (7,))
    want = [struct.unpack("<f", struct.pack("<I", b << 16))[0] for b in bits]
    assert got.dtype == torch.float32
    assert got.view(torch.int32).tolist() == [struct.unpack("<i", struct.pack("<f", v))[0] for v in want]
    kept = W.decode_tensor(raw, "BF16", (7,), stored_width=True)
    assert kept.dtype == torch.bfloat16 and kept.view(torch.int16).tolist() == \
        list(struct.unpack("<7h", raw))
    with pytest.raises(ValueError, match="unsupported safetensors dtype"):
        W.decode_tensor(b"\0\0", "F8_E4M3", (2,))
    assert W.is_quant_metadata("a.b.scales") and W.is_quant_metadata("x.biases")
    assert not W.is_quant_metadata("a.norm.weight") and not W.is_quant_metadata("a.A_log")


def _loc(shape, dtype="U32"):
    return W.TensorSpan("s", dtype, tuple(shape), 0, 0)


def test_linear_layout_rules():
    """The reference loader's conditions (expert_loader.py:95-141): a
    missing weight is a KeyError; biases without scales, an affine scheme
    without biases, biases for a scheme that has none (the float schemes),
    biases not shaped like the scales, weight and scale rows
    that differ, and a packed width other than groups * group_size * bits /
    32 are each a LayoutError (a ValueError); several at once are all
    named."""

    q4 = QuantScheme(4, 64)
    check = W.projection_is_quantized
    ok = {"p.weight": _loc((8, 16)), "p.scales": _loc((8, 2), "BF16"), "p.biases": _loc((8, 2), "BF16")}
    assert check(ok, "p", q4) is True
    assert check({"p.weight": _loc((8, 128), "BF16")}, "p", q4) is False
    with pytest.raises(KeyError, match="p.weight"):
        check({}, "p", q4)
    cases = [
        ({"p.weight": ok["p.weight"], "p.biases": ok["p.biases"]}, q4, "without the scales"),
        ({"p.weight": ok["p.weight"], "p.scales": ok["p.scales"]}, q4, "none are stored"),
        ({**ok, "p.scales": _loc((9, 2), "BF16"), "p.biases": _loc((9, 2), "BF16")}, q4,
         "leading dimensions"),
        ({**ok, "p.biases": _loc((8, 3), "BF16")}, q4, "differ in shape"),
        (ok, QuantScheme(8, 64), "pack into 32 words a row"),
    ]
    for index, scheme, msg in cases:
        with pytest.raises(W.LayoutError, match=msg):
            check(index, "p", scheme)
        assert issubclass(W.LayoutError, ValueError)
    # two problems at once: both reported
    with pytest.raises(W.LayoutError, match="differ in shape.*pack into 32"):
        check({**ok, "p.biases": _loc((8, 3), "BF16")}, "p", QuantScheme(8, 64))
    # modes without biases (mxfp4) need none
    mx = {"p.weight": _loc((8, 8)), "p.scales": _loc((8, 2), "U8")}
    assert check(mx, "p", QuantScheme(4, 32, "mxfp4")) is True
    # ... and biases stored beside them are a layout error
    with pytest.raises(W.LayoutError, match="mxfp4 scheme has no biases"):
        check({**mx, "p.biases": _loc((8, 2), "BF16")}, "p", QuantScheme(4, 32, "mxfp4"))
    nv = {"p.weight": _loc((8, 8)), "p.scales": _loc((8, 4), "U8")}
    assert check(nv, "p", QuantScheme(4, 16, "nvfp4")) is True


def test_hf_config_shapes_and_quantization():
    cfg = {"text_config": {"linear_num_key_heads": 16, "linear_num_value_heads": 32,
                           "linear_key_head_dim": 128, "linear_value_head_dim": 128,
                           "linear_conv_kernel_dim": 4},
           "quantization": {"bits": 4, "group_size": 64,
                            "m.layers.0.linear_attn.in_proj_a.weight": {"bits": 8},
                            "m.layers.0.linear_attn.out_proj": {"group_size": 32, "bits": 8}}}
    dims = W.linear_dims_from_hf(cfg)
    assert (dims.num_key_heads, dims.num_value_heads, dims.conv_dim) == (16, 32, 8192)
    q = W.quant_config_from_hf(cfg)
    assert q.default == QuantScheme(4, 64)
    assert q.quant_for("m.layers.0.linear_attn.in_proj_a") == QuantScheme(8, 64)
    assert q.quant_for("m.layers.0.linear_attn.out_proj") == QuantScheme(8, 32)
    assert q.quant_for("m.layers.0.linear_attn.in_proj_z") == QuantScheme(4, 64)
    assert q.quant_for("x", QuantScheme(8, 128)) == QuantScheme(8, 128)
    assert W.quant_config_from_hf({}).default == QuantScheme(4, 64)
    assert W.quant_config_from_hf({"quantization_config": {"bits": 8, "group_size": 32}}).default == \
        QuantScheme(8, 32)


def test_read_linear_and_truncated_shard(tmp_path):
    write_checkpoint(tmp_path, dense_b=True)
    with W.CheckpointReader(tmp_path) as reader:
        qkv = W.read_projection(reader, f"{PREFIX}.in_proj_qkv", QuantScheme(4, 32))
        assert qkv.quant == QuantScheme(4, 32) and set(qkv.tensors) == {"weight", "scales", "biases"}
        assert qkv.tensors["scales"].dtype == torch.bfloat16
        dense = W.read_projection(reader, f"{PREFIX}.in_proj_b", QuantScheme(4, 32))
        assert dense.quant is None and dense.tensors.dtype == torch.float32
    shard = tmp_path / "model-00002-of-00002.safetensors"
    shard.write_bytes(shard.read_bytes()[:-8])
    with W.CheckpointReader(tmp_path) as reader, pytest.raises(ValueError, match="truncated"):
        for name in reader.index:
            reader.read_tensor(name)
    with pytest.raises(FileNotFoundError):
        W.build_index(tmp_path / "missing")
