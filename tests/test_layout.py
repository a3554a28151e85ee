"""TensorWiseINT8 weight format and checkpoint loader: host logic on the CPU
(metadata parsing, errors, save/load round trip; no GPU compute)."""
import json

import pytest
import torch

from imagine_amd import layout as L


def _state(prefix="blk.linear.", conf=None, scale=True, n=4, k=8):
    st = {f"{prefix}weight": torch.arange(n * k, dtype=torch.int8).reshape(n, k)}
    if scale:
        st[f"{prefix}weight_scale"] = torch.full((n, 1), 0.5)
    if conf is not None:
        st[f"{prefix}comfy_quant"] = torch.tensor(list(json.dumps(conf).encode()), dtype=torch.uint8)
    return st


def test_int8_tensorwise_layer_loads_with_its_convrot_fields():
    st = _state(conf={"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 64})
    m = L.load_quantized_module(st, "blk.linear.", "cpu", torch.bfloat16)
    assert m.quant_format == "int8_tensorwise" and not m.full_precision
    w = m.weight
    assert isinstance(w, L.TensorWiseINT8Weight)
    assert w.convrot and w.convrot_groupsize == 64 and w.orig_dtype == torch.bfloat16
    assert w.qdata.dtype == torch.int8 and w.orig_shape == (4, 8)
    assert m.consumed == ("blk.linear.weight", "blk.linear.weight_scale")
    assert st == {}  # every key of the layer was consumed


def test_options_nested_in_params_and_python_truthiness():
    """quantized.rs:179-181: options are read at the top level, then in params;
    int() accepts numeric strings; convrot 0 / "" is false (group then 256)."""
    m = L.load_quantized_module(_state(conf={"format": "int8_tensorwise",
                                             "params": {"convrot": 1, "convrot_groupsize": " 16 "}}),
                                "blk.linear.", "cpu", torch.float16)
    assert m.weight.convrot and m.weight.convrot_groupsize == 16
    m = L.load_quantized_module(_state(conf={"format": "int8_tensorwise", "convrot": "", "convrot_groupsize": 64}),
                                "blk.linear.", "cpu", torch.float16)
    assert not m.weight.convrot and m.weight.convrot_groupsize == 256
    with pytest.raises(ValueError, match=r"invalid literal for int\(\) with base 10: 'x'"):
        L.load_quantized_module(_state(conf={"format": "int8_tensorwise", "convrot": True,
                                             "convrot_groupsize": "x"}), "blk.linear.", "cpu", torch.float16)


def test_loader_errors_follow_the_reference_messages():
    with pytest.raises(ValueError, match="^Unknown quantization format for layer blk.linear$"):
        L.load_quantized_module(_state(conf={"convrot": True}), "blk.linear.", "cpu", torch.bfloat16)
    with pytest.raises(ValueError, match="^Missing INT8 weight scale for layer blk.linear$"):
        L.load_quantized_module(_state(conf={"format": "int8_tensorwise"}, scale=False), "blk.linear.", "cpu",
                                torch.bfloat16)
    with pytest.raises(NotImplementedError):
        L.load_quantized_module(_state(conf={"format": "nvfp4"}), "blk.linear.", "cpu", torch.bfloat16)


def test_full_precision_flags():
    m = L.load_quantized_module(_state(conf={"format": "int8_tensorwise", "full_precision_matrix_mult": True}),
                                "blk.linear.", "cpu", torch.bfloat16)
    assert m.full_precision and m.full_precision_config
    m = L.load_quantized_module(_state(conf={"format": "int8_tensorwise"}), "blk.linear.", "cpu", torch.bfloat16,
                                disabled_formats=("int8_tensorwise",))
    assert m.full_precision and not m.full_precision_config


def test_plain_weight_and_missing_weight():
    st = {"a.weight": torch.ones(2, 3, dtype=torch.float32)}
    m = L.load_quantized_module(st, "a.", "cpu", torch.bfloat16)
    assert m.quant_format is None and m.weight.dtype == torch.bfloat16 and m.consumed == ("a.weight",)
    assert L.load_quantized_module({}, "b.", "cpu", torch.bfloat16).weight is None


def test_metadata_is_written_with_python_json_spacing():
    w = L.TensorWiseINT8Weight(torch.zeros(2, 256, dtype=torch.int8), torch.ones(2, 1), torch.bfloat16, (2, 256),
                               convrot=True, convrot_groupsize=256)
    assert bytes(L.comfy_quant_bytes(w).tolist()) == \
        b'{"format": "int8_tensorwise", "convrot": true, "convrot_groupsize": 256}'
    w.convrot = False
    assert bytes(L.comfy_quant_bytes(w).tolist()) == b'{"format": "int8_tensorwise"}'


def test_save_load_round_trip(tmp_path):
    q = torch.randint(-128, 128, (6, 512), dtype=torch.int8)
    s = torch.rand(6, 1)
    layers = {"blocks.0.attn.qkv.": L.TensorWiseINT8Weight(q, s, torch.bfloat16, (6, 512), convrot=True),
              "blocks.0.attn.out.": L.TensorWiseINT8Weight(q[:3], torch.tensor(0.25), torch.bfloat16, (3, 512)),
              "final.": torch.randn(4, 4)}
    path = tmp_path / "int8.safetensors"
    L.save_checkpoint(path, layers)
    got = L.load_checkpoint(path, "cpu", torch.bfloat16)
    qkv = got["blocks.0.attn.qkv."].weight
    assert torch.equal(qkv.qdata, q) and torch.equal(qkv.scale, s) and qkv.convrot and qkv.convrot_groupsize == 256
    out = got["blocks.0.attn.out."].weight
    assert torch.equal(out.qdata, q[:3]) and out.scale.item() == 0.25 and not out.convrot
    assert got["final."].quant_format is None and got["final."].weight.dtype == torch.bfloat16


def test_from_float_argument_rules():
    """layout_complete.rs:124-136 (checked before anything is quantized)."""
    w = torch.zeros(2, 256)
    with pytest.raises(ValueError, match="convrot is only supported when is_weight is True"):
        L.from_float(w, is_weight=False, convrot=True)
    with pytest.raises(ValueError, match="convrot is only supported when per_channel is True"):
        L.from_float(w, per_channel=False, convrot=True)
