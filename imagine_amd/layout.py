"""TensorWiseINT8 weights: the reference's INT8 weight format, its from_float
quantizers and its checkpoint loader, over the HIP library.

Format (``TensorWiseINT8Layout``, inference/src/layouts.rs:39-70): an int8
payload ``[N, K]`` (one row per output channel), an fp32 ``scale`` (``[N, 1]``
per channel, or a scalar), and the fields ``is_weight``, ``convrot``,
``convrot_groupsize`` and ``transposed`` (always false here).

Checkpoint (inference/src/checkpoint/quantized.rs:112-202): a linear layer
``<prefix>`` stores ``<prefix>weight`` (int8 ``[N, K]``), ``<prefix>weight_scale``
(fp32) and ``<prefix>comfy_quant``: the bytes of a JSON object such as
``{"format": "int8_tensorwise", "convrot": true, "convrot_groupsize": 256}``
(written by Python's ``json.dumps``, components/offload.rs:414-428) in a uint8
tensor.  Files are safetensors.
"""
import json
from dataclasses import dataclass

import torch

from . import ops

INT8_FORMAT = "int8_tensorwise"


@dataclass
class TensorWiseINT8Weight:
    """One quantized linear weight (TensorWiseINT8Layout)."""
    qdata: torch.Tensor
    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple
    is_weight: bool = True
    convrot: bool = False
    convrot_groupsize: int = 256
    transposed: bool = False

    def linear(self, x, bias=None, out_dtype=None, residual=None, residual_scale=None, **kw):
        """``int8_linear`` with this weight (its ConvRot fields included)."""
        return ops.int8_linear(x, self.qdata, self.scale, bias, out_dtype, convrot=self.convrot,
                               convrot_groupsize=self.convrot_groupsize, residual=residual,
                               residual_scale=residual_scale, **kw)


def from_float(w, is_weight=True, per_channel=False, convrot=False, convrot_groupsize=256, scale=None,
               scale_form="ieee"):
    """Quantize a float weight into a TensorWiseINT8Weight, choosing the
    quantizer as the reference's layout does (inference/src/layout_complete.rs:119-160):
    ConvRot weights by quantize_int8_convrot_weight, per-channel weights (or
    non-weights) rowwise, other weights tensorwise (with ``scale`` if given)."""
    if convrot and not is_weight:
        raise ValueError("convrot is only supported when is_weight is True")
    if convrot and not per_channel:
        raise ValueError("convrot is only supported when per_channel is True")
    if convrot:
        q, s = ops.quantize_convrot_weight(w, convrot_groupsize, scale_form=scale_form)
    elif not is_weight or per_channel:
        q, s = ops.quantize_rowwise(w, scale_form=scale_form)
        q = q.reshape(w.shape)
    else:
        q, s = ops.quantize_tensorwise(w, scale=scale, scale_form=scale_form)
    return TensorWiseINT8Weight(q, s, w.dtype, tuple(w.shape), is_weight, bool(convrot), int(convrot_groupsize))


# ---------------------------------------------------------------- checkpoint


@dataclass
class QuantizedModule:
    """What loading one linear's parameters yields (quantized.rs:42-49)."""
    weight: object = None
    quant_format: str = None
    full_precision: bool = False
    full_precision_config: bool = False
    consumed: tuple = ()


def _truth(v):
    """Python truthiness of a JSON value (quantized.rs:81-90)."""
    return bool(v)


def _int(v, default):
    """Python int() of a JSON value (quantized.rs:91-106)."""
    if v is None:
        return default
    if isinstance(v, bool):
        return int(v)
    if isinstance(v, (int, float)):
        return int(v)
    if isinstance(v, str):
        try:
            return int(v.strip())
        except ValueError:
            raise ValueError(f"invalid literal for int() with base 10: '{v}'") from None
    raise NotImplementedError("Python int conversion of quantization metadata")


def load_quantized_module(state, prefix, device, compute_dtype, original_shape=None, full_precision=False,
                          disabled_formats=()):
    """Pop ``<prefix>weight`` (and its scale and metadata) from ``state`` and
    build the layer's weight, as the reference's load_quantized_module
    (quantized.rs:107-202) does for unquantized and int8_tensorwise layers.
    Other quantization formats raise NotImplementedError."""
    out = QuantizedModule(full_precision=full_precision)
    consumed = []
    weight = state.pop(f"{prefix}weight", None)
    if weight is None:
        return out
    consumed.append(f"{prefix}weight")
    conf = state.pop(f"{prefix}comfy_quant", None)
    if conf is None:
        out.weight = weight.to(device=device, dtype=compute_dtype).detach()
        out.consumed = tuple(consumed)
        return out
    if conf.device.type != "cpu":
        raise TypeError("can't convert cuda:0 device type tensor to numpy. Use Tensor.cpu() to copy the tensor "
                        "to host memory first.")
    meta = json.loads(bytes(conf.contiguous().reshape(-1).view(torch.uint8).tolist()))
    name = prefix.rstrip(".")
    fmt = meta.get("format")
    if fmt is None:
        raise ValueError(f"Unknown quantization format for layer {name}")
    if not isinstance(fmt, str):
        raise NotImplementedError("Non-string quantization format")
    out.quant_format = fmt
    out.full_precision_config = _truth(meta.get("full_precision_matrix_mult"))
    if not out.full_precision:
        out.full_precision = out.full_precision_config
    if fmt in disabled_formats:
        out.full_precision = True
    params = meta.get("params") if isinstance(meta.get("params"), dict) else None

    def option(key):
        if key in meta:
            return meta[key]
        return params.get(key) if params else None

    if fmt != INT8_FORMAT:
        raise NotImplementedError(f"quantization format {fmt!r} is not part of this build")
    scale = state.pop(f"{prefix}weight_scale", None)
    if scale is None:
        raise ValueError(f"Missing INT8 weight scale for layer {name}")
    consumed.append(f"{prefix}weight_scale")
    rotated = _truth(option("convrot"))
    group = _int(option("convrot_groupsize"), 256) if rotated else 256
    shape = tuple(original_shape) if original_shape is not None else tuple(weight.shape)
    out.weight = TensorWiseINT8Weight(weight.to(device=device, dtype=torch.int8), scale.to(device=device),
                                      compute_dtype, shape, True, rotated, group)
    out.consumed = tuple(consumed)
    return out


def comfy_quant_bytes(layer):
    """The metadata tensor a TensorWiseINT8Weight is saved with
    (components/offload.rs:414-428, Python json.dumps spacing)."""
    conf = {"format": INT8_FORMAT}
    if layer.convrot:
        conf["convrot"] = True
        conf["convrot_groupsize"] = int(layer.convrot_groupsize)
    return torch.tensor(list(json.dumps(conf).encode()), dtype=torch.uint8)


def save_checkpoint(path, layers):
    """Write ``{prefix: TensorWiseINT8Weight | tensor}`` as a safetensors file
    in the checkpoint layout above (``prefix`` ends with '.' or is empty)."""
    from safetensors.torch import save_file
    tensors = {}
    for prefix, layer in layers.items():
        if isinstance(layer, TensorWiseINT8Weight):
            # copies: safetensors refuses tensors that share storage
            tensors[f"{prefix}weight"] = layer.qdata.detach().to("cpu", copy=True).contiguous()
            tensors[f"{prefix}weight_scale"] = layer.scale.detach().to("cpu", torch.float32, copy=True).contiguous()
            tensors[f"{prefix}comfy_quant"] = comfy_quant_bytes(layer)
        else:
            tensors[f"{prefix}weight"] = layer.detach().to("cpu", copy=True).contiguous()
    save_file(tensors, str(path))


def load_checkpoint(path, device, compute_dtype=torch.bfloat16, disabled_formats=()):
    """Load every linear weight of a safetensors checkpoint: ``{prefix:
    QuantizedModule}`` for each ``<prefix>weight`` key."""
    from safetensors.torch import load_file
    state = load_file(str(path), device="cpu")
    prefixes = [k[: -len("weight")] for k in list(state) if k.endswith("weight")]
    return {p: load_quantized_module(state, p, device, compute_dtype, disabled_formats=disabled_formats)
            for p in prefixes}
