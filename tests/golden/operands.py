"""Rebuild the reference fixtures' deterministic operands with numpy.

The reference's capture scripts build every operand from ``arange`` (no RNG),
so each fixture case stores only its parameters and expected bytes.  This
module restates those constructions in float32/int64 numpy arithmetic, which
is what torch does for a float32 tensor combined with Python scalars:

* ``inference/tools/reference_cuda_int8_m1.py:6-25``  (x, weight, scale, bias,
  residual, residual_scale by mode)
* ``inference/tools/reference_cuda_int8_gemm.py:7-24`` (fused/unaligned residual
  and bias modes)
* ``inference/tools/reference_cuda_int8_activation.py:7-16`` (activation cases)
* ``inference/tools/reference_primitives.py:357-365,388-391`` (quantizer cases)
* ``inference/tools/reference_int8_linear.py:18-30,75-92`` (int8_mm and eager
  int8_linear cases)
"""
import numpy as np

F32 = np.float32
DTYPES = {"torch.float32": "f32", "torch.float16": "f16", "torch.bfloat16": "bf16"}


def dtype_name(torch_name):
    return DTYPES[torch_name]


def _arange_f32(count):
    return np.arange(count, dtype=F32)


def base_x(shape):
    """((arange % 31) * 0.0137 - 0.1) in float32, reshaped; before the dtype cast."""
    count = int(np.prod(shape))
    a = _arange_f32(count)
    return ((a % F32(31)) * F32(0.0137) - F32(0.1)).reshape(shape)


def base_weight(n, k):
    return ((np.arange(n * k, dtype=np.int64) % 255) - 127).astype(np.int8).reshape(n, k)


def m1_operands(case):
    """Operands of reference_cuda_int8_m1.operands (values only; layout modes
    such as ``noncontiguous`` and ``unaligned_*`` change addresses, not values).

    Returns dict with x (f32 values, pre-cast), weight int8 [n,k], scale f32
    values (flat), bias f32 values or None, residual / residual_scale or None.
    """
    shape = case["shape"]
    k = shape[-1]
    n = case["n"]
    mode = case["mode"]
    x = base_x(shape)
    w = base_weight(n, k)
    size = n + 1 if mode == "bad_scale" else (n if mode in ("row_scale", "cpu_scale_bias", "noncontiguous") else 1)
    scale = np.full((size,), 0.03125, dtype=np.float64 if mode == "cpu_scale_bias" else F32)
    bias = None
    if mode in ("bias", "cpu_scale_bias"):
        if mode == "cpu_scale_bias":
            bias = np.arange(n, dtype=np.float64) * 0.015625
        else:
            bias = _arange_f32(n) * F32(0.015625)
    residual = residual_scale = None
    if mode in ("residual", "missing_residual_scale"):
        residual = np.full((*shape[:-1], n), 0.375, dtype=np.float64)
    if mode == "residual":
        residual_scale = np.arange(n, dtype=np.float64) * 0.0078125 + 0.5
    return dict(x=x, weight=w, scale=scale, bias=bias, residual=residual, residual_scale=residual_scale)


def gemm_operands(case):
    """reference_cuda_int8_gemm.operands: the m1 operands plus residual modes."""
    ops = m1_operands(case)
    mode = case["mode"]
    n = case["n"]
    if mode in ("fused_residual", "unaligned_residual", "unaligned_residual_scale"):
        ops["residual"] = np.full((*case["shape"][:-1], n), 0.375, dtype=F32)
        ops["residual_scale"] = _arange_f32(n) * F32(0.0078125) + F32(0.5)
        ops["residual_in_out_dtype"] = True
    if mode == "unaligned_bias":
        ops["bias"] = _arange_f32(n) * F32(0.015625)
    return ops


def activation_operands(case):
    """reference_cuda_int8_activation.operands."""
    shape = case["shape"]
    k = case["weight_k"]
    n = case["n"]
    x = base_x(shape)
    w = base_weight(n, k)
    scale = np.full((1,), 0.03125, dtype=F32)
    full = case["mode"] == "full"
    bias = _arange_f32(n) * F32(0.015625) if full else None
    residual = np.full((*shape[:-1], n), 0.375, dtype=F32) if full else None
    residual_scale = np.full((n,), 0.5, dtype=F32) if full else None
    return dict(x=x, weight=w, scale=scale, bias=bias, residual=residual,
                residual_scale=residual_scale, residual_in_out_dtype=True)


def quantizer_x_primitives():
    """reference_primitives.py:357-360: (arange(64)*0.125-4).reshape(4,16), row 0 zeroed."""
    x = (_arange_f32(64) * F32(0.125) - F32(4)).reshape(4, 16)
    x[0] = 0
    return x


def quantizer_x_native():
    """reference_primitives.py:388-389: (arange(256)*0.03125-4).reshape(4,64)."""
    return (_arange_f32(256) * F32(0.03125) - F32(4)).reshape(4, 64)


def int8_mm_operands(m, k, n):
    """reference_int8_linear.py:19-21."""
    a = ((np.arange(m * k, dtype=np.int64) % 31) - 15).astype(np.int8).reshape(m, k)
    b = ((np.arange(k * n, dtype=np.int64) % 29) - 14).astype(np.int8).reshape(k, n)
    return a, b


def eager_linear_operands(case):
    """reference_int8_linear._linear_case (:75-92) for modes without ConvRot."""
    shape = case["shape"]
    mode = case["mode"]
    width = shape[-1]
    input_shape = list(shape)
    if mode == "swiglu":
        input_shape[-1] *= 2
    count = int(np.prod(input_shape))
    x = (_arange_f32(count) * F32(0.03125) - F32(0.5)).reshape(input_shape)
    w = base_weight(17, width)
    nscale = 18 if mode == "bad_scale" else (17 if mode in ("row_scale", "convrot") else 1)
    scales = np.full((nscale,), 0.03125, dtype=np.float64)
    bias = np.arange(17, dtype=np.float64) * 0.125 if mode == "row_scale" else None
    return dict(x=x, weight=w, scale=scales, bias=bias)
