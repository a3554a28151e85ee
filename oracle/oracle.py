"""Python face of the oracle (TEST INFRASTRUCTURE ONLY).

Wraps the C restatement in ``oracle/w8a8_oracle.c`` (built into
``oracle/liboracle.so`` by ``oracle/Makefile``) with numpy arrays.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only to check or time the reference's
algorithm; the product library never does.

16-bit floating tensors travel as ``np.uint16`` bit arrays next to a dtype
name: ``"f32"`` (np.float32 values), ``"f16"`` or ``"bf16"`` (np.uint16 bits).
"""
import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
DTYPE_CODE = {"f32": 0, "f16": 1, "bf16": 2}

_lib = None


def build():
    """Compile the C restatement with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        f = _lib
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        f.w8o_quant_rowwise.argtypes = [p, i32, i64, i64, i32, i32, p, p]
        f.w8o_gemm_i32.argtypes = [p, p, i64, i64, i64, p]
        f.w8o_epilogue_kitchen.argtypes = [p, p, p, i64, p, p, i32, i64, i64, i32, i32]
        f.w8o_residual.argtypes = [p, p, p, i64, i32, i64, i64, i32]
        f.w8o_quant_tensorwise.argtypes = [p, i32, i64, p, i32, p, p]
        f.w8o_convrot_rotate.argtypes = [p, i32, i64, i64, i64, p, p]
        f.w8o_convrot_quant.argtypes = [p, i32, i64, i64, i64, i32, p, p, p]
        f.w8o_epilogue_eager.argtypes = [p, p, p, i64, p, p, i32, i64, i64]
        f.w8o_gelu_tanh_tensor.argtypes = [p, p, i32, i64]
        f.w8o_f32_to_bf16_n.argtypes = [p, p, i64]
        f.w8o_f32_to_f16_n.argtypes = [p, p, i64]
        f.w8o_gelu_tanh.argtypes = [ctypes.c_float]
        f.w8o_gelu_tanh.restype = ctypes.c_float
        f.w8o_tanh_cr.argtypes = [ctypes.c_float]
        f.w8o_tanh_cr.restype = ctypes.c_float
        f.w8o_input_act.argtypes = [p, i32, i64, i64, i32, p, ctypes.c_float, p]
        f.w8o_convrot_quant_act.argtypes = [p, i32, i64, i64, i64, i32, i32, p, ctypes.c_float, p, p, p]
        f.w8o_round_to.argtypes = [ctypes.c_float, i32]
        f.w8o_round_to.restype = ctypes.c_float
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _storage(dtype):
    return np.float32 if dtype == "f32" else np.uint16


def to_dtype(values_f32, dtype):
    """Round float32 values to ``dtype`` storage (bits for 16-bit types), RNE."""
    v = np.ascontiguousarray(values_f32, dtype=np.float32)
    if dtype == "f32":
        return v.copy()
    out = np.empty(v.shape, np.uint16)
    fn = lib().w8o_f32_to_bf16_n if dtype == "bf16" else lib().w8o_f32_to_f16_n
    fn(_ptr(v), _ptr(out), v.size)
    return out


def to_f32(storage, dtype):
    """Widen a tensor held in ``dtype`` storage to float32 values (exact)."""
    s = np.ascontiguousarray(storage)
    if dtype == "f32":
        return s.astype(np.float32)
    if dtype == "bf16":
        return (s.astype(np.uint32) << 16).view(np.float32)
    return s.view(np.float16).astype(np.float32)


def quant_rowwise(x, dtype, scale_mode=0, act=0):
    """Per-token absmax quantization of ``x`` [M, K] -> (q int8 [M, K], s fp32 [M]).

    scale_mode 0: IEEE amax/127 (the reference's CPU/eager path);
    scale_mode 1: amax * (1/127f) (the reference's CUDA kernel).
    act 1 applies gelu_tanh to x (rounded to its dtype) before quantizing.
    """
    x = np.ascontiguousarray(x, dtype=_storage(dtype))
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().w8o_quant_rowwise(_ptr(x), DTYPE_CODE[dtype], M, K, scale_mode, act, _ptr(q), _ptr(s))
    return q, s


def quant_tensorwise(x, dtype, scale=None, scale_mode=0):
    """Tensorwise quantization of ``x`` (any shape) -> (q int8, s fp32 scalar);
    ``scale`` (a float) replaces the computed scale."""
    x = np.ascontiguousarray(x, dtype=_storage(dtype))
    q = np.empty(x.shape, np.int8)
    s = np.empty((1,), np.float32)
    given = None if scale is None else np.array([scale], np.float32)
    lib().w8o_quant_tensorwise(_ptr(x), DTYPE_CODE[dtype], x.size, None if given is None else _ptr(given),
                               scale_mode, _ptr(q), _ptr(s))
    return q, s[0]


def convrot_fused_route(k, group):
    """The reference's fused-rotation predicate (cuda_linear.rs:404-417):
    group 256, K a multiple of 256 in [256, 16384]."""
    return group == 256 and k % 256 == 0 and 256 <= k <= 16384


def convrot_rotate(x, dtype, group):
    """dtype(x rotated per `group`-wide slice) -> same shape and storage."""
    x = np.ascontiguousarray(x, dtype=_storage(dtype))
    M, K = x.shape
    y = np.empty_like(x)
    work = np.empty((group,), np.float32)
    lib().w8o_convrot_rotate(_ptr(x), DTYPE_CODE[dtype], M, K, group, _ptr(y), _ptr(work))
    return y


def convrot_quant(x, dtype, group, scale_mode=0):
    """ConvRot activation quantization of ``x`` [M, K] -> (q, s), by the route
    the reference takes: the fused rotation (fp32 rotated values) where
    ``convrot_fused_route`` holds, else rotate (rounded to the dtype) then
    the plain per-token quantizer."""
    x = np.ascontiguousarray(x, dtype=_storage(dtype))
    M, K = x.shape
    if not convrot_fused_route(K, group):
        return quant_rowwise(convrot_rotate(x, dtype, group), dtype, scale_mode=scale_mode)
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    work = np.empty((K,), np.float32)
    lib().w8o_convrot_quant(_ptr(x), DTYPE_CODE[dtype], M, K, group, scale_mode, _ptr(q), _ptr(s),
                            _ptr(work))
    return q, s


ACT_CODE = {None: 0, "gelu_tanh": 1, "swiglu": 2, "rms_norm": 3, "situ": 4}


def input_act(x, dtype, act, weight=None, eps=0.0):
    """The eager input activation (int8_linear.rs:37-97) of [M, K] (or [M, 2K]
    for swiglu / situ) storage -> [M, K] storage of the dtype."""
    x = np.ascontiguousarray(x, dtype=_storage(dtype))
    code = ACT_CODE[act]
    M = x.shape[0]
    K = x.shape[1] // 2 if code in (2, 4) else x.shape[1]
    y = np.empty((M, K), _storage(dtype))
    wt = None if weight is None else np.ascontiguousarray(weight, dtype=_storage(dtype))
    lib().w8o_input_act(_ptr(x), DTYPE_CODE[dtype], M, K, code, _ptr(wt), float(eps), _ptr(y))
    return y


def convrot_quant_act(x, dtype, group, act, weight=None, eps=0.0, scale_mode=0):
    """ConvRot quantization with an input activation, by the reference's route:
    on the fused route the activation is fused in fp32 (int8_linear.cu:1175-1262),
    elsewhere it is applied eagerly (rounded to the dtype) before the rotation."""
    x = np.ascontiguousarray(x, dtype=_storage(dtype))
    code = ACT_CODE[act]
    M = x.shape[0]
    K = x.shape[1] // 2 if code in (2, 4) else x.shape[1]
    if code == 0 or not convrot_fused_route(K, group):
        xa = x if code == 0 else input_act(x, dtype, act, weight, eps)
        return convrot_quant(xa, dtype, group, scale_mode=scale_mode)
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    work = np.empty((K,), np.float32)
    wt = None if weight is None else np.ascontiguousarray(weight, dtype=_storage(dtype))
    lib().w8o_convrot_quant_act(_ptr(x), DTYPE_CODE[dtype], M, K, group, scale_mode, code, _ptr(wt), float(eps),
                                _ptr(q), _ptr(s), _ptr(work))
    return q, s


def convrot_quant_weight(w, dtype, group, scale_mode=0):
    """ConvRot weight quantization [N, K] by the reference's weight path
    (inference/src/convrot.rs:345-372): group 256 with K % 256 == 0 takes the
    fused numerics at any K (its Rowwise64 and Staged paths), other groups
    rotate then quantize rowwise (EagerRotation)."""
    w = np.ascontiguousarray(w, dtype=_storage(dtype))
    N, K = w.shape
    if not (group == 256 and K % 256 == 0):
        return quant_rowwise(convrot_rotate(w, dtype, group), dtype, scale_mode=scale_mode)
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    work = np.empty((K,), np.float32)
    lib().w8o_convrot_quant(_ptr(w), DTYPE_CODE[dtype], N, K, group, scale_mode, _ptr(q), _ptr(s), _ptr(work))
    return q, s


def gemm_i32(a, b):
    """Exact int32 C = A @ B.T for int8 A [M, K], B [N, K]."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    M, K = a.shape
    N, K2 = b.shape
    assert K == K2
    c = np.empty((M, N), np.int32)
    lib().w8o_gemm_i32(_ptr(a), _ptr(b), M, N, K, _ptr(c))
    return c


def epilogue_kitchen(acc, xs, ws, bias, out_dtype, contract=1, act=0):
    """GPU-route dequant: O((float(acc)*xs)*ws + bias) with one rounding.

    ``bias`` is in ``out_dtype`` storage or None; ``act`` 1 appends gelu_tanh.
    """
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    M, N = acc.shape
    xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1)
    ws = np.ascontiguousarray(ws, dtype=np.float32).reshape(-1)
    assert xs.size == M and ws.size in (1, N)
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=_storage(out_dtype)).reshape(-1)
        assert bias.size == N
    out = np.empty((M, N), _storage(out_dtype))
    lib().w8o_epilogue_kitchen(_ptr(acc), _ptr(xs), _ptr(ws), ws.size, _ptr(bias), _ptr(out),
                               DTYPE_CODE[out_dtype], M, N, contract, act)
    return out


def epilogue_eager(acc, xs, ws, bias_f32, out_dtype):
    """CPU-eager dequant: O(float(acc)*(xs*ws)) then + O(bias) in the output dtype."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    M, N = acc.shape
    xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1)
    ws = np.ascontiguousarray(ws, dtype=np.float32).reshape(-1)
    if bias_f32 is not None:
        bias_f32 = np.ascontiguousarray(bias_f32, dtype=np.float32).reshape(-1)
    out = np.empty((M, N), _storage(out_dtype))
    lib().w8o_epilogue_eager(_ptr(acc), _ptr(xs), _ptr(ws), ws.size, _ptr(bias_f32), _ptr(out),
                             DTYPE_CODE[out_dtype], M, N)
    return out


def gelu_tanh(x, dtype):
    """gelu_tanh of a tensor in ``dtype`` storage, rounded back to ``dtype``."""
    x = np.ascontiguousarray(x, dtype=_storage(dtype))
    y = np.empty_like(x)
    lib().w8o_gelu_tanh_tensor(_ptr(x), _ptr(y), DTYPE_CODE[dtype], x.size)
    return y


def residual(out, resid, rscale, dtype, contract=1):
    """out' = O(resid + out * rscale) in the output dtype (w8o_residual); all
    three in storage convention of ``dtype``; rscale of 1 or N entries."""
    out = np.ascontiguousarray(out).copy()
    m, n = out.shape
    resid = np.ascontiguousarray(resid, dtype=out.dtype).reshape(m, n)
    rscale = np.ascontiguousarray(rscale, dtype=out.dtype).reshape(-1)
    lib().w8o_residual(_ptr(out), _ptr(resid), _ptr(rscale), rscale.size, DTYPE_CODE[dtype], m, n, contract)
    return out


def linear_kitchen(x, x_dtype, w, ws, bias, out_dtype, scale_mode=0, input_act=0,
                   epilogue_act=0, contract=1, convrot_group=0):
    """Composed GPU-route linear: quantize -> int32 GEMM -> single-rounding epilogue.

    Returns (out, q, xs, acc) so callers can check every intermediate.
    """
    if convrot_group:
        q, xs = convrot_quant(x, x_dtype, convrot_group, scale_mode=scale_mode)
    else:
        q, xs = quant_rowwise(x, x_dtype, scale_mode=scale_mode, act=input_act)
    acc = gemm_i32(q, w)
    out = epilogue_kitchen(acc, xs, ws, bias, out_dtype, contract=contract, act=epilogue_act)
    return out, q, xs, acc


# ---------------------------------------------------------------- DiT block glue
# Bit-level restatements (numpy) of the glue's elementwise steps.  Each product
# of two 16-bit values is exact in fp32, so these are single roundings.

def modulate(x, s, dtype):
    """backend_bindings.rs:391-394 on storage arrays: T(x * T(1 + s)), s of
    x's last-dim width broadcast over the rows."""
    xf = to_f32(x, dtype)
    m = to_f32(to_dtype(np.float32(1.0) + to_f32(s, dtype), dtype), dtype)
    return to_dtype((xf * m).astype(np.float32), dtype)


def gated_residual(x, y, g, dtype):
    """numeric.rs:110-125 (ATen addcmul_) on storage arrays: T(fp32(x + y * g))."""
    v = (to_f32(x, dtype) + to_f32(y, dtype) * to_f32(g, dtype)).astype(np.float32)
    return to_dtype(v, dtype)


def adaln_single(x, scale, shift, eps, dtype, rms=False):
    """The single-rounding adaLN (the rounding structure of Kitchen's CUDA
    kernel, adaln.cu in the reference's native-source archive):
    T(fp32(y * fp32(1 + scale) + shift)) with y the fp32 normalised value and
    the multiply-add fused; the norm in float64 here, so this matches a fp32
    implementation to within one ulp of T."""
    xf = to_f32(x, dtype).astype(np.float64)
    if rms:
        y = xf / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
    else:
        mu = xf.mean(axis=-1, keepdims=True)
        var = ((xf - mu) ** 2).mean(axis=-1, keepdims=True)
        y = (xf - mu) / np.sqrt(var + eps)
    y = y.astype(np.float32).astype(np.float64)
    m = (np.float32(1.0) + to_f32(scale, dtype)).astype(np.float32).astype(np.float64)
    z = (y * m + to_f32(shift, dtype).astype(np.float64)).astype(np.float32)   # one rounding: fma
    return to_dtype(z, dtype)


def adaln(x, scale, shift, eps, dtype, rms=False):
    """backend_eager.rs:186-199 in float64 up to the roundings of the op order:
    y = T(norm(x)), T(y * T(1 + scale)), T(. + shift); x [n, d], scale and shift
    broadcast against it.  The fp32 reductions of the reference round the mean
    and rstd differently, so this matches it to within one ulp of T."""
    xf = to_f32(x, dtype).astype(np.float64)
    if rms:
        y = xf / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
    else:
        mu = xf.mean(axis=-1, keepdims=True)
        var = ((xf - mu) ** 2).mean(axis=-1, keepdims=True)
        y = (xf - mu) / np.sqrt(var + eps)
    y = to_f32(to_dtype(y.astype(np.float32), dtype), dtype)
    m = to_f32(to_dtype(np.float32(1.0) + to_f32(scale, dtype), dtype), dtype)
    z = to_f32(to_dtype((y * m).astype(np.float32), dtype), dtype)
    return to_dtype((z + to_f32(shift, dtype)).astype(np.float32), dtype)
