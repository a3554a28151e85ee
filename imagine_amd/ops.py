"""Torch-facing W8A8 operators over the C ABI (device memory and streams only).

``int8_linear`` mirrors the reference crate's operator: its kwargs, route
selection, argument conversions and error classes/messages follow
``inference/src/cuda_linear.rs:311-317,419-824`` (with the signature at
``inference/src/backend_signatures.rs:445-460``).  The arithmetic runs in the
HIP kernels of libw8a8_hip.so; torch only allocates tensors, converts dtypes
of small operands (scales, bias) and supplies the current stream.

The residual kwargs are fused into the GEMM / GEMV epilogue (or applied by
the HIP residual kernel).  ``convrot`` rotates the activations by the regular
Hadamard matrix of ``convrot_groupsize`` before quantizing them (fused into
the quantizer on the crate's fused route).  ``input_act`` is the crate's
input activation (gelu_tanh, swiglu, situ, rms_norm with ``input_act_weight``
and ``input_act_eps``), fused into the quantizer with the crate's eager
numerics, or in fp32 into the ConvRot quantizer on its fused route.
"""
import torch

from . import _lib

_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _dtype_code(dtype, what):
    if dtype not in _CODE:
        raise RuntimeError(f"{what} requires original floating dtype contract")
    return _CODE[dtype]


def _require_cuda(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("W8A8 HIP path requires device tensors on a ROCm GPU")


def _as_2d(x):
    if x.dim() == 2 and x.is_contiguous():
        return x
    if x.dim() == 0:
        raise IndexError("tuple index out of range")
    return x.reshape(-1, x.shape[-1]).contiguous()


def _weight_scale(ws, device):
    """cuda_linear.rs:530-540: fp32, contiguous, flattened, on the device."""
    if ws.device == device and ws.dtype == torch.float32 and ws.is_contiguous():
        return ws.reshape(-1)
    return ws.to(device=device, dtype=torch.float32).reshape(-1).contiguous()


def _bias(bias, device, dtype):
    """cuda_linear.rs:26-51,541-551: output dtype, contiguous, 16-byte aligned."""
    if bias is None:
        return None
    b = bias
    if b.device != device or b.dtype != dtype or not b.is_contiguous():
        b = b.to(device=device, dtype=dtype).contiguous()
    if b.data_ptr() % 16 != 0:
        b = b.clone()
    return b


# ---------------------------------------------------------------- primitives


def quantize_rowwise(x, scale_form="ieee", input_act=None):
    """Per-token quantization of a [M, K] device tensor -> (q int8 [M, K], s fp32 [M, 1]).

    The reference's ``quantize_int8_rowwise`` (int8_linear.cu:1322-1371).
    ``scale_form`` "ieee" (amax / 127, the reference CPU route) or "recip"
    (amax * (1/127), the reference CUDA kernel)."""
    _require_cuda(x)
    x = _as_2d(x)
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    flags = (_lib.SCALE_RECIP if scale_form == "recip" else 0) | (
        _lib.ACT_GELU_TANH if input_act == "gelu_tanh" else 0)
    _lib.check(_lib.load().w8a8_quantize_rowwise(
        _ptr(x), _dtype_code(x.dtype, "INT8 quantization"), _ptr(q), _ptr(s), M, K, flags,
        _stream(x.device)))
    return q, s


def _act_args(x, input_act, weight, eps):
    if input_act not in _lib.ACT_CODES:
        raise ValueError(f"Unsupported input_act {input_act!r}")
    act = _lib.ACT_CODES[input_act]
    w = None
    if act == 3:
        if weight is None:
            raise ValueError("input_act 'rms_norm' requires act_weight")
        w = weight.to(device=x.device, dtype=x.dtype).reshape(-1).contiguous()
    eps = torch.finfo(torch.float32).eps if eps is None else float(eps)
    return act, w, eps


def input_act(x, input_act, weight=None, eps=None):
    """The crate's eager input activation (int8_linear.rs:37-97) of a [M, K]
    (swiglu / situ: [M, 2K]) device tensor -> [M, K] in its dtype."""
    _require_cuda(x)
    x = _as_2d(x)
    act, w, eps = _act_args(x, input_act, weight, eps)
    M, width = x.shape
    K = width // 2 if act in (2, 4) else width
    y = torch.empty((M, K), dtype=x.dtype, device=x.device)
    _lib.check(_lib.load().w8a8_input_act(_ptr(x), _dtype_code(x.dtype, "input activation"), act, _ptr(w), eps,
                                          _ptr(y), M, K, _stream(x.device)))
    return y


def quantize_rowwise_act(x, input_act, weight=None, eps=None, convrot_group=0, scale_form="ieee"):
    """Per-token quantization of the activated input -> (q [M, K], s [M, 1]),
    by the crate's route: the eager activation fused into the quantizer, or
    (convrot_group) the ConvRot quantizer with the activation fused in fp32 on
    its fused route, else activated, rotated, then quantized."""
    _require_cuda(x)
    x = _as_2d(x)
    act, w, eps = _act_args(x, input_act, weight, eps)
    M, width = x.shape
    K = width // 2 if act in (2, 4) else width
    code = _dtype_code(x.dtype, "INT8 quantization")
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    aux_bytes = lib.w8a8_convrot_workspace_bytes(M, K, convrot_group, code) if convrot_group else 0
    aux = torch.empty(max(aux_bytes, 1), dtype=torch.uint8, device=x.device) if aux_bytes > 0 else None
    flags = _lib.SCALE_RECIP if scale_form == "recip" else 0
    _lib.check(lib.w8a8_quantize_rowwise_act(_ptr(x), code, act, _ptr(w), eps, _ptr(q), _ptr(s), M, K, convrot_group,
                                             flags, _ptr(aux), max(aux_bytes, 0), _stream(x.device)))
    return q, s


def convrot_rotate(x, group=256):
    """Regular Hadamard rotation of every ``group``-wide slice of the rows of a
    [M, K] device tensor, rounded to its dtype: the crate's rotate_activation
    (int8_utils.rs:97-106)."""
    _require_cuda(x)
    x = _as_2d(x)
    M, K = x.shape
    y = torch.empty_like(x)
    _lib.check(_lib.load().w8a8_convrot_rotate(_ptr(x), _dtype_code(x.dtype, "ConvRot rotation"), _ptr(y), M, K,
                                               group, _stream(x.device)))
    return y


def quantize_rowwise_convrot(x, group=256, scale_form="ieee"):
    """ConvRot activation quantization -> (q int8 [M, K], s fp32 [M, 1]) by the
    crate's route (cuda_linear.rs:586-599): fused rotation + quantization for
    group 256 and 256 <= K <= 16384 (Kitchen quantize_int8_rowwise_convrot64,
    int8_linear.cu:1204-1314), else rotate then quantize."""
    _require_cuda(x)
    x = _as_2d(x)
    M, K = x.shape
    code = _dtype_code(x.dtype, "INT8 quantization")
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    rot_bytes = lib.w8a8_convrot_workspace_bytes(M, K, group, code)
    rotated = torch.empty(max(rot_bytes, 1), dtype=torch.uint8, device=x.device) if rot_bytes > 0 else None
    flags = _lib.SCALE_RECIP if scale_form == "recip" else 0
    _lib.check(lib.w8a8_quantize_rowwise_convrot(_ptr(x), code, _ptr(q), _ptr(s), M, K, group, flags,
                                                 _ptr(rotated), max(rot_bytes, 0), _stream(x.device)))
    return q, s


def quantize_tensorwise(x, scale=None, scale_form="ieee"):
    """One scale for the whole tensor -> (q int8 of x's shape, s fp32 scalar):
    the reference's quantize_int8_tensorwise (inference/src/eager.rs:134-151).
    ``scale`` (a number or a one-element tensor) replaces the computed scale and
    is returned as given (an fp32 device tensor)."""
    _require_cuda(x)
    xc = x.contiguous()
    q = torch.empty(xc.shape, dtype=torch.int8, device=x.device)
    flags = _lib.SCALE_RECIP if scale_form == "recip" else 0
    if scale is None:
        s = torch.empty((), dtype=torch.float32, device=x.device)
    else:
        s = torch.as_tensor(scale).to(device=x.device, dtype=torch.float32).reshape(())  # read, not written
        flags |= _lib.GIVEN_SCALE
    _lib.check(_lib.load().w8a8_quantize_tensorwise(_ptr(xc), _dtype_code(xc.dtype, "INT8 quantization"), _ptr(q),
                                                    _ptr(s), xc.numel(), flags, _stream(x.device)))
    return q, s


def quantize_convrot_weight(w, group=256, scale_form="ieee"):
    """ConvRot weight quantization [N, K] -> (q int8 [N, K], s fp32 [N, 1]): the
    reference's quantize_int8_convrot_weight (inference/src/convrot.rs:378-429)."""
    _require_cuda(w)
    if w.dim() != 2:
        raise ValueError("ConvRot INT8 weight quantization expects a 2D weight tensor")
    w = w.contiguous()
    N, K = w.shape
    code = _dtype_code(w.dtype, "INT8 quantization")
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    s = torch.empty((N, 1), dtype=torch.float32, device=w.device)
    lib = _lib.load()
    rot_bytes = lib.w8a8_convrot_weight_workspace_bytes(N, K, group, code)
    rotated = torch.empty(rot_bytes, dtype=torch.uint8, device=w.device) if rot_bytes > 0 else None
    flags = _lib.SCALE_RECIP if scale_form == "recip" else 0
    _lib.check(lib.w8a8_quantize_convrot_weight(_ptr(w), code, _ptr(q), _ptr(s), N, K, group, flags,
                                                _ptr(rotated), max(rot_bytes, 0), _stream(w.device)))
    return q, s


def row_scales(x, scale_form="ieee"):
    """Row scales only (fp32 [M, 1]); the first pass of the fused quant+GEMM."""
    _require_cuda(x)
    x = _as_2d(x)
    M, K = x.shape
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    flags = _lib.SCALE_RECIP if scale_form == "recip" else 0
    _lib.check(_lib.load().w8a8_row_scales(_ptr(x), _dtype_code(x.dtype, "INT8 quantization"),
                                           _ptr(s), M, K, flags, _stream(x.device)))
    return s


def gemv_dequant(q, w, xs, ws, bias, out_dtype, gelu=False):
    """M = 1 / 2 GEMV + dequant (the reference's ``int8_gemv_dequant``)."""
    _require_cuda(q, w, xs, ws, bias)
    M, K = q.shape
    N = w.shape[0]
    out = torch.empty((M, N), dtype=out_dtype, device=q.device)
    _lib.check(_lib.load().w8a8_gemv_dequant(
        _ptr(q), _ptr(w), _ptr(xs), _ptr(ws), ws.numel(), _ptr(bias), _ptr(out),
        _dtype_code(out_dtype, "GEMV output"), M, N, K,
        _lib.ACT_GELU_TANH if gelu else 0, _stream(q.device)))
    return out


def gemm_config(m, n, k, tile=_lib.TILE_AUTO, gelu=False):
    """Name of the GEMM main loop ``gemm_dequant`` runs for an m x n x k product
    (16-byte aligned operands) when ``tile`` is requested: "256x192",
    "256x256", "384x192", "256x128", "regs" or "generic"."""
    flags = _lib.GEMM_TILE(tile) | (_lib.ACT_GELU_TANH if gelu else 0)
    code = _lib.load().w8a8_gemm_config(m, n, k, flags)
    if code < 0:
        raise ValueError(f"bad GEMM query {m}x{n}x{k} tile {tile}")
    return _lib.TILE_NAMES[code]


def gemm_dequant(q, w, xs, ws, bias, out_dtype, gelu=False, out=None, tile=_lib.TILE_AUTO):
    """INT8 GEMM + fused dequant epilogue (the reference's ``cutlass_int8_dequant``).
    ``tile`` requests a main loop (``_lib.TILE_*``; every one gives the same bits)."""
    _require_cuda(q, w, xs, ws, bias)
    M, K = q.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=q.device)
    _lib.check(_lib.load().w8a8_gemm_dequant(
        _ptr(q), _ptr(w), _ptr(xs), _ptr(ws), ws.numel(), _ptr(bias), _ptr(out),
        _dtype_code(out_dtype, "INT8 linear output"), M, N, K,
        (_lib.ACT_GELU_TANH if gelu else 0) | _lib.GEMM_TILE(tile), _stream(q.device)))
    return out


def gemm_i32(q, w, out=None, tile=_lib.TILE_AUTO):
    """INT8 GEMM with int32 output (the reference's ``cublas_gemm_int8``)."""
    _require_cuda(q, w)
    M, K = q.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=q.device)
    _lib.check(_lib.load().w8a8_gemm_dequant(
        _ptr(q), _ptr(w), None, None, 1, None, _ptr(out), _lib.F32, M, N, K,
        _lib.OUT_INT32 | _lib.GEMM_TILE(tile), _stream(q.device)))
    return out


def gemm_dequant_xq(x, xs, w, ws, bias, out_dtype, gelu=False, out=None):
    """GEMM that quantizes the 16-bit activation ``x`` inside its tile loads,
    given the row scales ``xs`` from :func:`row_scales`."""
    _require_cuda(x, xs, w, ws, bias)
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    _lib.check(_lib.load().w8a8_gemm_dequant_xq(
        _ptr(x), _dtype_code(x.dtype, "INT8 quantization"), _ptr(xs), _ptr(w), _ptr(ws), ws.numel(),
        _ptr(bias), _ptr(out), _dtype_code(out_dtype, "INT8 linear output"), M, N, K,
        _lib.ACT_GELU_TANH if gelu else 0, _stream(x.device)))
    return out


def _residual_operands(residual, scale, m, n, device, dtype):
    """The crate's conversions of the residual operands (cuda_linear.rs:707-722,
    int8_linear.rs:99-111): both in the output dtype, residual [M, N], scale flat."""
    r = residual.to(device=device, dtype=dtype).reshape(m, n).contiguous()
    s = scale.to(device=device, dtype=dtype).reshape(-1).contiguous()
    return r, s


def gemm_dequant_residual(q, w, xs, ws, bias, out_dtype, residual, residual_scale, out=None,
                          tile=_lib.TILE_AUTO):
    """INT8 GEMM + dequant + the pre-norm block's residual in one epilogue (the
    reference's ``cutlass_int8_dequant_residual``)."""
    _require_cuda(q, w, xs, ws, bias)
    M, K = q.shape
    N = w.shape[0]
    r, rs = _residual_operands(residual, residual_scale, M, N, q.device, out_dtype)
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=q.device)
    _lib.check(_lib.load().w8a8_gemm_dequant_residual(
        _ptr(q), _ptr(w), _ptr(xs), _ptr(ws), ws.numel(), _ptr(bias), _ptr(rs), rs.numel(), _ptr(r),
        _ptr(out), _dtype_code(out_dtype, "INT8 linear output"), M, N, K, _lib.GEMM_TILE(tile),
        _stream(q.device)))
    return out


def gemv_dequant_residual(q, w, xs, ws, bias, out_dtype, residual, residual_scale):
    """M = 1 / 2 GEMV + dequant + residual (``int8_gemv_dequant`` with residual)."""
    _require_cuda(q, w, xs, ws, bias)
    M, K = q.shape
    N = w.shape[0]
    r, rs = _residual_operands(residual, residual_scale, M, N, q.device, out_dtype)
    out = torch.empty((M, N), dtype=out_dtype, device=q.device)
    _lib.check(_lib.load().w8a8_gemv_dequant_residual(
        _ptr(q), _ptr(w), _ptr(xs), _ptr(ws), ws.numel(), _ptr(bias), _ptr(rs), rs.numel(), _ptr(r),
        _ptr(out), _dtype_code(out_dtype, "GEMV output"), M, N, K, 0, _stream(q.device)))
    return out


def dequantize_linear(acc, xs, ws, bias, out_dtype, gelu=False):
    """Standalone int32 -> out dequant (the reference's ``dequantize_int8_linear``)."""
    _require_cuda(acc, xs, ws, bias)
    M, N = acc.shape
    out = torch.empty((M, N), dtype=out_dtype, device=acc.device)
    _lib.check(_lib.load().w8a8_dequantize_linear(
        _ptr(acc), _ptr(xs), _ptr(ws), ws.numel(), _ptr(bias), _ptr(out),
        _dtype_code(out_dtype, "INT8 linear output"), M, N, _lib.ACT_GELU_TANH if gelu else 0,
        _stream(acc.device)))
    return out


# ---------------------------------------------------------------- operator


def route(m, k, n):
    """The reference's route choice (cuda_linear.rs:498-511, :836-860), non-ConvRot.

    Returns "m1", "gemv" or "gemm".  The M=1 route is a quantize + GEMV pair in
    the reference too (Kitchen int8_linear_m1, dlpack_bindings.cpp:3594-3660),
    so "m1" and "gemv" run the same kernels here."""
    if m == 1 and k % 4 == 0 and (k <= 2560 or (k == 6144 and n <= 128)):
        return "m1"
    if (m == 1 and k % 4 == 0) or (m == 2 and k % 16 == 0):
        return "gemv"
    return "gemm"


def apply_residual(out, residual, scale):
    """int8_linear.rs:99-111: residual.to(out).addcmul(out, scale.to(out)), in
    place on ``out`` by the HIP residual kernel (one fma per element, as the
    reference's GPU addcmul)."""
    if residual is None:
        return out
    if scale is None:
        raise ValueError("residual requires residual_scale")
    _require_cuda(out)
    out2 = out.reshape(-1, out.shape[-1])
    if not out2.is_contiguous():
        raise ValueError("apply_residual needs a contiguous output")
    m, n = out2.shape
    r, rs = _residual_operands(residual, scale, m, n, out.device, out.dtype)
    _lib.check(_lib.load().w8a8_residual_apply(
        _ptr(out2), _ptr(r), _ptr(rs), rs.numel(), _dtype_code(out.dtype, "residual"), m, n,
        _stream(out.device)))
    return out


def int8_linear(x, weight, weight_scale, bias=None, out_dtype=None, convrot=False,
                convrot_groupsize=256, input_act=None, input_act_weight=None, input_act_eps=None,
                residual=None, residual_scale=None, *, scale_form="ieee", fused_quant=False,
                workspace=None):
    """W8A8 linear: quantize x per token, INT8 GEMM/GEMV, dequant to ``out_dtype``.

    Same keyword arguments, in the same order, as the crate's
    ``("cuda", "int8_linear")`` operator (backend_signatures.rs:445-460).
    Extra keyword-only knobs: ``scale_form`` ("ieee" default, or "recip"),
    ``fused_quant`` (quantize inside the GEMM's tile loads), ``workspace`` (a
    preallocated uint8 device buffer of at least
    ``w8a8_int8_linear_workspace_bytes(M, K)`` bytes, 256-byte aligned).
    """
    if residual is not None and residual_scale is None:
        raise ValueError("int8_linear: residual requires residual_scale")
    if input_act not in _lib.ACT_CODES:
        raise ValueError(f"Unsupported input_act {input_act!r}")
    act = _lib.ACT_CODES[input_act]
    _require_cuda(x, weight)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    shape = x.shape
    x2 = _as_2d(x)
    weight = weight.contiguous()
    m, width = x2.shape
    gated = act in (2, 4)  # swiglu / situ: [gate | up] rows (cuda_linear.rs:450-455)
    k = width // 2 if gated else width
    n, kw = weight.shape
    fused_act = bool(convrot) and act != 0 and convrot_groupsize == 256 and k % 256 == 0 and 256 <= k <= 16384
    act_w = None
    if act == 3:
        if input_act_weight is None:
            # the reference's texts by route (cuda_linear.rs:404-417,459-481,558-599)
            if fused_act and m == 1:
                raise RuntimeError("int8 fused convrot GEMV: rms_norm activation requires a weight")
            if fused_act:
                raise RuntimeError("INT8 rowwise convrot64 rms_norm weight must have K elements")
            raise ValueError("input_act 'rms_norm' requires act_weight")
        act_w = input_act_weight.to(device=x.device, dtype=x2.dtype).reshape(-1).contiguous()
        if act_w.numel() != k:
            raise RuntimeError("INT8 rowwise convrot64 rms_norm weight must have K elements")
    if input_act_eps is None:
        if act == 3 and fused_act:
            raise TypeError("float() argument must be a string or a real number, not 'NoneType'")
        input_act_eps = torch.finfo(torch.float32).eps  # ATen rms_norm's default (opmath epsilon)
    if k != kw:
        raise AssertionError("Input and weight inner dimensions must match")
    out_code = _dtype_code(out_dtype, "GEMV output")
    r = route(m, k, n)
    ws = _weight_scale(weight_scale, x.device)
    if ws.numel() not in (1, n):
        if r == "gemm":
            ws.expand([n])  # raises the reference's torch expand error (cuda_linear.rs:702-706)
        raise RuntimeError("INT8 GEMV weight scale must be scalar or per-output-channel")
    if r == "gemv" and m == 2 and weight.data_ptr() % 16 != 0:
        weight = weight.clone()  # cuda_linear.rs:623-625
    b = _bias(bias, x.device, out_dtype)
    out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    lib = _lib.load()
    x_code = _dtype_code(x2.dtype, "INT8 quantization")
    if convrot:
        need = lib.w8a8_int8_linear_convrot_workspace_bytes(m, k, convrot_groupsize, x_code)
    else:
        need = lib.w8a8_int8_linear_workspace_bytes(m, k)
    if workspace is None or workspace.numel() < need or workspace.data_ptr() % 256 != 0:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    flags = (_lib.SCALE_RECIP if scale_form == "recip" else 0) | (
        _lib.ACT_GELU_TANH if input_act == "gelu_tanh" and not convrot else 0) | (
        _lib.FUSED_QUANT if fused_quant else 0)
    if act in (2, 3, 4) or (convrot and act != 0):
        r = rs = None
        if residual is not None:
            r, rs = _residual_operands(residual, residual_scale, m, n, x.device, out_dtype)
        _lib.check(lib.w8a8_int8_linear_act(
            _ptr(x2), x_code, act, _ptr(act_w), float(input_act_eps), _ptr(weight), _ptr(ws), ws.numel(), _ptr(b),
            _ptr(rs), 0 if rs is None else rs.numel(), _ptr(r), _ptr(out), out_code, m, n, k,
            convrot_groupsize if convrot else 0, flags & ~_lib.FUSED_QUANT, _ptr(workspace), workspace.numel(),
            _stream(x.device)))
    elif convrot:
        r = rs = None
        if residual is not None:
            r, rs = _residual_operands(residual, residual_scale, m, n, x.device, out_dtype)
        _lib.check(lib.w8a8_int8_linear_convrot(
            _ptr(x2), x_code, _ptr(weight), _ptr(ws), ws.numel(), _ptr(b), _ptr(rs),
            0 if rs is None else rs.numel(), _ptr(r), _ptr(out), out_code, m, n, k, convrot_groupsize, flags,
            _ptr(workspace), workspace.numel(), _stream(x.device)))
    elif residual is None:
        _lib.check(lib.w8a8_int8_linear(
            _ptr(x2), x_code, _ptr(weight), _ptr(ws), ws.numel(),
            _ptr(b), _ptr(out), out_code, m, n, k, flags, _ptr(workspace), workspace.numel(),
            _stream(x.device)))
    else:
        # fused into the epilogue: the reference's CUTLASS / M = 1 residual
        # routes and its eager addcmul round alike (one fma)
        r, rs = _residual_operands(residual, residual_scale, m, n, x.device, out_dtype)
        _lib.check(lib.w8a8_int8_linear_residual(
            _ptr(x2), x_code, _ptr(weight), _ptr(ws), ws.numel(),
            _ptr(b), _ptr(rs), rs.numel(), _ptr(r), _ptr(out), out_code, m, n, k, flags,
            _ptr(workspace), workspace.numel(), _stream(x.device)))
    if len(shape) == 2:
        return out
    return out.reshape(*shape[:-1], n)
