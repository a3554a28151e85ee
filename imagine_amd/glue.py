"""DiT block glue around the W8A8 linears, over the HIP kernels of
``csrc/w8a8_glue.hip``: the adaLN modulated norm, the gated residual and the
batch-one modulated INT8 linear.

Host-side mirrors of the reference's functions (same arguments, shape rules,
exception classes and messages):
  adaln / rms_adaln        inference/src/backend_eager.rs:176-229 (GPU branch),
                           its modulation() grouping :134-175
  modulated_norm           inference/src/models/qwen_image21/numeric.rs:63-107
  gated_residual           numeric.rs:110-125
  int8_linear_modulated    inference/src/backend_bindings.rs:329-405
All arithmetic runs in the HIP kernels; torch only allocates, reshapes and
slices.
"""
import torch

from . import _lib
from .ops import _bias, _dtype_code, _ptr, _require_cuda, _stream, _weight_scale, quantize_rowwise, route


def _modulation(t, x, n, d):
    """backend_eager.rs:134-175: ``t`` as [rows, d] with the number of
    consecutive rows of ``x`` that share a row of it, when ``t`` broadcasts
    over trailing leading dimensions of ``x``; else ``t`` expanded to [n, d]."""
    ts, xs = list(t.shape), list(x.shape)
    if not ts:
        raise IndexError("tuple index out of range")
    if ts[-1] == d and len(ts) <= len(xs):
        lead = [1] * (len(xs) - len(ts)) + ts[:-1]
        seen, groupable = False, True
        for s, xd in zip(lead, xs[:-1]):
            if s == xd:
                if xd != 1 and seen:
                    groupable = False
                    break
            elif s == 1:
                if xd != 1:
                    seen = True
            else:
                groupable = False
                break
        if groupable:
            rows = t.numel() // d
            if rows > 0 and n % rows == 0:
                return t.reshape(rows, d).contiguous(), n // rows
    return t.expand_as(x).reshape(n, d).contiguous(), 1


def adaln(x, scale, shift, eps, rms=False, single_rounding=False):
    """Kitchen's ``adaln`` / ``rms_adaln`` as the crate calls them on the GPU:
    ``T(T(T(norm(x)) * T(1 + scale)) + shift)`` over the last dimension (the
    crate's eager op order), scale and shift broadcast by ``_modulation``, in
    x's dtype.  ``single_rounding``: ``T(fma(norm, 1 + scale, shift))`` in fp32
    instead, the rounding structure of Kitchen's CUDA kernel."""
    shape = x.shape
    if len(shape) == 0:
        raise IndexError("tuple index out of range")
    d = shape[-1]
    if d == 0:
        raise ZeroDivisionError("integer division or modulo by zero")
    _require_cuda(x, scale, shift)
    for t, name in ((scale, "scale"), (shift, "shift")):
        if t.dtype != x.dtype:
            raise RuntimeError(f"adaln: {name} must have the dtype of x ({x.dtype}), got {t.dtype}")
    n = x.numel() // d
    inp = x.reshape(n, d).contiguous()
    sc, sg = _modulation(scale, x, n, d)
    sh, tg = _modulation(shift, x, n, d)
    out = torch.empty_like(inp)
    _lib.check(_lib.load().w8a8_adaln(
        _ptr(inp), _ptr(sc), _ptr(sh), _ptr(out), n, d, sg, tg, float(eps), _dtype_code(x.dtype, "adaln"),
        (_lib.ADALN_RMS if rms else 0) | (_lib.ADALN_SINGLE_ROUNDING if single_rounding else 0), _stream(x.device)))
    return out.reshape(shape)


def modulated_norm(x, scale, prefix, zero, eps, rms=False, single_rounding=False):
    """numeric.rs:63-107 (inference branch): adaln of every token with
    ``scale[1]``, then the first ``prefix`` tokens (dimension 1) again with
    ``scale[0]``; shift ``zero``.  ``rms`` selects rms_adaln."""
    out = adaln(x, scale[1], zero, eps, rms=rms, single_rounding=single_rounding)
    if prefix != 0:
        out[:, :prefix].copy_(adaln(x[:, :prefix], scale[0], zero, eps, rms=rms, single_rounding=single_rounding))
    return out


def _gate_rows(g, batch, d):
    """A gate that broadcasts over [batch, tokens, d] as [batch, d] rows."""
    if g.dim() == 3 and g.shape[1] != 1:
        raise RuntimeError("gated_residual: the gate must broadcast over the token dimension")
    return g.reshape(*([1] * (3 - g.dim())), *g.shape).expand(batch, 1, d).reshape(batch, d).contiguous()


def gated_residual(x, y, gate, prefix):
    """numeric.rs:110-125: ``x[:, prefix:] += y[:, prefix:] * gate[1]`` and
    ``x[:, :prefix] += y[:, :prefix] * gate[0]``, in place; returns x.
    x and y are [batch, tokens, d] in one dtype (the DiT's hidden states)."""
    _require_cuda(x, y, *gate)
    if x.dim() != 3 or y.shape != x.shape:
        raise RuntimeError("gated_residual: x and y must be [batch, tokens, d] of one shape")
    if y.dtype != x.dtype or any(g.dtype != x.dtype for g in gate):
        raise RuntimeError("gated_residual: y and the gates must have the dtype of x")
    if not x.is_contiguous():
        raise RuntimeError("gated_residual: x must be contiguous (it is updated in place)")
    batch, tokens, d = x.shape
    g0 = _gate_rows(gate[0], batch, d)
    g1 = _gate_rows(gate[1], batch, d)
    y = y.contiguous()
    p = max(0, min(int(prefix), tokens))
    _lib.check(_lib.load().w8a8_gated_residual(
        _ptr(x), _ptr(y), _ptr(g0), _ptr(g1), _ptr(x), batch, tokens, d, p,
        _dtype_code(x.dtype, "gated_residual"), _stream(x.device)))
    return x


def int8_linear_modulated(x, modulation_scale, weight, weight_scale, bias=None, out_dtype=None, convrot=False,
                          convrot_groupsize=256, *, scale_form="ieee", workspace=None):
    """Kitchen's batch-one ``int8_linear_modulated`` (backend_bindings.rs:329-405):
    ``int8_linear(x * (1 + modulation_scale), ...)`` with ``out_dtype``
    defaulting to bfloat16.  The modulation is applied inside the quantizer."""
    width = x.shape[-1]
    if modulation_scale.numel() != width:
        raise ValueError(
            f"modulation_scale must contain one batch-one row of {width} values, got {modulation_scale.numel()}")
    _require_cuda(x, modulation_scale, weight)
    if convrot:
        raise NotImplementedError("int8_linear_modulated with ConvRot is not part of this build")
    if modulation_scale.dtype != x.dtype:
        raise NotImplementedError("a modulation_scale dtype other than x's is not part of this build")
    out_dtype = torch.bfloat16 if out_dtype is None else out_dtype
    shape = x.shape
    x2 = x.reshape(-1, width).contiguous()
    mod = modulation_scale.reshape(-1).contiguous()
    weight = weight.contiguous()
    m, k = x2.shape
    n, kw = weight.shape
    if k != kw:
        raise AssertionError("Input and weight inner dimensions must match")
    out_code = _dtype_code(out_dtype, "GEMV output")
    ws = _weight_scale(weight_scale, x.device)
    if ws.numel() not in (1, n):
        if route(m, k, n) == "gemm":
            ws.expand([n])
        raise RuntimeError("INT8 GEMV weight scale must be scalar or per-output-channel")
    if route(m, k, n) == "gemv" and m == 2 and weight.data_ptr() % 16 != 0:
        weight = weight.clone()
    b = _bias(bias, x.device, out_dtype)
    out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    lib = _lib.load()
    need = lib.w8a8_int8_linear_workspace_bytes(m, k)
    if workspace is None or workspace.numel() < need or workspace.data_ptr() % 256 != 0:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    flags = _lib.SCALE_RECIP if scale_form == "recip" else 0
    _lib.check(lib.w8a8_int8_linear_modulated(
        _ptr(x2), _dtype_code(x2.dtype, "INT8 quantization"), _ptr(mod), _ptr(weight), _ptr(ws), ws.numel(),
        _ptr(b), _ptr(out), out_code, m, n, k, flags, _ptr(workspace), workspace.numel(), _stream(x.device)))
    return out.reshape(*shape[:-1], n)


def quantize_rowwise_modulated(x, modulation_scale, scale_form="ieee"):
    """The modulated quantizer alone: codes and row scales of T(x * T(1 + s))."""
    _require_cuda(x, modulation_scale)
    if modulation_scale.dtype != x.dtype or modulation_scale.numel() != x.shape[-1]:
        raise ValueError("modulation_scale must be one row of x's width in x's dtype")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    m, k = x2.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m, 1), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().w8a8_quantize_rowwise_modulated(
        _ptr(x2), _dtype_code(x2.dtype, "INT8 quantization"), _ptr(modulation_scale.reshape(-1).contiguous()),
        _ptr(q), _ptr(s), m, k, _lib.SCALE_RECIP if scale_form == "recip" else 0, _stream(x.device)))
    return q, s


def modulated_norm_quant(x, scale, prefix, shift, eps, rms=False, *, scale_form="ieee"):
    """``modulated_norm`` (numeric.rs:63-107) followed by the per-token INT8
    quantizer of the linear that consumes it, for x [batch, tokens, d]:
    returns (q int8 [batch * tokens, d], s fp32 [batch * tokens, 1]), equal bit
    for bit to ``quantize_rowwise(modulated_norm(x, scale, prefix, shift, eps))``.
    One kernel when the rows fit its register layout (16-byte aligned, at most
    2048 16-byte chunks), else those two steps.  ``shift`` is the one shift
    tensor of both token ranges, as the reference's ``zero``."""
    _require_cuda(x, *scale, shift)
    if x.dim() != 3:
        raise RuntimeError("modulated_norm_quant: x must be [batch, tokens, d]")
    if any(t.dtype != x.dtype for t in (*scale, shift)):
        raise RuntimeError("modulated_norm_quant: scale and shift must have the dtype of x")
    batch, tokens, d = x.shape
    esz = x.element_size()
    x = x.contiguous()
    s0, s1, h = _gate_rows(scale[0], batch, d), _gate_rows(scale[1], batch, d), _gate_rows(shift, batch, d)
    fits = (d * esz) % 16 == 0 and d * esz // 16 <= 2048 and x.data_ptr() % 16 == 0
    if not fits:
        n = modulated_norm(x, scale, prefix, shift, eps, rms=rms)
        return quantize_rowwise(n.reshape(batch * tokens, d), scale_form=scale_form)
    q = torch.empty((batch * tokens, d), dtype=torch.int8, device=x.device)
    s = torch.empty((batch * tokens, 1), dtype=torch.float32, device=x.device)
    p = max(0, min(int(prefix), tokens))
    _lib.check(_lib.load().w8a8_modulated_norm_quant(
        _ptr(x), _ptr(s0), _ptr(s1), _ptr(h), _ptr(h), _ptr(q), _ptr(s), batch, tokens, d, p, float(eps),
        _dtype_code(x.dtype, "adaln"), 1 if rms else 0, _lib.SCALE_RECIP if scale_form == "recip" else 0,
        _stream(x.device)))
    return q, s


def _rope(name, q, k, freqs_cis, q_scale, k_scale, epsilon, norm, inplace=False):
    """Checks, layout and launch shared by the non-split RoPE family; k None
    is the one-tensor form.  Returns packed (q_out, k_out or None)."""
    _require_cuda(*[t for t in (q, k, freqs_cis, q_scale) if t is not None])
    if q.dim() != 4 or (k is not None and k.shape != q.shape):
        raise RuntimeError(f"{name}: inputs must be [batch, seq, heads, head_dim] of one shape")
    b, s, h, d = q.shape
    if freqs_cis.dtype != torch.float32:
        raise NotImplementedError(f"{name}: freqs_cis in a dtype other than float32 is not part of this build")
    fs = tuple(freqs_cis.shape)
    if len(fs) != 6 or fs[0] not in (1, b) or fs[1] != s or fs[2] != 1 or fs[3:] != (d // 2, 2, 2):
        raise NotImplementedError(f"{name}: freqs_cis layout {fs} is not part of this build")
    if any(t is not None and t.dtype != q.dtype for t in (k, q_scale, k_scale)):
        raise RuntimeError(f"{name}: the second tensor and the scales must have the dtype of the first")
    rs = q.stride(1)
    if q.stride() != (s * rs, rs, d, 1) or (k is not None and k.stride() != q.stride()) or rs < h * d:
        if inplace:
            raise NotImplementedError(f"{name}: in place on this stride layout is not part of this build")
        q = q.contiguous()
        k = None if k is None else k.contiguous()
        rs = h * d
    f = freqs_cis.contiguous()
    if inplace:
        qo, ko = q, k
    else:
        qo = torch.empty((b, s, h, d), device=q.device, dtype=q.dtype)
        ko = None if k is None else torch.empty_like(qo)
    fpb = 1 if fs[0] == b and b > 1 else 0
    code = _dtype_code(q.dtype, name)
    if norm:
        qs = q_scale.reshape(-1).contiguous()
        ks = None if k is None else k_scale.reshape(-1).contiguous()
        _lib.check(_lib.load().w8a8_rms_rope(
            _ptr(q), _ptr(k), _ptr(f), _ptr(qs), _ptr(ks), _ptr(qo), _ptr(ko), b, s, h, d, rs, fpb,
            float(epsilon), code, _stream(q.device)))
    else:
        _lib.check(_lib.load().w8a8_apply_rope(
            _ptr(q), _ptr(k), _ptr(f), _ptr(qo), _ptr(ko), b, s, h, d, rs, fpb, code, _stream(q.device)))
    return qo, ko


def rms_rope(q, k, freqs_cis, q_scale, k_scale=None, epsilon=1e-6):
    """Kitchen's ``rms_rope`` (backend_rope.rs:364-440, the eager numerics of
    eager_rms :204-222 / eager_apply :146-159, non-split): RMSNorm of every
    head row of q and k with its weight, then the pairwise rotation by
    ``freqs_cis``.  q, k [B, S, H, D]; freqs_cis fp32 [B|1, S, 1, D/2, 2, 2]
    (the DiT's layout); scales [D].  q and k may be views whose heads are
    packed but whose tokens are further apart (q, k = qkv[:, :, 0],
    qkv[:, :, 1] of a [B, S, 3, H, D] QKV output): those are read in place.
    Returns packed (q_out, k_out)."""
    return _rope("rms_rope", q, k, freqs_cis, q_scale, q_scale if k_scale is None else k_scale, epsilon, True)


def rms_rope1(x, freqs_cis, scale, epsilon=1e-6):
    """Kitchen's ``rms_rope1`` (one tensor; backend_rope.rs:364-440): as
    ``rms_rope`` on x alone.  Returns the packed output."""
    return _rope("rms_rope1", x, None, freqs_cis, scale, None, epsilon, True)[0]


def apply_rope(xq, xk, freqs_cis):
    """Kitchen's ``apply_rope`` (backend_rope.rs:256-299, eager numerics
    eager_apply :146-159, non-split): the pairwise rotation alone of xq and xk
    [B, S, H, D] by fp32 ``freqs_cis`` [B|1, S, 1, D/2, 2, 2].  Returns packed
    (xq_out, xk_out)."""
    if xk is None:
        raise RuntimeError("apply_rope: xk is required (apply_rope1 takes one tensor)")
    return _rope("apply_rope", xq, xk, freqs_cis, None, None, 0.0, False)


def apply_rope1(x, freqs_cis):
    """Kitchen's ``apply_rope1`` (the DiT's attention-patch route,
    models/qwen_image21/dit.rs:460-480): ``apply_rope`` on one tensor."""
    return _rope("apply_rope1", x, None, freqs_cis, None, None, 0.0, False)[0]


def rms_rope_(q, k, freqs_cis, q_scale, k_scale=None, epsilon=1e-6):
    """Kitchen's in-place ``rms_rope_``: ``rms_rope`` written back over q and
    k (views into a QKV output included).  Returns (q, k)."""
    return _rope("rms_rope_", q, k, freqs_cis, q_scale, q_scale if k_scale is None else k_scale, epsilon, True,
                 inplace=True)


def rms_rope1_(x, freqs_cis, scale, epsilon=1e-6):
    """Kitchen's in-place ``rms_rope1_``.  Returns x."""
    return _rope("rms_rope1_", x, None, freqs_cis, scale, None, epsilon, True, inplace=True)[0]


def apply_rope_(xq, xk, freqs_cis):
    """Kitchen's in-place ``apply_rope_``.  Returns (xq, xk)."""
    if xk is None:
        raise RuntimeError("apply_rope_: xk is required (apply_rope1_ takes one tensor)")
    return _rope("apply_rope_", xq, xk, freqs_cis, None, None, 0.0, False, inplace=True)


def apply_rope1_(x, freqs_cis):
    """Kitchen's in-place ``apply_rope1_``.  Returns x."""
    return _rope("apply_rope1_", x, None, freqs_cis, None, None, 0.0, False, inplace=True)[0]
