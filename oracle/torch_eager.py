"""LibTorch-CPU restatement of the reference's eager INT8 linear (TEST INFRASTRUCTURE ONLY).

The reference's CPU route is a fixed sequence of ATen ops issued from Rust
through tch; this module issues the same ops in the same order from Python on
the CPU build of torch.  It is the ``cpu_baseline`` that ``bench.py`` times
(``kind: "port"``) and a second, independent restatement that the tests
compare the C oracle against bit for bit.  The product library never imports it.

Op sequence, with the reference lines it follows:
  int8_linear.rs:198-199   x = apply_input(x, act)            (gelu "tanh" only here)
  eager.rs:159-165         s = amax(|x|, -1).float() / 127, clamp_min(1e-30)
  eager.rs:94-109          sT = s.to(x.dtype); sT[sT == 0] = tiny(x.dtype)
  eager.rs:110-121,169     q = (x / sT).round_().clamp_(-128, 127).to(int8)
  int8_linear.rs:240       acc = _int_mm(q, weight.T.contiguous())   (K padded to 8)
  int8_linear.rs:248-261   out = (acc.float() * (xs * ws)).to(out)  in <=256 MiB row chunks
  int8_linear.rs:263-269   out = out + bias.to(out)
"""
import torch

TINY = {torch.float16: 6.103515625e-5, torch.bfloat16: torch.finfo(torch.float32).tiny,
        torch.float32: torch.finfo(torch.float32).tiny}


def quantize_rowwise(x):
    """eager.rs:159-171 on a 2-D tensor: returns (q int8 [M,K], s fp32 [M,1])."""
    s = x.abs().amax(dim=-1, keepdim=True).float().div(127.0).clamp_min(1e-30)
    sT = s.to(x.dtype)
    sT = torch.where(sT == 0, torch.full_like(sT, TINY[x.dtype]), sT)
    q = (x / sT).round_().clamp_(-128, 127).to(torch.int8)
    return q, s


def accumulate(q, wt):
    """int8_linear.rs:134-168 on the CPU: pad K to a multiple of 8, then _int_mm."""
    m, k = q.shape
    n = wt.shape[1]
    if m == 0 or k == 0:
        return torch._int_mm(q, wt)
    pk = (k + 7) // 8 * 8
    if pk != k:
        q = torch.cat([q, q.new_zeros(m, pk - k)], 1)
        wt = torch.cat([wt, wt.new_zeros(pk - k, n)], 0)
    return torch._int_mm(q, wt)


def int8_linear(x, weight, weight_scale, bias=None, out_dtype=torch.bfloat16, input_act=None):
    """The reference's CPU eager int8_linear (no ConvRot, no residual)."""
    if input_act == "gelu_tanh":
        x = torch.nn.functional.gelu(x, approximate="tanh")
    elif input_act is not None:
        raise ValueError(f"unsupported input_act {input_act!r}")
    width = x.shape[-1]
    weight = weight.contiguous()
    ws = weight_scale.to(torch.float32).reshape(-1)
    shape = x.shape
    q, xs = quantize_rowwise(x.reshape(-1, width))
    acc = accumulate(q, weight.t().contiguous())
    m, n = acc.shape
    chunk = max(1, min(m, 256 * 1024 * 1024 // (n * 4)))
    ws_row = ws.reshape(1, -1)
    parts = []
    for i in range(0, m, chunk):
        end = min(i + chunk, m)
        scale = xs[i:end].float() * ws_row
        parts.append((acc[i:end].float() * scale).to(out_dtype))
    out = torch.cat(parts, 0)
    if bias is not None:
        out = out + bias.to(out_dtype).reshape(1, -1)
    return out.reshape(*shape[:-1], weight.shape[0]), q, xs, acc


# ---------------------------------------------------------------- DiT block glue
# The reference's eager (CPU) routes of the glue around the linears, as the same
# ATen ops in the same order.

def adaln(x, scale, shift, eps, rms=False):
    """backend_eager.rs:186-199: norm over the last dim (layer_norm without
    affine, or rms_norm without weight), * (scale + 1), + shift; every op in
    x's dtype."""
    shape = [x.shape[-1]]
    if rms:
        normalized = torch.nn.functional.rms_norm(x, shape, None, eps)
    else:
        normalized = torch.nn.functional.layer_norm(x, shape, None, None, eps)
    return normalized.mul(scale.add(1)).add(shift)


def modulated_norm(x, scale, prefix, zero, eps):
    """numeric.rs:63-107 (inference branch) with the eager adaln."""
    out = adaln(x, scale[1], zero, eps)
    if prefix != 0:
        out[:, :prefix].copy_(adaln(x[:, :prefix], scale[0], zero, eps))
    return out


def gated_residual(x, y, gate, prefix):
    """numeric.rs:110-125: in-place addcmul_ on the two token ranges."""
    x[:, prefix:].addcmul_(y[:, prefix:], gate[1])
    if prefix != 0:
        x[:, :prefix].addcmul_(y[:, :prefix], gate[0])
    return x


def modulate(x, modulation_scale):
    """backend_bindings.rs:391-394: x * (modulation_scale + 1), the scale
    reshaped to broadcast over x's leading dims."""
    width = x.shape[-1]
    shape = [1] * (x.dim() - 1) + [width]
    return x.mul(modulation_scale.reshape(shape).add(1.0))


def rope_apply(x, f):
    """backend_rope.rs:146-159 (eager_apply, non-split): x in f's dtype viewed
    as pairs, out[2i + j] = f[i][j][0] x[2i] + f[i][j][1] x[2i + 1] (mul, then
    addcmul_), back to x's dtype."""
    shape = x.shape
    inp = x.to(f.dtype).reshape(*shape[:-1], -1, 1, 2)
    out = f[..., 0] * inp[..., 0]
    out.addcmul_(f[..., 1], inp[..., 1])
    return out.reshape(shape).to(x.dtype)


def rms_rope(q, k, freqs_cis, q_scale, k_scale, eps):
    """backend_rope.rs:204-222 (eager_rms, whole head rotated) on q and k."""
    def one(x, s):
        return rope_apply(torch.nn.functional.rms_norm(x, (x.shape[-1],), s, eps), freqs_cis)
    return one(q, q_scale), one(k, k_scale)
