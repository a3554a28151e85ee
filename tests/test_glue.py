"""DiT block glue on the CPU: the oracle's bit-level restatements against the
reference's eager ATen op sequences, the modulation grouping rule, and the
host-side argument errors (no device needed)."""
import numpy as np
import pytest
import torch

import imagine_amd as W
from imagine_amd import _lib
from imagine_amd.glue import _modulation
from oracle import oracle as O
from oracle import torch_eager as E

TD = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def storage(t, dtype):
    t = t.detach().contiguous()
    return t.numpy() if dtype == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def with_specials(t):
    """Random values plus zeros of both signs, tiny and large magnitudes."""
    t = t.clone()
    flat = t.view(-1)
    specials = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 3e4, -3e4, 1.0, -1.0, 0.5, -2.0])
    flat[: specials.numel()] = specials.to(t.dtype)
    return t


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_modulate_oracle_equals_aten(dtype):
    g = torch.Generator().manual_seed(31)
    x = with_specials(torch.randn(64, 768, generator=g) * 3).to(TD[dtype])
    s = (torch.randn(768, generator=g) * 0.7).to(TD[dtype])
    s[:4] = torch.tensor([-1.0, -0.999, 1e-4, 7.5]).to(TD[dtype])
    want = storage(E.modulate(x, s), dtype)
    got = O.modulate(storage(x, dtype), storage(s, dtype), dtype)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("prefix", [0, 5])
def test_gated_residual_oracle_equals_aten(dtype, prefix):
    g = torch.Generator().manual_seed(32 + prefix)
    x = with_specials(torch.randn(2, 24, 256, generator=g) * 4).to(TD[dtype])
    y = (torch.randn(2, 24, 256, generator=g) * 2).to(TD[dtype])
    g0 = (torch.randn(2, 1, 256, generator=g)).to(TD[dtype])
    g1 = (torch.randn(2, 1, 256, generator=g)).to(TD[dtype])
    want = storage(E.gated_residual(x.clone(), y, (g0, g1), prefix), dtype)
    xs, ys = storage(x, dtype), storage(y, dtype)
    got = xs.copy()
    got[:, prefix:] = O.gated_residual(xs[:, prefix:], ys[:, prefix:], storage(g1, dtype), dtype)
    if prefix:
        got[:, :prefix] = O.gated_residual(xs[:, :prefix], ys[:, :prefix], storage(g0, dtype), dtype)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("rms", [False, True])
def test_adaln_oracle_within_one_ulp_of_aten(dtype, rms):
    """The float64 restatement against ATen's layer_norm / rms_norm sequence:
    the two differ only in how the fp32 reductions round (one ulp at most)."""
    g = torch.Generator().manual_seed(33)
    x = (torch.randn(48, 3072, generator=g) * 2 + 0.3).to(TD[dtype])
    scale = (torch.randn(1, 3072, generator=g) * 0.5).to(TD[dtype])
    shift = (torch.randn(1, 3072, generator=g) * 0.1).to(TD[dtype])
    want = storage(E.adaln(x, scale, shift, 1e-6, rms), dtype)
    got = O.adaln(storage(x, dtype), storage(scale, dtype), storage(shift, dtype), 1e-6, dtype, rms)
    a = O.to_f32(got, dtype).astype(np.float64)
    b = O.to_f32(want, dtype).astype(np.float64)
    z = E.adaln(x, scale, torch.zeros_like(shift), 1e-6, rms).float().numpy()
    rel = {"bf16": 2.0**-7, "f16": 2.0**-10}[dtype]
    # two roundings after the norm: one ulp of the norm carries through, in
    # units of the value before the shift is added (which may cancel it)
    assert np.all(np.abs(a - b) <= 2 * np.maximum(np.abs(b), np.abs(z)) * rel + 1e-6)
    assert (got == want).mean() > 0.97


def test_adaln_oracle_is_a_normalisation():
    """Mathematical check of the restatement: with scale 0 and shift 0 every
    row has mean ~0 and variance ~1 (layer norm) or mean square ~1 (rms)."""
    g = torch.Generator().manual_seed(34)
    x = (torch.randn(16, 1024, generator=g) * 5 + 2).float().numpy()
    z = np.zeros((1, 1024), np.float32)
    ln = O.adaln(x, z, z, 1e-6, "f32").astype(np.float64)
    assert np.allclose(ln.mean(-1), 0, atol=1e-5) and np.allclose(ln.var(-1), 1, atol=1e-4)
    rms = O.adaln(x, z, z, 1e-6, "f32", rms=True).astype(np.float64)
    assert np.allclose((rms * rms).mean(-1), 1, atol=1e-4)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("rms", [False, True])
def test_adaln_single_rounding_oracle_against_fp32_torch(dtype, rms):
    """oracle.adaln_single against an independent fp32 evaluation of the same
    formula with ATen (layer_norm / rms_norm in fp32, then y * (1 + scale) +
    shift in fp32, rounded to T once): within one ulp of T, almost all
    bit-equal (the fp32 norm and the unfused multiply-add round differently in
    rare cases); and, with zero modulation, the same as rounding the norm."""
    g = torch.Generator().manual_seed(35)
    x = (torch.randn(48, 3072, generator=g) * 2 + 0.3).to(TD[dtype])
    scale = (torch.randn(1, 3072, generator=g) * 0.5).to(TD[dtype])
    shift = (torch.randn(1, 3072, generator=g) * 0.1).to(TD[dtype])
    xf = x.float()
    y = torch.nn.functional.rms_norm(xf, (3072,), eps=1e-6) if rms else torch.nn.functional.layer_norm(xf, (3072,), eps=1e-6)
    want = storage((y * (1 + scale.float()) + shift.float()).to(TD[dtype]), dtype)
    got = O.adaln_single(storage(x, dtype), storage(scale, dtype), storage(shift, dtype), 1e-6, dtype, rms)
    a, b = O.to_f32(got, dtype).astype(np.float64), O.to_f32(want, dtype).astype(np.float64)
    z = (y * (1 + scale.float())).numpy().astype(np.float64)   # before the shift, which may cancel it
    rel = {"bf16": 2.0**-7, "f16": 2.0**-10}[dtype]
    assert np.all(np.abs(a - b) <= np.maximum(np.abs(b), np.abs(z)) * rel + 1e-6)
    assert (got == want).mean() > 0.99
    zero = np.zeros((1, 3072), np.uint16)
    got0 = O.adaln_single(storage(x, dtype), zero, zero, 1e-6, dtype, rms)
    assert (got0 == storage(y.to(TD[dtype]), dtype)).mean() > 0.99
    # a dropped "1 +" or a sign slip would be far off
    assert not np.array_equal(got, O.adaln_single(storage(x, dtype), storage(scale, dtype), zero, 1e-6, dtype, rms))


def test_modulation_grouping_follows_the_reference_rule():
    x = torch.zeros(2, 5, 8)
    t, grp = _modulation(torch.ones(2, 1, 8), x, 10, 8)
    assert tuple(t.shape) == (2, 8) and grp == 5          # per batch row, shared by its tokens
    t, grp = _modulation(torch.ones(8), x, 10, 8)
    assert tuple(t.shape) == (1, 8) and grp == 10         # one row for all
    t, grp = _modulation(torch.ones(2, 5, 8), x, 10, 8)
    assert tuple(t.shape) == (10, 8) and grp == 1         # one row per token
    t, grp = _modulation(torch.arange(40.0).reshape(5, 8), x, 10, 8)
    assert tuple(t.shape) == (10, 8) and grp == 1         # broadcasts over a leading dim: expanded
    assert torch.equal(t[5:], t[:5])
    with pytest.raises(IndexError, match="tuple index out of range"):
        _modulation(torch.tensor(1.0), x, 10, 8)


def test_host_errors_match_the_reference():
    x = torch.zeros(2, 3, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="modulation_scale must contain one batch-one row of 8 values, got 7"):
        W.int8_linear_modulated(x, torch.zeros(7, dtype=torch.bfloat16), torch.zeros(4, 8, dtype=torch.int8),
                                torch.ones(4))
    with pytest.raises(ZeroDivisionError, match="integer division or modulo by zero"):
        W.adaln(torch.zeros(2, 0), torch.zeros(0), torch.zeros(0), 1e-6)
    with pytest.raises(IndexError):
        W.adaln(torch.tensor(1.0), torch.zeros(1), torch.zeros(1), 1e-6)


def test_c_entries_reject_bad_arguments():
    lib = _lib.load()
    assert lib.w8a8_adaln(None, None, None, None, 4, 0, 1, 1, 1e-6, _lib.BF16, 0, None) == _lib.ERR_VALUE
    assert lib.w8a8_last_error().decode() == "integer division or modulo by zero"
    assert lib.w8a8_adaln(None, None, None, None, 4, 8, 1, 1, 1e-6, _lib.BF16, 0, None) == _lib.ERR_VALUE
    assert lib.w8a8_adaln(None, None, None, None, 4, 8, 1, 1, 1e-6, 7, 0, None) == _lib.ERR_RUNTIME
    assert lib.w8a8_adaln(None, None, None, None, 0, 8, 1, 1, 1e-6, _lib.BF16, 0, None) == _lib.OK
    assert lib.w8a8_modulated_norm_quant(None, None, None, None, None, None, None, 2, 3, 0, 0, 1e-6, _lib.BF16, 0, 0,
                                         None) == _lib.ERR_VALUE
    assert lib.w8a8_modulated_norm_quant(None, None, None, None, None, None, None, 2, 3, 8, 0, 1e-6, _lib.BF16, 0, 0,
                                         None) == _lib.ERR_VALUE
    assert lib.w8a8_modulated_norm_quant(None, None, None, None, None, None, None, 0, 3, 8, 0, 1e-6, _lib.BF16, 0, 0,
                                         None) == _lib.OK
    assert lib.w8a8_gated_residual(None, None, None, None, None, 2, 3, 8, 0, _lib.BF16, None) == _lib.ERR_VALUE
    assert lib.w8a8_gated_residual(None, None, None, None, None, 0, 3, 8, 0, _lib.BF16, None) == _lib.OK
    assert lib.w8a8_quantize_rowwise_modulated(None, _lib.BF16, None, None, None, 2, 8, 0, None) == _lib.ERR_VALUE
    assert lib.w8a8_quantize_rowwise_modulated(None, _lib.BF16, None, None, None, 2, 8, _lib.ACT_GELU_TANH,
                                               None) == _lib.ERR_VALUE
    assert lib.w8a8_int8_linear_modulated(None, _lib.BF16, None, None, None, 1, None, None, _lib.BF16, 2, 4, 8,
                                          _lib.FUSED_QUANT, None, 0, None) == _lib.ERR_VALUE


def test_rope_apply_oracle_is_the_complex_rotation():
    """The eager rotation on fp32 pairs equals the complex product
    (x0 + i x1)(cos + i sin) in float64 to fp32 rounding, is the identity for
    zero angles, and keeps every pair's length."""
    g = torch.Generator().manual_seed(51)
    x = torch.randn(2, 7, 3, 16, generator=g)
    theta = torch.rand(7, 8, generator=g, dtype=torch.float64) * 6.3
    c, s = theta.cos(), theta.sin()
    f = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2).float()[None, :, None]  # [1,7,1,8,2,2]
    out = E.rope_apply(x, f).double()
    z = torch.complex(x[..., 0::2].double(), x[..., 1::2].double()) * torch.complex(c, s)[None, :, None]
    assert torch.allclose(out[..., 0::2], z.real, rtol=0, atol=1e-5)
    assert torch.allclose(out[..., 1::2], z.imag, rtol=0, atol=1e-5)
    ident = torch.zeros(1, 7, 1, 8, 2, 2)
    ident[..., 0, 0] = 1
    ident[..., 1, 1] = 1
    assert torch.equal(E.rope_apply(x, ident), x)
    n_in = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n_out = out[..., 0::2] ** 2 + out[..., 1::2] ** 2
    assert torch.allclose(n_out, n_in.double(), rtol=1e-5)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_rms_norm_with_weight_rounds_once(dtype):
    """ATen's rms_norm with a weight (what backend_rope.rs:216 calls) is
    T(x * rsqrt(mean(x^2) + eps) * w) with the weight product in fp32 and one
    rounding; rounding after the normalisation and again after the weight
    disagrees on about a quarter of the bf16 outputs."""
    g = torch.Generator().manual_seed(52)
    x = torch.randn(64, 128, generator=g).to(TD[dtype])
    w = (torch.randn(128, generator=g) * 0.5 + 1).to(TD[dtype])
    got = torch.nn.functional.rms_norm(x, (128,), w, 1e-6)
    xf = x.double()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    once = (xf * r * w.double()).to(TD[dtype])
    twice = ((xf * r).to(TD[dtype]).double() * w.double()).to(TD[dtype])
    assert (got == once).float().mean() > 0.99
    assert (got == twice).float().mean() < 0.95


def test_rms_rope_host_errors():
    q = torch.zeros(1, 4, 2, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        W.rms_rope(q, q, torch.zeros(1, 4, 1, 4, 2, 2), torch.ones(8, dtype=torch.bfloat16))   # CPU tensors
    lib = _lib.load()
    assert lib.w8a8_rms_rope(None, None, None, None, None, None, None, 1, 4, 2, 7, 14, 0, 1e-6, _lib.BF16,
                             None) == _lib.ERR_VALUE
    assert lib.w8a8_rms_rope(None, None, None, None, None, None, None, 0, 4, 2, 8, 16, 0, 1e-6, _lib.BF16,
                             None) == _lib.OK
    assert lib.w8a8_rms_rope(None, None, None, None, None, None, None, 1, 4, 2, 8, 16, 0, 1e-6, _lib.BF16,
                             None) == _lib.ERR_VALUE                  # null pointers
    assert lib.w8a8_rms_rope(None, None, None, None, None, None, None, 1, 4, 2, 8, 15, 0, 1e-6, _lib.BF16,
                             None) == _lib.ERR_VALUE                  # token rows overlap
    assert lib.w8a8_apply_rope(None, None, None, None, None, 1, 4, 2, 7, 14, 0, _lib.BF16, None) == _lib.ERR_VALUE
    assert lib.w8a8_apply_rope(None, None, None, None, None, 0, 4, 2, 8, 16, 0, _lib.BF16, None) == _lib.OK
    assert lib.w8a8_apply_rope(None, None, None, None, None, 1, 4, 2, 8, 16, 0, _lib.BF16, None) == _lib.ERR_VALUE
    assert lib.w8a8_apply_rope(None, None, None, None, None, 1, 4, 2, 8, 16, 0, 9, None) == _lib.ERR_RUNTIME
    with pytest.raises(RuntimeError):
        W.apply_rope1(q, torch.zeros(1, 4, 1, 4, 2, 2))                 # CPU tensors
    # q written in place but k not: refused before anything is launched or read
    assert lib.w8a8_rms_rope(4096, 8192, 12288, 16384, 16384, 4096, 20480, 1, 4, 2, 8, 16, 0, 1e-6, _lib.BF16,
                             None) == _lib.ERR_VALUE
    assert "in place" in lib.w8a8_last_error().decode()
