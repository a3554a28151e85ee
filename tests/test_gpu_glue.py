"""GPU parity of the DiT block glue kernels (w8a8_glue.hip) against the
reference's eager ATen op sequences (oracle/torch_eager.py) and the oracle.

Bar: the modulated quantizer's codes and scales and the modulated linear's
outputs bit-exact; the gated residual bit-exact for 16-bit dtypes (fp32 within
one ulp); adaLN within one ulp of the norm carried through its two roundings,
and at least 97% of outputs bit-equal (the fp32 mean / variance reductions
round in a different order than ATen's)."""
import numpy as np
import pytest
import torch

import imagine_amd as W
from oracle import oracle as O
from oracle import torch_eager as E

pytestmark = pytest.mark.gpu
TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    W._lib.load()
    yield
    torch.cuda.synchronize()


def storage(t, dtype):
    t = t.detach().cpu().contiguous()
    return t.numpy() if dtype == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def close(got, want, dtype, frac=0.97, before_add=None):
    """Two ulps of the larger of the result and the value before the last
    addition (``before_add``: adaLN's T(norm * (1 + scale)), where a shift
    of the opposite sign cancels), and ``frac`` of the outputs bit-equal."""
    a = O.to_f32(got, dtype).astype(np.float64)
    b = O.to_f32(want, dtype).astype(np.float64)
    mag = np.abs(b) if before_add is None else np.maximum(np.abs(b), np.abs(before_add))
    rel = {"bf16": 2.0**-7, "f16": 2.0**-10, "f32": 2.0**-22}[dtype]
    bad = np.abs(a - b) > 2 * mag * rel + 1e-6
    assert not bad.any(), f"{int(bad.sum())} outputs off; e.g. got {a[bad][:4]} want {b[bad][:4]}"
    assert (got == want).mean() > frac


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rms", [False, True])
def test_adaln_matches_eager_sequence(dtype, rms):
    g = torch.Generator().manual_seed(41)
    x = (torch.randn(2, 300, 3072, generator=g) * 2 + 0.25).to(TD[dtype])
    scale = (torch.randn(2, 1, 3072, generator=g) * 0.5).to(TD[dtype])
    shift = (torch.randn(2, 1, 3072, generator=g) * 0.1).to(TD[dtype])
    print(f"adaln {dtype} rms={rms} x={tuple(x.shape)}", flush=True)
    out = W.adaln(x.to(DEV), scale.to(DEV), shift.to(DEV), 1e-6, rms=rms)
    want = E.adaln(x, scale, shift, 1e-6, rms)
    z = E.adaln(x, scale, torch.zeros_like(shift), 1e-6, rms).float().numpy()
    # fp32 outputs carry the reduction-order differences unrounded: ulp bound only
    close(storage(out, dtype), storage(want, dtype), dtype, frac=0.0 if dtype == "f32" else 0.97,
          before_add=z)


def test_adaln_per_token_modulation_and_odd_width():
    """scale with one row per token (group 1), a width that is no multiple of
    the block size, and a [1, d] shift shared by all rows."""
    g = torch.Generator().manual_seed(42)
    x = (torch.randn(3, 7, 1000, generator=g)).to(torch.bfloat16)
    scale = (torch.randn(3, 7, 1000, generator=g) * 0.3).to(torch.bfloat16)
    shift = (torch.randn(1000, generator=g) * 0.3).to(torch.bfloat16)
    out = W.adaln(x.to(DEV), scale.to(DEV), shift.to(DEV), 1e-5)
    want = E.adaln(x, scale, shift, 1e-5)
    z = E.adaln(x, scale, torch.zeros_like(shift), 1e-5).float().numpy()
    close(storage(out, "bf16"), storage(want, "bf16"), "bf16", before_add=z)


def test_modulated_norm_with_text_prefix():
    """The DiT's norm1/norm2: text tokens (the prefix) take the first
    modulation, image tokens the second; shift zero."""
    g = torch.Generator().manual_seed(43)
    x = (torch.randn(2, 512, 3072, generator=g)).to(torch.bfloat16)
    s0 = (torch.randn(2, 1, 3072, generator=g) * 0.4).to(torch.bfloat16)
    s1 = (torch.randn(2, 1, 3072, generator=g) * 0.4).to(torch.bfloat16)
    zero = torch.zeros(2, 1, 3072, dtype=torch.bfloat16)
    out = W.modulated_norm(x.to(DEV), (s0.to(DEV), s1.to(DEV)), 256, zero.to(DEV), 1e-6)
    want = E.modulated_norm(x, (s0, s1), 256, zero, 1e-6)
    close(storage(out, "bf16"), storage(want, "bf16"), "bf16")


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("prefix", [0, 256])
def test_gated_residual_matches_addcmul(dtype, prefix):
    g = torch.Generator().manual_seed(44 + prefix)
    x = (torch.randn(2, 700, 3072, generator=g) * 3).to(TD[dtype])
    y = (torch.randn(2, 700, 3072, generator=g) * 2).to(TD[dtype])
    g0 = torch.randn(2, 1, 3072, generator=g).to(TD[dtype])
    g1 = torch.randn(2, 1, 3072, generator=g).to(TD[dtype])
    xd = x.to(DEV)
    ret = W.gated_residual(xd, y.to(DEV), (g0.to(DEV), g1.to(DEV)), prefix)
    assert ret.data_ptr() == xd.data_ptr()   # in place, as the reference
    want = E.gated_residual(x.clone(), y, (g0, g1), prefix)
    if dtype == "f32":
        close(storage(xd, dtype), storage(want, dtype), dtype, frac=0.0)
    else:
        assert np.array_equal(storage(xd, dtype), storage(want, dtype))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_modulated_quantizer_bit_exact(dtype):
    g = torch.Generator().manual_seed(45)
    x = (torch.randn(333, 3072, generator=g) * 2).to(TD[dtype])
    x[3] = 0
    s = (torch.randn(3072, generator=g) * 0.6).to(TD[dtype])
    q, xs = W.quantize_rowwise_modulated(x.to(DEV), s.to(DEV))
    xm = O.modulate(storage(x, dtype), storage(s, dtype), dtype)
    q_ref, xs_ref = O.quant_rowwise(xm, dtype)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(xs.cpu().numpy().reshape(-1), xs_ref)


@pytest.mark.parametrize("m", [1, 2, 300])
def test_int8_linear_modulated_bit_exact(m):
    """GEMV (M = 1, 2) and GEMM routes: the linear of the modulated input with
    the reference CUDA routes' epilogue, bit for bit; default out dtype bf16."""
    g = torch.Generator().manual_seed(46 + m)
    k, n = 3072, 1024
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    s = (torch.randn(k, generator=g) * 0.5).to(torch.bfloat16)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    ws = torch.rand(n, generator=g) * 9e-3 + 1e-3
    b = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    out = W.int8_linear_modulated(x.to(DEV), s.to(DEV), w.to(DEV), ws.to(DEV), b.to(DEV))
    assert out.dtype == torch.bfloat16
    xm = O.modulate(storage(x, "bf16"), storage(s, "bf16"), "bf16")
    want, _, _, _ = O.linear_kitchen(xm, "bf16", w.numpy(), ws.numpy(), storage(b, "bf16"), "bf16")
    assert np.array_equal(storage(out, "bf16"), want)


def test_glue_full_size_sampled_rows():
    """The DiT step's shape, [2, 9952, 3072] bf16 with the 256-token text
    prefix: modulated_norm and the gated residual on the GPU, 64 sampled token
    rows of each batch checked against the reference's ATen sequence on the
    CPU (rows are independent), and the whole output finite."""
    g = torch.Generator().manual_seed(47)
    B, T, D, P = 2, 9952, 3072, 256
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    y = (torch.randn(B, T, D, generator=g) * 0.5).to(torch.bfloat16)
    s0, s1, g0, g1 = ((torch.randn(B, 1, D, generator=g) * 0.3).to(torch.bfloat16) for _ in range(4))
    zero = torch.zeros(B, 1, D, dtype=torch.bfloat16)
    rows = torch.cat([torch.arange(0, 4), torch.arange(P - 2, P + 2),
                      torch.randperm(T, generator=g)[:56]]).sort().values
    norm = W.modulated_norm(x.to(DEV), (s0.to(DEV), s1.to(DEV)), P, zero.to(DEV), 1e-6)
    assert bool(torch.isfinite(norm).all())
    xs = x[:, rows]
    pref = int((rows < P).sum())
    want = E.modulated_norm(xs.clone(), (s0, s1), pref, zero, 1e-6)
    z = E.modulated_norm(xs.clone(), (s0, s1), pref, zero, 1e-6).float().numpy()
    close(storage(norm[:, rows.to(DEV)], "bf16"), storage(want, "bf16"), "bf16", before_add=z)
    xd = x.to(DEV)
    W.gated_residual(xd, y.to(DEV), (g0.to(DEV), g1.to(DEV)), P)
    want = E.gated_residual(xs.clone(), y[:, rows], (g0, g1), pref)
    assert np.array_equal(storage(xd[:, rows.to(DEV)], "bf16"), storage(want, "bf16"))


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rms", [False, True])
@pytest.mark.parametrize("prefix", [0, 256])
def test_modulated_norm_quant_equals_norm_then_quantizer(dtype, rms, prefix):
    """The fused norm + quantizer against the two library steps it replaces
    (adaLN with the text prefix, then the per-token quantizer): codes and
    row scales bit for bit."""
    g = torch.Generator().manual_seed(48 + prefix)
    x = (torch.randn(2, 700, 3072, generator=g) * 1.5 + 0.2).to(TD[dtype])
    s0, s1 = ((torch.randn(2, 1, 3072, generator=g) * 0.4).to(TD[dtype]) for _ in range(2))
    shift = (torch.randn(2, 1, 3072, generator=g) * 0.1).to(TD[dtype])
    xd = x.to(DEV)
    sc = (s0.to(DEV), s1.to(DEV))
    q, s = W.modulated_norm_quant(xd, sc, prefix, shift.to(DEV), 1e-6, rms=rms)
    n = W.modulated_norm(xd, sc, prefix, shift.to(DEV), 1e-6, rms=rms)
    q2, s2 = W.quantize_rowwise(n.reshape(-1, 3072))
    assert torch.equal(q, q2)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s2.cpu().numpy().view(np.uint32))


def test_modulated_norm_quant_odd_width_and_fallback():
    """A width of 1000 (125 chunks, fused kernel) and an unaligned width of 1001
    (two-step fallback), both equal to norm-then-quantize."""
    for d in (1000, 1001):
        g = torch.Generator().manual_seed(49 + d)
        x = torch.randn(1, 33, d, generator=g).to(torch.bfloat16).to(DEV)
        s0, s1 = ((torch.randn(1, 1, d, generator=g) * 0.3).to(torch.bfloat16).to(DEV) for _ in range(2))
        zero = torch.zeros(1, 1, d, dtype=torch.bfloat16, device=DEV)
        q, s = W.modulated_norm_quant(x, (s0, s1), 5, zero, 1e-6)
        q2, s2 = W.quantize_rowwise(W.modulated_norm(x, (s0, s1), 5, zero, 1e-6).reshape(-1, d))
        assert torch.equal(q, q2) and torch.equal(s, s2)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rms", [False, True])
def test_adaln_single_rounding_against_oracle(dtype, rms):
    """The single-rounding adaLN (T(fma(norm, 1 + scale, shift))) against the
    oracle's float64-norm restatement: within two ulps of T and (16-bit) at
    least 97% bit-equal; the fp32 row sums round in another order."""
    g = torch.Generator().manual_seed(60 + rms)
    x = (torch.randn(2, 300, 3072, generator=g) * 2 + 0.25).to(TD[dtype])
    scale = (torch.randn(2, 1, 3072, generator=g) * 0.5).to(TD[dtype])
    shift = (torch.randn(2, 1, 3072, generator=g) * 0.1).to(TD[dtype])
    out = W.adaln(x.to(DEV), scale.to(DEV), shift.to(DEV), 1e-6, rms=rms, single_rounding=True)
    xs, ss, hs = (storage(t, dtype).reshape(-1, 3072) for t in (x, scale, shift))
    want = np.concatenate([O.adaln_single(xs[b * 300:(b + 1) * 300], ss[b:b + 1], hs[b:b + 1], 1e-6, dtype, rms)
                           for b in range(2)])
    close(storage(out, dtype).reshape(-1, 3072), want, dtype, frac=0.0 if dtype == "f32" else 0.97)
    # and it is a different rounding from the eager route's three
    eager = storage(W.adaln(x.to(DEV), scale.to(DEV), shift.to(DEV), 1e-6, rms=rms), dtype).reshape(-1, 3072)
    if dtype != "f32":
        assert (eager != storage(out, dtype).reshape(-1, 3072)).any()


@pytest.mark.parametrize("rms", [False, True])
@pytest.mark.parametrize("prefix", [0, 256])
def test_modulated_norm_quant_against_oracle_chain(rms, prefix):
    """The fused norm + quantizer against the oracle chain (oracle.adaln, then
    oracle.quant_rowwise) on the rows where the library's adaLN equals
    oracle.adaln bit for bit (the fp32 row sums round in another order
    elsewhere): codes and scales bit for bit on those rows, and most rows
    qualify."""
    g = torch.Generator().manual_seed(70 + prefix)
    B, T, d = 2, 500, 3072
    x = (torch.randn(B, T, d, generator=g) * 1.5 + 0.2).to(torch.bfloat16)
    s0, s1 = ((torch.randn(B, 1, d, generator=g) * 0.4).to(torch.bfloat16) for _ in range(2))
    zero = torch.zeros(B, 1, d, dtype=torch.bfloat16)
    xd = x.to(DEV)
    q, s = W.modulated_norm_quant(xd, (s0.to(DEV), s1.to(DEV)), prefix, zero.to(DEV), 1e-6, rms=rms)
    n = storage(W.modulated_norm(xd, (s0.to(DEV), s1.to(DEV)), prefix, zero.to(DEV), 1e-6, rms=rms), "bf16")
    xs = storage(x, "bf16")
    want = np.empty_like(n)
    for b in range(B):
        for lo, hi, sc in ((0, prefix, s0), (prefix, T, s1)):
            if hi > lo:
                want[b, lo:hi] = O.adaln(xs[b, lo:hi], storage(sc[b], "bf16"), storage(zero[b], "bf16"), 1e-6, "bf16",
                                         rms)
    want = want.reshape(-1, d)
    agree = (n.reshape(-1, d) == want).all(axis=1)
    assert agree.mean() > 0.5, agree.mean()
    q_ref, s_ref = O.quant_rowwise(want[agree], "bf16")
    assert np.array_equal(q.cpu().numpy()[agree], q_ref)
    assert np.array_equal(s.cpu().numpy().reshape(-1)[agree].view(np.uint32), s_ref.view(np.uint32))


def _freqs(batch, seq, d, seed):
    g = torch.Generator().manual_seed(seed)
    theta = torch.rand(batch, seq, d // 2, generator=g, dtype=torch.float64) * 50.0
    c, s = theta.cos(), theta.sin()
    return torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2).float()[:, :, None]


_ROPE_CASES = [(dt, fb, lay, 128) for dt in ("bf16", "f16") for fb in (1, 2) for lay in ("packed", "qkv_view")] + [
    (dt, 1, "packed", D) for dt in ("bf16", "f16") for D in (64, 256, 96)]


@pytest.mark.parametrize("dtype,fb,layout,D", _ROPE_CASES)
def test_rms_rope_matches_eager_sequence(dtype, fb, layout, D):
    """QK RMSNorm + RoPE against the reference's eager sequence (rms_norm with
    weight, then the fp32 pair rotation) on the CPU: two ulps of the rotated
    pair's magnitude, and at least 97% of outputs bit-equal (the fp32 sum of
    squares rounds in another order).  q and k either packed or read in place
    as views into one [B, S, 3, H, D] QKV output; the 16-byte-per-lane rows
    (D = 64, 128, 256) and the pair-per-lane kernel (D = 96)."""
    g = torch.Generator().manual_seed(52 + fb)
    B, S, H = 2, 300, 24 if D == 128 else 5
    if layout == "packed":
        q = (torch.randn(B, S, H, D, generator=g) * 2).to(TD[dtype])
        k = (torch.randn(B, S, H, D, generator=g) * 0.5).to(TD[dtype])
        qd, kd = q.to(DEV), k.to(DEV)
    else:
        qkv = (torch.randn(B, S, 3, H, D, generator=g) * torch.tensor([2.0, 0.5, 1.0])[:, None, None]).to(TD[dtype])
        q, k = qkv[:, :, 0].contiguous(), qkv[:, :, 1].contiguous()
        qkv_d = qkv.to(DEV)
        qd, kd = qkv_d[:, :, 0], qkv_d[:, :, 1]
        assert qd.stride(1) == 3 * H * D
    qs = (1 + 0.1 * torch.randn(D, generator=g)).to(TD[dtype])
    ks = (1 + 0.1 * torch.randn(D, generator=g)).to(TD[dtype])
    f = _freqs(fb, S, D, seed=53)
    qo, ko = W.rms_rope(qd, kd, f.to(DEV), qs.to(DEV), ks.to(DEV), 1e-6)
    assert qo.is_contiguous() and ko.is_contiguous()
    wq, wk = E.rms_rope(q, k, f, qs, ks, 1e-6)
    for got, want, x, s in ((qo, wq, q, qs), (ko, wk, k, ks)):
        m = torch.nn.functional.rms_norm(x, (D,), s, 1e-6).float()
        mag = (m[..., 0::2].abs() + m[..., 1::2].abs()).repeat_interleave(2, -1).numpy()
        close(storage(got, dtype), storage(want, dtype), dtype, before_add=mag)


@pytest.mark.parametrize("case", ["f32", "bf16_unaligned"])
def test_rms_rope_pair_kernel_fp32_and_unaligned(case):
    """The pair-per-lane kernel on fp32 rows (nothing is rounded between the
    steps, so outputs agree up to the fp32 row-sum order: no bit-equal share
    asked) and on bf16 q / k that start 2 bytes off a 4-byte boundary
    (element-wise loads and stores)."""
    dtype = "f32" if case == "f32" else "bf16"
    g = torch.Generator().manual_seed(61)
    B, S, H, D = 2, 200, 6, 128
    q = (torch.randn(B, S, H, D, generator=g) * 2).to(TD[dtype])
    k = (torch.randn(B, S, H, D, generator=g) * 0.5).to(TD[dtype])

    def offset_by_one(t):
        buf = torch.zeros(t.numel() + 1, dtype=t.dtype, device=DEV)
        buf[1:] = t.reshape(-1).to(DEV)
        v = buf[1:].view(t.shape)
        assert v.data_ptr() % 4 == 2
        return v

    qd, kd = (q.to(DEV), k.to(DEV)) if case == "f32" else (offset_by_one(q), offset_by_one(k))
    qs = (1 + 0.1 * torch.randn(D, generator=g)).to(TD[dtype])
    ks = (1 + 0.1 * torch.randn(D, generator=g)).to(TD[dtype])
    f = _freqs(1, S, D, seed=62)
    qo, ko = W.rms_rope(qd, kd, f.to(DEV), qs.to(DEV), ks.to(DEV), 1e-6)
    wq, wk = E.rms_rope(q, k, f, qs, ks, 1e-6)
    for got, want, x, s in ((qo, wq, q, qs), (ko, wk, k, ks)):
        m = torch.nn.functional.rms_norm(x, (D,), s, 1e-6).float()
        mag = (m[..., 0::2].abs() + m[..., 1::2].abs()).repeat_interleave(2, -1).numpy()
        close(storage(got, dtype), storage(want, dtype), dtype, frac=0.0 if dtype == "f32" else 0.97,
              before_add=mag)


@pytest.mark.parametrize("op", ["apply_rope", "apply_rope1", "rms_rope1"])
@pytest.mark.parametrize("D", [128, 96])
def test_rope_family_matches_eager_sequence(op, D):
    """The rotation alone (apply_rope / apply_rope1) and the one-tensor
    rms_rope1 against the eager route on the CPU: two ulps of the rotated
    pair's magnitude and at least 97% bit-equal (the fp32 product sum may be
    contracted to an fma on either side); the 16-byte-per-lane (D = 128) and
    pair-per-lane (D = 96) kernels."""
    g = torch.Generator().manual_seed(71)
    B, S, H = 2, 150, 6
    x = (torch.randn(B, S, H, D, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(B, S, H, D, generator=g) * 0.5).to(torch.bfloat16)
    sc = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    f = _freqs(2, S, D, seed=72)
    fd = f.to(DEV)
    if op == "apply_rope":
        got = W.apply_rope(x.to(DEV), k.to(DEV), fd)
        want = (E.rope_apply(x, f), E.rope_apply(k, f))
    elif op == "apply_rope1":
        got = (W.apply_rope1(x.to(DEV), fd),)
        want = (E.rope_apply(x, f),)
    else:
        got = (W.rms_rope1(x.to(DEV), fd, sc.to(DEV), 1e-6),)
        want = (E.rms_rope(x, x, f, sc, sc, 1e-6)[0],)
    for a, b, src in zip(got, want, (x, k)):
        assert a.is_contiguous()
        m = torch.nn.functional.rms_norm(src, (D,), sc, 1e-6) if op == "rms_rope1" else src
        m = m.float()
        mag = (m[..., 0::2].abs() + m[..., 1::2].abs()).repeat_interleave(2, -1).numpy()
        close(storage(a, "bf16"), storage(b, "bf16"), "bf16", before_add=mag)


@pytest.mark.parametrize("op", ["rms_rope_", "apply_rope1_"])
def test_rope_in_place_forms(op):
    """The in-place forms write the eager route's result back over their
    inputs: rms_rope_ on q / k views into one [B, S, 3, H, 128] QKV output
    (the v third untouched; 16-byte-per-lane kernel), apply_rope1_ on a packed
    [B, S, H, 96] tensor (pair-per-lane kernel)."""
    g = torch.Generator().manual_seed(81)
    B, S, H = 2, 150, 6
    if op == "rms_rope_":
        D = 128
        qkv = (torch.randn(B, S, 3, H, D, generator=g) * 1.5).to(torch.bfloat16)
        sc = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
        f = _freqs(1, S, D, seed=82)
        qkv_d = qkv.to(DEV)
        rq, rk = W.rms_rope_(qkv_d[:, :, 0], qkv_d[:, :, 1], f.to(DEV), sc.to(DEV), sc.to(DEV), 1e-6)
        assert rq.data_ptr() == qkv_d[:, :, 0].data_ptr() and rk.data_ptr() == qkv_d[:, :, 1].data_ptr()
        q, k = qkv[:, :, 0].contiguous(), qkv[:, :, 1].contiguous()
        wq, wk = E.rms_rope(q, k, f, sc, sc, 1e-6)
        got = qkv_d.cpu()
        assert torch.equal(got[:, :, 2], qkv[:, :, 2])
        pairs = ((got[:, :, 0], wq, q), (got[:, :, 1], wk, k))
    else:
        D = 96
        x = (torch.randn(B, S, H, D, generator=g) * 2).to(torch.bfloat16)
        sc = None
        f = _freqs(2, S, D, seed=83)
        xd = x.to(DEV)
        r = W.apply_rope1_(xd, f.to(DEV))
        assert r.data_ptr() == xd.data_ptr()
        pairs = ((xd.cpu(), E.rope_apply(x, f), x),)
    for a, b, src in pairs:
        m = (torch.nn.functional.rms_norm(src, (D,), sc, 1e-6) if sc is not None else src).float()
        mag = (m[..., 0::2].abs() + m[..., 1::2].abs()).repeat_interleave(2, -1).numpy()
        close(storage(a, "bf16"), storage(b, "bf16"), "bf16", before_add=mag)
