"""GPU parity: every HIP kernel against the oracle on identical seeded inputs.

Bar: int8 codes, row scales and int32 accumulators bit-exact; epilogue
outputs bit-exact against the oracle's single-rounding form (the same formula
the reference's CUDA routes use), GELU included (GELU-tanh with a correctly
rounded tanh: every finite bf16 and fp16 input is checked exhaustively).
Also runs the reference's own CUDA golden payloads through the operator.
"""
import numpy as np
import pytest
import torch

import imagine_amd as W
from oracle import oracle as O
from tests.golden import fixtures as FX
from tests.golden import operands as OP

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
    """Host numpy storage of a tensor in oracle convention."""
    t = t.detach().cpu().contiguous()
    if dtype == "f32":
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def from_storage(a, dtype, device=DEV):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype != "f32":
        t = t.view(torch.int16).view(TD[dtype])
    return t.to(device)


def make_x(m, k, dtype, seed, dist="normal"):
    g = torch.Generator().manual_seed(seed)
    if dist == "normal":
        x = torch.randn(m, k, generator=g)
    else:  # Student-t(3) with 0.1% of channels x50
        z = torch.randn(m, k, generator=g)
        chi = torch.randn(m, k, 3, generator=g).pow(2).sum(-1)
        x = z / torch.sqrt(chi / 3.0)
        idx = torch.randperm(k, generator=g)[: max(1, k // 1000)]
        x[:, idx] *= 50.0
    if m > 3:
        x[3] = 0.0
    return x.to(TD[dtype])


def make_w(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)


def ulp_close(got, want, dtype, abs_floor=0.0):
    a = O.to_f32(got, dtype).astype(np.float64)
    b = O.to_f32(want, dtype).astype(np.float64)
    rel = {"bf16": 2.0**-7, "f16": 2.0**-10, "f32": 2.0**-23}[dtype]
    return np.abs(a - b) <= np.abs(b) * rel + abs_floor


# ---------------------------------------------------------------- quantizer

QUANT_SHAPES = [(1, 64), (2, 3072), (7, 3072), (256, 3072), (33, 12288), (5, 1001), (3, 20000),
                (9, 4096), (6, 9216), (4, 16)]


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", QUANT_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("form", ["ieee", "recip"])
def test_quantize_bit_exact(dtype, shape, form):
    m, k = shape
    x = make_x(m, k, dtype, seed=m * 31 + k, dist="student_t" if k == 12288 else "normal")
    q, s = W.quantize_rowwise(x.to(DEV), scale_form=form)
    q_ref, s_ref = O.quant_rowwise(storage(x, dtype), dtype, scale_mode=1 if form == "recip" else 0)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))


def test_quantize_unaligned_input_takes_generic_path():
    x = make_x(5, 3073, "bf16", seed=1)
    xd = x.to(DEV)[:, 1:]  # row stride 3073, start not 16-byte aligned
    xc = xd.contiguous()
    base = torch.empty(xc.numel() + 1, dtype=torch.bfloat16, device=DEV)
    xu = base[1:].view(5, 3072)
    xu.copy_(xc)
    assert xu.data_ptr() % 16 != 0
    q, s = W.quantize_rowwise(xu)
    q_ref, s_ref = O.quant_rowwise(storage(xc, "bf16"), "bf16")
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().reshape(-1), s_ref)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_quantize_gelu_input_act(dtype):
    """The GELU-tanh input activation (the reference's FFN-down input form):
    codes and scales bit for bit against the oracle."""
    x = make_x(64, 3072, dtype, seed=4)
    q, s = W.quantize_rowwise(x.to(DEV), input_act="gelu_tanh")
    q_ref, s_ref = O.quant_rowwise(storage(x, dtype), dtype, act=1)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("aligned", [True, False], ids=["vector", "generic"])
def test_quantize_gelu_every_16bit_pattern_bit_exact(dtype, aligned):
    """Every finite 16-bit input through the quantizer's GELU input
    activation: row i repeats pattern i eight times, so its scale is
    |T(gelu(x))| / 127 and its codes expose the activated value.  Codes and
    scales bit for bit against the oracle, on the vector kernel and (an
    unaligned copy) the generic one."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    bits = bits[np.isfinite(O.to_f32(bits, dtype))]
    rows = np.repeat(bits[:, None], 8, axis=1)
    xa = from_storage(rows, dtype)
    if not aligned:
        buf = torch.empty(rows.size + 8, dtype=TD[dtype], device=DEV)
        xu = buf[1:1 + rows.size].view(rows.shape)
        xu.copy_(xa)
        assert xu.data_ptr() % 16 != 0
        xa = xu
    q, s = W.quantize_rowwise(xa, input_act="gelu_tanh")
    q_ref, s_ref = O.quant_rowwise(rows, dtype, act=1)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_quantize_gelu_vector_and_generic_kernels_agree_for_every_bf16():
    """The bf16 GELU input activation of the vector quantizer (activated once,
    in registers, paired rounding) against the generic kernel's per-element
    evaluation, for all 65536 bf16 bit patterns: row i repeats pattern i eight
    times, so its scale |T(gelu(x))| / 127 and its codes expose the activated
    value.  An unaligned copy routes the same rows to the generic kernel."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    rows = np.repeat(bits[:, None], 8, axis=1)
    xa = from_storage(rows, "bf16")
    buf = torch.empty(rows.size + 8, dtype=torch.bfloat16, device=DEV)
    xu = buf[1:1 + rows.size].view(rows.shape)
    xu.copy_(xa)
    assert xa.data_ptr() % 16 == 0 and xu.data_ptr() % 16 != 0
    qa, sa = W.quantize_rowwise(xa, input_act="gelu_tanh")
    qu, su = W.quantize_rowwise(xu, input_act="gelu_tanh")
    assert np.array_equal(sa.cpu().numpy().view(np.uint32), su.cpu().numpy().view(np.uint32))
    assert np.array_equal(qa.cpu().numpy(), qu.cpu().numpy())


def test_row_scales_equal_quantizer_scales():
    x = make_x(100, 3072, "bf16", seed=9).to(DEV)
    _, s = W.quantize_rowwise(x)
    s2 = W.row_scales(x)
    assert torch.equal(s, s2)


def test_quantize_full_size_outlier_config_bit_exact():
    """M=11712, K=3072, Student-t(3) with 0.1% channels x50: every code and scale."""
    x = make_x(11712, 3072, "bf16", seed=3, dist="student_t")
    q, s = W.quantize_rowwise(x.to(DEV))
    q_ref, s_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))


# ---------------------------------------------------------------- GEMM

GEMM_SHAPES = [(256, 3072, 3072), (300, 200, 160), (1, 16, 16), (513, 257, 64), (64, 96, 48),
               (2, 2, 32), (4, 16, 20), (7, 9, 13), (257, 512, 1024), (37, 1000, 3072)]


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_gemm_int32_accumulators_bit_exact(shape):
    m, n, k = shape
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    b = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    c = W.gemm_i32(a.to(DEV), b.to(DEV))
    assert np.array_equal(c.cpu().numpy(), O.gemm_i32(a.numpy(), b.numpy()))


def test_gemm_int32_extremes_and_unaligned_operand():
    m, n, k = 64, 64, 3072
    a = torch.full((m, k), -128, dtype=torch.int8)
    b = torch.full((n, k), -128, dtype=torch.int8)
    c = W.gemm_i32(a.to(DEV), b.to(DEV))
    assert (c.cpu() == k * 128 * 128).all()
    g = torch.Generator().manual_seed(2)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    base = torch.empty(m * k + 3, dtype=torch.int8, device=DEV)
    au = base[3:].view(m, k)
    au.copy_(a.to(DEV))
    c = W.gemm_i32(au, b.to(DEV))
    assert np.array_equal(c.cpu().numpy(), O.gemm_i32(a.numpy(), b.numpy()))


@pytest.mark.parametrize("odt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("ws_scalar", [False, True])
def test_gemm_dequant_epilogue_bit_exact(odt, with_bias, ws_scalar):
    m, n, k = 300, 520, 1024
    x = make_x(m, k, "bf16", seed=5)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=6)
    g = torch.Generator().manual_seed(7)
    ws = (torch.rand(1 if ws_scalar else n, generator=g) * 9e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=g) * 0.02).to(TD[odt]) if with_bias else None
    out = W.gemm_dequant(torch.from_numpy(q_ref).to(DEV), w.to(DEV),
                         torch.from_numpy(xs_ref).to(DEV), ws.to(DEV),
                         None if bias is None else bias.to(DEV), TD[odt])
    want = O.epilogue_kitchen(O.gemm_i32(q_ref, w.numpy()), xs_ref, ws.numpy(),
                              None if bias is None else storage(bias, odt), odt)
    assert np.array_equal(storage(out, odt), want)


@pytest.mark.parametrize("odt", ["bf16", "f16", "f32"])
def test_gemm_gelu_epilogue_bit_exact(odt):
    """GELU-tanh epilogue, bit for bit against the oracle (fp32 outputs too:
    their tanh is the double-precision tanh rounded once)."""
    m, n, k = 260, 384, 768
    x = make_x(m, k, "bf16", seed=8)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=9)
    ws = torch.full((n,), 0.004)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(1)) * 0.02).to(TD[odt])
    out = W.gemm_dequant(torch.from_numpy(q_ref).to(DEV), w.to(DEV), torch.from_numpy(xs_ref).to(DEV),
                         ws.to(DEV), bias.to(DEV), TD[odt], gelu=True)
    want = O.epilogue_kitchen(O.gemm_i32(q_ref, w.numpy()), xs_ref, ws.numpy(), storage(bias, odt),
                              odt, act=1)
    assert np.array_equal(storage(out, odt), want)


def test_gemm_full_size_sampled_rows_bit_exact():
    """11712 x 3072 x 12288 (the FFN-up shape): int32 accumulators and bf16
    outputs of 48 sampled rows against the oracle, whole output finite."""
    m, k, n = 11712, 3072, 12288
    x = make_x(m, k, "bf16", seed=2)
    w = make_w(n, k, seed=3)
    ws = (torch.rand(n, generator=torch.Generator().manual_seed(4)) * 9e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(5)) * 0.02).to(torch.bfloat16)
    xd, wd = x.to(DEV), w.to(DEV)
    q, xs = W.quantize_rowwise(xd)
    acc = W.gemm_i32(q, wd)
    out = W.gemm_dequant(q, wd, xs, ws.to(DEV), bias.to(DEV), torch.bfloat16)
    rows = np.sort(np.random.default_rng(0).choice(m, 48, replace=False))
    rows[-1] = m - 1  # last (ragged) tile
    q_ref, xs_ref = O.quant_rowwise(storage(x[rows], "bf16"), "bf16")
    acc_ref = O.gemm_i32(q_ref, w.numpy())
    assert np.array_equal(acc.cpu().numpy()[rows], acc_ref)
    want = O.epilogue_kitchen(acc_ref, xs_ref, ws.numpy(), storage(bias, "bf16"), "bf16")
    assert np.array_equal(storage(out, "bf16")[rows], want)
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("mode", ["bf16", "bf16_gelu", "f16", "f32", "bf16_residual", "int32"])
def test_gemm_n3072_tiles_sampled_rows(mode):
    """M = 11712, N = 3072 (the out-proj / FFN-down width, where the default
    tile choice takes 384 x 192 tiles, 256 x 192 with GELU), K = 512: every
    epilogue mode on 64 sampled rows against the oracle, bit for bit."""
    m, k, n = 11712, 512, 3072
    odt = {"bf16_gelu": "bf16", "bf16_residual": "bf16", "int32": "f32"}.get(mode, mode)
    x = make_x(m, k, "bf16", seed=61)
    w = make_w(n, k, seed=62)
    g = torch.Generator().manual_seed(63)
    ws = (torch.rand(n, generator=g) * 9e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=g) * 0.5).to(TD[odt])
    xd, wd = x.to(DEV), w.to(DEV)
    q, xs = W.quantize_rowwise(xd)
    rows = np.sort(np.random.default_rng(1).choice(m, 64, replace=False))
    rows[0], rows[-1] = 0, m - 1
    q_ref, xs_ref = O.quant_rowwise(storage(x[rows], "bf16"), "bf16")
    acc_ref = O.gemm_i32(q_ref, w.numpy())
    if mode == "int32":
        acc = W.gemm_i32(q, wd)
        assert np.array_equal(acc.cpu().numpy()[rows], acc_ref)
        return
    if mode == "bf16_residual":
        resid, rscale = _residual_inputs(m, n, "bf16", seed=64)
        out = W.gemm_dequant_residual(q, wd, xs, ws.to(DEV), bias.to(DEV), torch.bfloat16, resid.to(DEV),
                                      rscale.to(DEV))
        lin = O.epilogue_kitchen(acc_ref, xs_ref, ws.numpy(), storage(bias, "bf16"), "bf16")
        want = O.residual(lin, storage(resid, "bf16")[rows], storage(rscale, "bf16"), "bf16")
        assert np.array_equal(storage(out, "bf16")[rows], want)
        return
    out = W.gemm_dequant(q, wd, xs, ws.to(DEV), bias.to(DEV), TD[odt], gelu=mode == "bf16_gelu")
    want = O.epilogue_kitchen(acc_ref, xs_ref, ws.numpy(), storage(bias, odt), odt,
                              act=1 if mode == "bf16_gelu" else 0)
    assert np.array_equal(storage(out, odt)[rows], want)


# ---------------------------------------------------------------- GEMV

GEMV_SHAPES =[(2, 18432, 3072), (1, 4, 3072), (2, 17, 16), (1, 129, 6144), (2, 4, 2560),
               (1, 33, 20), (2, 5, 64), (2, 300, 12288), (1, 64, 2564)]


@pytest.mark.parametrize("shape", GEMV_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("odt", ["bf16", "f32"])
def test_gemv_bit_exact(shape, odt):
    m, n, k = shape
    x = make_x(m, k, "bf16", seed=n + k)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=n)
    ws = (torch.rand(n, generator=torch.Generator().manual_seed(k)) * 9e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.02).to(TD[odt])
    out = W.gemv_dequant(torch.from_numpy(q_ref).to(DEV), w.to(DEV), torch.from_numpy(xs_ref).to(DEV),
                         ws.to(DEV), bias.to(DEV), TD[odt])
    want = O.epilogue_kitchen(O.gemm_i32(q_ref, w.numpy()), xs_ref, ws.numpy(), storage(bias, odt), odt)
    assert np.array_equal(storage(out, odt), want)


def test_gemv_unaligned_weight():
    m, n, k = 2, 40, 3072
    x = make_x(m, k, "bf16", seed=1)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=2)
    base = torch.empty(n * k + 1, dtype=torch.int8, device=DEV)
    wu = base[1:].view(n, k)
    wu.copy_(w.to(DEV))
    ws = torch.full((1,), 0.03125, device=DEV)
    out = W.gemv_dequant(torch.from_numpy(q_ref).to(DEV), wu, torch.from_numpy(xs_ref).to(DEV), ws,
                         None, torch.bfloat16)
    want = O.epilogue_kitchen(O.gemm_i32(q_ref, w.numpy()), xs_ref, np.float32([0.03125]), None, "bf16")
    assert np.array_equal(storage(out, "bf16"), want)


# ---------------------------------------------------------------- fused quant + GEMM


@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("shape", [(300, 520, 1024), (11712, 3072, 3072), (64, 12288, 3072)],
                         ids=lambda s: "x".join(map(str, s)))
def test_fused_quant_gemm_equals_unfused(xdt, shape):
    m, n, k = shape
    x = make_x(m, k, xdt, seed=11, dist="student_t").to(DEV)
    w = make_w(n, k, seed=12).to(DEV)
    ws = (torch.rand(n, generator=torch.Generator().manual_seed(13)) * 9e-3 + 1e-3).to(DEV)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(14)) * 0.02).to(torch.bfloat16).to(DEV)
    q, xs = W.quantize_rowwise(x)
    ref = W.gemm_dequant(q, w, xs, ws, bias, torch.bfloat16)
    xs2 = W.row_scales(x)
    fused = W.gemm_dequant_xq(x, xs2, w, ws, bias, torch.bfloat16)
    assert torch.equal(xs, xs2)
    assert torch.equal(ref.view(torch.int16), fused.view(torch.int16))


def test_dequantize_linear_bit_exact():
    m, n = 33, 70
    g = torch.Generator().manual_seed(1)
    acc = torch.randint(-2**24, 2**24, (m, n), generator=g, dtype=torch.int32)
    xs = torch.rand(m, generator=g) * 0.1
    ws = torch.rand(n, generator=g) * 0.01
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.float16)
    out = W.dequantize_linear(acc.to(DEV), xs.to(DEV), ws.to(DEV), bias.to(DEV), torch.float16)
    want = O.epilogue_kitchen(acc.numpy(), xs.numpy(), ws.numpy(), storage(bias, "f16"), "f16")
    assert np.array_equal(storage(out, "f16"), want)


@pytest.mark.parametrize("tile", [W._lib.TILE_AUTO, W._lib.TILE_256x256, W._lib.TILE_256x192, W._lib.TILE_384x192,
                                  W._lib.TILE_256x128, W._lib.TILE_REGS, W._lib.TILE_GENERIC],
                         ids=lambda t: W._lib.TILE_NAMES[t])
@pytest.mark.parametrize("odt", ["bf16", "f16"])
def test_gemm_gelu_epilogue_every_preactivation(odt, tile):
    """Every finite 16-bit pre-activation through the GEMM's GELU epilogue.
    Zero codes make the accumulators 0, so the pre-activation of channel n is
    fma(0 * xs, ws, bias[n]) = bias[n] exactly; the bias takes every finite bit
    pattern of the output dtype (the saturated tails, the cancelling negative
    tail, subnormals and signed zeros included).  Bit for bit against the
    oracle, on the staged epilogue of each DMA tile with one block per CU
    (256x256 and 256x192 look bf16 GELU up in an LDS table for magnitudes
    2^-18 to 2^14, 384x192 evaluates it), of the two-blocks-per-CU one
    (256x128), and on the register-staged and generic main loops."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    bits = bits[np.isfinite(O.to_f32(bits, odt))]
    n = (len(bits) + 255) // 256 * 256
    bias = np.resize(bits, n)
    m, k = 64, 128
    q = torch.zeros(m, k, dtype=torch.int8)
    w = torch.zeros(n, k, dtype=torch.int8)
    xs = torch.full((m,), 0.75)
    ws = torch.full((n,), 1.25)
    out = W.gemm_dequant(q.to(DEV), w.to(DEV), xs.to(DEV), ws.to(DEV), from_storage(bias, odt),
                         TD[odt], gelu=True, tile=tile)
    want = O.epilogue_kitchen(np.zeros((m, n), np.int32), xs.numpy(), ws.numpy(), bias, odt, act=1)
    assert np.array_equal(storage(out, odt), want)


@pytest.mark.parametrize("odt", ["bf16", "f16"])
def test_gemv_gelu_epilogue_bit_exact(odt):
    m, n, k = 2, 4096, 3072
    x = make_x(m, k, "bf16", seed=21)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=22)
    ws = torch.full((n,), 0.003)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(23)) * 0.5).to(TD[odt])
    out = W.gemv_dequant(torch.from_numpy(q_ref).to(DEV), w.to(DEV), torch.from_numpy(xs_ref).to(DEV),
                         ws.to(DEV), bias.to(DEV), TD[odt], gelu=True)
    want = O.epilogue_kitchen(O.gemm_i32(q_ref, w.numpy()), xs_ref, ws.numpy(), storage(bias, odt),
                              odt, act=1)
    assert np.array_equal(storage(out, odt), want)


def test_dequantize_linear_gelu_bit_exact():
    """Dequant + GELU over a wide range of pre-activations, the saturated
    negative tail included (values down to about -12)."""
    m, n = 64, 512
    g = torch.Generator().manual_seed(5)
    acc = torch.randint(-2**22, 2**22, (m, n), generator=g, dtype=torch.int32)
    xs = torch.rand(m, generator=g) * 1e-3
    ws = torch.rand(n, generator=g) * 3e-3
    bias = (torch.randn(n, generator=g) * 0.5).to(torch.bfloat16)
    out = W.dequantize_linear(acc.to(DEV), xs.to(DEV), ws.to(DEV), bias.to(DEV), torch.bfloat16, gelu=True)
    want = O.epilogue_kitchen(acc.numpy(), xs.numpy(), ws.numpy(), storage(bias, "bf16"), "bf16", act=1)
    assert np.array_equal(storage(out, "bf16"), want)


def _residual_inputs(m, n, odt, seed):
    g = torch.Generator().manual_seed(seed)
    resid = (torch.randn(m, n, generator=g) * 2.0).to(TD[odt])
    rscale = (torch.rand(n, generator=g) * 1.5 + 0.25).to(TD[odt])
    return resid, rscale


@pytest.mark.parametrize("odt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rs_scalar", [False, True])
@pytest.mark.parametrize("shape", [(300, 512, 768), (11712, 3072, 3072)])
def test_gemm_residual_epilogue_bit_exact(odt, rs_scalar, shape):
    """GEMM + dequant + residual, bit for bit against the oracle's
    O(fma(O(lin), rscale, resid)) on the whole output (full size, the out-proj
    shape of the DiT block: the whole bf16 output, 64 sampled rows of the
    fp16 and fp32 ones)."""
    m, n, k = shape
    if m > 1000 and odt != "bf16":
        rows = np.sort(np.random.default_rng(7).choice(m, 64, replace=False))
        rows[0], rows[-1] = 0, m - 1
    else:
        rows = np.arange(m)
    x = make_x(m, k, "bf16", seed=31)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=32)
    ws = (torch.rand(n, generator=torch.Generator().manual_seed(33)) * 9e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(34)) * 0.02).to(TD[odt])
    resid, rscale = _residual_inputs(m, n, odt, 35)
    if rs_scalar:
        rscale = rscale[:1]
    out = W.gemm_dequant_residual(torch.from_numpy(q_ref).to(DEV), w.to(DEV), torch.from_numpy(xs_ref).to(DEV),
                                  ws.to(DEV), bias.to(DEV), TD[odt], resid.to(DEV), rscale.to(DEV))
    lin = O.epilogue_kitchen(O.gemm_i32(q_ref[rows], w.numpy()), xs_ref[rows], ws.numpy(), storage(bias, odt), odt)
    want = O.residual(lin, storage(resid, odt)[rows], storage(rscale, odt), odt)
    assert np.array_equal(storage(out, odt)[rows], want)


def test_gemm_residual_unaligned_operands_take_the_direct_epilogue():
    """A residual and a scale that are not 16-byte aligned (the reference's
    unaligned_residual / unaligned_residual_scale modes) give the same bits."""
    m, n, k = 200, 264, 512
    x = make_x(m, k, "bf16", seed=41)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=42)
    ws = torch.full((n,), 0.004)
    resid, rscale = _residual_inputs(m, n, "bf16", 43)
    rbuf = torch.empty(m * n + 1, dtype=torch.bfloat16, device=DEV)
    rbuf[1:] = resid.reshape(-1).to(DEV)
    sbuf = torch.empty(n + 3, dtype=torch.bfloat16, device=DEV)
    sbuf[3:] = rscale.to(DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    # device operands are held in names for the whole call: a temporary's
    # memory could be handed to the next temporary before the launch reads it
    qd, wd = torch.from_numpy(q_ref).to(DEV), w.to(DEV)
    xsd, wsd = torch.from_numpy(xs_ref).to(DEV), ws.to(DEV)
    lib = W._lib.load()
    W._lib.check(lib.w8a8_gemm_dequant_residual(
        qd.data_ptr(), wd.data_ptr(), xsd.data_ptr(), wsd.data_ptr(), n, None, sbuf[3:].data_ptr(), n,
        rbuf[1:].data_ptr(), out.data_ptr(), W._lib.BF16, m, n, k, 0, torch.cuda.current_stream().cuda_stream))
    lin = O.epilogue_kitchen(O.gemm_i32(q_ref, w.numpy()), xs_ref, ws.numpy(), None, "bf16")
    want = O.residual(lin, storage(resid, "bf16"), storage(rscale, "bf16"), "bf16")
    assert np.array_equal(storage(out, "bf16"), want)


@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("odt", ["bf16", "f32"])
def test_gemv_residual_epilogue_bit_exact(m, odt):
    n, k = 1536, 3072
    x = make_x(m, k, "bf16", seed=51)
    q_ref, xs_ref = O.quant_rowwise(storage(x, "bf16"), "bf16")
    w = make_w(n, k, seed=52)
    ws = (torch.rand(n, generator=torch.Generator().manual_seed(53)) * 9e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(54)) * 0.02).to(TD[odt])
    resid, rscale = _residual_inputs(m, n, odt, 55)
    out = W.gemv_dequant_residual(torch.from_numpy(q_ref).to(DEV), w.to(DEV), torch.from_numpy(xs_ref).to(DEV),
                                  ws.to(DEV), bias.to(DEV), TD[odt], resid.to(DEV), rscale.to(DEV))
    lin = O.epilogue_kitchen(O.gemm_i32(q_ref, w.numpy()), xs_ref, ws.numpy(), storage(bias, odt), odt)
    want = O.residual(lin, storage(resid, odt), storage(rscale, odt), odt)
    assert np.array_equal(storage(out, odt), want)


@pytest.mark.parametrize("odt", ["bf16", "f16", "f32"])
def test_residual_apply_bit_exact(odt):
    m, n = 37, 1000
    g = torch.Generator().manual_seed(61)
    out = (torch.randn(m, n, generator=g) * 3).to(TD[odt])
    resid, rscale = _residual_inputs(m, n, odt, 62)
    got = W.apply_residual(out.clone().to(DEV), resid.to(DEV), rscale.to(DEV))
    want = O.residual(storage(out, odt), storage(resid, odt), storage(rscale, odt), odt)
    assert np.array_equal(storage(got, odt), want)


# ---------------------------------------------------------------- ConvRot

CONVROT_SHAPES = [(37, 256), (5, 3072), (64, 3072), (3, 6144), (9, 12288), (2, 16384), (1, 4096)]


def _convrot_check(x, dtype, group, scale_form):
    q, s = W.quantize_rowwise_convrot(x, group, scale_form=scale_form)
    q_ref, s_ref = O.convrot_quant(storage(x, dtype), dtype, group,
                                   scale_mode=1 if scale_form == "recip" else 0)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("scale_form", ["ieee", "recip"])
@pytest.mark.parametrize("shape", CONVROT_SHAPES)
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_convrot_quant_fused_route_bit_exact(dtype, shape, scale_form):
    """Fused rotation + quantization (group 256): codes and scales bit for bit
    against the oracle, outlier-heavy rows included."""
    m, k = shape
    x = make_x(m, k, dtype, seed=71 + k, dist="student_t")
    _convrot_check(x.to(DEV), dtype, 256, scale_form)


def test_convrot_quant_full_size_bit_exact():
    """11712 tokens x 3072 channels (the DiT block's activation), bf16."""
    x = make_x(11712, 3072, "bf16", seed=73, dist="student_t")
    _convrot_check(x.to(DEV), "bf16", 256, "ieee")


@pytest.mark.parametrize("k", [3072, 16384])
def test_convrot_quant_unaligned_input_bit_exact(k):
    """An input that is not 16-byte aligned takes the row-in-LDS kernel."""
    m = 3
    x = make_x(m, k, "bf16", seed=75)
    buf = torch.empty(m * k + 1, dtype=torch.bfloat16, device=DEV)
    buf[1:] = x.reshape(-1).to(DEV)
    _convrot_check(buf[1:].view(m, k), "bf16", 256, "recip")


CONVROT_ROTATE_CASES = [(7, 256, 4), (7, 1024, 16), (5, 3072, 64), (3, 16640, 256), (2, 4096, 1024),
                        (3, 48, 16), (4, 16640, 64), (2, 768, 256)]


@pytest.mark.parametrize("m,k,group", CONVROT_ROTATE_CASES)
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_convrot_rotate_bit_exact(dtype, m, k, group):
    x = make_x(m, k, dtype, seed=91 + group)
    y = W.convrot_rotate(x.to(DEV), group)
    assert np.array_equal(storage(y, dtype), O.convrot_rotate(storage(x, dtype), dtype, group))


@pytest.mark.parametrize("m,k,group", [(4, 256, 64), (3, 16640, 256), (5, 1024, 16)])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_convrot_quant_rotate_route_bit_exact(dtype, m, k, group):
    x = make_x(m, k, dtype, seed=97 + k, dist="student_t")
    _convrot_check(x.to(DEV), dtype, group, "recip")


@pytest.mark.parametrize("m,n,k", [(300, 512, 3072), (2, 1536, 3072), (1, 640, 4096), (64, 256, 16640)])
def test_operator_convrot_equals_quantizer_then_linear(m, n, k):
    """The ConvRot operator is the ConvRot quantizer followed by the GEMM/GEMV
    with its epilogue, bit for bit, residual included."""
    x = make_x(m, k, "bf16", seed=101).to(DEV)
    w = make_w(n, k, seed=102).to(DEV)
    ws = (torch.rand(n, generator=torch.Generator().manual_seed(103)) * 9e-3 + 1e-3).to(DEV)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(104)) * 0.02).to(torch.bfloat16).to(DEV)
    resid, rscale = _residual_inputs(m, n, "bf16", 105)
    resid, rscale = resid.to(DEV), rscale.to(DEV)
    out = W.int8_linear(x, w, ws, bias, torch.bfloat16, convrot=True, convrot_groupsize=256,
                        residual=resid, residual_scale=rscale)
    q, s = W.quantize_rowwise_convrot(x, 256)
    if W.route(m, k, n) == "gemm":
        want = W.gemm_dequant_residual(q, w, s, ws, bias, torch.bfloat16, resid, rscale)
    else:
        want = W.gemv_dequant_residual(q, w, s, ws, bias, torch.bfloat16, resid, rscale)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


# ---------------------------------------------------------------- operator vs reference payloads


def _run_fixture(c, ops, scale_form, fused, convrot=False):
    xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
    x = from_storage(O.to_dtype(ops["x"], xd), xd)
    w = torch.from_numpy(ops["weight"]).to(DEV)
    ws = torch.from_numpy(np.asarray(ops["scale"])).to(DEV)
    bias = None if ops["bias"] is None else torch.from_numpy(np.asarray(ops["bias"])).to(DEV)
    r = None if ops["residual"] is None else torch.from_numpy(np.asarray(ops["residual"])).to(DEV)
    rs = None if ops["residual_scale"] is None else torch.from_numpy(np.asarray(ops["residual_scale"])).to(DEV)
    out = W.int8_linear(x, w, ws, bias, TD[od], convrot=convrot, convrot_groupsize=c.get("group", 256),
                        input_act=c.get("activation"), residual=r, residual_scale=rs, scale_form=scale_form,
                        fused_quant=fused)
    assert list(out.shape) == c["output_shape"]
    return storage(out, od).reshape(-1), FX.payload(c, od)


@pytest.mark.parametrize("section", sorted(FX.SECTIONS))
@pytest.mark.parametrize("scale_form", ["ieee", "recip"])
def test_operator_reproduces_reference_cuda_payloads(section, scale_form):
    n = 0
    for c, ops in FX.linear_cases(section):
        got, want = _run_fixture(c, ops, scale_form, fused=False)
        assert np.array_equal(got, want), c
        n += 1
    assert n > 100


@pytest.mark.parametrize("section", ["cuda_int8_gemm", "cuda_int8_gemv", "cuda_int8_m1"])
@pytest.mark.parametrize("fused", [False, True])
def test_operator_reproduces_reference_residual_payloads(section, fused):
    """Residual modes (fused, unaligned residual / scale, eager fallback) through
    the operator, residual fused into the epilogue (or, with the fused
    quantizer, applied by the residual kernel)."""
    n = 0
    for c, ops in FX.linear_cases(section, residual=True):
        got, want = _run_fixture(c, ops, "ieee", fused=fused)
        assert np.array_equal(got, want), c
        n += 1
    assert n >= 36


@pytest.mark.parametrize("section", ["cuda_int8_gemm", "cuda_int8_gemv", "cuda_int8_m1", "cuda_int8_activation"])
def test_operator_reproduces_reference_convrot_payloads(section):
    """ConvRot cases without an input activation, with and without a residual,
    through the operator with the CUDA scale form: bit for bit, except fp32
    inputs off the fused route (the reference rotates those with a library
    GEMM whose summation order is not restated), which agree within 2^-7."""
    exact = close = 0
    for residual in (False, True):
        for c, ops in FX.linear_cases(section, residual=residual, convrot=True):
            if c.get("activation"):
                continue
            got, want = _run_fixture(c, ops, "recip", fused=False, convrot=True)
            od = OP.dtype_name(c["output_dtype"])
            if OP.dtype_name(c["dtype"]) == "f32" and not O.convrot_fused_route(c["shape"][-1], c["group"]):
                a, b = O.to_f32(got, od).astype(np.float64), O.to_f32(want, od).astype(np.float64)
                assert np.abs(a - b).max() <= 2.0**-7 * np.abs(b).max(), c
                close += 1
            else:
                assert np.array_equal(got, want), c
                exact += 1
    assert exact >= 60


def test_operator_fused_quant_reproduces_gemm_payloads():
    n = 0
    for c, ops in FX.linear_cases("cuda_int8_gemm"):
        got, want = _run_fixture(c, ops, "ieee", fused=True)
        assert np.array_equal(got, want), c
        n += 1
    assert n > 100


def test_operator_error_cases_match_reference_classes():
    n = 0
    for section in ("cuda_int8_gemm", "cuda_int8_gemv", "cuda_int8_m1"):
        for c, ops in FX.linear_cases(section, with_errors=True):
            xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
            x = from_storage(O.to_dtype(ops["x"], xd), xd)
            w = torch.from_numpy(ops["weight"]).to(DEV)
            ws = torch.from_numpy(np.asarray(ops["scale"])).to(DEV)
            r = None if ops["residual"] is None else torch.from_numpy(ops["residual"]).to(DEV)
            rs = None if ops["residual_scale"] is None else torch.from_numpy(ops["residual_scale"]).to(DEV)
            exc = {"ValueError": ValueError, "RuntimeError": RuntimeError}[c["error"]]
            with pytest.raises(exc) as info:
                W.int8_linear(x, w, ws, None, TD[od], residual=r, residual_scale=rs)
            # Messages are compared for the reference's default policy (CUTLASS
            # enabled); with COMFY_KITCHEN_DISABLE_CUTLASS the reference reports a
            # bad GEMM scale from its cuBLAS dequant instead (same class).
            if not c.get("disable_cutlass"):
                assert str(info.value)[:48] == c["message"][:48], (c, str(info.value))
            n += 1
    assert n > 100
