"""Pin the oracle (CPU restatement) before trusting it.

Every oracle function is checked against (a) the reference's own golden vectors
and (b) independent facts: numpy/torch CPU rounding, brute-force integer
arithmetic, the LibTorch-CPU op sequence the reference's CPU route issues.
Several checks are run against a deliberately wrong variant too, to show the
check can tell the difference.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_eager as TE
from tests.golden import fixtures as FX
from tests.golden import operands as OP

TORCH_DTYPE = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _to_torch(storage, dtype):
    t = torch.from_numpy(np.ascontiguousarray(storage))
    return t if dtype == "f32" else t.view(torch.int16).view(TORCH_DTYPE[dtype])


def _storage(t, dtype):
    t = t.contiguous()
    return t.numpy() if dtype == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def _tie_patterns(low_bits):
    """All float32 bit patterns whose low bits below the 16-bit mantissa cut
    equal one of the given values (ties, just below/above ties, exact)."""
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    pats = np.concatenate([hi | np.uint32(v) for v in low_bits])
    return pats.view(np.float32)


# ---------------------------------------------------------------- rounding


def test_f16_rounding_matches_numpy_on_all_tie_classes():
    vals = _tie_patterns([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF])
    vals = vals[np.isfinite(vals)]
    ours = O.to_dtype(vals, "f16")
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_bf16_rounding_matches_torch_on_all_tie_classes():
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    pats = np.concatenate([hi | np.uint32(v) for v in (0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF)])
    vals = pats.view(np.float32)
    vals = vals[np.isfinite(vals)]
    ours = O.to_dtype(vals, "bf16")
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------- quantizer


def test_quant_matches_reference_rowwise_golden_vectors():
    """reference_primitives.py:357-365: eager rowwise quant, CPU and CUDA devices,
    zero first row.  CPU captures need the IEEE scale; CUDA-device eager captures
    are reproduced by both forms on this data."""
    n = 0
    for c in FX.load()["int8_rowwise"]:
        if c["seed"] is not None:
            continue
        xd = OP.dtype_name(c["dtype"])
        x = O.to_dtype(OP.quantizer_x_primitives(), xd)
        q, s = O.quant_rowwise(x, xd, scale_mode=0)
        assert q.view(np.uint8).reshape(-1).tolist() == c["payload"], c
        assert s.view(np.uint8).tolist() == c["scale"], c
        n += 1
    assert n == 6


def test_tensorwise_quant_matches_reference_golden_vectors():
    """reference_primitives.py:357-365: eager tensorwise quant (CPU and CUDA
    devices) with a recalculated, a zero and an explicit scale; a zero scale
    divides by the dtype's tiny, saturating every nonzero code."""
    n = 0
    for c in FX.load()["int8_tensorwise"]:
        xd = OP.dtype_name(c["dtype"])
        x = O.to_dtype(OP.quantizer_x_primitives(), xd)
        given = {"recalculate": None, "zero": 0.0, "explicit": 0.03125}[c["scale_mode"]]
        q, s = O.quant_tensorwise(x, xd, scale=given, scale_mode=0)
        assert q.view(np.uint8).reshape(-1).tolist() == c["payload"], c
        assert np.array([s], np.float32).view(np.uint8).tolist() == c["scale"], c
        n += 1
    assert n == 36


def test_quant_matches_reference_cuda_kernel_golden_vectors():
    """reference_primitives.py:388-391: Kitchen's quantize_int8_rowwise kernel."""
    cases = [c for c in FX.load()["native_int8_rowwise"] if c["seed"] is None]
    assert len(cases) == 3
    for c in cases:
        xd = OP.dtype_name(c["dtype"])
        q, s = O.quant_rowwise(O.to_dtype(OP.quantizer_x_native(), xd), xd, scale_mode=1)
        assert q.view(np.uint8).reshape(-1).tolist() == c["payload"]
        assert s.view(np.uint8).tolist() == c["scale"]


def _student_t_outliers(m, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.distributions.StudentT(3.0).sample((m, k)) if False else None
    # StudentT.sample has no generator argument; build t(3) from normals instead.
    z = torch.randn(m, k, generator=g)
    chi = torch.randn(m, k, 3, generator=g).pow(2).sum(-1)
    x = z / torch.sqrt(chi / 3.0)
    idx = torch.randperm(k, generator=g)[: max(1, k // 1000)]
    x[:, idx] *= 50.0
    return x


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("dist", ["normal", "student_t"])
def test_quant_bit_exact_vs_libtorch_cpu_sequence(dtype, dist):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(64, 3072, generator=g) if dist == "normal" else _student_t_outliers(64, 3072, 7)
    x[3] = 0.0  # zero row exercises the 1e-30 clamp and the tiny substitution
    xt = x.to(TORCH_DTYPE[dtype])
    q_ref, s_ref = TE.quantize_rowwise(xt)
    storage = xt.numpy() if dtype == "f32" else xt.view(torch.int16).numpy().view(np.uint16)
    q, s = O.quant_rowwise(storage, dtype, scale_mode=0)
    assert np.array_equal(q, q_ref.numpy())
    assert np.array_equal(s.view(np.uint32), s_ref.reshape(-1).numpy().view(np.uint32))


def test_quant_scale_forms_are_distinguished():
    """The IEEE form and the reciprocal-multiply form differ on real data; the
    LibTorch-CPU check above must fail for the wrong one."""
    x = torch.randn(256, 512, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    _, s_ref = TE.quantize_rowwise(x)
    _, s_wrong = O.quant_rowwise(x.view(torch.int16).numpy().view(np.uint16), "bf16", scale_mode=1)
    assert not np.array_equal(s_wrong.view(np.uint32), s_ref.reshape(-1).numpy().view(np.uint32))


def test_quant_with_gelu_input_act_vs_libtorch_cpu():
    x = torch.randn(32, 1024, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    xa = torch.nn.functional.gelu(x, approximate="tanh")
    q_ref, s_ref = TE.quantize_rowwise(xa)
    q, s = O.quant_rowwise(x.view(torch.int16).numpy().view(np.uint16), "bf16", act=1)
    # gelu's tanh may differ by one fp32 ulp between libm and ATen's vector tanh;
    # after bf16 rounding that almost never shows; require >= 99.99% exact codes.
    assert (q != q_ref.numpy()).mean() < 1e-4
    assert np.array_equal(s.view(np.uint32), s_ref.reshape(-1).numpy().view(np.uint32))


# ---------------------------------------------------------------- GEMM


def test_gemm_i32_brute_force_including_extremes():
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, size=(7, 37), dtype=np.int64).astype(np.int8)
    b = rng.integers(-128, 128, size=(5, 37), dtype=np.int64).astype(np.int8)
    a[0, :] = -128
    b[0, :] = -128
    c = O.gemm_i32(a, b)
    ref = [[sum(int(a[i, k]) * int(b[j, k]) for k in range(37)) for j in range(5)] for i in range(7)]
    assert c.tolist() == ref
    assert c[0, 0] == 37 * 128 * 128


def test_gemm_i32_matches_reference_int8_mm_golden_vectors():
    n = 0
    for c in FX.load()["int8_mm"]:
        if "error" in c or c["m"] * c["n"] == 0:
            continue
        a, b = OP.int8_mm_operands(c["m"], c["k"], c["n"])
        got = O.gemm_i32(a, np.ascontiguousarray(b.T))
        assert got.reshape(-1).view(np.uint8).tolist() == c["payload"]
        n += 1
    assert n == 18


def test_gemm_i32_matches_torch_int_mm():
    g = torch.Generator().manual_seed(5)
    a = torch.randint(-128, 128, (48, 256), generator=g, dtype=torch.int8)
    b = torch.randint(-128, 128, (40, 256), generator=g, dtype=torch.int8)
    ref = torch._int_mm(a, b.t().contiguous())
    assert np.array_equal(O.gemm_i32(a.numpy(), b.numpy()), ref.numpy())


# ---------------------------------------------------------------- epilogues


@pytest.mark.parametrize("section", sorted(FX.SECTIONS))
def test_kitchen_route_linear_matches_reference_cuda_payloads(section):
    """Quantize -> int32 GEMM -> single-rounding epilogue reproduces every
    no-residual, non-ConvRot Kitchen CUDA payload (GEMM, GEMV, M=1 and
    input-activation routes; fp32/fp16/bf16 inputs and outputs)."""
    n = 0
    for c, ops in FX.linear_cases(section):
        xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
        x = O.to_dtype(ops["x"], xd)
        x2 = x.reshape(-1, x.shape[-1])
        ws = np.asarray(ops["scale"], np.float32).reshape(-1)
        bias = None if ops["bias"] is None else O.to_dtype(np.asarray(ops["bias"], np.float32), od)
        act = 1 if c.get("activation") == "gelu_tanh" else 0
        out, _, _, _ = O.linear_kitchen(x2, xd, ops["weight"], ws, bias, od, input_act=act)
        assert np.array_equal(out.reshape(-1), FX.payload(c, od)), c
        n += 1
    assert n > 100


def _residual_case_outputs(section, contract):
    """(got, want) per residual-mode CUDA case: the composed route, then the
    residual step with the given rounding (oracle w8o_residual)."""
    for c, ops in FX.linear_cases(section, residual=True):
        xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
        x = O.to_dtype(ops["x"], xd)
        x2 = x.reshape(-1, x.shape[-1])
        ws = np.asarray(ops["scale"], np.float32).reshape(-1)
        bias = None if ops["bias"] is None else O.to_dtype(np.asarray(ops["bias"], np.float32), od)
        out, _, _, _ = O.linear_kitchen(x2, xd, ops["weight"], ws, bias, od)
        r = O.to_dtype(np.asarray(ops["residual"], np.float32).reshape(out.shape), od)
        s = O.to_dtype(np.asarray(ops["residual_scale"], np.float32).reshape(-1), od)
        yield c, O.residual(out, r, s, od, contract=contract).reshape(-1), FX.payload(c, od)


@pytest.mark.parametrize("section", ["cuda_int8_gemm", "cuda_int8_gemv", "cuda_int8_m1"])
def test_residual_matches_reference_cuda_payloads(section):
    """O(fma(O(lin), rscale, resid)) reproduces every residual-mode payload of
    the reference (fused CUTLASS residual, unaligned residual / scale, and the
    eager fallback on the GEMM, GEMV and M=1 routes)."""
    n = 0
    for c, got, want in _residual_case_outputs(section, contract=1):
        assert np.array_equal(got, want), c
        n += 1
    assert n >= 36


def test_residual_rounding_form_is_distinguished():
    """The payloads tell the single-fma residual from a rounded product: the
    fp32-output cases fail with the product rounded before the add."""
    mismatched = sum(not np.array_equal(got, want)
                     for _, got, want in _residual_case_outputs("cuda_int8_gemm", contract=0))
    assert mismatched > 0


def test_eager_route_linear_matches_reference_eager_payloads():
    """reference_int8_linear.py: eager int8_linear on CPU (IEEE scale) and on a
    CUDA device (torch's CUDA division by a scalar multiplies by the reciprocal,
    so those captures need the reciprocal scale form)."""
    seen = {"cpu": 0, "cuda:0": 0}
    for c in FX.load()["eager_int8_linear"]:
        if "error" in c or c["mode"] not in ("plain", "gelu_tanh"):
            continue
        ops = OP.eager_linear_operands(c)
        xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
        x = O.to_dtype(ops["x"], xd)
        mode = 0 if c["device"] == "cpu" else 1
        q, xs = O.quant_rowwise(x.reshape(-1, x.shape[-1]), xd, scale_mode=mode,
                                act=1 if c["mode"] == "gelu_tanh" else 0)
        out = O.epilogue_eager(O.gemm_i32(q, ops["weight"]), xs, ops["scale"].astype(np.float32), None, od)
        assert np.array_equal(out.reshape(-1), FX.payload(c, od)), c
        seen[c["device"]] += 1
    assert seen == {"cpu": 12, "cuda:0": 12}


def test_eager_epilogue_bit_exact_vs_libtorch_cpu_with_bias():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(33, 320, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (70, 320), generator=g, dtype=torch.int8)
    ws = torch.rand(70, generator=g) * 9e-3 + 1e-3
    bias = (torch.randn(70, generator=g) * 0.02).to(torch.bfloat16)
    out_ref, q_ref, xs_ref, acc_ref = TE.int8_linear(x, w, ws, bias, torch.bfloat16)
    q, xs = O.quant_rowwise(x.view(torch.int16).numpy().view(np.uint16), "bf16")
    acc = O.gemm_i32(q, w.numpy())
    assert np.array_equal(acc, acc_ref.numpy())
    out = O.epilogue_eager(acc, xs, ws.numpy(), bias.float().numpy(), "bf16")
    assert np.array_equal(out, out_ref.view(torch.int16).numpy().view(np.uint16))
    # The GPU-route single rounding differs from the eager double rounding
    # somewhere, by at most one bf16 ulp at the magnitude of the larger of the
    # result and the pre-bias value (the eager route rounds that one first).
    single = O.epilogue_kitchen(acc, xs, ws.numpy(), bias.view(torch.int16).numpy().view(np.uint16), "bf16")
    pre = O.epilogue_eager(acc, xs, ws.numpy(), None, "f32")
    a, b = O.to_f32(single, "bf16"), O.to_f32(out, "bf16")
    mag = np.maximum(np.abs(b), np.abs(pre))
    assert (np.abs(a - b) <= mag * 2.0**-7).all()
    assert (single != out).any()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_gelu_tanh_equals_aten_on_every_16bit_value_outside_the_saturated_tail(dtype):
    """Every finite bf16 / fp16 input: the oracle's gelu_tanh equals ATen's
    gelu(approximate="tanh") bit for bit, except in the negative tail where
    1 + tanh(u) is one fp32 ulp or zero.  There ATen's vector tanh saturates
    to -1 a little earlier than the correctly rounded tanh (u ~ -8.7, x in
    [-5.2, -5.0]), giving -0.0 where the oracle gives about -1.5e-7; both are
    below 2^-22 in magnitude."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = O.to_f32(bits, dtype)
    bits = bits[np.isfinite(vals)]
    vals = O.to_f32(bits, dtype)
    ours = O.gelu_tanh(bits, dtype)
    ref = torch.nn.functional.gelu(_to_torch(bits, dtype), approximate="tanh")
    ref = ref.view(torch.int16).numpy().view(np.uint16)
    diff = ours != ref
    assert diff.sum() <= 32
    assert ((vals[diff] > -5.2) & (vals[diff] < -5.0)).all()
    assert (np.abs(O.to_f32(ours[diff], dtype)) < 2.0**-22).all()
    assert (O.to_f32(ref[diff], dtype) == 0).all()


def test_tanh_is_correctly_rounded_against_long_double():
    """The oracle's tanh is the fp32 nearest the true tanh: checked against an
    independent 80-bit long double evaluation (numpy longdouble) over every
    argument gelu_tanh forms from a bf16 or fp16 input, plus 2^20 random fp32
    arguments.  Only arguments whose true value lies within 2^-40 relative of
    a rounding midpoint could be decided differently; none occur."""
    args = []
    for dt in ("bf16", "f16"):
        bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
        x = O.to_f32(bits, dt)
        x = x[np.isfinite(x)]
        with np.errstate(all="ignore"):
            inner = np.float32(1.41421356237309504880 * 1.12837916709551257390 * 0.5) * (
                x + np.float32(0.044715) * (x * x * x))
        args.append(inner[np.isfinite(inner)])
    rng = np.random.default_rng(5)
    args.append((rng.standard_normal(1 << 20) * 4).astype(np.float32))
    u = np.concatenate(args)
    got = np.array([O.lib().w8o_tanh_cr(float(v)) for v in u[:: max(1, len(u) // 200000)]], np.float32)
    u = u[:: max(1, len(u) // 200000)]
    ld = np.tanh(u.astype(np.longdouble))
    want = ld.astype(np.float32)   # one rounding from 64-bit significands
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- ConvRot


def _hadamard_f64(G):
    """int8_utils.rs:21-58 restated in float64: Kronecker powers of H4 over sqrt(G)."""
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.float64)
    h = h4
    while h.shape[0] < G:
        h = np.kron(h, h4)
    return h / np.sqrt(G)


@pytest.mark.parametrize("G", [4, 16, 64, 256, 1024])
def test_convrot_stages_equal_dense_hadamard_matmul(G):
    """The radix-4 stage order computes x . H_G: against a float64 dense
    product (fp32 rounding only), H_G orthogonal and symmetric, and rotating
    twice gives x back."""
    rng = np.random.default_rng(G)
    x = rng.standard_normal((5, 2 * G)).astype(np.float32)
    h = _hadamard_f64(G)
    assert np.allclose(h @ h.T, np.eye(G), atol=1e-12) and np.array_equal(h, h.T)
    want = (x.astype(np.float64).reshape(5, 2, G) @ h).reshape(5, 2 * G)
    got = O.convrot_rotate(x, "f32", G)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    back = O.convrot_rotate(got, "f32", G)
    assert np.abs(back - x).max() <= 1e-5 * np.abs(x).max()


def test_convrot_stage_sign_rows_are_distinguished():
    """A one-hot row picks out one row of H_256: the signs, positions and scale
    of every output are those of the dense matrix (a transposed H4 or a wrong
    stride fails here)."""
    h = _hadamard_f64(256)
    for i in (0, 1, 5, 17, 100, 255):
        x = np.zeros((1, 256), np.float32)
        x[0, i] = 1.0
        assert np.array_equal(O.convrot_rotate(x, "f32", 256)[0], h[i].astype(np.float32))


def test_convrot_route_predicate_matches_reference_native_calls():
    """The fused route is taken exactly where the reference's captures called
    quantize_int8_rowwise_convrot64 (GEMM and GEMV sections)."""
    n = 0
    for section in ("cuda_int8_gemm", "cuda_int8_gemv"):
        for c in FX.load()[section]:
            if not c.get("convrot") or "error" in c or not c.get("native_calls"):
                continue
            names = [nc["name"] if isinstance(nc, dict) else nc for nc in c["native_calls"]]
            fused = "quantize_int8_rowwise_convrot64" in names
            assert O.convrot_fused_route(c["shape"][-1], c["group"]) == fused, c
            n += 1
    assert n > 200


def _convrot_case_outputs(section, scale_mode, residual):
    for c, ops in FX.linear_cases(section, residual=residual, convrot=True):
        if c.get("activation"):
            continue
        xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
        x = O.to_dtype(ops["x"], xd)
        x2 = x.reshape(-1, x.shape[-1])
        ws = np.asarray(ops["scale"], np.float32).reshape(-1)
        bias = None if ops["bias"] is None else O.to_dtype(np.asarray(ops["bias"], np.float32), od)
        out, _, _, _ = O.linear_kitchen(x2, xd, ops["weight"], ws, bias, od, scale_mode=scale_mode,
                                        convrot_group=c["group"])
        if residual:
            r = O.to_dtype(np.asarray(ops["residual"], np.float32).reshape(out.shape), od)
            s = O.to_dtype(np.asarray(ops["residual_scale"], np.float32).reshape(-1), od)
            out = O.residual(out, r, s, od)
        yield c, xd, od, out.reshape(-1), FX.payload(c, od)


def _library_summed_case(c, xd):
    """fp32 inputs off the fused route: the reference rotates with its GEMM
    library (x @ H in fp32), whose summation order is not restated here."""
    return xd == "f32" and not O.convrot_fused_route(c["shape"][-1], c["group"])


@pytest.mark.parametrize("section", ["cuda_int8_gemm", "cuda_int8_gemv", "cuda_int8_m1",
                                     "cuda_int8_activation"])
def test_convrot_linear_matches_reference_cuda_payloads(section):
    """Every ConvRot payload without an input activation (with and without a
    residual) bit for bit, with the CUDA scale form; fp32 inputs off the fused
    route agree within 2^-7 relative (their rotation is a library GEMM)."""
    exact = close = 0
    for residual in (False, True):
        for c, xd, od, got, want in _convrot_case_outputs(section, 1, residual):
            if _library_summed_case(c, xd):
                a, b = O.to_f32(got, od).astype(np.float64), O.to_f32(want, od).astype(np.float64)
                assert np.abs(a - b).max() <= 2.0**-7 * np.abs(b).max(), c
                close += 1
            else:
                assert np.array_equal(got, want), c
                exact += 1
    assert exact >= 60


def test_convrot_scale_form_is_distinguished_on_the_rotate_route():
    """The 16-bit rotate-route payloads need the CUDA scale form amax*(1/127):
    the IEEE form misses some of them, while the fused route matches both."""
    misses = {True: 0, False: 0}
    for c, xd, od, got, want in _convrot_case_outputs("cuda_int8_gemm", 0, False):
        if xd == "f32":
            continue
        misses[O.convrot_fused_route(c["shape"][-1], c["group"])] += not np.array_equal(got, want)
    assert misses[True] == 0 and misses[False] > 0


# ---------------------------------------------------------------- input activations


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_input_act_swiglu_and_situ_equal_aten_op_chains(dtype):
    """The eager SwiGLU and SiTU (int8_linear.rs:44-75) against the ATen op
    chains the crate issues, on every 16-bit gate value (with a few up values)
    and on random pairs: bit for bit."""
    td = {"bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    bits = bits[np.isfinite(O.to_f32(bits, dtype))]
    g = torch.Generator().manual_seed(12)
    rand_a = (torch.randn(50000, generator=g) * 20).to(td).view(torch.int16).numpy().view(np.uint16)
    rand_b = (torch.randn(50000, generator=g) * 5).to(td).view(torch.int16).numpy().view(np.uint16)
    for ups in (1.0, -1.5, 3.25):
        up = np.full(bits.shape, O.to_dtype(np.float32([ups]), dtype)[0], np.uint16)
        pairs = [(bits, up), (up, bits), (rand_a, rand_b)]
        for a, b in pairs:
            at, bt = _to_torch(a, dtype), _to_torch(b, dtype)
            sw = (torch.nn.functional.silu(at) * bt).view(torch.int16).numpy().view(np.uint16)
            gated = (bt / 4.).tanh_().mul_(4.).mul_(bt.sigmoid())
            si = (at / 25.).tanh_().mul_(25.).mul_(gated).view(torch.int16).numpy().view(np.uint16)
            row = np.concatenate([a, b])[None, :]
            assert np.array_equal(O.input_act(row, dtype, "swiglu")[0], sw)
            assert np.array_equal(O.input_act(row, dtype, "situ")[0], si)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_input_act_rms_norm_within_one_ulp_of_aten(dtype):
    """rms_norm with a weight (int8_linear.rs:77-95) against ATen's: within one
    ulp for 16-bit outputs, two for fp32 (ATen sums the squares in fp32 in its
    own order; the oracle's mean is the exactly rounded one), mostly
    bit-equal."""
    td = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    g = torch.Generator().manual_seed(13)
    x = (torch.randn(64, 3072, generator=g) * 3).to(td)
    w = (1 + 0.2 * torch.randn(3072, generator=g)).to(td)
    ref = torch.nn.functional.rms_norm(x, [3072], w, 1e-6)
    got = O.input_act(_storage(x, dtype), dtype, "rms_norm", _storage(w, dtype), 1e-6)
    a = O.to_f32(got, dtype).astype(np.float64)
    b = ref.float().numpy().astype(np.float64)
    rel = {"bf16": 2.0**-7, "f16": 2.0**-10, "f32": 2.0**-21}[dtype]   # fp32: two ulps (rsqrt rounding)
    assert (np.abs(a - b) <= np.abs(b) * rel).all()
    assert (got.reshape(-1) == _storage(ref, dtype).reshape(-1)).mean() > (0.97 if dtype != "f32" else 0.7)


def _activation_chain(c, ops):
    """The crate's route for an activation case (cuda_linear.rs:450-481,586-619)
    on the oracle, CUDA scale form."""
    xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
    act, k, n, group = c.get("activation"), c["weight_k"], c["n"], c["group"]
    x = O.to_dtype(ops["x"].reshape(-1, ops["x"].shape[-1]), xd)
    weight = O.to_dtype(np.ones(k, np.float32), xd) if act == "rms_norm" else None
    if c["convrot"]:
        q, s = O.convrot_quant_act(x, xd, group, act, weight, 0.0, scale_mode=1)
    else:
        q, s = O.quant_rowwise(O.input_act(x, xd, act, weight, 0.0) if act else x, xd, scale_mode=1)
    acc = O.gemm_i32(q, ops["weight"])
    bias = None if ops["bias"] is None else O.to_dtype(ops["bias"], od)
    out = O.epilogue_kitchen(acc, s, ops["scale"].astype(np.float32), bias, od)
    if ops["residual"] is not None:
        out = O.residual(out, O.to_dtype(ops["residual"].reshape(-1, n), od), O.to_dtype(ops["residual_scale"], od), od)
    return out.reshape(-1), FX.payload(c, od), od


def test_activation_payloads_reproduce_on_the_oracle():
    """The reference's swiglu / situ / rms_norm / gelu CUDA payloads
    (plain and bias + residual modes), routed as the crate routes them:
      * eager route (no ConvRot, or ConvRot off its fused route), 16-bit
        inputs: every case bit for bit;
      * fp32 inputs on the eager route: ATen's vectorised exp / tanh differ
        from the correctly rounded ones in the last bits: within 4e-6;
      * the fused ConvRot route: Kitchen's kernel uses fast-math exp / tanh /
        rsqrt (parity unpinned there): 16-bit RMSNorm bit for bit, the rest
        within 4e-4 of the largest output."""
    counts = {"exact": 0, "fp32_close": 0, "fused_close": 0}
    for c in FX.load()["cuda_int8_activation"]:
        if "error" in c or c.get("activation") is None:
            continue
        got, want, od = _activation_chain(c, OP.activation_operands(c))
        fused = c["convrot"] and O.convrot_fused_route(c["weight_k"], c["group"])
        xd = OP.dtype_name(c["dtype"])
        if np.array_equal(got, want):
            counts["exact"] += 1
            continue
        a, b = O.to_f32(got, od).astype(np.float64), O.to_f32(want, od).astype(np.float64)
        err = np.abs(a - b).max() / np.abs(b).max()
        if fused:
            assert not (c["activation"] == "rms_norm" and xd != "f32"), c
            assert err <= 4e-4, (c, err)
            counts["fused_close"] += 1
        else:
            assert xd == "f32", c
            assert err <= 4e-6, (c, err)
            counts["fp32_close"] += 1
    assert counts["exact"] >= 600, counts
