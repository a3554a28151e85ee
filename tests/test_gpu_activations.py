"""GPU parity of the linear's input activations (SwiGLU, SiTU, RMSNorm, and
GELU on the ConvRot route) against the oracle, and the operator against the
reference's activation payloads.

Bar: the eager activations (the crate's ATen op chains, int8_linear.rs:37-97)
and everything downstream of them bit for bit against the oracle, every
dtype; the fused ConvRot route (Kitchen's kernel, int8_linear.cu:1175-1262)
bit for bit against the oracle's restatement.  Against the reference's own
payloads: 16-bit inputs on the eager route bit for bit; fp32 inputs there
within 4e-6 (ATen's vector exp / tanh); the fused ConvRot route within 4e-4
of the largest output (Kitchen compiles it with fast-math exp / tanh / rsqrt,
which no fixture pins), 16-bit RMSNorm there bit for bit.
"""
import numpy as np
import pytest
import torch

import imagine_amd as W
from oracle import oracle as O
from tests.golden import fixtures as FX
from tests.golden import operands as OP

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    W._lib.load()
    yield
    torch.cuda.synchronize()


def storage(t, dtype):
    t = t.detach().cpu().contiguous()
    return t.numpy() if dtype == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def from_storage(a, dtype, device=DEV):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype != "f32":
        t = t.view(torch.int16).view(TD[dtype])
    return t.to(device)


def gated_rows(dtype, seed):
    """[gate | up] rows: every finite 16-bit gate with fixed up values, every
    up value with fixed gates, and random pairs (fp32: random only)."""
    g = torch.Generator().manual_seed(seed)
    ra = (torch.randn(8192, generator=g) * 20).to(TD[dtype])
    rb = (torch.randn(8192, generator=g) * 5).to(TD[dtype])
    pairs = [(storage(ra, dtype), storage(rb, dtype))]
    if dtype != "f32":
        bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
        bits = bits[np.isfinite(O.to_f32(bits, dtype))]
        for v in (1.0, -1.5, 3.25):
            fixed = np.full(bits.shape, O.to_dtype(np.float32([v]), dtype)[0], np.uint16)
            pairs += [(bits, fixed), (fixed, bits)]
    rows = []
    width = 256
    for a, b in pairs:
        n = (len(a) // width) * width
        a2, b2 = a[:n].reshape(-1, width), b[:n].reshape(-1, width)
        rows.append(np.concatenate([a2, b2], axis=1))
    return np.concatenate(rows)


@pytest.mark.parametrize("act", ["swiglu", "situ"])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_gated_input_act_bit_exact(act, dtype):
    rows = gated_rows(dtype, seed=3)
    y = W.input_act(from_storage(rows, dtype), act)
    assert np.array_equal(storage(y, dtype), O.input_act(rows, dtype, act))


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("k", [64, 3072, 12288])
def test_rms_norm_input_act_bit_exact(dtype, k):
    g = torch.Generator().manual_seed(k)
    x = (torch.randn(33, k, generator=g) * 4).to(TD[dtype])
    w = (1 + 0.3 * torch.randn(k, generator=g)).to(TD[dtype])
    y = W.input_act(x.to(DEV), "rms_norm", w.to(DEV), 1e-6)
    assert np.array_equal(storage(y, dtype), O.input_act(storage(x, dtype), dtype, "rms_norm", storage(w, dtype), 1e-6))


@pytest.mark.parametrize("act", ["gelu_tanh", "swiglu", "situ", "rms_norm"])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_quantize_with_input_act_bit_exact(act, dtype):
    """The activation fused into the per-token quantizer (no ConvRot): codes
    and scales of act(x) bit for bit."""
    m, k = 40, 3072
    width = 2 * k if act in ("swiglu", "situ") else k
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(m, width, generator=g) * 2).to(TD[dtype])
    w = (1 + 0.3 * torch.randn(k, generator=g)).to(TD[dtype]) if act == "rms_norm" else None
    q, s = W.quantize_rowwise_act(x.to(DEV), act, None if w is None else w.to(DEV), 1e-6)
    xa = O.input_act(storage(x, dtype), dtype, act, None if w is None else storage(w, dtype), 1e-6)
    q_ref, s_ref = O.quant_rowwise(xa, dtype)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("act", ["gelu_tanh", "swiglu", "situ", "rms_norm"])
@pytest.mark.parametrize("group,k", [(256, 3072), (256, 256), (64, 1024)], ids=["fused3072", "fused256", "rotate64"])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_convrot_quantize_with_input_act_bit_exact(act, group, k, dtype):
    """ConvRot with an input activation, both routes: the fused one (the
    activation in fp32 inside the rotation) and the rotate one (eager
    activation, rotation in the dtype, plain quantizer), against the oracle."""
    m = 9
    width = 2 * k if act in ("swiglu", "situ") else k
    g = torch.Generator().manual_seed(group + k)
    x = (torch.randn(m, width, generator=g) * 2).to(TD[dtype])
    w = (1 + 0.3 * torch.randn(k, generator=g)).to(TD[dtype]) if act == "rms_norm" else None
    q, s = W.quantize_rowwise_act(x.to(DEV), act, None if w is None else w.to(DEV), 1e-6, convrot_group=group,
                                  scale_form="recip")
    q_ref, s_ref = O.convrot_quant_act(storage(x, dtype), dtype, group, act, None if w is None else storage(w, dtype),
                                       1e-6, scale_mode=1)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_ffn_down_with_swiglu_at_dit_width_sampled_rows():
    """The reference DiT's FFN-down form (dit.rs:327-336): int8_linear on a
    [M, 2 * 12288] SwiGLU input, M = 600 (the GEMM route), against the oracle
    chain on sampled rows."""
    m, k, n = 600, 12288, 3072
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(m, 2 * k, device=DEV, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=g)
    ws = torch.rand(n, device=DEV, generator=g) * 9e-3 + 1e-3
    b = (torch.randn(n, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    out = W.int8_linear(x, w, ws, b, torch.bfloat16, input_act="swiglu")
    rows = np.array([0, 1, 77, 300, 599])
    xa = O.input_act(storage(x[rows], "bf16"), "bf16", "swiglu")
    q_ref, s_ref = O.quant_rowwise(xa, "bf16")
    want = O.epilogue_kitchen(O.gemm_i32(q_ref, w.cpu().numpy()), s_ref, ws.cpu().numpy(), storage(b, "bf16"), "bf16")
    assert np.array_equal(storage(out[rows], "bf16"), want)


# ---------------------------------------------------------------- the reference's payloads


def _run_case(c):
    ops = OP.activation_operands(c)
    xd, od = OP.dtype_name(c["dtype"]), OP.dtype_name(c["output_dtype"])
    x = from_storage(O.to_dtype(ops["x"], xd), xd)
    w = torch.from_numpy(ops["weight"]).to(DEV)
    ws = torch.from_numpy(np.asarray(ops["scale"])).to(DEV)
    bias = None if ops["bias"] is None else torch.from_numpy(np.asarray(ops["bias"])).to(DEV)
    r = None if ops["residual"] is None else torch.from_numpy(np.asarray(ops["residual"])).to(DEV)
    rs = None if ops["residual_scale"] is None else torch.from_numpy(np.asarray(ops["residual_scale"])).to(DEV)
    act = c.get("activation")
    aw = None
    if act == "rms_norm" and c["mode"] != "missing_norm_weight":
        aw = torch.ones(c["shape"][-1], dtype=TD[xd], device=DEV)
    out = W.int8_linear(x, w, ws, bias, TD[od], convrot=c["convrot"], convrot_groupsize=c["group"], input_act=act,
                        input_act_weight=aw, input_act_eps=0.0, residual=r, residual_scale=rs, scale_form="recip")
    return out, od


def test_operator_reproduces_reference_activation_payloads():
    counts = {"exact": 0, "fp32_close": 0, "fused_close": 0}
    for c in FX.load()["cuda_int8_activation"]:
        act = c.get("activation")
        if "error" in c or act is None or (act == "gelu_tanh" and not c["convrot"]):
            continue
        out, od = _run_case(c)
        assert list(out.shape) == c["output_shape"]
        got, want = storage(out, od).reshape(-1), FX.payload(c, od)
        if np.array_equal(got, want):
            counts["exact"] += 1
            continue
        fused = c["convrot"] and O.convrot_fused_route(c["weight_k"], c["group"])
        xd = OP.dtype_name(c["dtype"])
        a, b = O.to_f32(got, od).astype(np.float64), O.to_f32(want, od).astype(np.float64)
        err = np.abs(a - b).max() / np.abs(b).max()
        if fused:
            assert not (act == "rms_norm" and xd != "f32"), c
            assert err <= 4e-4, (c, err)
            counts["fused_close"] += 1
        else:
            assert xd == "f32", c
            assert err <= 4e-6, (c, err)
            counts["fp32_close"] += 1
    print(counts)
    assert counts["exact"] >= 500, counts


def test_operator_missing_norm_weight_errors_match_reference():
    n = 0
    for c in FX.load()["cuda_int8_activation"]:
        if c.get("mode") != "missing_norm_weight":
            continue
        exc = {"ValueError": ValueError, "RuntimeError": RuntimeError}[c["error"]]
        with pytest.raises(exc) as info:
            _run_case(c)
        assert str(info.value) == c["message"], (c, str(info.value))
        n += 1
    assert n == 126
