"""The scratch-free operator entry, w8a8_int8_linear_noalloc, through the C ABI
against w8a8_int8_linear with a caller-allocated workspace: bit for bit, on
calls in a row whose later inputs are smaller (stale scratch contents from an
earlier call would show), over the GEMM and GEMV routes and the flags it
takes; and the size limit it enforces."""
import pytest
import torch

from imagine_amd import _lib as L

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def lib():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return L.load()


def _operands(m, k, n, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=g)
    ws = torch.rand(n, device=DEV, generator=g) * 9e-3 + 1e-3
    b = (torch.randn(n, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    return x, w, ws, b


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("flags", [0, L.ACT_GELU_TANH, L.SCALE_RECIP], ids=["plain", "gelu_input", "recip"])
def test_noalloc_equals_workspace_entry_on_calls_in_a_row(lib, flags):
    # GEMM route, then a smaller GEMM, then the M = 2 and M = 1 GEMV routes
    shapes = [(640, 3072, 1536), (37, 3072, 1536), (2, 3072, 1536), (1, 3072, 1536)]
    for i, (m, k, n) in enumerate(shapes):
        x, w, ws, b = _operands(m, k, n, seed=10 + i)
        got = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
        want = torch.empty_like(got)
        L.check(lib.w8a8_int8_linear_noalloc(x.data_ptr(), L.BF16, w.data_ptr(), ws.data_ptr(), n, b.data_ptr(),
                                             got.data_ptr(), L.BF16, m, n, k, flags, _stream()))
        need = lib.w8a8_int8_linear_workspace_bytes(m, k)
        buf = torch.empty(need + 256, device=DEV, dtype=torch.uint8)
        off = (-buf.data_ptr()) % 256
        L.check(lib.w8a8_int8_linear(x.data_ptr(), L.BF16, w.data_ptr(), ws.data_ptr(), n, b.data_ptr(),
                                     want.data_ptr(), L.BF16, m, n, k, flags, buf.data_ptr() + off, need, _stream()))
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (m, k, n, flags)


def test_noalloc_rejects_inputs_beyond_its_scratch(lib):
    cap = lib.w8a8_int8_linear_noalloc_max_bytes()
    assert cap == 64 << 20
    m, k, n = 16384, 4096, 64  # codes alone are exactly the scratch size; the scales do not fit
    assert lib.w8a8_int8_linear_workspace_bytes(m, k) > cap
    x, w, ws, b = _operands(1, 16, n, seed=1)   # never read: the size check comes first
    out = torch.empty(1, n, device=DEV, dtype=torch.bfloat16)
    rc = lib.w8a8_int8_linear_noalloc(x.data_ptr(), L.BF16, w.data_ptr(), ws.data_ptr(), n, b.data_ptr(),
                                      out.data_ptr(), L.BF16, m, n, k, 0, _stream())
    assert rc == L.ERR_VALUE
    assert "fixed scratch" in lib.w8a8_last_error().decode()
    # the largest input that fits runs (M x K codes plus scales within 64 MiB)
    m, k, n = 16000, 4096, 256
    assert lib.w8a8_int8_linear_workspace_bytes(m, k) <= cap
    x, w, ws, b = _operands(m, k, n, seed=2)
    got = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    L.check(lib.w8a8_int8_linear_noalloc(x.data_ptr(), L.BF16, w.data_ptr(), ws.data_ptr(), n, b.data_ptr(),
                                         got.data_ptr(), L.BF16, m, n, k, 0, _stream()))
    want = torch.empty_like(got)
    need = lib.w8a8_int8_linear_workspace_bytes(m, k)
    buf = torch.empty(need + 256, device=DEV, dtype=torch.uint8)
    off = (-buf.data_ptr()) % 256
    L.check(lib.w8a8_int8_linear(x.data_ptr(), L.BF16, w.data_ptr(), ws.data_ptr(), n, b.data_ptr(),
                                 want.data_ptr(), L.BF16, m, n, k, 0, buf.data_ptr() + off, need, _stream()))
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
