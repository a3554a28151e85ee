"""GPU parity of every GEMM main loop, and of the full-size GEMMs the benchmark
and the DiT step run, against the oracle.

Each main loop (W8A8_GEMM_TILE_*) is requested explicitly and the test checks
through w8a8_gemm_config that it is the one that ran; the full-size shapes
check that the automatic choice is the main loop the benchmark's figures are
quoted for.  Codes, scales, int32 accumulators and every epilogue output
(GELU included) are compared bit for bit.  Full-size shapes compare sampled rows (the first, the last and random ones)
and check the whole output is finite.
"""
import numpy as np
import pytest
import torch

import imagine_amd as W
from imagine_amd import _lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    L.load()
    yield
    torch.cuda.synchronize()


def storage(t, dtype):
    t = t.detach().cpu().contiguous()
    if dtype == "f32":
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def dev_gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def dev_x(m, k, seed, scale=1.0):
    return (torch.randn(m, k, device=DEV, generator=dev_gen(seed)) * scale).to(torch.bfloat16)


def dev_w(n, k, seed):
    return torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=dev_gen(seed))


def dev_scales(n, seed):
    return torch.rand(n, device=DEV, generator=dev_gen(seed)) * 9e-3 + 1e-3


def sample_rows(m, count, seed):
    rows = np.sort(np.random.default_rng(seed).choice(m, count, replace=False))
    rows[0], rows[-1] = 0, m - 1
    return rows


# ---------------------------------------------------------------- every main loop

TILES = [L.TILE_256x192, L.TILE_256x256, L.TILE_384x192, L.TILE_256x128, L.TILE_REGS, L.TILE_GENERIC]
MODES = ["bf16", "bf16_gelu", "f16_gelu", "f16", "f32", "f32_gelu", "bf16_residual", "f16_residual", "int32"]


@pytest.mark.parametrize("shape", [(600, 800, 512), (300, 260, 256)], ids=["staged", "direct"])
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("tile", TILES, ids=lambda t: L.TILE_NAMES[t])
def test_every_main_loop_bit_exact(tile, mode, shape):
    """Each main loop, requested through its flag, on a shape every main loop
    takes (K a multiple of 128; ragged last tiles in M and N), against the
    oracle on the whole output.  N = 800 takes the LDS-staged epilogue of the
    DMA main loops, N = 260 (not a multiple of 8) their direct one."""
    m, n, k = shape
    assert W.gemm_config(m, n, k, tile) == L.TILE_NAMES[tile]
    odt = {"int32": "f32"}.get(mode, mode.split("_")[0])
    x = dev_x(m, k, seed=1, scale=1.5)
    w = dev_w(n, k, seed=2)
    ws = dev_scales(n, seed=3)
    bias = (torch.randn(n, device=DEV, generator=dev_gen(4)) * 0.5).to(TD[odt])
    q, xs = W.quantize_rowwise(x)
    qh, xsh = q.cpu().numpy(), xs.cpu().numpy().reshape(-1)
    acc = O.gemm_i32(qh, w.cpu().numpy())
    if mode == "int32":
        got = W.gemm_i32(q, w, tile=tile)
        assert np.array_equal(got.cpu().numpy(), acc)
        return
    if mode.endswith("_residual"):
        g = dev_gen(5)
        resid = (torch.randn(m, n, device=DEV, generator=g) * 2).to(TD[odt])
        rscale = (torch.rand(n, device=DEV, generator=g) + 0.25).to(TD[odt])
        got = W.gemm_dequant_residual(q, w, xs, ws, bias, TD[odt], resid, rscale, tile=tile)
        lin = O.epilogue_kitchen(acc, xsh, ws.cpu().numpy(), storage(bias, odt), odt)
        want = O.residual(lin, storage(resid, odt), storage(rscale, odt), odt)
    else:
        gelu = mode.endswith("_gelu")
        got = W.gemm_dequant(q, w, xs, ws, bias, TD[odt], gelu=gelu, tile=tile)
        want = O.epilogue_kitchen(acc, xsh, ws.cpu().numpy(), storage(bias, odt), odt, act=1 if gelu else 0)
    assert np.array_equal(storage(got, odt), want)


PERSIST_MODES = ["bf16", "bf16_gelu", "f16", "f16_gelu", "bf16_residual", "f16_residual"]


@pytest.mark.parametrize("mode", PERSIST_MODES)
@pytest.mark.parametrize("tile", [L.TILE_256x256, L.TILE_256x192], ids=lambda t: L.TILE_NAMES[t])
def test_persistent_tile_loop_bit_exact(tile, mode):
    """The main loops that loop over output tiles (one block per CU), on a
    shape with more tiles than the GPU has CUs (306 and 396 tiles; ragged
    last tiles in M and N), so blocks take a second tile after their first
    epilogue: every output mode, 48 sampled rows (all columns) against the
    oracle."""
    m, n, k = 4100, 4392, 256
    assert W.gemm_config(m, n, k, tile) == L.TILE_NAMES[tile]
    odt = mode.split("_")[0]
    x = dev_x(m, k, seed=31, scale=1.5)
    w = dev_w(n, k, seed=32)
    ws = dev_scales(n, seed=33)
    bias = (torch.randn(n, device=DEV, generator=dev_gen(34)) * 0.5).to(TD[odt])
    q, xs = W.quantize_rowwise(x)
    rows = sample_rows(m, 48, seed=35)
    qh, xsh = q[rows].cpu().numpy(), xs.cpu().numpy().reshape(-1)[rows]
    acc = O.gemm_i32(qh, w.cpu().numpy())
    if mode.endswith("_residual"):
        g = dev_gen(36)
        resid = (torch.randn(m, n, device=DEV, generator=g) * 2).to(TD[odt])
        rscale = (torch.rand(n, device=DEV, generator=g) + 0.25).to(TD[odt])
        got = W.gemm_dequant_residual(q, w, xs, ws, bias, TD[odt], resid, rscale, tile=tile)
        lin = O.epilogue_kitchen(acc, xsh, ws.cpu().numpy(), storage(bias, odt), odt)
        want = O.residual(lin, storage(resid[rows], odt), storage(rscale, odt), odt)
    else:
        gelu = mode.endswith("_gelu")
        got = W.gemm_dequant(q, w, xs, ws, bias, TD[odt], gelu=gelu, tile=tile)
        want = O.epilogue_kitchen(acc, xsh, ws.cpu().numpy(), storage(bias, odt), odt, act=1 if gelu else 0)
    assert np.array_equal(storage(got[rows], odt), want)


def test_requested_tile_falls_back_when_k_does_not_fit():
    """A 128-byte-K-tile main loop requested for K = 192 runs the 64-byte one;
    K = 48 runs the register-staged loop; K = 13 the generic kernel."""
    assert W.gemm_config(512, 512, 192, L.TILE_256x256) == "256x128"
    assert W.gemm_config(512, 512, 48, L.TILE_256x192) == "regs"
    assert W.gemm_config(512, 512, 13, L.TILE_384x192) == "generic"


# ---------------------------------------------------------------- full-size shapes

# (name, M, K, N, GELU epilogue, main loop the automatic choice must take)
FULL = [
    ("ffn_up_M11712", 11712, 3072, 12288, True, "256x256"),
    ("qkv_M11712", 11712, 3072, 9216, False, "384x192"),
    ("out_M11712", 11712, 3072, 3072, False, "384x192"),
    ("ffn_down_M11712", 11712, 12288, 3072, False, "384x192"),
    ("qkv_M19904", 19904, 3072, 9216, False, "256x256"),
    ("ffn_up_M19904", 19904, 3072, 12288, True, "256x256"),
    ("out_M19904", 19904, 3072, 3072, False, "256x256"),
    ("ffn_down_M19904", 19904, 12288, 3072, False, "256x256"),
]


@pytest.mark.parametrize("name,m,k,n,gelu,tile", FULL, ids=[f[0] for f in FULL])
def test_full_size_gemm_sampled_rows_bit_exact(name, m, k, n, gelu, tile):
    """The block linear set at M = 11712 (the benchmark's workload) and at
    M = 19904 (the DiT step's): quantize, then the GEMM with bias (and the
    GELU epilogue for FFN-up) on the automatically chosen main loop; codes,
    scales and outputs of 40 sampled rows bit for bit against the oracle."""
    assert W.gemm_config(m, n, k, gelu=gelu) == tile
    x = dev_x(m, k, seed=11)
    w = dev_w(n, k, seed=12)
    ws = dev_scales(n, seed=13)
    bias = (torch.randn(n, device=DEV, generator=dev_gen(14)) * 0.02).to(torch.bfloat16)
    q, xs = W.quantize_rowwise(x)
    out = W.gemm_dequant(q, w, xs, ws, bias, torch.bfloat16, gelu=gelu)
    rows = sample_rows(m, 40, seed=m + n)
    xr = storage(x[rows], "bf16")
    q_ref, xs_ref = O.quant_rowwise(xr, "bf16")
    assert np.array_equal(q[rows].cpu().numpy(), q_ref)
    assert np.array_equal(xs[rows].cpu().numpy().reshape(-1).view(np.uint32), xs_ref.view(np.uint32))
    acc = O.gemm_i32(q_ref, w.cpu().numpy())
    want = O.epilogue_kitchen(acc, xs_ref, ws.cpu().numpy(), storage(bias, "bf16"), "bf16", act=1 if gelu else 0)
    assert np.array_equal(storage(out[rows], "bf16"), want)
    assert torch.isfinite(out.float()).all()


def test_dit_block_ffn_chain_M19904_sampled_rows_bit_exact():
    """The FFN half of a DiT block at M = 19904 (2 x (5600 + 4096 + 256)
    tokens): fused modulated norm + quantizer -> FFN-up GEMM with the GELU
    epilogue (256 x 256 tiles) -> quantizer -> FFN-down GEMM (256 x 256 tiles)
    -> gated residual.  The oracle follows the same chain on 24 sampled rows
    from the library's codes of each stage: GEMM + epilogue + GELU,
    requantization of the whole 12288-wide row, second GEMM, gated residual,
    every value bit for bit."""
    B, T, D, F, prefix = 2, 9952, 3072, 12288, 256
    g = dev_gen(21)
    x = torch.randn(B, T, D, device=DEV, generator=g).to(torch.bfloat16)
    mod = [(torch.randn(B, 1, D, device=DEV, generator=g) * 0.3).to(torch.bfloat16) for _ in range(6)]
    w_up, w_down = dev_w(F, D, seed=22), dev_w(D, F, seed=23)
    ws_up, ws_down = dev_scales(F, seed=24), dev_scales(D, seed=25)
    b_up = (torch.randn(F, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    b_down = (torch.randn(D, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    zero = torch.zeros(B, 1, D, device=DEV, dtype=torch.bfloat16)
    q2, s2 = W.modulated_norm_quant(x, (mod[0], mod[1]), prefix, zero, 1e-6)
    assert W.gemm_config(B * T, F, D, gelu=True) == "256x256"
    assert W.gemm_config(B * T, D, F) == "256x256"
    up = W.gemm_dequant(q2, w_up, s2, ws_up, b_up, torch.bfloat16, gelu=True)
    q3, s3 = W.quantize_rowwise(up)
    down = W.gemm_dequant(q3, w_down, s3, ws_down, b_down, torch.bfloat16)
    gate = (mod[2], mod[3])
    res = W.gated_residual(x.clone(), down.view(B, T, D), gate, prefix)
    rows = sample_rows(B * T, 24, seed=7)
    q2h, s2h = q2[rows].cpu().numpy(), s2[rows].cpu().numpy().reshape(-1)
    acc = O.gemm_i32(q2h, w_up.cpu().numpy())
    up_ref = O.epilogue_kitchen(acc, s2h, ws_up.cpu().numpy(), storage(b_up, "bf16"), "bf16", act=1)
    up_rows = storage(up[rows], "bf16")
    assert np.array_equal(up_rows, up_ref)
    q3_ref, s3_ref = O.quant_rowwise(up_rows, "bf16")
    assert np.array_equal(s3[rows].cpu().numpy().reshape(-1).view(np.uint32), s3_ref.view(np.uint32))
    assert np.array_equal(q3[rows].cpu().numpy(), q3_ref)
    acc2 = O.gemm_i32(q3_ref, w_down.cpu().numpy())
    down_ref = O.epilogue_kitchen(acc2, s3_ref, ws_down.cpu().numpy(), storage(b_down, "bf16"), "bf16")
    assert np.array_equal(storage(down[rows], "bf16"), down_ref)
    # gated residual: x + down * gate, gate0 for tokens < prefix (per batch row)
    xr = storage(x.reshape(B * T, D)[rows], "bf16")
    gates = np.stack([storage(gate[0].reshape(B, D), "bf16"), storage(gate[1].reshape(B, D), "bf16")])
    bt = rows // T
    tt = rows % T
    gsel = gates[(tt >= prefix).astype(int), bt]
    want = O.gated_residual(xr, down_ref, gsel, "bf16")
    assert np.array_equal(storage(res.reshape(B * T, D)[rows], "bf16"), want)
