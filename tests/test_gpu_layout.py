"""GPU parity of the weight quantizers (tensorwise, ConvRot weight) against
the oracle, and the checkpoint loader end to end: from_float -> safetensors ->
load -> int8_linear."""
import numpy as np
import pytest
import torch

import imagine_amd as W
from imagine_amd import layout as L
from oracle import oracle as O
from tests.test_gpu_parity import DEV, TD, make_x, storage

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    W._lib.load()
    yield
    torch.cuda.synchronize()


@pytest.mark.parametrize("given", [None, 0.0, 0.03125])
@pytest.mark.parametrize("shape", [(12288, 3072), (37, 1001), (3, 8), (1, 1)])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_tensorwise_quant_bit_exact(dtype, shape, given):
    x = make_x(*shape, dtype, seed=11 + shape[1], dist="student_t")
    q, s = W.quantize_tensorwise(x.to(DEV), scale=given)
    q_ref, s_ref = O.quant_tensorwise(storage(x, dtype), dtype, scale=given)
    assert np.float32(s.item()).view(np.uint32) == np.float32(s_ref).view(np.uint32)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_tensorwise_quant_unaligned_and_recip_form():
    m, k = 5, 3000
    x = make_x(m, k, "bf16", seed=13)
    buf = torch.empty(m * k + 1, dtype=torch.bfloat16, device=DEV)
    buf[1:] = x.reshape(-1).to(DEV)
    q, s = W.quantize_tensorwise(buf[1:].view(m, k), scale_form="recip")
    q_ref, s_ref = O.quant_tensorwise(storage(x, "bf16"), "bf16", scale_mode=1)
    assert s.item() == s_ref and np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("n,k,group", [(64, 3072, 256), (32, 16640, 256), (8, 20480, 256), (4, 65536, 256),
                                       (48, 1024, 64), (16, 768, 16)])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_convrot_weight_quant_bit_exact(dtype, n, k, group):
    """Weights take the fused numerics for group 256 at any K (the reference's
    Rowwise64 / Staged weight paths), the rotate route otherwise."""
    w = make_x(n, k, dtype, seed=17 + k)
    q, s = W.quantize_convrot_weight(w.to(DEV), group)
    q_ref, s_ref = O.convrot_quant_weight(storage(w, dtype), dtype, group)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("convrot,per_channel", [(True, True), (False, True), (False, False)])
def test_from_float_save_load_linear(tmp_path, convrot, per_channel):
    """A bf16 weight through from_float, a safetensors file and the loader
    gives the same layer output as the in-memory weight, and that output
    equals the oracle's linear on the oracle's quantized weight."""
    n, k, m = 192, 768, 40
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(21)) * 0.05).to(torch.bfloat16)
    x = make_x(m, k, "bf16", seed=22)
    layer = L.from_float(w.to(DEV), per_channel=per_channel, convrot=convrot)
    path = tmp_path / "w.safetensors"
    L.save_checkpoint(path, {"blk.fc.": layer})
    loaded = L.load_checkpoint(path, DEV, torch.bfloat16)["blk.fc."].weight
    assert loaded.convrot == convrot
    out = loaded.linear(x.to(DEV))
    assert torch.equal(out.view(torch.int16), layer.linear(x.to(DEV)).view(torch.int16))
    ws = storage(w, "bf16")
    if convrot:
        qw, sw = O.convrot_quant_weight(ws, "bf16", 256)
    elif per_channel:
        qw, sw = O.quant_rowwise(ws, "bf16")
    else:
        qw, s1 = O.quant_tensorwise(ws, "bf16")
        sw = np.array([s1], np.float32)
    want, _, _, _ = O.linear_kitchen(storage(x, "bf16"), "bf16", qw, sw, None, "bf16",
                                     convrot_group=256 if convrot else 0)
    assert np.array_equal(storage(out, "bf16"), want)
