"""The C-ABI library loads, exports every symbol include/w8a8.h declares, and
rejects invalid arguments before touching the GPU (no device needed)."""
import ctypes
import re
from pathlib import Path

import pytest

from imagine_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "w8a8.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(w8a8_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_workspace_size():
    lib = _lib.load()
    assert b"gfx950" in lib.w8a8_version()
    assert lib.w8a8_int8_linear_workspace_bytes(11712, 3072) == 11712 * 3072 + 4 * 11712
    assert lib.w8a8_int8_linear_workspace_bytes(3, 5) == 256 + 12
    assert lib.w8a8_int8_linear_workspace_bytes(-1, 5) == -1


def test_noalloc_entry_rejects_inputs_beyond_its_scratch_before_touching_memory():
    lib = _lib.load()
    assert lib.w8a8_int8_linear_noalloc_max_bytes() == 64 << 20
    rc = lib.w8a8_int8_linear_noalloc(None, 2, None, None, 1, None, None, 2, 16384, 64, 4096, 0, None)
    assert rc == _lib.ERR_VALUE
    assert "fixed scratch of 67108864 bytes" in lib.w8a8_last_error().decode()


def test_kitchen_bridge_exports_the_bridge_symbols_and_rejects_unknown_names():
    """libimagine_kitchen.so loads like the crate loads its bridge and answers
    an unknown name with the bridge's code and text (no device touched)."""
    bridge = ctypes.CDLL(str(_lib.LIB_PATH.parent / "libimagine_kitchen.so"), mode=ctypes.RTLD_LOCAL)
    text = re.sub(r"/\*.*?\*/", "", (HEADER.parent / "imagine_kitchen.h").read_text(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(imagine_[a-z_]+)\s*\(", text)))
    assert declared == ["imagine_kitchen_call", "imagine_last_accelerator_code", "imagine_last_error",
                        "imagine_last_metadata"]
    for name in declared:
        assert hasattr(bridge, name), name
    bridge.imagine_kitchen_call.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_size_t,
                                            ctypes.POINTER(ctypes.c_int64)]
    bridge.imagine_last_error.restype = ctypes.c_char_p
    out = ctypes.c_int64(0)
    assert bridge.imagine_kitchen_call(b"no_such_kernel", None, 0, ctypes.byref(out)) == -1
    assert bridge.imagine_last_error() == b"Unknown Kitchen kernel"
    assert bridge.imagine_kitchen_call(b"cutlass_int8_dequant", None, 0, ctypes.byref(out)) == -1
    assert bridge.imagine_last_error() == b"Kernel argument count mismatch"


def _err(rc):
    return rc, _lib.load().w8a8_last_error().decode()


def test_argument_errors_return_reference_codes_and_messages():
    lib = _lib.load()
    # negative dimension -> ValueError code
    assert _err(lib.w8a8_quantize_rowwise(None, 2, None, None, -1, 4, 0, None))[0] == _lib.ERR_VALUE
    # unknown flag bits
    assert _err(lib.w8a8_quantize_rowwise(None, 2, None, None, 1, 4, 1 << 30, None))[0] == _lib.ERR_VALUE
    # bad dtype code
    rc, msg = _err(lib.w8a8_quantize_rowwise(None, 7, None, None, 1, 4, 0, None))
    assert rc == _lib.ERR_RUNTIME and "dtype" in msg
    # GEMV: M must be 1 or 2 (dlpack_bindings.cpp:3545-3547)
    rc, msg = _err(lib.w8a8_gemv_dequant(None, None, None, None, 1, None, None, 2, 3, 4, 16, 0, None))
    assert rc == _lib.ERR_RUNTIME and msg == "INT8 GEMV dequant expects M == 1 or M == 2"
    # GEMV: weight scale size
    rc, msg = _err(lib.w8a8_gemv_dequant(None, None, None, None, 3, None, None, 2, 2, 4, 16, 0, None))
    assert msg == "INT8 GEMV weight scale must be scalar or per-output-channel"
    # operator: GEMM route needs K % 4 == 0 (cublas_gemm_int8.cu:161)
    rc, msg = _err(lib.w8a8_int8_linear(None, 2, None, None, 1, None, None, 2, 4, 16, 15, 0, None, 0, None))
    assert rc == _lib.ERR_RUNTIME and msg.startswith("INT8 GEMM not supported on this GPU")
    # operator: workspace too small
    rc, msg = _err(lib.w8a8_int8_linear(None, 2, None, None, 1, None, None, 2, 4, 16, 64, 0, None, 10, None))
    assert rc == _lib.ERR_VALUE and "workspace" in msg
    # residual entries: a residual without its scale (int8_linear.rs:107), a
    # scale of neither 1 nor N entries, and an output activation with a residual
    buf = ctypes.c_void_p(16)  # never dereferenced: every call below fails its checks first
    rc, msg = _err(lib.w8a8_gemm_dequant_residual(None, None, None, None, 1, None, None, 1, buf, None, 2,
                                                  4, 8, 64, 0, None))
    assert rc == _lib.ERR_VALUE and msg == "residual requires residual_scale"
    rc, msg = _err(lib.w8a8_gemm_dequant_residual(None, None, None, None, 1, None, buf, 3, buf, None, 2,
                                                  4, 8, 64, 0, None))
    assert rc == _lib.ERR_RUNTIME and "residual_scale" in msg
    rc, _ = _err(lib.w8a8_gemv_dequant_residual(None, None, None, None, 1, None, buf, 1, buf, None, 2,
                                                1, 8, 64, _lib.ACT_GELU_TANH, None))
    assert rc == _lib.ERR_VALUE
    rc, msg = _err(lib.w8a8_residual_apply(buf, None, buf, 1, 2, 4, 8, None))
    assert rc == _lib.ERR_VALUE and msg == "residual requires residual_scale"
    rc, msg = _err(lib.w8a8_int8_linear_residual(None, 2, None, None, 1, None, buf, 5, buf, None, 2, 4, 8,
                                                 64, 0, None, 0, None))
    assert rc == _lib.ERR_RUNTIME and "residual_scale" in msg
    # ConvRot groups: a power of 4 (int8_utils.rs:36-46) that divides K (:60-73)
    for group in (0, 2, 8, 32, 48, -4):
        rc, msg = _err(lib.w8a8_convrot_rotate(buf, 2, buf, 2, 256, group, None))
        assert rc == _lib.ERR_VALUE and msg == f"Regular Hadamard size must be a power of 4, got {group}"
    rc, msg = _err(lib.w8a8_quantize_rowwise_convrot(buf, 2, buf, buf, 2, 336, 64, 0, None, 0, None))
    assert rc == _lib.ERR_VALUE and msg == "features 336 not divisible by group_size 64"
    rc, msg = _err(lib.w8a8_quantize_rowwise_convrot(buf, 2, buf, buf, 2, 256, 64, 0, None, 0, None))
    assert rc == _lib.ERR_VALUE and "rotated buffer" in msg  # off the fused route it needs the buffer
    rc, _ = _err(lib.w8a8_int8_linear_convrot(buf, 2, buf, buf, 1, None, None, 0, None, buf, 2, 4, 8, 256, 256,
                                              _lib.ACT_GELU_TANH, buf, 1 << 20, None))
    assert rc == _lib.ERR_VALUE
    assert lib.w8a8_convrot_workspace_bytes(4, 3072, 256, 2) == 0
    assert lib.w8a8_convrot_workspace_bytes(4, 16640, 256, 2) == 4 * 16640 * 2
    assert lib.w8a8_convrot_workspace_bytes(4, 256, 64, 0) == 4 * 256 * 4
    assert lib.w8a8_int8_linear_convrot_workspace_bytes(3, 256, 64, 2) == 768 + 256 + 3 * 256 * 2
    # empty outputs are a no-op success, nothing launched
    assert lib.w8a8_gemm_dequant(None, None, None, None, 1, None, None, 2, 0, 16, 64, 0, None) == 0
    assert lib.w8a8_quantize_rowwise(None, 2, None, None, 0, 64, 0, None) == 0


def test_check_maps_codes_to_reference_exception_classes():
    lib = _lib.load()
    lib.w8a8_quantize_rowwise(None, 2, None, None, -1, 4, 0, None)
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_VALUE)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_RUNTIME)
    with pytest.raises(IndexError):
        _lib.check(_lib.ERR_INDEX)


def test_route_selection_matches_reference_selectors():
    """cuda_int8_m1_selection fixtures + the GEMV/GEMM predicates."""
    from imagine_amd.ops import route
    from tests.golden import fixtures as FX
    for c in FX.load()["cuda_int8_m1_selection"]:
        if c["convrot"]:
            continue
        m, k = c["shape"][0], c["shape"][-1]
        assert (route(m, k, c["n"]) == "m1") == c["native_m1_called"], c
    assert route(2, 3072, 18432) == "gemv"
    assert route(1, 2564, 4) == "gemv"
    assert route(2, 20, 16) == "gemm"
    assert route(11712, 3072, 12288) == "gemm"
