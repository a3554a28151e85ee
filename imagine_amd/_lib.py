"""ctypes binding of libw8a8_hip.so (the C ABI declared in include/w8a8.h).

The library is built in-tree by ``imagine_amd/build.py``.  Loading fails
loudly when it is missing: there is no fallback implementation.
"""
import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libw8a8_hip.so"

F32, F16, BF16 = 0, 1, 2
OK, ERR_RUNTIME, ERR_OOM, ERR_ACCELERATOR, ERR_VALUE, ERR_INDEX = 0, -1, -9, -10, -20, -21
SCALE_RECIP = 1 << 0
ACT_GELU_TANH = 1 << 1
OUT_INT32 = 1 << 2
FUSED_QUANT = 1 << 3
ROUTE_GEMM = 1 << 4
GIVEN_SCALE = 1 << 5
# input activation codes
ACT_CODES = {None: 0, "gelu_tanh": 1, "swiglu": 2, "rms_norm": 3, "situ": 4}
# w8a8_adaln mode bits
ADALN_RMS, ADALN_SINGLE_ROUNDING = 1, 2
# GEMM main loops (flag bits 8..11: GEMM_TILE(code))
TILE_AUTO, TILE_256x192, TILE_256x256, TILE_384x192, TILE_256x128, TILE_REGS, TILE_GENERIC = range(7)
TILE_NAMES = {TILE_AUTO: "auto", TILE_256x192: "256x192", TILE_256x256: "256x256", TILE_384x192: "384x192",
              TILE_256x128: "256x128", TILE_REGS: "regs", TILE_GENERIC: "generic"}


def GEMM_TILE(code):
    return code << 8

# Every symbol include/w8a8.h declares, with (restype, argtypes).
_p, _i, _i64, _u32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32
SIGNATURES = {
    "w8a8_last_error": (ctypes.c_char_p, []),
    "w8a8_last_accelerator_code": (_i, []),
    "w8a8_version": (ctypes.c_char_p, []),
    "w8a8_quantize_rowwise": (_i, [_p, _i, _p, _p, _i64, _i64, _u32, _p]),
    "w8a8_row_scales": (_i, [_p, _i, _p, _i64, _i64, _u32, _p]),
    "w8a8_input_act": (_i, [_p, _i, _i, _p, ctypes.c_double, _p, _i64, _i64, _p]),
    "w8a8_quantize_rowwise_act": (_i, [_p, _i, _i, _p, ctypes.c_double, _p, _p, _i64, _i64, _i64, _u32, _p, _i64, _p]),
    "w8a8_int8_linear_act": (_i, [_p, _i, _i, _p, ctypes.c_double, _p, _p, _i64, _p, _p, _i64, _p, _p, _i, _i64, _i64,
                                  _i64, _i64, _u32, _p, _i64, _p]),
    "w8a8_gemv_dequant": (_i, [_p, _p, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64, _u32, _p]),
    "w8a8_gemm_dequant": (_i, [_p, _p, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64, _u32, _p]),
    "w8a8_gemm_config": (_i, [_i64, _i64, _i64, _u32]),
    "w8a8_gemm_dequant_xq": (_i, [_p, _i, _p, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64, _u32, _p]),
    "w8a8_dequantize_linear": (_i, [_p, _p, _p, _i64, _p, _p, _i, _i64, _i64, _u32, _p]),
    "w8a8_int8_linear_workspace_bytes": (_i64, [_i64, _i64]),
    "w8a8_int8_linear": (_i, [_p, _i, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64, _u32, _p, _i64, _p]),
    "w8a8_int8_linear_noalloc_max_bytes": (_i64, []),
    "w8a8_int8_linear_noalloc": (_i, [_p, _i, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64, _u32, _p]),
    "w8a8_gemm_dequant_residual": (_i, [_p, _p, _p, _p, _i64, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64,
                                        _u32, _p]),
    "w8a8_gemv_dequant_residual": (_i, [_p, _p, _p, _p, _i64, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64,
                                        _u32, _p]),
    "w8a8_residual_apply": (_i, [_p, _p, _p, _i64, _i, _i64, _i64, _p]),
    "w8a8_int8_linear_residual": (_i, [_p, _i, _p, _p, _i64, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64,
                                       _u32, _p, _i64, _p]),
    "w8a8_convrot_rotate": (_i, [_p, _i, _p, _i64, _i64, _i64, _p]),
    "w8a8_convrot_workspace_bytes": (_i64, [_i64, _i64, _i64, _i]),
    "w8a8_quantize_rowwise_convrot": (_i, [_p, _i, _p, _p, _i64, _i64, _i64, _u32, _p, _i64, _p]),
    "w8a8_int8_linear_convrot_workspace_bytes": (_i64, [_i64, _i64, _i64, _i]),
    "w8a8_int8_linear_convrot": (_i, [_p, _i, _p, _p, _i64, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64, _i64,
                                      _u32, _p, _i64, _p]),
    "w8a8_quantize_tensorwise": (_i, [_p, _i, _p, _p, _i64, _u32, _p]),
    "w8a8_convrot_weight_workspace_bytes": (_i64, [_i64, _i64, _i64, _i]),
    "w8a8_quantize_convrot_weight": (_i, [_p, _i, _p, _p, _i64, _i64, _i64, _u32, _p, _i64, _p]),
    "w8a8_adaln": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, ctypes.c_double, _i, _i, _p]),
    "w8a8_gated_residual": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, _p]),
    "w8a8_rms_rope": (_i, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i, ctypes.c_double, _i, _p]),
    "w8a8_apply_rope": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i, _i, _p]),
    "w8a8_modulated_norm_quant": (_i, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, ctypes.c_double, _i,
                                       _i, _u32, _p]),
    "w8a8_quantize_rowwise_modulated": (_i, [_p, _i, _p, _p, _p, _i64, _i64, _u32, _p]),
    "w8a8_int8_linear_modulated": (_i, [_p, _i, _p, _p, _p, _i64, _p, _p, _i, _i64, _i64, _i64, _u32, _p, _i64,
                                        _p]),
}

_lib = None


class W8A8Error(RuntimeError):
    """Accelerator or runtime failure reported by the library (code != 0)."""

    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


def load(path=None):
    """Load the library (once) and declare every exported signature."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} is not built: run `python -m imagine_amd.build` (hipcc, gfx950). "
            "The W8A8 path has no CPU fallback.")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(rc):
    """Map a return code to the exception class the reference raises for it."""
    if rc == OK:
        return
    msg = load().w8a8_last_error().decode()
    if rc == ERR_VALUE:
        raise ValueError(msg)
    if rc == ERR_INDEX:
        raise IndexError(msg)
    if rc == ERR_OOM:
        raise MemoryError(msg)
    raise W8A8Error(rc, msg)
