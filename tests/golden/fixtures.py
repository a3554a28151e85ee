"""Access to the committed reference golden vectors and their rebuilt operands."""
import gzip
import json
from functools import lru_cache
from pathlib import Path

import numpy as np

from . import operands as OP

PATH = Path(__file__).resolve().parent / "kitchen_int8_fixtures.json.gz"

# Modes that carry the pre-norm residual (residual + residual_scale).
RESIDUAL_MODES = {"residual", "fused_residual", "unaligned_residual", "unaligned_residual_scale"}
SECTIONS = {
    "cuda_int8_gemm": OP.gemm_operands,
    "cuda_int8_gemv": OP.m1_operands,
    "cuda_int8_m1": OP.m1_operands,
    "cuda_int8_activation": OP.activation_operands,
}


@lru_cache(maxsize=1)
def load():
    return json.load(gzip.open(PATH))


def linear_cases(section, with_errors=False, residual=False, convrot=False):
    """End-to-end cases of a CUDA section whose activation is None or
    gelu_tanh: without a residual, or (residual=True) only the residual modes;
    non-ConvRot cases, or (convrot=True) only the ConvRot ones.
    Yields (case, operands)."""
    for c in load()[section]:
        if bool(c.get("convrot")) != convrot:
            continue
        if c.get("activation") not in (None, "gelu_tanh"):
            continue
        if section == "cuda_int8_activation" and c["mode"] == "full":
            continue
        if (c["mode"] in RESIDUAL_MODES) != residual:
            continue
        if ("error" in c) != with_errors:
            continue
        yield c, SECTIONS[section](c)


def payload(c, dtype):
    """Expected output bytes as an array of the output storage type."""
    raw = np.array(c["payload"], dtype=np.uint8)
    return raw.view(np.float32 if dtype == "f32" else np.uint16)
