"""Exhaustive CPU proof that the quantizer's reciprocal-based division gives
the IEEE result for every 16-bit input pair the kernel can see, and that the
uncorrected product x * RN(1/d) already gives the IEEE int8 code."""
import subprocess
import tempfile
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "divide_check.c"


@pytest.fixture(scope="module")
def checker():
    with tempfile.TemporaryDirectory() as tmp:
        exe = Path(tmp) / "divide_check"
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-std=c99", "-o", str(exe), str(SRC), "-lm"],
                       check=True)
        yield exe


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_reciprocal_division_exact_for_all_reachable_pairs(checker, dtype):
    r = subprocess.run([str(checker), dtype], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout
    assert "code_mismatches=0 quotient_mismatches=0 product_code_mismatches=0" in r.stdout
