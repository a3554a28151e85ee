"""The C and C++ callers of the boundary, on the GPU (each a process of its
own): tests/cpp/w8a8_c_harness (plain C over include/w8a8.h) and
tests/cpp/kitchen_bridge_test (the reference crate's imagine_kitchen_call
argument lists through libimagine_kitchen.so), each checked against the oracle."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle" / "liboracle.so"


def _run(args):
    r = subprocess.run([str(a) for a in args], capture_output=True, text=True, timeout=180)
    print(r.stdout)
    print(r.stderr[-2000:])
    return r


def test_c_harness_over_the_header():
    r = _run([ROOT / "tests" / "cpp" / "w8a8_c_harness", ORACLE])
    assert r.returncode == 0 and "OK: 0 failure(s)" in r.stdout, r.stdout


def test_kitchen_bridge_with_the_crates_argument_lists():
    r = _run([ROOT / "tests" / "cpp" / "kitchen_bridge_test", ROOT / "imagine_amd" / "libimagine_kitchen.so", ORACLE])
    assert r.returncode == 0 and "OK: 0 failure(s)" in r.stdout, r.stdout
    assert r.stdout.count("PASS") >= 30
