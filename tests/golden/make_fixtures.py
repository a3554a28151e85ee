"""Extract the reference's INT8 golden vectors into one small committed fixture file.

Run in a container where the reference checkout is mounted at /root/reference:

    python tests/golden/make_fixtures.py

Sources (data only, nothing from the reference is imported or executed):

* ``inference/fixtures/kitchen-038-upgrade.json.gz`` (committed in the reference):
  sections ``cuda_int8_activation`` (1386 cases), ``cuda_int8_m1`` (504) and
  ``cuda_int8_m1_selection`` (5).  Captured from Kitchen 0.2.38 on an SM89 GPU by
  ``inference/tools/reference_cuda_int8_activation.py`` and ``reference_cuda_int8_m1.py``.
* ``inference/fixtures/stage-1/oracles.tar.gz.part-*`` member ``runtime/primitives.json``
  (streamed; only this member is read, and only its first ~99 MB).  Sections
  ``int8`` (rowwise cases), ``native_quantizers`` (``int8_rowwise`` cases), ``int8_mm``,
  ``eager_int8_linear``, ``cuda_int8_gemv`` and ``cuda_int8_gemm``.  Generators:
  ``inference/tools/reference_primitives.py:357-365,388-391``,
  ``reference_int8_linear.py:18-92``, ``reference_cuda_int8_gemv.py:7-47`` and
  ``reference_cuda_int8_gemm.py:7-77``.

Every case keeps only its parameters and expected bytes: the operands are
deterministic functions of the parameters (rebuilt in ``tests/golden/operands.py``).
"""
import gzip
import json
import subprocess
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "kitchen_int8_fixtures.json.gz"

# Byte offsets of the top-level keys inside runtime/primitives.json (one JSON line).
SECTION_OFFSETS = {
    "int8": 73_618,
    "native_quantizers": 172_977,
    "int8_mm": 44_607_355,
    "eager_int8_linear": 44_719_859,
    "cuda_int8_gemv": 95_841_055,
    "cuda_int8_gemm": 96_162_061,
}
HEAD_BYTES = 99_000_000


def _archived_sections():
    parts = sorted((REF / "inference/fixtures/stage-1").glob("oracles.tar.gz.part-*"))
    cat = subprocess.Popen(["cat", *map(str, parts)], stdout=subprocess.PIPE)
    tar = subprocess.Popen(["tar", "xzOf", "-", "runtime/primitives.json"],
                           stdin=cat.stdout, stdout=subprocess.PIPE)
    cat.stdout.close()
    head = tar.stdout.read(HEAD_BYTES)
    tar.stdout.close()
    tar.kill()
    cat.kill()
    text = head.decode("utf-8", errors="replace")
    dec = json.JSONDecoder()
    out = {}
    for key, off in SECTION_OFFSETS.items():
        tag = f'"{key}":'
        assert text[off:off + len(tag)] == tag, f"offset of {key} moved"
        start = off + len(tag)
        while text[start] in " \n":
            start += 1
        out[key], _ = dec.raw_decode(text, start)
    return out


def main():
    committed = json.load(gzip.open(REF / "inference/fixtures/kitchen-038-upgrade.json.gz"))
    archived = _archived_sections()
    fixtures = {
        "provenance": {
            "committed": "inference/fixtures/kitchen-038-upgrade.json.gz "
                         f"(kitchen {committed['kitchen_version']}, rev {committed['reference_revision']})",
            "archived": "inference/fixtures/stage-1/oracles.tar.gz.part-* -> runtime/primitives.json",
        },
        "cuda_int8_activation": committed["sections"]["cuda_int8_activation"],
        "cuda_int8_m1": committed["sections"]["cuda_int8_m1"],
        "cuda_int8_m1_selection": committed["sections"]["cuda_int8_m1_selection"],
        "int8_rowwise": [c for c in archived["int8"] if c["rowwise"]],
        # tensorwise quantizer, deterministic rounding only (seed None or 0)
        "int8_tensorwise": [c for c in archived["int8"] if not c["rowwise"] and not c["seed"]],
        "native_int8_rowwise": [c for c in archived["native_quantizers"]
                                if c.get("operation") == "int8_rowwise"],
        "int8_mm": archived["int8_mm"],
        "eager_int8_linear": archived["eager_int8_linear"],
        "cuda_int8_gemv": archived["cuda_int8_gemv"],
        "cuda_int8_gemm": archived["cuda_int8_gemm"],
    }
    for c in fixtures["int8_rowwise"] + fixtures["int8_tensorwise"]:
        c.pop("decoded", None)
    raw = json.dumps(fixtures, separators=(",", ":")).encode()
    with gzip.GzipFile(OUT, "wb", mtime=0) as f:
        f.write(raw)
    print(OUT, {k: len(v) for k, v in fixtures.items() if isinstance(v, list)},
          f"{OUT.stat().st_size} bytes")


if __name__ == "__main__":
    main()
