"""The fp16 GELU table the kernels look up (imagine_amd/gelu_tables.py, built
into the library) against the oracle's gelu_tanh on every fp16 pattern, and
its closed forms beyond the table."""
import numpy as np

from imagine_amd import gelu_tables as G
from oracle import oracle as O


def test_fp16_table_and_closed_forms_equal_the_oracle_on_every_pattern():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = O.to_f32(bits, "f16")
    want = O.gelu_tanh(bits, "f16")       # scalar C: NaN payloads kept (quieted)
    tab = G.table()
    a = bits.astype(np.int64) & 0x7FFF
    inside = a < G.F16_HI
    idx = (bits.astype(np.int64) >> 15) * G.F16_HI + np.minimum(a, G.F16_HI - 1)
    got = np.where(inside, tab[idx], G.closed_form(bits)).astype(np.uint16)
    finite_or_inf = ~np.isnan(x)
    assert np.array_equal(got[finite_or_inf], want[finite_or_inf])
    nan = np.isnan(x)
    assert np.array_equal(got[nan], bits[nan] | 0x200)


def test_header_declares_the_table_the_kernels_index():
    text = G.header_text()
    assert f"kGeluF16Table[{2 * G.F16_HI}]" in text
    assert "kGeluF16Hi = 0x4600u" in text
