"""Pin the IQ4_NL oracle (oracle_dequantize_iq4_nl, cpp/fast_dequant.cpp:40-65).

* The 16 table values against the reference's own sources, read as text when
  the reference tree is present (fast_dequant.cpp:4-9 and the AVX2 file's copy,
  fast_dequant_avx2.cpp:34-39, which must agree with each other).
* The layout by one-hot probes against the block layout stated in the
  reference (fast_dequant_avx2.cpp:3-10; fast_dequant.cpp:56-61): value i
  takes the low nibble of byte i, value 16 + i its high nibble, and a nibble
  n yields scale * table[n].
* The scale: a power-of-two FP16 scale scales the table exactly, and every
  FP16 bit pattern of the scale (subnormals included) decodes as IEEE binary16.
* The row geometry of the export: rows of cols / 32 blocks, row r at
  dst + r * cols, columns past the last whole block untouched.
"""
from __future__ import annotations

import re

import numpy as np
import pytest

from conftest import REFERENCE


def _block(d, qs):
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:] = qs
    return b


def _table(oracle_mod):
    """table[n] as the oracle decodes it: d = 1, every value the nibble n."""
    out = []
    for n in range(16):
        v = oracle_mod.dequantize_iq4_nl(_block(1.0, np.full(16, n | (n << 4), np.uint8)), 1, 32)[0]
        assert np.all(v == v[0])
        out.append(v[0])
    return np.array(out, np.float32)


def _reference_tables():
    found = []
    for name in ("fast_dequant.cpp", "fast_dequant_avx2.cpp"):
        path = REFERENCE / "cpp" / name
        if not path.exists():
            pytest.skip("reference tree not present")
        m = re.search(r"kvalues_iq4_nl\[16\]\s*=\s*\{([^}]*)\}", path.read_text())
        assert m, name
        found.append(np.array([float(v.strip().rstrip("f")) for v in m.group(1).split(",") if v.strip()],
                              dtype=np.float32))
    return found


def test_table_is_the_reference_libraries_table(oracle_mod):
    a, b = _reference_tables()
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(_table(oracle_mod), a)


def test_table_shape(oracle_mod):
    t = _table(oracle_mod)
    assert t[0] == -1.0 and t[15] == 1.0
    assert np.all(np.diff(t) > 0)              # strictly increasing, 8 negative and 8 positive entries
    assert np.sum(t < 0) == 7 and np.sum(t > 0) == 9


def test_one_hot_layout(oracle_mod):
    t = _table(oracle_mod)
    d = 0.375
    for i in range(16):
        for hi in (0, 1):
            for n in (1, 7, 15):
                qs = np.zeros(16, np.uint8)
                qs[i] = n << 4 if hi else n
                v = oracle_mod.dequantize_iq4_nl(_block(d, qs), 1, 32)[0]
                want = np.full(32, np.float32(d) * t[0], np.float32)
                want[i + 16 * hi] = np.float32(d) * t[n]
                np.testing.assert_array_equal(v, want)


def test_scale_decoding(oracle_mod):
    t = _table(oracle_mod)
    qs = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    for e in range(-14, 16):
        v = oracle_mod.dequantize_iq4_nl(_block(2.0 ** e, qs), 1, 32)[0]
        np.testing.assert_array_equal(v[:16], t * np.float32(2.0 ** e))
        np.testing.assert_array_equal(v[16:], t[::-1] * np.float32(2.0 ** e))
    bits = np.arange(0, 0x7C00, 97, dtype=np.uint16)          # positive finite halves, subnormals included
    blocks = np.zeros((bits.size, 18), np.uint8)
    blocks[:, 0:2] = bits.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = 0xFF                                       # every value table[15] = 1.0
    v = oracle_mod.dequantize_iq4_nl(blocks, bits.size, 32)
    np.testing.assert_array_equal(v[:, 0], bits.view(np.float16).astype(np.float32))


def test_row_geometry(oracle_mod):
    rng = np.random.default_rng(1)
    rows, cols = 3, 70                                         # two whole blocks per row, 6 columns left over
    raw = rng.integers(0, 256, size=rows * 2 * 18, dtype=np.uint8)
    raw.reshape(-1, 18)[:, 0:2] = np.array([0.5], np.float16).view(np.uint8)
    v = oracle_mod.dequantize_iq4_nl(raw, rows, cols)
    flat = oracle_mod.dequantize_iq4_nl(raw, rows * 2, 32).reshape(rows, 64)
    np.testing.assert_array_equal(v[:, :64], flat)
    np.testing.assert_array_equal(v[:, 64:], 0.0)             # untouched (the wrapper zero-fills)
