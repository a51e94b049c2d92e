"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so that a plausible slip in the oracle's restatement of
cpp/dequant_k.cpp fails at least one of them:

* FP16<->FP32 conversion against NumPy's IEEE binary16 conversion (a textbook
  routine): all 65,536 halves, and FP32 values around every rounding boundary.
* Block decoders against an independent, vectorised restatement of the
  published gguf.quants dequantizers (oracle/gguf_quants_np.py): bit-exact on
  random and edge blocks.
* Block decoders against the reference's own measured bit maps
  (cpp/dequant_k_tables.h, read as text when the reference tree is present)
  by one-bit probes, the way tools/derive_k_tables.py measured them.
* Field-level closed forms: blocks packed from known (d, dmin, scales, quants)
  decode to d*sc*q - dmin*m exactly.
* The test procedure of tools/test_dequant_k.py:112-156 (first block
  identical, FP32 within 1e-6, FP16 within 1e-3, n+1 rejected with -1).
* Q8_0 quantize -> dequantize round trip with the gguf quantizer
  (tools/_kquant_ref.txt:378-395), which excludes the legacy -128 offset.
"""
from __future__ import annotations

import re

import numpy as np
import pytest

from conftest import REFERENCE

TYPES = [8, 11, 12, 13, 14]
NAMES = {8: "Q8_0", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}
BLOCK = {8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
D_OFF = {8: 0, 11: 108, 12: 0, 13: 0, 14: 208}


def put_f16(buf: np.ndarray, off: int, value) -> None:
    buf[..., off:off + 2] = np.array(value, dtype=np.float16).reshape(-1, 1).view(np.uint8).reshape(
        buf[..., off:off + 2].shape)


def random_blocks(rng, t, n):
    bs, pb = BLOCK[t]
    data = rng.integers(0, 256, size=(n, pb), dtype=np.uint8)
    put_f16(data, D_OFF[t], rng.uniform(-0.5, 0.5, n))
    if t in (12, 13):
        put_f16(data, 2, rng.uniform(-0.2, 0.2, n))
    return data


def edge_blocks(t):
    """d/dmin at zero, negative zero, subnormal, tiny, max; quant bytes at 0x00/0xFF/patterns."""
    bs, pb = BLOCK[t]
    d_bits = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x1234]
    fills = [0x00, 0xFF, 0x55, 0xAA, 0x0F, 0xF0]
    out = []
    for db in d_bits:
        for f in fills:
            blk = np.full(pb, f, dtype=np.uint8)
            blk[D_OFF[t]:D_OFF[t] + 2] = np.array([db], np.uint16).view(np.uint8)
            if t in (12, 13):
                blk[2:4] = np.array([d_bits[(d_bits.index(db) + 3) % len(d_bits)]], np.uint16).view(np.uint8)
            out.append(blk)
    return np.stack(out)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- f16 <-> f32

def test_f16_to_f32_all_halves(oracle_mod):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle_mod.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    assert np.array_equal(bits(got), bits(want))


def test_f32_to_f16_rounding_boundaries(oracle_mod):
    rng = np.random.default_rng(7)
    # every half value, its neighbours, and the exact midpoints between halves
    h = np.arange(0, 0x7C00, dtype=np.uint32)
    f = h.astype(np.uint16).view(np.float16).astype(np.float32)
    nxt = (h + 1).astype(np.uint16).view(np.float16).astype(np.float32)
    mid = ((f.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)  # exact in FP32
    cand = np.concatenate([f, mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf)),
                           np.float32([65504, 65519.996, 65520, 65536, 1e30, 2.0 ** -25, 2.0 ** -26,
                                       np.nextafter(np.float32(2.0 ** -25), np.float32(1)), 1e-40, 0.0])])
    rnd = rng.integers(0, 2 ** 32, 400_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    cand = np.concatenate([cand, -cand, rnd[np.isfinite(rnd)]])
    got = oracle_mod.f32_to_f16_bits(cand)
    with np.errstate(over="ignore"):
        want = cand.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------- decoders vs NumPy gguf style

@pytest.mark.parametrize("t", TYPES)
def test_decoders_match_gguf_restatement(oracle_mod, t):
    from oracle import gguf_quants_np as gq

    rng = np.random.default_rng(100 + t)
    blocks = np.concatenate([random_blocks(rng, t, 512), edge_blocks(t)])
    got = oracle_mod.dequant(t, blocks)
    want = gq.dequantize(blocks, t)
    assert got.shape == want.shape
    assert np.array_equal(bits(got), bits(want)), f"{NAMES[t]}: {np.sum(bits(got) != bits(want))} values differ"
    got16 = oracle_mod.dequant(t, blocks, want_f16=True)
    with np.errstate(over="ignore"):
        want16 = want.astype(np.float16)
    assert np.array_equal(got16.view(np.uint16), want16.view(np.uint16))


# ----------------------------------------------- one-bit probes vs the tables

def _parse_tables():
    path = REFERENCE / "cpp" / "dequant_k_tables.h"
    if not path.exists():
        pytest.skip("reference tree not present")
    text = path.read_text()
    tables = {}
    for name, body in re.findall(r"static const uint8_t (\w+)\[256\] = \{([^}]*)\}", text):
        tables[name] = np.array([int(v) for v in body.split(",")], dtype=np.int64)
    return tables


def _probe(oracle_mod, t, base: np.ndarray, byte_range):
    """For each output, the bytes/bits whose flip changes it and by how much."""
    ref = oracle_mod.dequant(t, base[None]).astype(np.float64)
    effects = {}
    for byte in byte_range:
        for bit in range(8):
            blk = base.copy()
            blk[byte] ^= np.uint8(1 << bit)
            delta = oracle_mod.dequant(t, blk[None]).astype(np.float64) - ref
            for i in np.nonzero(delta)[0]:
                effects.setdefault(int(i), []).append((byte, bit, delta[i]))
    return effects


def _field(effects_i, lo_byte, hi_byte):
    """(byte, lowest bit, width, weight of the lowest bit) of the field in [lo, hi)."""
    e = [(b, bit, d) for b, bit, d in effects_i if lo_byte <= b < hi_byte]
    assert e, "no field found"
    byte = {b for b, _, _ in e}
    assert len(byte) == 1
    low = min(bit for _, bit, _ in e)
    return byte.pop(), low, len(e), [d for _, bit, d in e if bit == low][0]


def test_q6k_bit_map_matches_reference_tables(oracle_mod):
    tab = _parse_tables()
    base = np.zeros(210, np.uint8)
    base[192:208] = 1                      # int8 scales = 1
    base[208:210] = np.array([1.0], np.float16).view(np.uint8)
    eff = _probe(oracle_mod, 14, base, range(0, 192))
    for i in range(256):
        b1, s1, w1, u1 = _field(eff[i], 0, 128)
        b2, s2, w2, u2 = _field(eff[i], 128, 192)
        assert (b1, s1, w1, u1) == (tab["Q6_K_B1"][i], tab["Q6_K_S1"][i], 4, 1.0), i
        assert (b2, s2, w2, abs(u2)) == (tab["Q6_K_B2"][i], tab["Q6_K_S2"][i], 2, 16.0), i


def test_q3k_bit_map_matches_reference_tables(oracle_mod):
    tab = _parse_tables()
    base = np.zeros(110, np.uint8)
    base[96:104] = 0x11                    # scale low nibbles = 1
    base[104:108] = 0xAA                   # scale high bits = 2  -> scale = 33 - 32 = 1
    base[108:110] = np.array([1.0], np.float16).view(np.uint8)
    eff = _probe(oracle_mod, 11, base, range(0, 96))
    for i in range(256):
        b1, s1, w1, u1 = _field(eff[i], 0, 32)      # hmask bit
        b2, s2, w2, u2 = _field(eff[i], 32, 96)     # 2-bit quant
        assert (b1, s1, w1, u1) == (tab["Q3_K_B1"][i], tab["Q3_K_S1"][i], 1, 4.0), i
        assert (b2, s2, w2, u2) == (tab["Q3_K_B2"][i], tab["Q3_K_S2"][i], 2, 1.0), i


def test_q5k_bit_map_matches_reference_tables(oracle_mod):
    tab = _parse_tables()
    base = np.zeros(176, np.uint8)
    base[0:2] = np.array([1.0], np.float16).view(np.uint8)   # d = 1, dmin = 0
    base[4:8] = 1                          # sc[0..3] = 1, mins 0
    base[12:16] = 0x01                     # sc[4..7] = 1, mins 0
    eff = _probe(oracle_mod, 13, base, range(16, 176))
    for i in range(256):
        b1, s1, w1, u1 = _field(eff[i], 16, 48)     # 1-bit field weighted 2^O1
        b2, s2, w2, u2 = _field(eff[i], 48, 176)    # 4-bit field weighted 2^O2
        assert (b1, s1, w1, u1) == (tab["Q5_K_B1"][i], tab["Q5_K_S1"][i], tab["Q5_K_W1"][i],
                                    2.0 ** tab["Q5_K_O1"][i]), i
        assert (b2, s2, w2, u2) == (tab["Q5_K_B2"][i], tab["Q5_K_S2"][i], tab["Q5_K_W2"][i],
                                    2.0 ** tab["Q5_K_O2"][i]), i


# ---------------------------------------------------- field-level closed forms

def _pack_scale_min_k4(sc, mn):
    """12 bytes holding eight 6-bit scales and mins (layout diagram of
    tools/_kquant_ref.txt:482-494): bytes 0-3 = sc[0:4] | (sc[4:8] top 2 bits) << 6,
    bytes 4-7 = mn[0:4] | (mn[4:8] top 2 bits) << 6, bytes 8-11 = sc[4:8] low
    nibble | mn[4:8] low nibble << 4."""
    s = np.zeros(12, np.uint8)
    s[0:4] = sc[0:4] | ((sc[4:8] >> 4) << 6)
    s[4:8] = mn[0:4] | ((mn[4:8] >> 4) << 6)
    s[8:12] = (sc[4:8] & 15) | ((mn[4:8] & 15) << 4)
    return s


@pytest.mark.parametrize("seed", range(4))
def test_q4k_closed_form(oracle_mod, seed):
    rng = np.random.default_rng(seed)
    d, dmin = np.float16(rng.uniform(0.001, 0.1)), np.float16(rng.uniform(0.001, 0.1))
    sc, mn = rng.integers(0, 64, 8).astype(np.uint8), rng.integers(0, 64, 8).astype(np.uint8)
    q = rng.integers(0, 16, 256).astype(np.uint8)
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d]).view(np.uint8)
    blk[2:4] = np.array([dmin]).view(np.uint8)
    blk[4:16] = _pack_scale_min_k4(sc, mn)
    for g in range(4):          # 64 values per 32 bytes: low nibble first, then high
        blk[16 + 32 * g:48 + 32 * g] = q[64 * g:64 * g + 32] | (q[64 * g + 32:64 * g + 64] << 4)
    j = np.arange(256) // 32
    want = (np.float32(d) * sc[j].astype(np.float32)) * q.astype(np.float32) - np.float32(dmin) * mn[j].astype(np.float32)
    assert np.array_equal(bits(oracle_mod.dequant(12, blk)), bits(want))


@pytest.mark.parametrize("seed", range(4))
def test_q6k_closed_form(oracle_mod, seed):
    rng = np.random.default_rng(seed)
    d = np.float16(rng.uniform(-0.1, 0.1))
    sc = rng.integers(-128, 128, 16).astype(np.int8)
    q = rng.integers(-32, 32, 256)
    u = (q + 32).astype(np.uint8)
    blk = np.zeros(210, np.uint8)
    for h in range(2):          # per 128 values: 64 ql bytes, 32 qh bytes
        v = u[128 * h:128 * h + 128].reshape(4, 32)
        blk[64 * h:64 * h + 32] = (v[0] & 15) | ((v[2] & 15) << 4)
        blk[64 * h + 32:64 * h + 64] = (v[1] & 15) | ((v[3] & 15) << 4)
        blk[128 + 32 * h:160 + 32 * h] = (v[0] >> 4) | ((v[1] >> 4) << 2) | ((v[2] >> 4) << 4) | ((v[3] >> 4) << 6)
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = np.array([d]).view(np.uint8)
    want = (np.float32(d) * sc[np.arange(256) // 16].astype(np.float32)) * q.astype(np.float32)
    assert np.array_equal(bits(oracle_mod.dequant(14, blk)), bits(want))


@pytest.mark.parametrize("seed", range(4))
def test_q3k_closed_form(oracle_mod, seed):
    rng = np.random.default_rng(seed)
    d = np.float16(rng.uniform(-0.1, 0.1))
    sc = rng.integers(-32, 32, 16)
    q = rng.integers(-4, 4, 256)
    u = (q + 4).astype(np.uint8)            # 3-bit: bit 2 is the hmask bit
    blk = np.zeros(110, np.uint8)
    for i in range(256):
        blk[i % 32] |= ((u[i] >> 2) & 1) << (i // 32)
        h, s, l = i // 128, (i // 32) % 4, i % 32
        blk[32 + 32 * h + l] |= (u[i] & 3) << (2 * s)
    us = (sc + 32).astype(np.uint8)         # 6-bit biased scales
    blk[96:104] = (us[0:8] & 15) | ((us[8:16] & 15) << 4)
    for j in range(16):
        blk[104 + (j % 4)] |= (us[j] >> 4) << (2 * (j // 4))
    blk[108:110] = np.array([d]).view(np.uint8)
    want = (np.float32(d) * sc[np.arange(256) // 16].astype(np.float32)) * q.astype(np.float32)
    assert np.array_equal(bits(oracle_mod.dequant(11, blk)), bits(want))


def test_q5k_closed_form(oracle_mod):
    rng = np.random.default_rng(3)
    d, dmin = np.float16(0.0371), np.float16(0.0059)
    sc, mn = rng.integers(0, 64, 8).astype(np.uint8), rng.integers(0, 64, 8).astype(np.uint8)
    q = rng.integers(0, 32, 256).astype(np.uint8)
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([d]).view(np.uint8)
    blk[2:4] = np.array([dmin]).view(np.uint8)
    blk[4:16] = _pack_scale_min_k4(sc, mn)
    for i in range(256):
        blk[16 + i % 32] |= ((q[i] >> 4) & 1) << (i // 32)
    for g in range(4):
        blk[48 + 32 * g:80 + 32 * g] = (q[64 * g:64 * g + 32] & 15) | ((q[64 * g + 32:64 * g + 64] & 15) << 4)
    j = np.arange(256) // 32
    want = (np.float32(d) * sc[j].astype(np.float32)) * q.astype(np.float32) - np.float32(dmin) * mn[j].astype(np.float32)
    assert np.array_equal(bits(oracle_mod.dequant(13, blk)), bits(want))


def test_q8_0_quantize_roundtrip(oracle_mod):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 32)) * 0.05).astype(np.float32)
    d = np.abs(x).max(axis=1, keepdims=True) / 127
    qs = np.round(x / d).astype(np.int8)
    blocks = np.concatenate([d.astype(np.float16).view(np.uint8), qs.view(np.uint8)], axis=1)
    y = oracle_mod.dequant(8, blocks).reshape(64, 32).astype(np.float64)
    d16 = d.astype(np.float16).astype(np.float64)
    # |q*d16 - x| <= |q*d - x| + 127*|d16 - d| <= d/2 + 127*|d16 - d|
    bound = d / 2 + 127 * np.abs(d16 - d) + 1e-7
    assert np.all(np.abs(y - x) <= bound)
    # the legacy layout's -128 offset would shift every value by 128*d
    assert np.abs(y - x).max() < 0.01 * np.abs(x).max()


# ------------------------------------- procedure of tools/test_dequant_k.py

@pytest.mark.parametrize("t", TYPES)
def test_reference_dequant_procedure(oracle_mod, t):
    from oracle import gguf_quants_np as gq

    L = oracle_mod.lib()
    bs, pb = BLOCK[t]
    assert L.oracle_dequant_k_supported(t) == 1
    assert L.oracle_dequant_k_block_size(t) == bs
    data = random_blocks(np.random.default_rng(t), t, 8).reshape(-1)
    n = data.nbytes // pb * bs
    ref = gq.dequantize(data, t).astype(np.float64)
    rc, out32 = oracle_mod.dequant_k(t, data, n, False)
    assert rc == 0 and not np.isnan(out32).any()
    assert np.array_equal(out32[:bs].astype(np.float64), ref[:bs])
    assert oracle_mod.max_relative_error(out32, ref) < 1e-6
    rc, out16 = oracle_mod.dequant_k(t, data, n, True)
    assert rc == 0 and oracle_mod.max_relative_error(out16.astype(np.float32), ref) < 1e-3
    assert oracle_mod.dequant_k(t, data, n + 1, False)[0] == -1
    assert oracle_mod.dequant_k(t, data, 0, False)[0] == -1
    assert oracle_mod.dequant_k(99, data, n, False)[0] == -1
    assert L.oracle_dequant_k_supported(99) == 0 and L.oracle_dequant_k_block_size(99) == 0
