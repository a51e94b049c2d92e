"""The decode fast path's integer-digit dot products, built for the host, against the oracle (CPU only).

tests/cpu/lane_check.cpp compiles kquant_lane.h -- the same __host__
__device__ code the gfx950 kernels run, with v_dot4_i32_i8 emulated -- and
computes full row dot products lane by lane (4 lanes of 64 weights per
super-block).  They must match the FP64 dot product of the oracle-dequantized
row within the digit error (two int8 digits: |x - x'| <= 1.6e-5 of each
16-column run's maximum) plus FP32 rounding of the sums.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import PKG_DIR, ROOT, build_check_library

# |x - (s/254)(254 x0 + x1)| <= s/508 with s = run max / 127, plus FP32 rounding of X = x * 127/max
DIGIT_ERR = 1.0 / (127 * 508) + 2.0 ** -22

SRC = ROOT / "tests" / "cpu" / "lane_check.cpp"
OUT = ROOT / "tests" / "cpu" / "_build" / "liblanecheck.so"


@pytest.fixture(scope="module")
def chk():
    deps = [SRC, PKG_DIR / "csrc" / "kquant_lane.h", PKG_DIR / "csrc" / "kquant_device.h"]
    L = C.CDLL(str(build_check_library(SRC, OUT, deps)))
    L.mqh_cpu_row_dot.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    L.mqh_cpu_row_dot.restype = C.c_float
    L.mqh_cpu_digit_roundtrip.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
    L.mqh_cpu_lane_cover.argtypes = [C.c_int, C.c_void_p]
    L.mqh_cpu_lane_w16.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    return L


def activations(rng, n, kind):
    if kind == "normal":
        return rng.standard_normal(n).astype(np.float32)
    if kind == "heavy":
        return (rng.standard_t(2, n) * 10.0 ** rng.uniform(-3, 3, n)).astype(np.float32)
    if kind == "sparse":
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.random(n) < 0.7] = 0.0
        return x
    return (rng.standard_normal(n) * 1e4).astype(np.float32)


@pytest.mark.parametrize("t", [8, 11, 12, 13, 14])
@pytest.mark.parametrize("kind", ["normal", "heavy", "sparse", "large"])
def test_row_dot_matches_oracle(chk, oracle_mod, t, kind):
    from flash_moe_hip.synthetic import random_tensor

    rng = np.random.default_rng(100 * t + len(kind))
    for ncols in (256, 512, 2048):
        rows = random_tensor(rng, t, 8, ncols).reshape(8, -1)
        w = oracle_mod.dequant(t, rows).reshape(8, ncols).astype(np.float64)
        for r in range(8):
            x = activations(rng, ncols, kind)
            got = chk.mqh_cpu_row_dot(t, rows[r].ctypes.data, ncols, x.ctypes.data)
            want = float(w[r] @ x.astype(np.float64))
            # digit error <= 1/(127*508) of the run max per value, plus FP32 rounding of the sums
            gmax = np.abs(x.reshape(-1, 16)).max(axis=1).repeat(16).astype(np.float64)
            bound = DIGIT_ERR * float(np.abs(w[r]) @ gmax) + 1e-6 * float(np.abs(w[r] * x).sum()) + 1e-30
            assert abs(got - want) <= bound, (ncols, r, got, want, bound)


def test_digit_roundtrip_bound(chk):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(4096), rng.standard_t(1, 4096) * 1e3,
                        np.zeros(64), np.full(32, 1e-30), np.full(32, -3e30)]).astype(np.float32)
    out = np.empty_like(x)
    chk.mqh_cpu_digit_roundtrip(x.ctypes.data, x.size, out.ctypes.data)
    gmax = np.abs(x.reshape(-1, 16)).max(axis=1).repeat(16)
    err = np.abs(out.astype(np.float64) - x)
    assert np.all(err <= DIGIT_ERR * gmax + 1e-45)
    # the bound is tight: two digits do not reconstruct every value exactly
    nz = gmax > 0
    assert (err[nz] / gmax[nz]).max() > 0.3 * DIGIT_ERR


@pytest.mark.parametrize("t", [8, 11, 12, 13, 14])
def test_lanes_cover_each_column_once(chk, t):
    count = np.zeros(256, np.int32)
    chk.mqh_cpu_lane_cover(t, count.ctypes.data)
    assert np.all(count == 1)


@pytest.mark.parametrize("t", [8, 11, 12, 13, 14])
def test_fp16_graph_lane_weights_bit_exact(chk, oracle_mod, t):
    """The FP16 graph's weight operands (lane_w16): for every lane of a 256-column
    unit, each weight is the oracle's dequantized value rounded to FP16 (the
    reference's round_weights, moe_quant_dot.cpp:154-157), bit for bit, and the
    lanes cover each column once -- on random units and on units whose scales
    make products land on FP16 rounding ties and subnormals."""
    from flash_moe_hip.synthetic import random_tensor
    from flash_moe_hip.quant_types import block_info

    rng = np.random.default_rng(300 + t)
    bs, pb = block_info(t)
    unit_bytes = 8 * pb if t == 8 else pb
    units = [random_tensor(rng, t, 1, 256, scale=s) for s in (0.01, 1.0, 1e-5, 37.0) for _ in range(8)]
    for unit in units:
        unit = np.ascontiguousarray(unit[:unit_bytes])
        bits = np.zeros(256, np.uint16)
        cols = np.zeros(256, np.int32)
        chk.mqh_cpu_lane_w16(t, unit.ctypes.data, bits.ctypes.data, cols.ctypes.data)
        assert sorted(cols.tolist()) == list(range(256))
        want = oracle_mod.f32_to_f16_bits(oracle_mod.dequant(t, unit, 256))
        np.testing.assert_array_equal(bits, np.asarray(want, np.uint16)[cols])


def test_q4k_q5k_fp16_weight_product_exact():
    """The premise that lets the FP16 graph's Q4_K/Q5_K weights be one fused
    multiply-add, fmaf(d1, q, -m1) = RN(RN(d1 q) - m1): for every finite FP16 d,
    every 6-bit scale sc and every 5-bit quant q, d1 = RN32(d sc) equals d sc
    exactly and RN32(d1 q) equals d1 q exactly (so the reference's first rounding
    never changes the value).  The min term m1 = RN32(dmin m) is the same product
    form, covered by the first check."""
    d = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    d = d[np.isfinite(d)]
    q = np.arange(32, dtype=np.float64)
    for sc in range(64):
        d1_64 = d * sc
        d1 = d1_64.astype(np.float32)
        assert np.array_equal(d1.astype(np.float64), d1_64), sc
        prod32 = (d1[:, None] * q[None, :].astype(np.float32)).astype(np.float64)
        assert np.array_equal(prod32, d1_64[:, None] * q[None, :]), sc
