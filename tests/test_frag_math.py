"""The prefill GEMM's exact-integer MFMA operands, built for the host, against the oracle (CPU only).

tests/cpu/frag_check.cpp compiles kquant_frag.h -- the same __host__ __device__
code the gfx950 prefill kernels run -- and emulates one wave lane by lane with
the documented MFMA register layouts: each lane loads its contiguous byte runs
of a super-block, unpacks the 8 consecutive columns it owns in each of the 8
steps as exact FP16 integers sc*q (Q6_K: a split pair), the token rows enter as
power-of-two-scaled FP16 high (+ low) planes read at the same columns, the
Q4_K/Q5_K min term goes through the sub-block sums, and d / dmin are applied
per super-block (Q8_0: each step is one 32-column block, its int8 quants the
exact operand and its own d applied to the step's product).  Every column of a super-block must be dealt exactly once.
The result must match the FP64 product of the oracle-dequantized rows to FP32
rounding: the decomposition itself is exact, unlike FP16-rounded weights
(which miss the 1e-3 bar on Q4_K through cancellation of the min offsets).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import PKG_DIR, ROOT, build_check_library

SRC = ROOT / "tests" / "cpu" / "frag_check.cpp"
OUT = ROOT / "tests" / "cpu" / "_build" / "libfragcheck.so"


@pytest.fixture(scope="module")
def chk():
    deps = [SRC, PKG_DIR / "csrc" / "kquant_frag.h", PKG_DIR / "csrc" / "kquant_device.h"]
    L = C.CDLL(str(build_check_library(SRC, OUT, deps)))
    L.mqh_cpu_frag_gemm.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    L.mqh_cpu_frag_gemm.restype = None
    L.mqh_cpu_frag_cover.argtypes = [C.c_int, C.c_void_p]
    return L


def bf16(x: np.ndarray) -> np.ndarray:
    """Round FP32 to BF16 (nearest even), back as FP32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def tokens(rng, n, K, kind):
    if kind == "normal":
        return rng.standard_normal((n, K)).astype(np.float32)
    if kind == "heavy":
        return (rng.standard_t(2, (n, K)) * 10.0 ** rng.uniform(-3, 3, (n, 1))).astype(np.float32)
    if kind == "sparse":
        x = rng.standard_normal((n, K)).astype(np.float32)
        x[rng.random((n, K)) < 0.8] = 0.0
        x[0] = 0.0                                   # an all-zero token
        return x
    return (rng.standard_normal((n, K)) * 5e4).astype(np.float32)   # activations near the FP16 limit


def frag_gemm(chk, t, rows, K, x, split):
    out = np.zeros((x.shape[0], 16), np.float32)
    chk.mqh_cpu_frag_gemm(t, rows.ctypes.data, K, np.ascontiguousarray(x).ctypes.data, x.shape[0], split,
                          out.ctypes.data)
    return out


# -11: Q3_K with the gate/up kernel's operand form (11: the down kernel's, quant bits in place)
@pytest.mark.parametrize("t", [11, -11, 12, 13, 14, 8])
@pytest.mark.parametrize("kind", ["normal", "heavy", "sparse", "large"])
@pytest.mark.parametrize("split", [1, 0], ids=["fp32-x", "bf16-x"])
def test_frag_gemm_matches_oracle(chk, oracle_mod, t, kind, split):
    from flash_moe_hip.synthetic import random_tensor

    rng = np.random.default_rng(1000 * abs(t) + 10 * len(kind) + split)
    for K in (256, 512, 2048):
        rows = random_tensor(rng, abs(t), 16, K)
        w = oracle_mod.dequant(abs(t), rows).reshape(16, K).astype(np.float64)
        x = tokens(rng, 16, K, kind)
        if not split:
            x = bf16(x)
        got = frag_gemm(chk, t, rows, K, x, split)
        want = x.astype(np.float64) @ w.T
        # FP32 rounding of the per-block sums: a few ulp of sum |w x| per output
        bound = 1e-6 * (np.abs(x.astype(np.float64)) @ np.abs(w).T) + 1e-30
        assert np.all(np.abs(got - want) <= bound), (K, float(np.max(np.abs(got - want) / bound)))


def test_fp16_rounded_weights_would_fail(oracle_mod):
    """Why the operands are integers: FP16-rounded Q4_K weights alone cost close
    to (or more than) the 1e-3 bar on the benchmark expert shape."""
    from flash_moe_hip.synthetic import random_tensor

    rng = np.random.default_rng(5)
    H = 2048
    rows = random_tensor(rng, 12, 64, H)
    w = oracle_mod.dequant(12, rows).reshape(64, H).astype(np.float64)
    w16 = w.astype(np.float16).astype(np.float64)
    x = bf16(rng.standard_normal((16, H)).astype(np.float32)).astype(np.float64)
    ref = x @ w.T
    err = np.abs(x @ w16.T - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert err.max() > 2e-4


def test_all_zero_rows(chk):
    x = np.zeros((4, 256), np.float32)
    rows = np.zeros(16 * 144, np.uint8)
    out = frag_gemm(chk, 12, rows, 256, x, 1)
    assert np.all(out == 0.0)


@pytest.mark.parametrize("t", [11, 12, 13, 14, 8])
def test_lanes_cover_each_column_once(chk, t):
    count = np.zeros(256, np.int32)
    chk.mqh_cpu_frag_cover(t, count.ctypes.data)
    assert np.all(count == 1)
