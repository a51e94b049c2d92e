"""GPU drop-in moe_quant_expert / NativeExpert against the oracle.

Tolerance: max relative error (dequant.py:198-202) <= 1e-3 for outputs, the
bar for FP32-accumulated GEMV; the observed error in the FP32 graph is ~1e-6.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from test_oracle_expert import TRIPLES, kat_expert

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def native(hip):
    from flash_moe_hip.native_expert import NativeExpert

    return NativeExpert()


@pytest.mark.parametrize("kinds", TRIPLES)
@pytest.mark.parametrize("fp16", [0, 1])
def test_kat_triples(native, oracle_mod, kinds, fp16):
    print(f"expert kinds={kinds} fp16={fp16}", flush=True)
    rng = np.random.default_rng(31 + sum(kinds))
    k = dict(zip(("gate", "up", "down"), kinds))
    tensors = kat_expert(rng, kinds)
    scale = .005 if fp16 else 1.0
    x = (rng.standard_normal(256) * scale).astype(np.float32)
    want = oracle_mod.expert_forward(tensors, k, x, 256, 256, fp16)
    native.fp16_graph = fp16
    got = native.forward(tensors, k, x, 256, 256)
    err = oracle_mod.max_relative_error(got, want)
    print(f"  max rel err {err:.3e}", flush=True)
    assert err <= TOL


def test_single_expert_benchmark_shape(native, oracle_mod):
    """Q4_K 512x2048 / 2048x512 expert, x ~ N(0,1), seed 0: FP32 graph within
    tolerance; FP16 graph reports the same -4 the reference reports."""
    from flash_moe_hip.synthetic import config1_expert

    tensors, kinds, x = config1_expert(0)
    want = oracle_mod.expert_forward(tensors, kinds, x, 2048, 512, 0)
    native.fp16_graph = 0
    got = native.forward(tensors, kinds, x, 2048, 512)
    err = oracle_mod.max_relative_error(got, want)
    print(f"config-1 expert max rel err {err:.3e}", flush=True)
    assert err <= TOL
    native.fp16_graph = 1
    with pytest.raises(RuntimeError, match="status -4"):
        native.forward(tensors, kinds, x, 2048, 512)


def test_concurrent_calls_are_bit_identical(native, oracle_mod):
    rng = np.random.default_rng(5)
    kinds = (12, 13, 14)
    k = dict(zip(("gate", "up", "down"), kinds))
    tensors = kat_expert(rng, kinds)
    x = (rng.standard_normal(256) * .005).astype(np.float32)
    native.fp16_graph = 1
    with ThreadPoolExecutor(4) as pool:
        results = list(pool.map(lambda _: native.forward(tensors, k, x, 256, 256), range(8)))
    for r in results:
        np.testing.assert_array_equal(r, results[0])
    with pytest.raises(RuntimeError, match="status -2"):
        native.forward(tensors, dict(k, gate=999), x, 256, 256)
    with pytest.raises(ValueError):
        native.forward(tensors, k, x[:255], 256, 256)


def test_loader_contract(hip):
    from flash_moe_hip.native_expert import NativeExpert, load_native_expert

    types = {0: dict(gate=11, up=11, down=11)}
    assert isinstance(load_native_expert("native", None, "GPU", types), NativeExpert)
    assert load_native_expert("openvino", None, "GPU", types) is None
    assert load_native_expert("auto", None, "CPU", types) is None
    with pytest.raises(RuntimeError):
        load_native_expert("native", None, "GPU", {0: dict(gate=999, up=11, down=11)})
    with pytest.raises(RuntimeError):
        load_native_expert("native", "/nonexistent/lib.so", "GPU", types)
    with pytest.raises(ValueError):
        load_native_expert("bogus", None, "GPU", types)


@pytest.mark.parametrize("fp16", [0, 1])
@pytest.mark.parametrize("down", [12, 14, 8])
def test_non_finite_row_leaves_later_rows_untouched(hip, oracle_mod, fp16, down):
    """moe_quant_expert through the C ABI with a down row whose scale is
    +inf: -4, the rows before it within tolerance of the oracle's, that row
    non-finite, and every later row as the caller left it -- the reference's
    row-loop side effects (moe_quant_dot.cpp:207-211), which the oracle pins."""
    from test_oracle_expert import poison_row

    print(f"non-finite expert row: down={down} fp16={fp16}", flush=True)
    rng = np.random.default_rng(40 + down + fp16)
    kinds = (12, 12, down)
    k = dict(zip(("gate", "up", "down"), kinds))
    tensors = poison_row(kat_expert(rng, kinds), down, 100, 256)
    x = (rng.standard_normal(256) * (.005 if fp16 else 1.0)).astype(np.float32)
    want = np.full(256, 7.0, np.float32)
    rc_o, _ = oracle_mod.moe_quant_expert(tensors, k, x, 256, 256, fp16, out=want)
    assert rc_o == -4
    arrs = [np.ascontiguousarray(tensors[r], dtype=np.uint8) for r in ("gate", "up", "down")]
    got = np.full(256, 7.0, np.float32)
    rc = hip.moe_quant_expert(kinds[0], arrs[0].ctypes.data, arrs[0].nbytes, kinds[1], arrs[1].ctypes.data,
                              arrs[1].nbytes, kinds[2], arrs[2].ctypes.data, arrs[2].nbytes, x.ctypes.data, 256, 256,
                              got.ctypes.data, fp16)
    assert rc == -4
    assert oracle_mod.max_relative_error(got[:100], want[:100]) <= TOL
    assert not np.isfinite(got[100])
    np.testing.assert_array_equal(got[101:], 7.0)
