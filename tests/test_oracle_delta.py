"""The DeltaNet recurrence oracle (oracle/delta_oracle.c, cpp/moe_delta.cpp:18-69).

Pinned three ways: bit for bit against the reference's own kernel compiled
from its source (oracle/_ref, where the reference tree was present at build
time); against the float64 closed form of gated_deltanet.py:264-298 (arXiv
2412.06464 eq. 10) within FP32 rounding; and by two invariants that a dropped
term, a wrong sign or a swapped operand would break: with beta = 0 the step is
a pure decay read by q, and with gate = 0, beta = 1 and a unit key the updated
state maps k to v exactly (the delta rule overwrites what the state recalled).
"""
from __future__ import annotations

import numpy as np
import pytest

SHAPES = [(32, 128, 128), (3, 7, 9), (4, 5, 200), (2, 3, 1), (1, 2, 1024), (256, 1, 8), (5, 16, 15)]


def inputs(rng, nv, dv, dk):
    q = (rng.standard_normal((nv, dk)) * 0.05).astype(np.float32)
    k = (rng.standard_normal((nv, dk)) * 0.05).astype(np.float32)
    v = (rng.standard_normal((nv, dv)) * 0.1).astype(np.float32)
    beta = rng.uniform(0.01, 0.99, nv).astype(np.float32)
    gate = (-rng.uniform(0.001, 5, nv)).astype(np.float32)
    return q, k, v, beta, gate


@pytest.mark.parametrize("shape", SHAPES)
def test_oracle_is_the_reference_kernel_bit_for_bit(oracle_mod, shape):
    if oracle_mod.reference_delta_lib() is None:
        pytest.skip("the reference kernel was not built here (no reference tree at build time)")
    rng = np.random.default_rng(sum(shape))
    nv, dv, dk = shape
    a = (rng.standard_normal(shape) * 0.01).astype(np.float32)
    b = a.copy()
    for _ in range(40):
        args = inputs(rng, nv, dv, dk)
        r1, o1 = oracle_mod.delta_heads(a, *args)
        r2, o2 = oracle_mod.reference_delta_heads(b, *args)
        assert r1 == r2 == 0
        np.testing.assert_array_equal(o1, o2)
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("shape", SHAPES)
def test_oracle_matches_the_float64_closed_form(oracle_mod, shape):
    rng = np.random.default_rng(7 + sum(shape))
    nv, dv, dk = shape
    st = (rng.standard_normal(shape) * 0.01).astype(np.float32)
    s64 = st.astype(np.float64)
    for _ in range(40):
        q, k, v, beta, gate = inputs(rng, nv, dv, dk)
        rc, out = oracle_mod.delta_heads(st, q, k, v, beta, gate)
        assert rc == 0
        want = np.stack([oracle_mod.delta_step_numpy(s64[h], q[h].astype(np.float64), k[h].astype(np.float64),
                                                     v[h].astype(np.float64), float(beta[h]), float(gate[h]))
                         for h in range(nv)])
        # the reference's own tolerance against NumPy (tools/test_optimized_inference.py:211-212)
        np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-7)
        np.testing.assert_allclose(st, s64, rtol=1e-4, atol=1e-7)


def test_zero_beta_is_a_pure_decay(oracle_mod):
    rng = np.random.default_rng(3)
    nv, dv, dk = 4, 6, 24
    st = rng.standard_normal((nv, dv, dk)).astype(np.float32)
    q, k, v, _, gate = inputs(rng, nv, dv, dk)
    decay = np.exp(gate.astype(np.float64))
    want_state = (st.astype(np.float64) * decay[:, None, None]).astype(np.float32)
    rc, out = oracle_mod.delta_heads(st, q, k, v, np.zeros(nv, np.float32), gate)
    assert rc == 0
    np.testing.assert_array_equal(st, want_state)   # one double product, rounded once
    np.testing.assert_allclose(out, np.einsum("hrj,hj->hr", want_state.astype(np.float64), q), rtol=1e-5,
                               atol=1e-7)


def test_unit_key_writes_the_value(oracle_mod):
    rng = np.random.default_rng(4)
    nv, dv, dk = 3, 5, 16
    st = rng.standard_normal((nv, dv, dk)).astype(np.float32)
    k = np.zeros((nv, dk), np.float32)
    for h in range(nv):
        k[h, (3 * h + 1) % dk] = 1.0
    q = k.copy()                                   # read back along the same key
    v = rng.standard_normal((nv, dv)).astype(np.float32)
    rc, out = oracle_mod.delta_heads(st, q, k, v, np.ones(nv, np.float32), np.zeros(nv, np.float32))
    assert rc == 0
    # S_new k = S k + (v - S k)(k.k) = v for a unit key: fl(s + fl(v - s)) is v
    # within one rounding of the larger magnitude
    tol = 2.0 ** -22 * np.maximum(np.abs(v), 4.0)
    assert np.all(np.abs(out - v) <= tol)
    for h in range(nv):
        assert np.all(np.abs(st[h][:, (3 * h + 1) % dk] - v[h]) <= tol[h])


def test_status_codes(oracle_mod):
    st = np.zeros((2, 3, 4), np.float32)
    q = k = np.zeros((2, 4), np.float32)
    v = np.zeros((2, 3), np.float32)
    b = g = np.zeros(2, np.float32)
    assert oracle_mod.delta_heads(st, q, k, v, b, g)[0] == 0
    v_bad = v.copy()
    v_bad[1, 2] = np.nan
    rc, out = oracle_mod.delta_heads(st, q, k, v_bad, np.ones(2, np.float32), g)
    assert rc == -2
    np.testing.assert_array_equal(out[0], 0.0)     # rows before the bad one were written
    L = oracle_mod.lib()
    assert L.oracle_delta_heads(None, q.ctypes.data, k.ctypes.data, v.ctypes.data, b.ctypes.data, g.ctypes.data,
                                v.ctypes.data, 2, 4, 3) == -1
    for heads, dk, dv in ((0, 4, 3), (257, 4, 3), (2, 0, 3), (2, 1025, 3), (2, 4, 0), (2, 4, 1025)):
        assert L.oracle_delta_heads(st.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, b.ctypes.data,
                                    g.ctypes.data, v.ctypes.data, heads, dk, dv) == -1


def test_first_non_finite_row_stops_the_step(oracle_mod):
    """A NaN value in head 2, row 5 of a 4 x 8 x 16 step: the oracle returns -2
    with the state rows up to and including that row updated, the outputs
    before it written, and that row's output and every later row's state and
    output as the caller had them (moe_delta.cpp:30-66: the row loop returns
    before the output store).  Against the reference kernel built from its
    source as well, bit for bit, where it was built."""
    rng = np.random.default_rng(12)
    nv, dv, dk = 4, 8, 16
    q, k, v, beta, gate = inputs(rng, nv, dv, dk)
    v[2, 5] = np.nan
    bad = 2 * dv + 5
    st0 = (rng.standard_normal((nv, dv, dk)) * 0.01).astype(np.float32)
    st = st0.copy()
    out = np.full((nv, dv), 7.0, np.float32)
    rc, _ = oracle_mod.delta_heads(st, q, k, v, beta, gate, out=out)
    assert rc == -2
    clean = st0.copy()
    v_ok = v.copy()
    v_ok[2, 5] = 0.0
    _, out_ok = oracle_mod.delta_heads(clean, q, k, v_ok, beta, gate)
    rows, orow = st.reshape(-1, dk), out.reshape(-1)
    np.testing.assert_array_equal(rows[:bad], clean.reshape(-1, dk)[:bad])   # earlier rows: a normal step
    assert not np.isfinite(rows[bad]).all()                                  # the bad row's state: updated
    np.testing.assert_array_equal(rows[bad + 1:], st0.reshape(-1, dk)[bad + 1:])
    np.testing.assert_array_equal(orow[:bad], out_ok.reshape(-1)[:bad])
    np.testing.assert_array_equal(orow[bad:], 7.0)
    if oracle_mod.reference_delta_lib() is not None:
        st_r = st0.copy()
        out_r = np.full((nv, dv), 7.0, np.float32)
        rc_r, _ = oracle_mod.reference_delta_heads(st_r, q, k, v, beta, gate, out=out_r)
        assert rc_r == -2
        np.testing.assert_array_equal(st_r, st)
        np.testing.assert_array_equal(out_r, out)
