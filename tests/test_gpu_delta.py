"""DeltaNet decode recurrence on the GPU (mqh_delta_heads, moe_delta_heads)
against the oracle (oracle/delta_oracle.c, itself bit-identical to the
reference's cpp/moe_delta.cpp).

The kernel keeps the reference's summation order and separate roundings, so
state and outputs must equal the oracle's bit for bit after 40 steps.  With
gate = 0 the decay is exactly 1; with random gates it is the device's double
exp(gate), which agrees with the host libm's on every seeded input here (a
last-bit difference there would be the only admissible deviation).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(32, 128, 128), (3, 7, 9), (4, 5, 200), (2, 3, 1), (1, 2, 1024), (256, 1, 8), (5, 16, 15), (16, 64, 64)]


def inputs(rng, nv, dv, dk, zero_gate=False):
    q = (rng.standard_normal((nv, dk)) * 0.05).astype(np.float32)
    k = (rng.standard_normal((nv, dk)) * 0.05).astype(np.float32)
    v = (rng.standard_normal((nv, dv)) * 0.1).astype(np.float32)
    beta = rng.uniform(0.01, 0.99, nv).astype(np.float32)
    gate = np.zeros(nv, np.float32) if zero_gate else (-rng.uniform(0.001, 5, nv)).astype(np.float32)
    return q, k, v, beta, gate


@pytest.mark.parametrize("zero_gate", [True, False], ids=["decay1", "random-gate"])
@pytest.mark.parametrize("shape", SHAPES)
def test_device_state_matches_oracle(oracle_mod, shape, zero_gate):
    import torch
    from flash_moe_hip.native_expert import DeltaState

    rng = np.random.default_rng(sum(shape) + int(zero_gate))
    nv, dv, dk = shape
    host = (rng.standard_normal(shape) * 0.01).astype(np.float32)
    dev = DeltaState(nv, dv, dk, state=host)
    print(f"delta heads={nv} value_dim={dv} key_dim={dk} zero_gate={zero_gate}", flush=True)
    for step in range(40):
        args = inputs(rng, nv, dv, dk, zero_gate)
        rc, want = oracle_mod.delta_heads(host, *args)
        assert rc == 0
        got = dev.step(*[torch.from_numpy(a).cuda() for a in args]).cpu().numpy()
        st = dev.state.cpu().numpy()
        np.testing.assert_array_equal(got, want, err_msg=f"step {step}")
        np.testing.assert_array_equal(st, host, err_msg=f"step {step}")
    assert dev.status() == 0


def test_host_pointer_drop_in_matches_oracle(oracle_mod):
    """NativeExpert.delta (moe_delta_heads through host pointers), the
    reference's NativeDelta contract."""
    from flash_moe_hip.native_expert import NativeExpert

    native = NativeExpert().delta
    assert native is not None
    rng = np.random.default_rng(11)
    for nv, dv, dk in ((32, 128, 128), (3, 7, 9)):
        a = (rng.standard_normal((nv, dv, dk)) * 0.01).astype(np.float32)
        b = a.copy()
        for _ in range(10):
            args = inputs(rng, nv, dv, dk, zero_gate=True)
            rc, want = oracle_mod.delta_heads(a, *args)
            got = native.forward(b, *args)
            np.testing.assert_array_equal(got, want)
            np.testing.assert_array_equal(b, a)
        with pytest.raises(ValueError):
            native.forward(b, *inputs(rng, nv, dv, dk + 1))


def test_non_finite_output_is_reported(oracle_mod):
    import torch
    from flash_moe_hip import _lib
    from flash_moe_hip.native_expert import DeltaState, NativeExpert

    rng = np.random.default_rng(12)
    nv, dv, dk = 4, 8, 16
    q, k, v, beta, gate = inputs(rng, nv, dv, dk)
    v[2, 5] = np.nan
    state = np.zeros((nv, dv, dk), np.float32)
    lib = _lib.load()
    out = np.empty((nv, dv), np.float32)
    rc = lib.moe_delta_heads(state.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, beta.ctypes.data,
                             gate.ctypes.data, out.ctypes.data, nv, dk, dv)
    assert rc == -2
    # the reference's side effects (moe_delta.cpp:30-66), which the oracle pins:
    # state rows up to and including the bad one updated, outputs before it
    # written, everything after it as the caller left it -- bit for bit
    st0 = (rng.standard_normal((nv, dv, dk)) * 0.01).astype(np.float32)
    st_o, out_o = st0.copy(), np.full((nv, dv), 7.0, np.float32)
    assert oracle_mod.delta_heads(st_o, q, k, v, beta, gate, out=out_o)[0] == -2
    st_g, out_g = st0.copy(), np.full((nv, dv), 7.0, np.float32)
    rc = lib.moe_delta_heads(st_g.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, beta.ctypes.data,
                             gate.ctypes.data, out_g.ctypes.data, nv, dk, dv)
    assert rc == -2
    np.testing.assert_array_equal(st_g, st_o)
    np.testing.assert_array_equal(out_g, out_o)
    np.testing.assert_array_equal(out_g.reshape(-1)[2 * dv + 5:], 7.0)
    with pytest.raises(RuntimeError, match="status -2"):
        NativeExpert().delta.forward(np.zeros((nv, dv, dk), np.float32), q, k, v, beta, gate)
    dev = DeltaState(nv, dv, dk)
    dev.step(*[torch.from_numpy(a).cuda() for a in (q, k, v, beta, gate)])
    assert dev.status() == -4
    v[2, 5] = 0.1
    dev.reset()
    dev.step(*[torch.from_numpy(a).cuda() for a in (q, k, v, beta, gate)])
    assert dev.status() == 0
