"""Seeded sweep of layer configurations through every device path, against the oracle.

Each case draws the routed and shared types (all six decodable types, gate type =
up type), hidden and intermediate sizes, expert count, top-k and token count,
then checks: the fused decode on the default and generic paths
(max relative error <= 1e-3 per token against the oracle's run_moe_layer); the
grouped prefill where its kernels take the layer (same bar); and the routed
decode, bit for bit against route() followed by decode().  Layers with IQ4_NL
(which the reference's moe_quant_expert does not take) are checked against the
float64 SwiGLU of the oracle-dequantized weights instead.
"""
from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import _f64_expert, host_expert, make_layer, oracle_layer

pytestmark = pytest.mark.gpu

TOL = 1e-3
TYPES = (8, 11, 12, 13, 14, 20)


def draw(seed):
    rng = np.random.default_rng(seed)
    gt, dt = (int(v) for v in rng.choice(TYPES, 2))
    H = int(rng.choice([256, 512, 1024, 2048]))
    I = int(rng.choice([256, 512, 1024]))
    E = int(rng.choice([4, 16, 64]))
    k = int(rng.choice([1, 2, 4, 8]))
    k = min(k, E)
    T = int(rng.choice([1, 3, 8]))
    sh = rng.choice(["none", "same", "q6k"])
    shared = None if sh == "none" else ({"gate": gt, "up": gt, "down": dt} if sh == "same"
                                        else {"gate": 14, "up": 14, "down": 14})
    return dict(types={"gate": gt, "up": gt, "down": dt}, H=H, I=I, E=E, k=k, T=T, shared=shared)


@pytest.mark.parametrize("seed", range(24))
def test_layer_sweep(hip, oracle_mod, seed):
    import torch
    from flash_moe_hip.moe_gpu import MoeRunner

    c = draw(1000 + seed)
    print(f"sweep {seed}: {c}", flush=True)
    layer, host, shared = make_layer(seed, c["E"], c["H"], c["I"], c["types"], shared_types=c["shared"])
    rng = np.random.default_rng(seed + 7)
    T, k, E, H = c["T"], c["k"], c["E"], c["H"]
    X = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    ws = rng.dirichlet(np.ones(k), size=T).astype(np.float32)
    types_used = set(c["types"].values()) | (set(c["shared"].values()) if c["shared"] else set())
    if 20 in types_used:
        def ref(t):
            y = sum(float(w) * _f64_expert(oracle_mod, host_expert(host, layer, int(e)), c["types"], X[t], H, c["I"])
                    for e, w in zip(ids[t], ws[t]))
            if shared is not None:
                g = 1.0 / (1.0 + np.exp(-float(X[t].astype(np.float64) @ shared["gate_inp"])))
                y = y + g * _f64_expert(oracle_mod, {r: shared[r] for r in ("gate", "up", "down")}, shared["types"],
                                        X[t], H, shared["intermediate"])
            return y.astype(np.float32)
        want = [ref(t) for t in range(T)]
    else:
        want = [oracle_layer(oracle_mod, layer, host, shared, X[t], ids[t].tolist(), ws[t].tolist())
                for t in range(T)]
    runner = MoeRunner()
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (X, ids, ws))
    for path in (0, 1):
        old = hip.mqh_set_decode_path(path)
        try:
            y = runner.decode(layer, xd, idd, wd).cpu().numpy()
        finally:
            hip.mqh_set_decode_path(old)
        assert runner.status() == 0
        for t in range(T):
            err = oracle_mod.max_relative_error(y[t], want[t])
            assert err <= TOL, (seed, path, t, err)
    if MoeRunner.prefill_supported(layer):
        yp = runner.prefill(layer, xd, idd, wd).cpu().numpy()
        assert runner.status() == 0
        for t in range(T):
            err = oracle_mod.max_relative_error(yp[t], want[t])
            assert err <= TOL, (seed, "prefill", t, err)
    layer.router_weights = (rng.standard_normal((H, E)) * 0.05).astype(np.float32)
    yr, rid, rw = runner.decode_routed(layer, xd, k)
    y2 = runner.decode(layer, xd, rid, rw)
    torch.cuda.synchronize()
    assert runner.status() == 0
    np.testing.assert_array_equal(yr.cpu().numpy(), y2.cpu().numpy())
