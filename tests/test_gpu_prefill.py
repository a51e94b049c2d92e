"""Grouped-GEMM prefill (mqh_moe_prefill) against the oracle.

The oracle is the reference's run_moe_sequence arithmetic (moe_layer.py:110-195):
every (token, slot) pair through moe_quant_expert, ``result[t] += w * y`` in
top-k order (FP32), then ``+ sigmoid(x . g_inp) * shared(x)``.  Tolerance: max
relative error <= 1e-3 per token; the kernels' integer MFMA operands are exact,
so the measured error is FP32 summation noise and is also held to 1e-4.
"""
from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import host_expert, make_layer, oracle_layer

pytestmark = pytest.mark.gpu

TOL = 1e-3
TIGHT = 1e-4


def bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def routing(rng, T, E, k):
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32) + 0.05
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def run_prefill(layer, X, ids, ws, x_bf16=False, use_shared=True, runner=None):
    import torch

    from flash_moe_hip.moe_gpu import MoeRunner

    runner = runner or MoeRunner()
    x = torch.from_numpy(np.ascontiguousarray(X, np.float32)).cuda()
    if x_bf16:
        x = x.to(torch.bfloat16)
    tid = torch.from_numpy(np.ascontiguousarray(ids, np.int32)).cuda()
    tw = torch.from_numpy(np.ascontiguousarray(ws, np.float32)).cuda()
    y = runner.prefill(layer, x, tid, tw, use_shared=use_shared)
    return y.cpu().numpy(), runner.status()


def check(oracle_mod, layer, host, shared, X, ids, ws, got, label):
    worst = 0.0
    for t in range(X.shape[0]):
        want = oracle_layer(oracle_mod, layer, host, shared, X[t], list(ids[t]), list(ws[t]))
        worst = max(worst, oracle_mod.max_relative_error(got[t], want))
    print(f"  {label}: max rel err {worst:.3e}", flush=True)
    assert worst <= TOL
    assert worst <= TIGHT
    return worst


@pytest.fixture(scope="module")
def bench_shape_layer(hip):
    # 16 experts of the benchmark shape: gate/up Q4_K [512x2048], down Q6_K, shared the same
    types = {"gate": 12, "up": 12, "down": 14}
    return make_layer(11, 16, 2048, 512, types, shared_types=types)


@pytest.mark.parametrize("x_bf16", [True, False], ids=["bf16", "fp32"])
def test_prefill_bench_shape(bench_shape_layer, oracle_mod, x_bf16):
    layer, host, shared = bench_shape_layer
    rng = np.random.default_rng(3)
    T = 40
    X = rng.standard_normal((T, 2048)).astype(np.float32)
    if x_bf16:
        X = bf16(X)
    ids, ws = routing(rng, T, 16, 8)
    print(f"prefill T={T} E=16 top8 bf16={x_bf16}", flush=True)
    got, st = run_prefill(layer, X, ids, ws, x_bf16=x_bf16)
    assert st == 0
    check(oracle_mod, layer, host, shared, X, ids, ws, got, "bench shape")


@pytest.mark.parametrize("types", [(11, 11), (13, 12), (14, 14), (12, 13), (11, 14), (12, 11)])
# (intermediate 256 .. 2048: 4 .. 32 row chunks, so one to fifteen two-chunk
# workgroups a tile ahead of the one-chunk ones in the gate/up launch)
@pytest.mark.parametrize("shape", [(256, 256), (512, 1024), (1024, 256), (256, 2048), (2048, 1024)])
def test_prefill_type_pairs(oracle_mod, hip, types, shape):
    gt, dt = types
    H, I = shape
    kinds = {"gate": gt, "up": gt, "down": dt}
    layer, host, shared = make_layer(100 + gt + dt + H // 256 + I, 8, H, I, kinds, shared_types=kinds)
    rng = np.random.default_rng(gt * dt + H + I)
    T = 21
    X = rng.standard_normal((T, H)).astype(np.float32)
    ids, ws = routing(rng, T, 8, 3)
    print(f"prefill types={types} H={H} I={I} T={T}", flush=True)
    got, st = run_prefill(layer, X, ids, ws)
    assert st == 0
    check(oracle_mod, layer, host, shared, X, ids, ws, got, f"types {types} shape {shape}")


def test_prefill_multi_tile_experts_and_repeats(oracle_mod, hip):
    """More than 16 tokens per expert (several tiles per expert), the same
    workspace reused for a larger then a smaller prompt."""
    from flash_moe_hip.moe_gpu import MoeRunner

    kinds = {"gate": 12, "up": 12, "down": 14}
    layer, host, shared = make_layer(21, 4, 512, 256, kinds, shared_types=kinds)
    runner = MoeRunner()
    rng = np.random.default_rng(8)
    for T in (70, 9):
        X = rng.standard_normal((T, 512)).astype(np.float32)
        ids, ws = routing(rng, T, 4, 2)
        print(f"prefill multi-tile T={T}", flush=True)
        got, st = run_prefill(layer, X, ids, ws, runner=runner)
        assert st == 0
        check(oracle_mod, layer, host, shared, X, ids, ws, got, f"T={T}")


def test_prefill_single_token_matches_decode(bench_shape_layer, oracle_mod):
    import torch

    from flash_moe_hip.moe_gpu import MoeRunner

    layer, host, shared = bench_shape_layer
    rng = np.random.default_rng(4)
    X = rng.standard_normal((1, 2048)).astype(np.float32)
    ids, ws = routing(rng, 1, 16, 8)
    got, st = run_prefill(layer, X, ids, ws)
    assert st == 0
    check(oracle_mod, layer, host, shared, X, ids, ws, got, "T=1")
    runner = MoeRunner()
    y = runner.decode(layer, torch.from_numpy(X).cuda(), torch.from_numpy(ids).cuda(),
                      torch.from_numpy(ws).cuda()).cpu().numpy()
    assert oracle_mod.max_relative_error(got[0], y[0]) <= TIGHT


def test_prefill_without_shared_and_without_gate(oracle_mod, hip):
    kinds = {"gate": 14, "up": 14, "down": 12}
    layer, host, shared = make_layer(31, 8, 256, 512, kinds, shared_types=kinds)
    rng = np.random.default_rng(9)
    T = 17
    X = rng.standard_normal((T, 256)).astype(np.float32)
    ids, ws = routing(rng, T, 8, 4)
    got, st = run_prefill(layer, X, ids, ws, use_shared=False)
    assert st == 0
    check(oracle_mod, layer, host, None, X, ids, ws, got, "no shared")
    # shared expert without the sigmoid gate vector: scale 1
    layer.shared.gate_inp = None
    shared_nogate = dict(shared)
    got, st = run_prefill(layer, X, ids, ws)
    assert st == 0
    worst = 0.0
    for t in range(T):
        outs = [oracle_mod.expert_forward(host_expert(host, layer, e), layer.types, X[t], 256, 512) for e in ids[t]]
        sh = oracle_mod.expert_forward({r: shared_nogate[r] for r in ("gate", "up", "down")}, kinds, X[t], 256, 512)
        want = oracle_mod.combine(outs, list(ws[t]), sh)
        worst = max(worst, oracle_mod.max_relative_error(got[t], want))
    print(f"  shared without gate: max rel err {worst:.3e}", flush=True)
    assert worst <= TIGHT


def test_prefill_shared_of_other_type_goes_through_decode(oracle_mod, hip):
    kinds = {"gate": 12, "up": 12, "down": 14}
    sh_kinds = {"gate": 14, "up": 14, "down": 14}
    layer, host, shared = make_layer(41, 8, 512, 256, kinds, shared_types=sh_kinds, sh_I=512)
    rng = np.random.default_rng(10)
    T = 12
    X = rng.standard_normal((T, 512)).astype(np.float32)
    ids, ws = routing(rng, T, 8, 2)
    got, st = run_prefill(layer, X, ids, ws)
    assert st == 0
    check(oracle_mod, layer, host, shared, X, ids, ws, got, "shared via decode")


def test_prefill_bad_expert_id_flags(oracle_mod, hip):
    kinds = {"gate": 12, "up": 12, "down": 14}
    layer, host, shared = make_layer(51, 8, 256, 256, kinds, shared_types=kinds)
    rng = np.random.default_rng(12)
    T = 5
    X = rng.standard_normal((T, 256)).astype(np.float32)
    ids, ws = routing(rng, T, 8, 2)
    ids[2, 1] = 8          # out of range
    got, st = run_prefill(layer, X, ids, ws)
    assert st == -9
    # the valid tokens are still right
    for t in (0, 1, 3, 4):
        want = oracle_layer(oracle_mod, layer, host, shared, X[t], list(ids[t]), list(ws[t]))
        assert oracle_mod.max_relative_error(got[t], want) <= TIGHT


def test_backend_moe_tokens_uses_prefill(oracle_mod, hip):
    """run_moe_sequence through HipExpertBackend.moe_tokens on a multi-token prompt."""
    from flash_moe_hip.backend import HipExpertBackend
    from flash_moe_hip.moe_layer import run_moe_sequence
    from flash_moe_hip.shared_expert import SharedExpert

    kinds = {"gate": 12, "up": 12, "down": 14}
    layer, host, shared = make_layer(61, 16, 512, 256, kinds, shared_types=kinds)
    rng = np.random.default_rng(13)
    W = (rng.standard_normal((512, 16)) * 0.05).astype(np.float32)

    class Router:
        def route(self, x):
            return oracle_mod.route(x, W, 4)

    backend = HipExpertBackend({0: layer})
    sh = SharedExpert.from_backend(backend)
    X = rng.standard_normal((24, 512)).astype(np.float32)
    got = run_moe_sequence(0, X, Router(), backend, 512, 256, shared_expert=sh)
    worst = 0.0
    for t in range(24):
        ids, ws = oracle_mod.route(X[t], W, 4)
        want = oracle_layer(oracle_mod, layer, host, shared, X[t], ids, ws)
        worst = max(worst, oracle_mod.max_relative_error(got[t], want))
    print(f"  run_moe_sequence via prefill: max rel err {worst:.3e}", flush=True)
    assert worst <= TIGHT


def _sweep_case(seed):
    rng = np.random.default_rng(5000 + seed)
    gt, dt = (int(v) for v in rng.choice([11, 12, 13, 14], 2))
    T = int(rng.choice([5, 17, 33]))
    H = int(rng.choice([256, 512, 1024]))
    I = int(rng.choice([256, 512]))
    E = int(rng.choice([8, 32, 96]))
    k = int(rng.choice([1, 3, 8]))
    sh = str(rng.choice(["none", "same", "q6k"]))
    return gt, dt, T, H, I, E, k, sh, bool(rng.integers(2))


@pytest.mark.parametrize("seed", range(12))
def test_prefill_sweep(oracle_mod, hip, seed):
    """Seeded prefill cases with ragged token counts (the route pass stages four
    tokens a workgroup and cuts 16-token tiles, so 5, 17 and 33 tokens leave
    partial staging groups and tiles), BF16 or FP32 tokens, every prefill type
    as gate/up and as down, with no shared expert, one of the routed types or a
    Q6_K one: every token against the oracle."""
    gt, dt, T, H, I, E, k, sh, xb = _sweep_case(seed)
    kinds = {"gate": gt, "up": gt, "down": dt}
    st = None if sh == "none" else (kinds if sh == "same" else {"gate": 14, "up": 14, "down": 14})
    layer, host, shared = make_layer(7000 + seed, E, H, I, kinds, shared_types=st)
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((T, H)).astype(np.float32)
    if xb:
        X = bf16(X)
    ids, ws = routing(rng, T, E, k)
    print(f"prefill sweep {seed}: types {gt}/{dt} T={T} H={H} I={I} E={E} k={k} shared={sh} bf16={xb}", flush=True)
    got, st_ = run_prefill(layer, X, ids, ws, x_bf16=xb)
    assert st_ == 0
    check(oracle_mod, layer, host, shared, X, ids, ws, got, f"sweep {seed}")


@pytest.mark.parametrize("routed", [(11, 11), (12, 8), (13, 14), (12, 11), (11, 8)])
@pytest.mark.parametrize("shape", [(256, 256), (512, 1024), (1024, 2048), (2048, 512)])
def test_prefill_q6k_shared_beside_other_routed_types(oracle_mod, hip, routed, shape):
    """A Q6_K shared expert in the grouped launches beside routed experts of
    other types (its tiles run their own instance of the GEMM body), and Q8_0
    down projections (per-block scales applied per MFMA step): every token
    against the oracle, BF16 tokens for even intermediate sizes (the high
    plane only) and FP32 tokens for the others (both planes)."""
    from flash_moe_hip.moe_gpu import MoeRunner

    gt, dt = routed
    H, I = shape
    kinds = {"gate": gt, "up": gt, "down": dt}
    q6 = {"gate": 14, "up": 14, "down": 14}
    layer, host, shared = make_layer(700 + gt + dt + H // 256 + I, 12, H, I, kinds, shared_types=q6)
    assert MoeRunner._shared_in_prefill(layer)
    rng = np.random.default_rng(gt * 31 + dt + H + I)
    T = 37
    x_bf16 = (I // 256) % 2 == 0
    X = rng.standard_normal((T, H)).astype(np.float32)
    if x_bf16:
        X = bf16(X)
    ids, ws = routing(rng, T, 12, 4)
    print(f"prefill routed={routed} + Q6_K shared H={H} I={I} T={T} bf16={x_bf16}", flush=True)
    got, st = run_prefill(layer, X, ids, ws, x_bf16=x_bf16)
    assert st == 0
    check(oracle_mod, layer, host, shared, X, ids, ws, got, f"routed {routed} shape {shape}")


@pytest.mark.parametrize("shape", [(512, 256), (2048, 1024)])
def test_prefill_q8_0_down_without_shared(oracle_mod, hip, shape):
    """Q8_0 down projections with no shared expert, and the shared expert
    switched off on a layer that has one (use_shared=False)."""
    H, I = shape
    kinds = {"gate": 12, "up": 12, "down": 8}
    layer, host, shared = make_layer(750 + H + I, 6, H, I, kinds, shared_types={"gate": 14, "up": 14, "down": 14})
    rng = np.random.default_rng(H + I)
    T = 23
    X = rng.standard_normal((T, H)).astype(np.float32)
    ids, ws = routing(rng, T, 6, 3)
    print(f"prefill Q8_0 down, no shared, H={H} I={I}", flush=True)
    got, st = run_prefill(layer, X, ids, ws, use_shared=False)
    assert st == 0
    check(oracle_mod, layer, host, None, X, ids, ws, got, f"Q8_0 down {shape}")
