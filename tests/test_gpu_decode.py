"""Fused decode (all routed experts + shared expert in one call) against the oracle.

The oracle layer is the reference's run_moe_layer arithmetic: each routed
expert through moe_quant_expert, ``combined += w_k * y_k`` in top-k order
(FP32), plus ``sigmoid(x . g_inp) * shared(x)``.  Tolerance: max relative
error <= 1e-3.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3
ROLES = ("gate", "up", "down")


def make_layer(seed, n_experts, H, I, types, shared_types=None, sh_I=None, scale=0.01):
    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.synthetic import random_stack

    rng = np.random.default_rng(seed)
    shapes = {"gate": (I, H), "up": (I, H), "down": (H, I)}
    host = {r: random_stack(rng, types[r], n_experts, *shapes[r], scale=scale) for r in ROLES}
    shared = None
    if shared_types is not None:
        sh_I = sh_I or I
        sshapes = {"gate": (sh_I, H), "up": (sh_I, H), "down": (H, sh_I)}
        shared = {r: random_stack(rng, shared_types[r], 1, *sshapes[r], scale=scale) for r in ROLES}
        shared.update(types=shared_types, intermediate=sh_I,
                      gate_inp=(rng.standard_normal(H) * 0.02).astype(np.float32))
    layer = ExpertLayer.from_host(host, types, n_experts, H, I, shared=shared)
    return layer, host, shared


def host_expert(host, layer, e):
    return {r: host[r][e * layer.expert_bytes(r):(e + 1) * layer.expert_bytes(r)] for r in ROLES}


def oracle_layer(oracle_mod, layer, host, shared, x, ids, weights, fp16=0, shared_semantics="kernel"):
    H, I = layer.hidden, layer.intermediate
    outs = [oracle_mod.expert_forward(host_expert(host, layer, e), layer.types, x, H, I, fp16) for e in ids]
    sh_out = None
    if shared is not None:
        gate = oracle_mod._sigmoid(np.float32(x @ shared["gate_inp"]).reshape(()))
        if shared_semantics == "kernel":
            y = oracle_mod.expert_forward({r: shared[r] for r in ROLES}, shared["types"], x, H,
                                          shared["intermediate"], 0)
            sh_out = (gate * y).astype(np.float32)
        else:   # reference SharedExpert: FP16-dequantized weights promoted to FP32
            si = shared["intermediate"]
            w = {r: oracle_mod.dequant(shared["types"][r], shared[r], want_f16=True).astype(np.float32)
                 for r in ROLES}
            sh_out = oracle_mod.shared_expert_forward(x, w["gate"].reshape(si, H), w["up"].reshape(si, H),
                                                      w["down"].reshape(H, si), shared["gate_inp"])
    return oracle_mod.combine(outs, weights, sh_out)


def run(layer, X, ids, ws, fp16=0, use_shared=True):
    import torch

    from flash_moe_hip.moe_gpu import MoeRunner

    runner = MoeRunner()
    x = torch.from_numpy(np.ascontiguousarray(X, np.float32)).cuda()
    tid = torch.from_numpy(np.ascontiguousarray(ids, np.int32)).cuda() if ids is not None else None
    tw = torch.from_numpy(np.ascontiguousarray(ws, np.float32)).cuda() if ws is not None else None
    y = runner.decode(layer, x, tid, tw, fp16_graph=fp16, use_shared=use_shared)
    out = y.cpu().numpy()
    return out, runner.status()


@pytest.fixture(params=[0, 1], ids=["two-kernel", "generic"])
def path(request, hip):
    """Run the test through the two integer-digit kernels and the generic kernels."""
    old = hip.mqh_set_decode_path(request.param)
    yield request.param
    hip.mqh_set_decode_path(old)


def expect_kernels(hip):
    """Every decode launches two kernels (gate/up + SwiGLU, then down + combine)."""
    assert hip.mqh_last_decode_kernels() == 2


def test_removed_decode_path_rejected(hip):
    """Only paths 0 (fast kernels) and 1 (generic kernels) exist."""
    old = hip.mqh_set_decode_path(0)
    assert hip.mqh_set_decode_path(2) == -1
    assert hip.mqh_set_decode_path(old) == 0


@pytest.fixture(scope="module")
def decode_layer(hip):
    # 32 experts of the benchmark shape: gate/up Q4_K [512x2048], down Q6_K, shared the same
    types = {"gate": 12, "up": 12, "down": 14}
    return make_layer(7, 32, 2048, 512, types, shared_types=types)


def test_one_token_top8_plus_shared(decode_layer, oracle_mod, hip, path):
    layer, host, shared = decode_layer
    rng = np.random.default_rng(1)
    x = rng.standard_normal(2048).astype(np.float32)
    W = (rng.standard_normal((2048, 32)) * 0.02).astype(np.float32)
    ids, ws = oracle_mod.route(x, W, 8)
    print(f"decode 1 token path={path} ids={ids}", flush=True)
    got, st = run(layer, x[None], np.array([ids]), np.array([ws]))
    assert st == 0
    expect_kernels(hip)
    want = oracle_layer(oracle_mod, layer, host, shared, x, ids, ws)
    err = oracle_mod.max_relative_error(got[0], want)
    print(f"  max rel err (kernel semantics) {err:.3e}", flush=True)
    assert err <= TOL
    want_ref = oracle_layer(oracle_mod, layer, host, shared, x, ids, ws, shared_semantics="reference")
    err_ref = oracle_mod.max_relative_error(got[0], want_ref)
    print(f"  max rel err (reference shared semantics) {err_ref:.3e}", flush=True)
    assert err_ref <= TOL


def test_shared_only_and_no_shared(decode_layer, oracle_mod, path):
    layer, host, shared = decode_layer
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    got, st = run(layer, x, None, None)
    assert st == 0
    for t in range(3):
        want = oracle_layer(oracle_mod, layer, host, shared, x[t], [], [])
        assert oracle_mod.max_relative_error(got[t], want) <= TOL
    ids = np.array([[3, 5], [0, 31], [7, 7]])
    ws = np.array([[0.75, 0.25], [0.5, 0.5], [0.1, 0.9]])
    got, st = run(layer, x, ids, ws, use_shared=False)
    assert st == 0
    for t in range(3):
        want = oracle_layer(oracle_mod, layer, host, None, x[t], ids[t], ws[t])
        assert oracle_mod.max_relative_error(got[t], want) <= TOL


def test_bad_expert_id_is_reported(decode_layer, path):
    layer, _, _ = decode_layer
    x = np.ones((1, 2048), np.float32)
    _, st = run(layer, x, np.array([[1, 32]]), np.array([[0.5, 0.5]]))
    assert st == -9
    _, st = run(layer, x, np.array([[1, 2]]), np.array([[0.5, 0.5]]))
    assert st == 0


def test_batched_tokens_q3k(hip, oracle_mod, path):
    """16 tokens through an all-Q3_K layer, top-8 of N(0,1) logits (experts overlap)."""
    types = {"gate": 11, "up": 11, "down": 11}
    layer, host, shared = make_layer(11, 24, 2048, 512, types, shared_types=types)
    rng = np.random.default_rng(3)
    X = rng.standard_normal((16, 2048)).astype(np.float32)
    logits = rng.standard_normal((16, 24)).astype(np.float32)
    ids = np.argsort(-logits, axis=1)[:, :8]
    sel = np.take_along_axis(logits, ids, 1).astype(np.float64)
    ws = np.exp(sel - sel.max(1, keepdims=True))
    ws /= ws.sum(1, keepdims=True)
    got, st = run(layer, X, ids, ws)
    assert st == 0
    expect_kernels(hip)
    worst = 0.0
    for t in range(16):
        want = oracle_layer(oracle_mod, layer, host, shared, X[t], ids[t].tolist(), ws[t].tolist())
        worst = max(worst, oracle_mod.max_relative_error(got[t], want))
    print(f"batched q3k path={path} worst max rel err {worst:.3e}", flush=True)
    assert worst <= TOL


def test_fp16_graph_routed_experts(hip, oracle_mod):
    """FP16 graph on the routed experts (small-magnitude inputs as in the reference KAT),
    FP32 graph on the shared expert."""
    types = {"gate": 12, "up": 13, "down": 14}
    layer, host, shared = make_layer(13, 8, 256, 256, types, shared_types={"gate": 14, "up": 14, "down": 14},
                                     scale=0.002)
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(256) * 0.005).astype(np.float32)
    ids, ws = [5, 1, 2], [0.5, 0.3, 0.2]
    got, st = run(layer, x[None], np.array([ids]), np.array([ws]), fp16=1)
    assert st == 0
    want = oracle_layer(oracle_mod, layer, host, shared, x, ids, ws, fp16=1)
    err = oracle_mod.max_relative_error(got[0], want)
    print(f"fp16 graph max rel err {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("types", [(12, 14), (11, 11), (13, 12), (14, 14), (12, 13), (11, 14)])
def test_fast_type_pairs(hip, oracle_mod, types):
    """Every (gate/up, down) type pair of the two-kernel path, 3 tokens, at
    several shapes, against the oracle."""
    gu, dn = types
    t = {"gate": gu, "up": gu, "down": dn}
    for H, I in ((256, 256), (2048, 512), (512, 1024), (1024, 256), (1024, 1024), (2048, 1024)):
        layer, host, shared = make_layer(29 + gu + dn, 6, H, I, t, shared_types=t)
        rng = np.random.default_rng(H + I)
        X = rng.standard_normal((3, H)).astype(np.float32)
        ids = np.array([[0, 5, 2], [3, 3, 1], [4, 0, 5]])
        ws = np.array([[0.5, 0.3, 0.2], [0.6, 0.2, 0.2], [0.4, 0.4, 0.2]])
        want = [oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist())
                for tok in range(3)]
        print(f"fast types={types} H={H} I={I}", flush=True)
        old = hip.mqh_set_decode_path(0)
        try:
            got, st = run(layer, X, ids, ws)
            expect_kernels(hip)
        finally:
            hip.mqh_set_decode_path(old)
        assert st == 0
        for tok in range(3):
            err = oracle_mod.max_relative_error(got[tok], want[tok])
            assert err <= TOL, (types, H, I, tok, err)


@pytest.mark.parametrize("types,sh_types", [((12, 8), (14, 14)), ((8, 8), (8, 8)), ((8, 14), (14, 14)),
                                            ((11, 8), (11, 8)), ((13, 8), None)])
def test_fast_q8_0(hip, oracle_mod, types, sh_types):
    """Q8_0 gate/up or down projections in the integer-digit kernels (the
    reference model's first layer has a Q8_0 down projection), 3 tokens, against
    the oracle and against the generic kernels."""
    gu, dn = types
    t = {"gate": gu, "up": gu, "down": dn}
    st_ = None if sh_types is None else {"gate": sh_types[0], "up": sh_types[0], "down": sh_types[1]}
    for H, I in ((256, 256), (2048, 512), (512, 1024), (1024, 2048)):
        layer, host, shared = make_layer(31 + gu + dn, 6, H, I, t, shared_types=st_)
        rng = np.random.default_rng(H + 3 * I)
        X = rng.standard_normal((3, H)).astype(np.float32)
        ids = np.array([[0, 5, 2], [3, 3, 1], [4, 0, 5]])
        ws = np.array([[0.5, 0.3, 0.2], [0.6, 0.2, 0.2], [0.4, 0.4, 0.2]])
        want = [oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist())
                for tok in range(3)]
        got = {}
        for path in (0, 1):
            print(f"q8_0 types={types} shared={sh_types} H={H} I={I} path={path}", flush=True)
            old = hip.mqh_set_decode_path(path)
            try:
                got[path], st = run(layer, X, ids, ws)
            finally:
                hip.mqh_set_decode_path(old)
            assert st == 0
            for tok in range(3):
                err = oracle_mod.max_relative_error(got[path][tok], want[tok])
                assert err <= TOL, (types, H, I, path, tok, err)
        assert not np.array_equal(got[0], got[1])   # the digit kernels ran, not the FP32 ones


def test_fast_repeated_launches_share_workspace(decode_layer, oracle_mod, hip):
    """Back-to-back launches on one workspace with no host synchronisation in
    between, read once at the end: each result is its own."""
    import torch

    from flash_moe_hip.moe_gpu import MoeRunner

    layer, host, shared = decode_layer
    rng = np.random.default_rng(9)
    runner = MoeRunner()
    xs = [rng.standard_normal((1, 2048)).astype(np.float32) for _ in range(5)]
    ids = [rng.permutation(32)[:8].reshape(1, 8) for _ in range(5)]
    ws = [rng.dirichlet(np.ones(8)).astype(np.float32).reshape(1, 8) for _ in range(5)]
    xd = [torch.from_numpy(v).cuda() for v in xs]
    idd = [torch.from_numpy(v.astype(np.int32)).cuda() for v in ids]
    wd = [torch.from_numpy(v).cuda() for v in ws]
    ys = []
    for k in range(5):
        ys.append(runner.decode(layer, xd[k], idd[k], wd[k]))
    expect_kernels(hip)
    assert runner.status() == 0
    for k in range(5):
        want = oracle_layer(oracle_mod, layer, host, shared, xs[k][0], ids[k][0].tolist(), ws[k][0].tolist())
        assert oracle_mod.max_relative_error(ys[k].cpu().numpy()[0], want) <= TOL


@pytest.mark.parametrize("routed", [(12, 14), (11, 11), (13, 12), (14, 14)])
def test_shared_expert_q6k_with_other_routed_types(hip, oracle_mod, routed):
    """The reference model's layout: routed experts Q4_K/Q3_K (down Q6_K, Q3_K),
    the shared expert all Q6_K.  The fast kernels run the shared slot with its
    own type; 3 tokens (one row group per wave in kernel B) and 16 tokens (four
    or two), against the oracle and the generic kernels."""
    gu, dn = routed
    t = {"gate": gu, "up": gu, "down": dn}
    sh = {"gate": 14, "up": 14, "down": 14}
    layer, host, shared = make_layer(90 + gu + dn, 12, 2048, 512, t, shared_types=sh)
    rng = np.random.default_rng(gu * 10 + dn)
    for T in (3, 16):
        X = rng.standard_normal((T, 2048)).astype(np.float32)
        ids = np.stack([rng.permutation(12)[:8] for _ in range(T)])
        ws = rng.dirichlet(np.ones(8), size=T).astype(np.float32)
        print(f"mixed shared types routed={routed} T={T}", flush=True)
        got, st = run(layer, X, ids, ws)
        assert st == 0
        old = hip.mqh_set_decode_path(1)
        try:
            gen, st = run(layer, X, ids, ws)
        finally:
            hip.mqh_set_decode_path(old)
        assert st == 0
        for tok in range(T):
            want = oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist())
            assert oracle_mod.max_relative_error(got[tok], want) <= TOL, (routed, T, tok)
            assert oracle_mod.max_relative_error(got[tok], gen[tok]) <= TOL, (routed, T, tok)


@pytest.mark.parametrize("H,I,k,T", [(512, 512, 9, 1), (512, 512, 8, 2), (512, 256, 4, 4)])
def test_partial_last_workgroup(hip, oracle_mod, H, I, k, T):
    """Shapes whose gate/up work items do not fill the last workgroup of a
    token (3, 5 and 3 waves per workgroup; that workgroup also computes the
    shared expert's sigmoid gate): against the oracle and the generic kernels."""
    t = {"gate": 12, "up": 12, "down": 14}
    layer, host, shared = make_layer(300 + H + k + T, 16, H, I, t, shared_types=t)
    rng = np.random.default_rng(H + I + k + T)
    X = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.permutation(16)[:k] for _ in range(T)])
    ws = rng.dirichlet(np.ones(k), size=T).astype(np.float32)
    print(f"partial last workgroup H={H} I={I} k={k} T={T}", flush=True)
    old = hip.mqh_set_decode_path(0)
    try:
        got, st = run(layer, X, ids, ws)
        assert st == 0
        assert hip.mqh_last_decode_kernels() == 2
        hip.mqh_set_decode_path(1)
        gen, st = run(layer, X, ids, ws)
        assert st == 0
    finally:
        hip.mqh_set_decode_path(old)
    for tok in range(T):
        want = oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist())
        assert oracle_mod.max_relative_error(got[tok], want) <= TOL, (H, I, k, T, tok)
        assert oracle_mod.max_relative_error(got[tok], gen[tok]) <= TOL, (H, I, k, T, tok)


def _f64_expert(oracle_mod, tensors, types, x, H, I):
    g = oracle_mod.dequant(types["gate"], tensors["gate"]).astype(np.float64).reshape(I, H)
    u = oracle_mod.dequant(types["up"], tensors["up"]).astype(np.float64).reshape(I, H)
    d = oracle_mod.dequant(types["down"], tensors["down"]).astype(np.float64).reshape(H, I)
    gx, ux = g @ x.astype(np.float64), u @ x.astype(np.float64)
    return d @ (gx * oracle_mod._sigmoid(gx) * ux)   # the oracle's overflow-free sigmoid


@pytest.mark.parametrize("types", [(20, 20), (12, 20), (20, 14)])
def test_iq4_nl_layer(hip, oracle_mod, types):
    """IQ4_NL experts (the reference decodes IQ4_NL in its fast_dequant library
    and runs the matmuls elsewhere) through the fused decode, against the
    float64 SwiGLU of the oracle-dequantized weights: routed and shared
    experts, 3 tokens, and the routed-on-device form."""
    import torch
    from flash_moe_hip.moe_gpu import MoeRunner

    gu, dn = types
    t = {"gate": gu, "up": gu, "down": dn}
    E, H, I = 6, 512, 256
    layer, host, shared = make_layer(41 + gu + dn, E, H, I, t, shared_types=t)
    rng = np.random.default_rng(43)
    X = rng.standard_normal((3, H)).astype(np.float32)
    ids = np.array([[0, 5, 2], [3, 3, 1], [4, 0, 5]])
    ws = np.array([[0.5, 0.3, 0.2], [0.6, 0.2, 0.2], [0.4, 0.4, 0.2]])
    print(f"iq4_nl types={types}", flush=True)
    got, st = run(layer, X, ids, ws)
    assert st == 0
    sh_t = {r: shared[r] for r in ROLES}
    for tok in range(3):
        ys = [_f64_expert(oracle_mod, host_expert(host, layer, int(e)), t, X[tok], H, I) for e in ids[tok]]
        gate = 1.0 / (1.0 + np.exp(-float(X[tok].astype(np.float64) @ shared["gate_inp"])))
        want = sum(float(w) * y for w, y in zip(ws[tok], ys)) + gate * _f64_expert(oracle_mod, sh_t, t, X[tok], H, I)
        err = oracle_mod.max_relative_error(got[tok], want.astype(np.float32))
        assert err <= TOL, (types, tok, err)
    layer.router_weights = (rng.standard_normal((H, E)) * 0.05).astype(np.float32)
    runner = MoeRunner()
    y, rid, rw = runner.decode_routed(layer, torch.from_numpy(X).cuda(), 3)
    torch.cuda.synchronize()
    assert runner.status() == 0
    y2 = runner.decode(layer, torch.from_numpy(X).cuda(), rid, rw)
    np.testing.assert_array_equal(y.cpu().numpy(), y2.cpu().numpy())


def test_edge_inputs(hip, oracle_mod):
    """Empty token batches, more slots than the digit kernels take (top-20 runs
    the FP32 kernels), a hidden/intermediate pair outside the digit kernels'
    sizes, and a non-finite token reported as -4 (moe_quant_dot.cpp:209-210)."""
    import torch
    from flash_moe_hip.moe_gpu import MoeRunner

    runner = MoeRunner()
    types = {"gate": 12, "up": 12, "down": 14}
    layer, host, shared = make_layer(51, 24, 512, 256, types, shared_types=types)
    empty = torch.empty((0, 512), dtype=torch.float32, device="cuda")
    y = runner.decode(layer, empty, torch.empty((0, 4), dtype=torch.int32, device="cuda"),
                      torch.empty((0, 4), dtype=torch.float32, device="cuda"))
    assert tuple(y.shape) == (0, 512)
    layer.router_weights = np.zeros((512, 24), np.float32)
    y, i, w = runner.decode_routed(layer, empty, 4)
    assert tuple(y.shape) == (0, 512) and tuple(i.shape) == (0, 4)

    rng = np.random.default_rng(52)
    X = rng.standard_normal((2, 512)).astype(np.float32)
    ids = np.stack([rng.permutation(24)[:20] for _ in range(2)])
    ws = rng.dirichlet(np.ones(20), size=2)
    print("top-20 decode", flush=True)
    got, st = run(layer, X, ids, ws)
    assert st == 0
    for t in range(2):
        want = oracle_layer(oracle_mod, layer, host, shared, X[t], ids[t].tolist(), ws[t].tolist())
        assert oracle_mod.max_relative_error(got[t], want) <= TOL

    layer2, host2, shared2 = make_layer(53, 5, 768, 768, types, shared_types=types)
    X2 = rng.standard_normal((2, 768)).astype(np.float32)
    ids2 = np.array([[0, 4], [2, 2]])
    ws2 = np.array([[0.7, 0.3], [0.5, 0.5]])
    print("H=768 I=768 decode", flush=True)
    got2, st = run(layer2, X2, ids2, ws2)
    assert st == 0
    for t in range(2):
        want = oracle_layer(oracle_mod, layer2, host2, shared2, X2[t], ids2[t].tolist(), ws2[t].tolist())
        assert oracle_mod.max_relative_error(got2[t], want) <= TOL

    X3 = X.copy()
    X3[1, 7] = np.inf
    print("non-finite token", flush=True)
    _, st = run(layer, X3, ids[:, :8], ws[:, :8] / ws[:, :8].sum(1, keepdims=True))
    assert st == -4


@pytest.mark.parametrize("types", [(12, 14), (11, 11), (13, 12), (14, 14), (8, 8), (12, 8), (11, 14)])
def test_fp16_graph_fast_kernels(hip, oracle_mod, types):
    """The FP16 graph (fp16_graph=1, the reference's production decode) in the
    integer-decode kernels' FP16 mode: every routed weight decoded with the
    reference's arithmetic and rounded to FP16, FP16 activations, FP32 sums, and
    the rounding points of moe_quant_dot.cpp:189-211; the shared expert in the
    FP32 graph.  Against the oracle's FP16 graph at the north star's 1e-3 (the
    reference's own check allows 0.005, test_optimized_inference.py:231-290;
    observed ~1e-4) and against the generic kernels' FP16 graph, 3 tokens at several shapes, scales as the reference's
    FP16-graph check (d ~ 0.002, x ~ 0.05)."""
    gu, dn = types
    t = {"gate": gu, "up": gu, "down": dn}
    for H, I in ((256, 256), (2048, 512), (512, 1024), (1024, 2048)):
        layer, host, shared = make_layer(41 + gu + dn, 6, H, I, t, shared_types=t, scale=0.002)
        rng = np.random.default_rng(H + 5 * I)
        X = (rng.standard_normal((3, H)) * 0.05).astype(np.float32)
        ids = np.array([[0, 5, 2], [3, 3, 1], [4, 0, 5]])
        ws = np.array([[0.5, 0.3, 0.2], [0.6, 0.2, 0.2], [0.4, 0.4, 0.2]])
        want = [oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist(), fp16=1)
                for tok in range(3)]
        got = {}
        for path in (0, 1):
            print(f"fp16 graph types={types} H={H} I={I} path={path}", flush=True)
            old = hip.mqh_set_decode_path(path)
            try:
                got[path], st = run(layer, X, ids, ws, fp16=1)
            finally:
                hip.mqh_set_decode_path(old)
            assert st == 0
            for tok in range(3):
                err = oracle_mod.max_relative_error(got[path][tok], want[tok])
                assert err <= TOL, (types, H, I, path, tok, err)
        assert oracle_mod.max_relative_error(got[0], got[1]) <= TOL


@pytest.mark.parametrize("T,k,sh", [(8, 4, "same"), (8, 8, "q6k"), (16, 8, "same"), (16, 4, "q6k"), (16, 2, "same"),
                                    (12, 3, "same")])
def test_balanced_down_kernel(hip, oracle_mod, T, k, sh):
    """Many tokens with a shared expert (hidden 2048, intermediate 512): the down
    kernel gives each wave two (T >= 8) or four (T >= 16) row groups and, when
    top_k is at least that, deals the shared expert's row groups to the first
    waves (k = 2 at T = 16 keeps one wave per slot; k = 3 at T = 12 gives
    waves 0-1 the shared rows).  Every token against the oracle and the generic
    kernels."""
    H, I, E = 2048, 512, 32
    t = {"gate": 11, "up": 11, "down": 11}
    st = t if sh == "same" else {"gate": 14, "up": 14, "down": 14}
    layer, host, shared = make_layer(900 + T + k, E, H, I, t, shared_types=st)
    rng = np.random.default_rng(T * 10 + k)
    X = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    ws = rng.dirichlet(np.ones(k), size=T).astype(np.float32)
    print(f"balanced down T={T} k={k} shared={sh}", flush=True)
    old = hip.mqh_set_decode_path(0)
    try:
        got, s0 = run(layer, X, ids, ws)
        hip.mqh_set_decode_path(1)
        gen, s1 = run(layer, X, ids, ws)
    finally:
        hip.mqh_set_decode_path(old)
    assert s0 == 0 and s1 == 0
    for tok in range(T):
        want = oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist())
        # the integer-digit kernels' activation error (<= 1.6e-5 of a 16-column
        # run's max per value) reaches ~1e-4 of the output on these Q3_K layers
        assert oracle_mod.max_relative_error(got[tok], want) <= 2e-4, (T, k, sh, tok)
        assert oracle_mod.max_relative_error(got[tok], gen[tok]) <= TOL, (T, k, sh, tok)
    # a token's result does not depend on the batch it came in: the first and
    # last tokens alone (one wave per slot, one row group a wave) give the same bits
    old = hip.mqh_set_decode_path(0)
    try:
        for tok in (0, T - 1):
            one, s2 = run(layer, X[tok:tok + 1], ids[tok:tok + 1], ws[tok:tok + 1])
            assert s2 == 0
            assert np.array_equal(one[0].view(np.uint32), got[tok].view(np.uint32)), (T, k, sh, tok)
    finally:
        hip.mqh_set_decode_path(old)


@pytest.mark.parametrize("gt", [12, 13, 14, 8])
def test_batched_uniform_types(hip, oracle_mod, gt):
    """Uniform-type layers (gate/up type gt, down Q6_K, the shared expert of the
    routed types) at 4 and 16 tokens, where kernel A gives each wave two items
    (Q4_K, Q8_0) or one (Q5_K, Q6_K: two would spill): every token against the
    oracle and the generic kernels, and the first and last tokens run alone give
    the same bits."""
    H, I, E, K = 2048, 512, 24, 8
    t = {"gate": gt, "up": gt, "down": 14}
    layer, host, shared = make_layer(700 + gt, E, H, I, t, shared_types=t)
    rng = np.random.default_rng(gt)
    for T in (4, 16):
        X = rng.standard_normal((T, H)).astype(np.float32)
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
        ws = rng.dirichlet(np.ones(K), size=T).astype(np.float32)
        print(f"batched uniform gate/up type {gt} T={T}", flush=True)
        old = hip.mqh_set_decode_path(0)
        try:
            got, s0 = run(layer, X, ids, ws)
            hip.mqh_set_decode_path(1)
            gen, s1 = run(layer, X, ids, ws)
            hip.mqh_set_decode_path(0)
            alone = [run(layer, X[i:i + 1], ids[i:i + 1], ws[i:i + 1]) for i in (0, T - 1)]
        finally:
            hip.mqh_set_decode_path(old)
        assert s0 == 0 and s1 == 0 and all(s == 0 for _, s in alone)
        for tok in range(T):
            want = oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist())
            assert oracle_mod.max_relative_error(got[tok], want) <= TOL, (gt, T, tok)
            assert oracle_mod.max_relative_error(got[tok], gen[tok]) <= TOL, (gt, T, tok)
        for (one, _), tok in zip(alone, (0, T - 1)):
            assert np.array_equal(one[0].view(np.uint32), got[tok].view(np.uint32)), (gt, T, tok)


@pytest.mark.parametrize("fp16", [0, 1])
@pytest.mark.parametrize("shape", [(1024, 1024, 4), (512, 2048, 2)], ids=["h1024-i1024-k4", "h512-i2048-k2"])
@pytest.mark.parametrize("routed,shared_t", [((12, 14), (12, 14)), ((11, 11), (14, 14))])
def test_one_token_shared_item_on_two_waves_narrow(hip, oracle_mod, routed, shared_t, shape, fp16):
    """The two-wave shared item at 16 and 8 lanes per row: one token at hidden
    1024 / intermediate 1024 with top-4 and hidden 512 / intermediate 2048 with
    top-2, where kernel A also deals one wave a slot (top_k + 1 slots, one row
    group of every slot a workgroup); against the oracle and the generic
    kernels, both graphs."""
    gu, dn = routed
    t = {"gate": gu, "up": gu, "down": dn}
    sh = {"gate": shared_t[0], "up": shared_t[0], "down": shared_t[1]}
    H, I, K = shape
    E = 12
    layer, host, shared = make_layer(600 + H + K + gu + shared_t[0] + fp16, E, H, I, t, shared_types=sh,
                                     scale=0.002 if fp16 else 0.01)
    rng = np.random.default_rng(H + I + gu + fp16)
    X = (rng.standard_normal((1, H)) * (0.05 if fp16 else 1.0)).astype(np.float32)
    ids = rng.permutation(E)[:K][None]
    ws = rng.dirichlet(np.ones(K), size=1).astype(np.float32)
    print(f"one token, H={H} I={I} K={K} routed={routed} shared={shared_t} fp16={fp16}", flush=True)
    old = hip.mqh_set_decode_path(0)
    try:
        got, s0 = run(layer, X, ids, ws, fp16=fp16)
        assert hip.mqh_last_decode_path() == 0
        hip.mqh_set_decode_path(1)
        gen, s1 = run(layer, X, ids, ws, fp16=fp16)
    finally:
        hip.mqh_set_decode_path(old)
    assert s0 == 0 and s1 == 0
    want = oracle_layer(oracle_mod, layer, host, shared, X[0], ids[0].tolist(), ws[0].tolist(), fp16=fp16)
    assert oracle_mod.max_relative_error(got[0], want) <= TOL, (shape, routed, shared_t, fp16)
    assert oracle_mod.max_relative_error(got[0], gen[0]) <= TOL, (shape, routed, shared_t, fp16)


@pytest.mark.parametrize("fp16", [0, 1])
@pytest.mark.parametrize("routed,shared_t", [((12, 14), (12, 14)), ((12, 14), (14, 14)), ((11, 11), (14, 14)),
                                              ((12, 8), (14, 14))])
def test_one_token_shared_item_on_two_waves(hip, oracle_mod, routed, shared_t, fp16):
    """One token at hidden 2048 / intermediate 512 with top-8 + shared: kernel A
    deals one wave a slot and gives the shared expert's item to two waves (gate
    rows, up rows) whose second to finish applies SwiGLU.  The headline types
    and the reference model's three mixes with a Q6_K shared expert, both
    graphs, against the oracle and the generic kernels; a second call checks
    that the hand-over counter starts from zero in every launch."""
    gu, dn = routed
    t = {"gate": gu, "up": gu, "down": dn}
    sh = {"gate": shared_t[0], "up": shared_t[0], "down": shared_t[1]}
    H, I, E, K = 2048, 512, 24, 8
    layer, host, shared = make_layer(500 + gu + dn + 3 * shared_t[0] + fp16, E, H, I, t, shared_types=sh,
                                     scale=0.002 if fp16 else 0.01)
    rng = np.random.default_rng(gu + 5 * dn + shared_t[0] + fp16)
    for call in range(2):
        X = (rng.standard_normal((1, H)) * (0.05 if fp16 else 1.0)).astype(np.float32)
        ids = rng.permutation(E)[:K][None]
        ws = rng.dirichlet(np.ones(K), size=1).astype(np.float32)
        print(f"one token, routed={routed} shared={shared_t} fp16={fp16} call={call}", flush=True)
        old = hip.mqh_set_decode_path(0)
        try:
            got, s0 = run(layer, X, ids, ws, fp16=fp16)
            assert hip.mqh_last_decode_path() == 0
            expect_kernels(hip)
            hip.mqh_set_decode_path(1)
            gen, s1 = run(layer, X, ids, ws, fp16=fp16)
        finally:
            hip.mqh_set_decode_path(old)
        assert s0 == 0 and s1 == 0
        want = oracle_layer(oracle_mod, layer, host, shared, X[0], ids[0].tolist(), ws[0].tolist(), fp16=fp16)
        assert oracle_mod.max_relative_error(got[0], want) <= TOL, (routed, shared_t, fp16, call)
        assert oracle_mod.max_relative_error(got[0], gen[0]) <= TOL, (routed, shared_t, fp16, call)


@pytest.mark.parametrize("fp16", [0, 1])
@pytest.mark.parametrize("routed", [(12, 12), (11, 11), (12, 14), (8, 8)])
def test_intermediate_2048_twelve_slots(hip, oracle_mod, routed, fp16):
    """Intermediate 2048 with the most slots kernel B's digit LDS admits there:
    11 routed experts and a Q6_K shared expert (12 waves, 768 threads, the
    kernel's launch bound at that width).  Both graphs, 2 tokens, against the
    oracle and the generic kernels."""
    gu, dn = routed
    t = {"gate": gu, "up": gu, "down": dn}
    sh = {"gate": 14, "up": 14, "down": 14}
    H, I, E, K = 1024, 2048, 16, 11
    layer, host, shared = make_layer(300 + gu + dn + fp16, E, H, I, t, shared_types=sh,
                                     scale=0.002 if fp16 else 0.01)
    rng = np.random.default_rng(gu + 7 * dn + fp16)
    X = (rng.standard_normal((2, H)) * (0.05 if fp16 else 1.0)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(2)])
    ws = rng.dirichlet(np.ones(K), size=2).astype(np.float32)
    tol = TOL
    print(f"intermediate 2048, 12 slots, routed={routed} fp16={fp16}", flush=True)
    old = hip.mqh_set_decode_path(0)
    try:
        got, s0 = run(layer, X, ids, ws, fp16=fp16)
        expect_kernels(hip)
        assert hip.mqh_last_decode_path() == 0   # the 12-slot maximum runs on the fast kernels
        hip.mqh_set_decode_path(1)
        gen, s1 = run(layer, X, ids, ws, fp16=fp16)
        assert hip.mqh_last_decode_path() == 1
    finally:
        hip.mqh_set_decode_path(old)
    assert s0 == 0 and s1 == 0
    for tok in range(2):
        want = oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist(), fp16=fp16)
        assert oracle_mod.max_relative_error(got[tok], want) <= tol, (routed, fp16, tok)
        assert oracle_mod.max_relative_error(got[tok], gen[tok]) <= tol, (routed, fp16, tok)


def test_intermediate_2048_over_slot_limit_falls_back(hip, oracle_mod):
    """13 slots at intermediate 2048 (12 routed + shared) exceed kernel B's digit
    LDS: the layer runs on the generic kernels instead, with status 0 and the
    oracle's result."""
    t = {"gate": 12, "up": 12, "down": 14}
    H, I, E, K = 1024, 2048, 16, 12
    layer, host, shared = make_layer(333, E, H, I, t, shared_types=t)
    rng = np.random.default_rng(333)
    X = rng.standard_normal((2, H)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(2)])
    ws = rng.dirichlet(np.ones(K), size=2).astype(np.float32)
    print("intermediate 2048, 13 slots (generic fallback)", flush=True)
    old = hip.mqh_set_decode_path(0)
    try:
        got, st = run(layer, X, ids, ws)
        assert hip.mqh_last_decode_path() == 1   # the generic kernels ran, not the fast ones
    finally:
        hip.mqh_set_decode_path(old)
    assert st == 0
    for tok in range(2):
        want = oracle_layer(oracle_mod, layer, host, shared, X[tok], ids[tok].tolist(), ws[tok].tolist())
        assert oracle_mod.max_relative_error(got[tok], want) <= TOL, tok
