"""Pin the oracle's fused expert and the Python-side semantics (CPU only).

* FP32 graph: agrees with an FP64 brute force over the gguf-restated weights
  (dequantize, then two matrix products) -- a dropped term, a transposed
  operand or a wrong activation would be far outside the tolerance.
* FP16 graph: the known-answer procedure of
  tools/test_optimized_inference.py:231-262 (8 type triples, uniform random
  blocks with d=0.002/dmin=0.001, x*0.005, expected value with FP16 rounding at
  every graph point, max relative error < 0.005), plus bit-identical results
  across threads.
* Status codes of moe_quant_dot.cpp:177-212, including -4 for the benchmark's
  single-expert workload in FP16-graph mode (outputs overflow FP16).
* Router invariants of tools/test_router.py:146-178 and the shared-expert
  norm ratio of tools/test_shared_expert.py:103-113.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from oracle import gguf_quants_np as gq

BLOCK = {8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
TRIPLES = [(8, 11, 12), (11, 12, 13), (12, 13, 14), (13, 14, 8), (14, 8, 11), (12, 12, 14), (12, 12, 8),
           (11, 11, 11)]


def kat_expert(rng, kinds, hidden=256, inter=256):
    """Expert tensors as the reference KAT builds them (test_optimized_inference.py:241-247)."""
    tensors = {}
    for name, kind in zip(("gate", "up", "down"), kinds):
        rows, cols = (inter, hidden) if name != "down" else (hidden, inter)
        bs, size = BLOCK[kind]
        raw = rng.integers(0, 256, (rows * (cols // bs), size), np.uint8)
        offset = size - 2 if kind in (11, 14) else 0
        raw[:, offset:offset + 2] = np.frombuffer(np.float16(.002).tobytes(), np.uint8)
        if kind in (12, 13):
            raw[:, 2:4] = np.frombuffer(np.float16(.001).tobytes(), np.uint8)
        tensors[name] = raw.reshape(-1)
    return tensors


def weights_of(tensors, kinds, hidden, inter):
    g = gq.dequantize(tensors["gate"], kinds["gate"]).reshape(inter, hidden)
    u = gq.dequantize(tensors["up"], kinds["up"]).reshape(inter, hidden)
    d = gq.dequantize(tensors["down"], kinds["down"]).reshape(hidden, inter)
    return g, u, d


def fp64_expert(tensors, kinds, x, hidden, inter):
    g, u, d = (w.astype(np.float64) for w in weights_of(tensors, kinds, hidden, inter))
    x = np.asarray(x, np.float64)
    gv, uv = g @ x, u @ x
    return d @ (gv / (1 + np.exp(-gv)) * uv)


@pytest.mark.parametrize("kinds", TRIPLES)
def test_fp32_graph_matches_fp64_brute_force(oracle_mod, kinds):
    rng = np.random.default_rng(sum(kinds))
    k = dict(zip(("gate", "up", "down"), kinds))
    tensors = kat_expert(rng, kinds)
    x = rng.standard_normal(256).astype(np.float32)
    y = oracle_mod.expert_forward(tensors, k, x, 256, 256, 0)
    assert oracle_mod.max_relative_error(y, fp64_expert(tensors, k, x, 256, 256)) < 2e-6


def test_benchmark_single_expert_fp32(oracle_mod):
    """Q4_K [512x2048]/[2048x512], x ~ N(0,1), seed 0: FP32 graph agrees with FP64;
    the FP16 graph overflows (status -4), as the reference does on these inputs."""
    from flash_moe_hip.synthetic import config1_expert

    tensors, kinds, x = config1_expert(0)
    rc, y = oracle_mod.moe_quant_expert(tensors, kinds, x, 2048, 512, 0)
    assert rc == 0
    assert oracle_mod.max_relative_error(y, fp64_expert(tensors, kinds, x, 2048, 512)) < 2e-6
    assert np.abs(y).max() > 65504          # beyond the FP16 range
    rc16, _ = oracle_mod.moe_quant_expert(tensors, kinds, x, 2048, 512, 1)
    assert rc16 == -4


def round16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("kinds", TRIPLES)
def test_fp16_graph_known_answer(oracle_mod, kinds):
    rng = np.random.default_rng(17 + sum(kinds))
    k = dict(zip(("gate", "up", "down"), kinds))
    tensors = kat_expert(rng, kinds)
    w = [round16(a) for a in weights_of(tensors, k, 256, 256)]
    x = round16((rng.standard_normal(256) * .005).astype(np.float32))
    g, u = round16(x @ w[0].T), round16(x @ w[1].T)
    act = round16(round16(g * round16(1 / (1 + np.exp(-g)))) * u)
    expected = round16(act @ w[2].T)
    with ThreadPoolExecutor(4) as pool:
        results = list(pool.map(lambda _: oracle_mod.expert_forward(tensors, k, x, 256, 256, 1), range(8)))
    err = np.max(np.abs(results[0] - expected)) / max(1e-12, np.max(np.abs(expected)))
    assert err < .005
    for r in results:
        np.testing.assert_array_equal(r, results[0])


def test_status_codes(oracle_mod):
    rng = np.random.default_rng(0)
    k = {"gate": 12, "up": 12, "down": 14}
    t = kat_expert(rng, (12, 12, 14))
    x = np.zeros(256, np.float32)
    call = oracle_mod.moe_quant_expert
    assert call(t, k, x, 256, 256, 0)[0] == 0
    assert call(t, k, x, 256, 256, 2)[0] == -1
    assert call(t, k, x, 0, 256, 0)[0] == -1
    assert call(t, k, x, 65537, 256, 0)[0] == -1
    assert call(t, dict(k, gate=999), x, 256, 256, 0)[0] == -2
    bad = dict(t, up=t["up"][:-1])
    assert call(bad, k, x, 256, 256, 0)[0] == -3
    # cols % block: hidden 288 is a multiple of 32 but not of 256
    assert call(t, k, np.zeros(288, np.float32), 288, 256, 0)[0] == -2


# ------------------------------------------------------------------ router

def test_router_invariants_and_package_parity(oracle_mod):
    from flash_moe_hip.router import ExpertRouter, softmax_all_experts

    rng = np.random.default_rng(11)
    W = (rng.standard_normal((2048, 256)) * 0.02).astype(np.float32)
    r = ExpertRouter(2048, 256, top_k=8, gate_weights=W, gate_dtype=np.float32)
    for _ in range(16):
        x = rng.standard_normal(2048).astype(np.float32)
        idx, w = oracle_mod.route(x, W, 8)
        assert len(idx) == 8 and len(set(idx)) == 8 and all(0 <= i < 256 for i in idx)
        assert all(v > 0 for v in w) and abs(sum(w) - 1) < 1e-6
        assert list(w) == sorted(w, reverse=True)
        scores = x @ W
        p = softmax_all_experts(scores)
        assert np.abs(np.asarray(w) - p[idx] / p[idx].sum()).max() < 1e-9
        assert r.route(x) == (idx, w)
        assert r.route(x.tolist()) == (idx, w)
    # GGUF (n_expert, n_embd) order is transposed on load
    r2 = ExpertRouter(2048, 256, top_k=8, gate_weights=W.T.copy(), gate_dtype=np.float32)
    assert r2.route(x) == r.route(x)


def test_router_nonfinite_scores_fall_back_to_uniform(oracle_mod):
    W = np.zeros((4, 4), np.float32)
    x = np.array([np.inf, 0, 0, 0], np.float32)
    with np.errstate(all="ignore"):
        idx, w = oracle_mod.route(x, W, 2)
    assert w == [0.5, 0.5]


# ----------------------------------------------------- shared expert, combine

def test_shared_expert_norm_ratio_is_the_sigmoid(oracle_mod):
    rng = np.random.default_rng(3)
    H, I = 256, 128
    wg, wu = (rng.standard_normal((I, H)) * .05).astype(np.float32), (rng.standard_normal((I, H)) * .05).astype(np.float32)
    wd = (rng.standard_normal((H, I)) * .05).astype(np.float32)
    gi = (rng.standard_normal(H) * .02).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    scaled = oracle_mod.shared_expert_forward(x, wg, wu, wd, gi)
    unscaled = oracle_mod.shared_expert_forward(x, wg, wu, wd, None)
    ratio = np.linalg.norm(scaled) / np.linalg.norm(unscaled)
    assert abs(ratio - 1 / (1 + np.exp(-float(x @ gi)))) < 1e-4
    off = oracle_mod.shared_expert_forward(x, wg, wu, wd, -1e4 * np.sign(x))
    assert float(np.abs(off).max()) == 0.0


def test_combine_order_and_weight_cast(oracle_mod):
    rng = np.random.default_rng(4)
    ys = [rng.standard_normal(64).astype(np.float32) * 1e3 for _ in range(8)]
    w = list(rng.dirichlet(np.ones(8)))
    got = oracle_mod.combine(ys, w)
    want = np.zeros(64, np.float32)
    for y, v in zip(ys, w):
        want = (want + (np.float32(v) * y).astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(got, want)
    ref64 = sum(np.float64(v) * y.astype(np.float64) for y, v in zip(ys, w))
    assert oracle_mod.max_relative_error(got, ref64) < 1e-6


SCALE_OFFSET = {8: 0, 11: 108, 12: 0, 13: 0, 14: 208}   # byte offset of each block's FP16 d


def poison_row(tensors, kind, row, cols, role="down"):
    """A copy of ``tensors`` whose ``role`` matrix has every block of ``row``
    scaled by FP16 +inf, so that row's output is not finite."""
    bs, size = BLOCK[kind]
    raw = np.array(tensors[role], dtype=np.uint8).reshape(-1, size)
    per_row = cols // bs
    off = SCALE_OFFSET[kind]
    raw[row * per_row:(row + 1) * per_row, off:off + 2] = np.frombuffer(np.float16(np.inf).tobytes(), np.uint8)
    return dict(tensors, **{role: raw.reshape(-1)})


@pytest.mark.parametrize("fp16", [0, 1])
@pytest.mark.parametrize("down", [12, 14, 8])
def test_first_non_finite_row_stops_the_expert(oracle_mod, fp16, down):
    """A down row with an infinite scale: the oracle returns -4 with the rows
    before it as a clean run computes them, that row non-finite, and every
    later row as the caller had it (moe_quant_dot.cpp:207-211: the row is
    stored, then checked, then the loop returns)."""
    rng = np.random.default_rng(40 + down + fp16)
    kinds = (12, 12, down)
    k = dict(zip(("gate", "up", "down"), kinds))
    tensors = kat_expert(rng, kinds)
    x = (rng.standard_normal(256) * (.005 if fp16 else 1.0)).astype(np.float32)
    r0 = 100
    rc, clean = oracle_mod.moe_quant_expert(tensors, k, x, 256, 256, fp16)
    assert rc == 0
    out = np.full(256, 7.0, np.float32)
    rc, _ = oracle_mod.moe_quant_expert(poison_row(tensors, down, r0, 256), k, x, 256, 256, fp16, out=out)
    assert rc == -4
    np.testing.assert_array_equal(out[:r0], clean[:r0])
    assert not np.isfinite(out[r0])
    np.testing.assert_array_equal(out[r0 + 1:], 7.0)
