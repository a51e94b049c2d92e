"""Top-k routing on the device (mqh_route) against the oracle's ExpertRouter.route.

The oracle is router.py:140-170: FP32 scores ``x @ W``, the top k of
np.argsort in descending order, and the float64 softmax over the selected
scores (uniform weights when that sum is not finite).  The kernel sums each
score in a fixed order, so on random data a score differs from NumPy's BLAS
sum by FP32 rounding only: ids must agree wherever the float64 scores have no
near-tie (gap > 1e-4) at the compared ranks, and weights agree within 2e-6
absolute.  On integer-valued inputs every score is exact in any order, so ids
and weights must agree exactly (weights to one FP32 ulp of the float64
softmax).  NumPy's order among equal scores is unspecified: there the test
checks the scores by rank and the kernel's own rule (ascending expert id).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def gpu_route(x, w, k, with_scores=False):
    """mqh_route on x [T,H] and the reference-layout router weights w [H,E]
    (handed to the device as the GGUF stores them: [E,H])."""
    import torch
    from flash_moe_hip import _lib

    lib = _lib.load()
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    wt = torch.from_numpy(np.ascontiguousarray(np.asarray(w, dtype=np.float32).T)).cuda()
    T, H = xt.shape
    E = wt.shape[0]
    print(f"mqh_route T={T} H={H} E={E} k={k}", flush=True)
    scores = torch.full((T, E), -7.0, dtype=torch.float32, device="cuda")
    ids = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
    wts = torch.full((T, k), -1.0, dtype=torch.float32, device="cuda")
    rc = lib.mqh_route(xt.data_ptr(), T, H, wt.data_ptr(), E, k, scores.data_ptr(), ids.data_ptr(), wts.data_ptr(),
                       torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "mqh_route")
    torch.cuda.synchronize()
    if with_scores:
        return ids.cpu().numpy(), wts.cpu().numpy(), scores.cpu().numpy()
    return ids.cpu().numpy(), wts.cpu().numpy()


@pytest.mark.parametrize("T,H,E,k", [
    (1, 2048, 128, 8),
    (5, 1536, 60, 4),
    (3, 2500, 256, 8),      # three LDS chunks, the last ragged
    (2, 48, 16, 2),         # hidden below one wavefront
    (4, 512, 1024, 16),     # the largest expert count
    (64, 1024, 64, 6),
    (2, 256, 8, 8),         # every expert selected
    (3, 128, 1, 1),
    (33, 2048, 256, 8),     # first size on the one-wave-per-row score layout
    (130, 768, 200, 8),     # ragged token groups and expert groups
])
def test_route_random_matches_oracle(oracle_mod, T, H, E, k):
    rng = np.random.default_rng(T * 7919 + H * 31 + E)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((H, E)) / np.sqrt(H)).astype(np.float32)
    ids, wts, scores = gpu_route(x, w, k, with_scores=True)
    s64 = x.astype(np.float64) @ w.astype(np.float64)
    bound = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64)
    assert np.all(np.abs(scores - s64) <= 4e-6 * bound)      # FP32 summation error only
    exact = 0
    for t in range(T):
        o_ids, o_w = oracle_mod.route(x[t], w, k)
        assert len(set(ids[t].tolist())) == k and ids[t].min() >= 0 and ids[t].max() < E
        # ranks agree in score (a near-tie may swap two experts)
        np.testing.assert_allclose(s64[t][ids[t]], s64[t][o_ids], rtol=0, atol=1e-4)
        order = np.sort(s64[t])[::-1]
        gaps = np.abs(np.diff(order[:k + 1])) if k < E else np.abs(np.diff(order))
        if gaps.size == 0 or gaps.min() > 1e-4:
            assert ids[t].tolist() == list(o_ids), f"token {t}"
            np.testing.assert_allclose(wts[t], o_w, rtol=0, atol=2e-6)
            exact += 1
        np.testing.assert_allclose(wts[t].sum(), 1.0, atol=1e-5)
    assert exact >= max(1, T // 2)


def test_route_exact_scores_match_bit_for_bit(oracle_mod):
    """Integer x and W times 2^-7: every product and partial sum is exact in
    FP32, so the scores are exact in any summation order."""
    rng = np.random.default_rng(7)
    T, H, E, k = 16, 1000, 96, 8
    x = rng.integers(-8, 9, size=(T, H)).astype(np.float32)
    w = (rng.integers(-8, 9, size=(H, E)) * 2.0 ** -7).astype(np.float32)
    ids, wts, scores = gpu_route(x, w, k, with_scores=True)
    s64 = x.astype(np.float64) @ w.astype(np.float64)
    np.testing.assert_array_equal(scores, s64.astype(np.float32))
    checked = 0
    for t in range(T):
        top = np.sort(s64[t])[::-1][:k + 1]
        if len(np.unique(top)) < k + 1:
            continue    # a tie at the top: covered by the tie test
        o_ids, o_w = oracle_mod.route(x[t], w, k)
        assert ids[t].tolist() == list(o_ids)
        np.testing.assert_array_max_ulp(wts[t], np.asarray(o_w, dtype=np.float32), maxulp=1)
        checked += 1
    assert checked >= T // 2


def test_route_ties_take_ascending_expert_ids(oracle_mod):
    """Exactly equal scores: the device takes the lower expert id first.  The
    reference's np.argsort(s)[-k:][::-1] (router.py:156, the default unstable
    sort) orders exact ties as its sort implementation leaves them, which
    depends on the NumPy build, so only the set of tied experts and the score
    at every rank are compared with the oracle; the ascending order is this
    kernel's own, documented rule."""
    H, E, k = 64, 32, 6
    rng = np.random.default_rng(11)
    x = rng.integers(0, 3, size=(2, H)).astype(np.float32)
    w = rng.integers(-2, 3, size=(H, E)).astype(np.float32)
    # experts 3, 9, 17 and 30 share one column far above the rest: four equal top scores
    for e in (3, 9, 17, 30):
        w[:, e] = 4.0
    ids, wts = gpu_route(x, w, k)
    for t in range(2):
        o_ids, o_w = oracle_mod.route(x[t], w, k)
        s = x[t] @ w
        np.testing.assert_array_equal(s[ids[t]], s[o_ids])          # the same scores at every rank
        assert set(ids[t][:4].tolist()) == set(o_ids[:4]) == {3, 9, 17, 30}   # the same tied experts
        assert ids[t][:4].tolist() == [3, 9, 17, 30]                # this kernel's order: ascending
        if s[o_ids[k - 1]] != np.sort(s)[::-1][k]:                  # no tie across the k-th rank
            assert set(ids[t].tolist()) == set(o_ids)
        np.testing.assert_allclose(wts[t], o_w, rtol=0, atol=1e-7)


def test_route_nan_scores_rank_first_with_uniform_weights(oracle_mod):
    rng = np.random.default_rng(5)
    H, E, k = 256, 64, 4
    x = rng.standard_normal((1, H)).astype(np.float32)
    w = (rng.standard_normal((H, E)) / 16).astype(np.float32)
    w[10, 40] = np.nan
    w[3, 7] = np.nan
    ids, wts = gpu_route(x, w, k)
    o_ids, o_w = oracle_mod.route(x[0], w, k)
    assert set(ids[0][:2].tolist()) == set(o_ids[:2]) == {7, 40}
    assert ids[0][:2].tolist() == [7, 40]
    assert ids[0][2:].tolist() == list(o_ids[2:])
    np.testing.assert_array_equal(wts[0], np.float32(o_w))
    np.testing.assert_array_equal(wts[0], np.full(k, 0.25, np.float32))


@pytest.mark.parametrize("T,E,k", [(4096, 256, 8), (1024, 1024, 16), (2048, 60, 4)])
def test_route_select_is_the_top_k_of_its_scores_at_scale(T, E, k):
    """Size-independent: every token's ids are exactly the top k of the scores
    the kernel wrote (score descending, then expert ascending), and its weights
    the float64 softmax of those scores; the scores are x . W within FP32
    summation error."""
    H = 2048
    rng = np.random.default_rng(T + E)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((H, E)) * 0.02).astype(np.float32)
    ids, wts, scores = gpu_route(x, w, k, with_scores=True)
    s64 = x.astype(np.float64) @ w.astype(np.float64)
    bound = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64)
    assert np.all(np.abs(scores - s64) <= 4e-6 * bound)
    order = np.lexsort((np.broadcast_to(np.arange(E), scores.shape), -scores), axis=1)[:, :k]
    np.testing.assert_array_equal(ids, order)
    sel = np.take_along_axis(scores, order, axis=1).astype(np.float64)
    e = np.exp(sel - sel.max(axis=1, keepdims=True))
    want = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    np.testing.assert_allclose(wts, want, rtol=0, atol=1e-7)


def test_routed_decode_many_tokens_equals_route_then_decode():
    """64 tokens: every gate/up workgroup's own top-k in the prologue picks the
    same experts as the select kernel, so the outputs are bit-identical."""
    import torch
    from flash_moe_hip import _lib
    from flash_moe_hip.moe_gpu import MoeRunner
    from test_gpu_decode import make_layer

    E, H, I, k, T = 256, 1024, 256, 8, 64
    types = {"gate": 12, "up": 12, "down": 14}
    layer, _, _ = make_layer(5, E, H, I, types, shared_types={"gate": 14, "up": 14, "down": 14})
    rng = np.random.default_rng(6)
    layer.router_weights = (rng.standard_normal((H, E)) * 0.03).astype(np.float32)
    xd = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).cuda()
    runner = MoeRunner()
    lib = _lib.load()
    outs = []
    for _ in range(3):
        y, ids, wts = runner.decode_routed(layer, xd, k)
        torch.cuda.synchronize()
        assert lib.mqh_last_route_kernels() == 1
        outs.append((y.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()))
    ids2, wts2 = runner.route(layer, xd, k)
    y2 = runner.decode(layer, xd, ids2, wts2)
    torch.cuda.synchronize()
    assert runner.status() == 0
    for y, ids, wts in outs:
        np.testing.assert_array_equal(ids, ids2.cpu().numpy())
        np.testing.assert_array_equal(wts, wts2.cpu().numpy())
        np.testing.assert_array_equal(y, y2.cpu().numpy())


@pytest.mark.parametrize("E,types,sh_types,T,path,route_kernels", [
    (256, (12, 12, 14), (14, 14, 14), 1, 0, 1),     # the headline layer: select in the gate/up prologue
    (256, (12, 12, 14), (14, 14, 14), 16, 0, 1),
    (64, (11, 11, 11), (11, 11, 11), 5, 0, 1),
    (16, (13, 13, 12), None, 3, 0, 1),
    (300, (12, 12, 14), (14, 14, 14), 2, 0, 2),     # more experts than the prologue holds
    (32, (12, 12, 8), None, 2, 0, 1),               # Q8_0 down
    (32, (12, 12, 14), (12, 12, 14), 3, 1, 2),      # generic kernels forced
], ids=["E256-T1", "E256-T16", "E64-q3k", "E16-noshared", "E300", "q8down", "generic"])
def test_routed_decode_matches_the_oracle_layer(oracle_mod, E, types, sh_types, T, path, route_kernels):
    """Routing and the experts on the device in one call, against the oracle's
    route + run_moe_layer, and bit for bit against route() then decode()."""
    import torch
    from flash_moe_hip import _lib
    from flash_moe_hip.moe_gpu import MoeRunner
    from test_gpu_decode import make_layer, oracle_layer

    H, I, k = 512, 256, 8
    tdict = dict(zip(("gate", "up", "down"), types))
    sdict = dict(zip(("gate", "up", "down"), sh_types)) if sh_types else None
    layer, host, shared = make_layer(21 + E + T, E, H, I, tdict, shared_types=sdict)
    rng = np.random.default_rng(22 + E)
    layer.router_weights = (rng.standard_normal((H, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, H)).astype(np.float32)
    lib = _lib.load()
    old = lib.mqh_set_decode_path(path)
    try:
        runner = MoeRunner()
        xd = torch.from_numpy(X).cuda()
        print(f"routed decode E={E} types={types} T={T} path={path}", flush=True)
        y, ids, wts = runner.decode_routed(layer, xd, k)
        torch.cuda.synchronize()
        assert lib.mqh_last_route_kernels() == route_kernels
        assert runner.status() == 0
        ids2, wts2 = runner.route(layer, xd, k)
        y2 = runner.decode(layer, xd, ids2, wts2)
        torch.cuda.synchronize()
        assert runner.status() == 0
    finally:
        lib.mqh_set_decode_path(old)
    y, ids, wts = y.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    np.testing.assert_array_equal(ids, ids2.cpu().numpy())
    np.testing.assert_array_equal(wts, wts2.cpu().numpy())
    np.testing.assert_array_equal(y, y2.cpu().numpy())
    for t in range(T):
        o_ids, o_w = oracle_mod.route(X[t], layer.router_weights, k)
        assert ids[t].tolist() == list(o_ids), f"token {t}"
        np.testing.assert_allclose(wts[t], o_w, rtol=0, atol=2e-6)
        ref = oracle_layer(oracle_mod, layer, host, shared, X[t], o_ids, o_w)
        err = np.abs(y[t] - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err <= 1e-3, f"token {t}: {err}"
