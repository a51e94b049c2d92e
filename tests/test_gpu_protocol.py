"""The reference's call patterns into HipExpertBackend, against the oracle.

``run_moe_layer`` / ``run_moe_sequence`` (src/flash_moe/moe_layer.py:39-195)
reach the experts three ways, and each is driven here:

* fused: ``backend.moe_layer`` / ``moe_tokens`` (this package's fast hooks);
* protocol, one token: ``backend.forward`` per routed expert, fanned out on
  ``backend._moe_executor`` threads (moe_layer.py:74-94), plus the shared
  expert's own ``forward``;
* protocol, a sequence: tokens bucketed per expert, ``forward`` for a bucket of
  one and ``forward_batch`` for more (moe_layer.py:125-170), the shared expert
  per token below 16 tokens and batched from 16 to 128 (:177-194).

The protocol branches are reached through a proxy that hides the fused hooks,
exactly the attribute set a reference caller sees.  Each result is compared
with the oracle's run_moe_layer arithmetic at max relative error <= 1e-3.
Also: ``forward`` from many threads at once is deterministic and
thread-independent (the reference's test_optimized_inference.py:257-262), and
the shared expert and routers built from a GGUF file with the reference's
constructors match the oracle.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from test_gpu_decode import TOL, make_layer, oracle_layer

pytestmark = pytest.mark.gpu

H, I, E, K = 1024, 256, 24, 8
TYPES = {"gate": 12, "up": 12, "down": 14}


class ProtocolOnly:
    """The reference backend protocol only (no fused hooks)."""

    def __init__(self, backend):
        self._b = backend
        self.store = backend.store
        self._moe_executor = backend._moe_executor

    def forward(self, *a):
        return self._b.forward(*a)

    def forward_batch(self, *a):
        return self._b.forward_batch(*a)

    def prefetch_weights(self, keys):
        return self._b.prefetch_weights(keys)


class ForwardOnly:
    """A backend without forward_batch (run_moe_sequence then stacks run_moe_layer)."""

    def __init__(self, backend):
        self._b = backend
        self.store = None
        self._moe_executor = None   # run_moe_layer makes a pool of its own

    def forward(self, *a):
        return self._b.forward(*a)


@pytest.fixture(scope="module")
def setup(oracle_mod, hip):
    from flash_moe_hip.backend import HipExpertBackend
    from flash_moe_hip.shared_expert import SharedExpert

    layer, host, shared = make_layer(81, E, H, I, TYPES, shared_types={"gate": 14, "up": 14, "down": 14})
    rng = np.random.default_rng(82)
    W = (rng.standard_normal((H, E)) * 0.05).astype(np.float32)

    class Router:
        top_k = K

        def route(self, x):
            return oracle_mod.route(x, W, K)

    backend = HipExpertBackend({5: layer}, fp16_graph=0)   # the FP32 graph: checked against the FP32 oracle
    sh = SharedExpert.from_backend(backend)
    yield layer, host, shared, Router(), backend, sh
    backend.close()


def _want(oracle_mod, layer, host, shared, router, x):
    ids, ws = router.route(x)
    return oracle_layer(oracle_mod, layer, host, shared, x, ids, ws)


@pytest.mark.parametrize("via", ["fused", "protocol", "forward-only"])
def test_run_moe_layer(setup, oracle_mod, via):
    from flash_moe_hip.moe_layer import run_moe_layer

    layer, host, shared, router, backend, sh = setup
    b = {"fused": backend, "protocol": ProtocolOnly(backend), "forward-only": ForwardOnly(backend)}[via]
    rng = np.random.default_rng(83)
    for i in range(3):
        x = rng.standard_normal(H).astype(np.float32)
        print(f"run_moe_layer via {via} token {i}", flush=True)
        got = run_moe_layer(5, x, router, b, H, I, shared_expert=sh)
        err = oracle_mod.max_relative_error(got, _want(oracle_mod, layer, host, shared, router, x))
        assert got.dtype == np.float32 and got.shape == (H,)
        assert err <= TOL, (via, i, err)


@pytest.mark.parametrize("T", [1, 5, 20])
@pytest.mark.parametrize("via", ["fused", "protocol", "forward-only"])
def test_run_moe_sequence(setup, oracle_mod, via, T):
    from flash_moe_hip.moe_layer import run_moe_sequence

    layer, host, shared, router, backend, sh = setup
    b = {"fused": backend, "protocol": ProtocolOnly(backend), "forward-only": ForwardOnly(backend)}[via]
    rng = np.random.default_rng(84 + T)
    X = rng.standard_normal((T, H)).astype(np.float32)
    print(f"run_moe_sequence via {via} T={T}", flush=True)
    got = run_moe_sequence(5, X, router, b, H, I, shared_expert=sh)
    assert got.shape == (T, H)
    worst = max(oracle_mod.max_relative_error(got[t], _want(oracle_mod, layer, host, shared, router, X[t]))
                for t in range(T))
    assert worst <= TOL, (via, T, worst)


def test_forward_threads_deterministic(setup, oracle_mod):
    """8 threads x 6 rounds of forward() on different experts: every result equals
    the single-threaded one bit for bit and the oracle's expert within 1e-3."""
    from flash_moe_hip.key import ExpertKey

    layer, host, shared, router, backend, sh = setup
    rng = np.random.default_rng(85)
    xs = rng.standard_normal((8, H)).astype(np.float32)
    keys = [ExpertKey(5, int(e)) for e in rng.permutation(E)[:8]]
    single = [backend.forward(keys[j], xs[j], H, I) for j in range(8)]
    with ThreadPoolExecutor(8) as pool:
        for rnd in range(6):
            print(f"threaded forward round {rnd}", flush=True)
            outs = list(pool.map(lambda j: backend.forward(keys[j], xs[j], H, I), range(8)))
            for j in range(8):
                assert np.array_equal(outs[j], single[j]), (rnd, j)
    from test_gpu_decode import host_expert

    for j in range(8):
        want = oracle_mod.expert_forward(host_expert(host, layer, keys[j].expert), TYPES, xs[j], H, I, 0)
        assert oracle_mod.max_relative_error(single[j], want) <= TOL


def test_forward_batch_and_shared(setup, oracle_mod):
    from flash_moe_hip.key import ExpertKey
    from test_gpu_decode import host_expert

    layer, host, shared, router, backend, sh = setup
    rng = np.random.default_rng(86)
    X = rng.standard_normal((7, H)).astype(np.float32)
    y = backend.forward_batch(ExpertKey(5, 3), X, H, I)
    assert backend.forward_batch(ExpertKey(5, 3), X[:0], H, I).shape == (0, H)
    for t in range(7):
        want = oracle_mod.expert_forward(host_expert(host, layer, 3), TYPES, X[t], H, I, 0)
        assert oracle_mod.max_relative_error(y[t], want) <= TOL
    ys = sh.forward_batch(5, X)
    y1 = sh.forward(5, X[2])
    for t in range(7):
        gate = oracle_mod._sigmoid(np.float32(X[t] @ shared["gate_inp"]).reshape(()))
        want = (gate * oracle_mod.expert_forward({r: shared[r] for r in ("gate", "up", "down")}, shared["types"],
                                                 X[t], H, I, 0)).astype(np.float32)
        assert oracle_mod.max_relative_error(ys[t], want) <= TOL
    assert np.array_equal(y1, ys[2])
    assert sh.forward(6, X[0]) is None   # no such layer


def test_shared_expert_and_routers_from_gguf(tmp_path, oracle_mod, hip):
    """SharedExpert(gguf_path, num_layers, hidden, intermediate) and
    routers_from_gguf(tmap, ...) with the reference's constructors, on a file
    packed with the reference model's tensor names: the shared contribution
    equals the oracle's, the routers equal ExpertRouter over the same gate, and
    a layer without the shared matrices raises KeyError."""
    from flash_moe_hip.gguf_file import GGUFFile
    from flash_moe_hip.router import ExpertRouter, routers_from_gguf
    from flash_moe_hip.shared_expert import SharedExpert
    from flash_moe_hip.synthetic import random_stack
    from test_gguf_file import F32, STR, pack_gguf, write

    rng = np.random.default_rng(87)
    Hs, Is, Es = 512, 256, 8
    tensors, want = [], {}
    for layer in range(2):
        sg, su, sd = (random_stack(rng, 14, 1, *shape) for shape in ((Is, Hs), (Is, Hs), (Hs, Is)))
        gi = (rng.standard_normal(Hs) * 0.05).astype(np.float32)
        gate = rng.standard_normal((Es, Hs)).astype(np.float32)
        tensors += [(f"blk.{layer}.ffn_gate_shexp.weight", (Hs, Is), 14, sg.tobytes()),
                    (f"blk.{layer}.ffn_up_shexp.weight", (Hs, Is), 14, su.tobytes()),
                    (f"blk.{layer}.ffn_down_shexp.weight", (Is, Hs), 14, sd.tobytes()),
                    (f"blk.{layer}.ffn_gate_inp_shexp.weight", (Hs,), 0, gi.tobytes()),
                    (f"blk.{layer}.ffn_gate_inp.weight", (Hs, Es), 0, gate.tobytes())]
        want[layer] = (sg, su, sd, gi, gate)
    path = write(tmp_path, pack_gguf([("general.architecture", STR, "qwen3moe")], tensors))
    sh = SharedExpert(path, 2, Hs, Is)
    with pytest.raises(KeyError):
        SharedExpert(path, 3, Hs, Is)
    routers = routers_from_gguf(GGUFFile(path).tensor_map(), 2, Hs, Es, 4)
    with pytest.raises(KeyError):
        routers_from_gguf(GGUFFile(path).tensor_map(), 3, Hs, Es, 4)
    X = rng.standard_normal((3, Hs)).astype(np.float32)
    for layer in range(2):
        sg, su, sd, gi, gate = want[layer]
        got = sh.forward_batch(layer, X)
        gi16 = gi.astype(np.float16).astype(np.float32)   # SharedExpert._load's storage (shared_expert.py:173)
        assert np.array_equal(sh.layers[layer].gate_inp.cpu().numpy(), gi16)
        for t in range(3):
            g = oracle_mod._sigmoid(np.float32(X[t] @ gi16).reshape(()))
            ref = (g * oracle_mod.expert_forward({"gate": sg, "up": su, "down": sd},
                                                 {"gate": 14, "up": 14, "down": 14}, X[t], Hs, Is, 0))
            assert oracle_mod.max_relative_error(got[t], ref.astype(np.float32)) <= TOL
        ref_router = ExpertRouter(Hs, Es, top_k=4, gate_weights=gate)
        for t in range(3):
            assert routers[layer].route(X[t])[0] == ref_router.route(X[t])[0]
        assert np.array_equal(routers[layer].gate_weights, ref_router.gate_weights)
    # an F16 shared matrix (the reference dequantizes nothing for it) is refused
    # when the layer is loaded, with the tensor's name
    f16 = rng.standard_normal((Is, Hs)).astype(np.float16)
    bad = [(n.replace("blk.1.", "blk.0."), d, t, b) for n, d, t, b in tensors if n.startswith("blk.1.")]
    bad[0] = ("blk.0.ffn_gate_shexp.weight", (Hs, Is), 1, f16.tobytes())
    with pytest.raises(ValueError, match="ffn_gate_shexp"):
        SharedExpert(write(tmp_path, pack_gguf([], bad), "f16_shared.gguf"), 1, Hs, Is)


@pytest.mark.parametrize("via", ["fused", "protocol"])
def test_backend_default_is_the_fp16_graph(oracle_mod, hip, via):
    """HipExpertBackend defaults to the reference decode's numerics, the
    native FP16 graph (native_expert.py:33-34): run_moe_layer through the fused
    hook and through forward() fan-out, at the reference's FP16-graph check
    magnitudes (d ~ 0.002, x ~ 0.05), against the oracle's FP16-graph experts
    at max relative error <= 5e-4, and nearer to them than to the oracle's FP32
    graph (the two graphs differ by 5-8e-4 here), so the graph is told apart.
    No shared expert: it runs the FP32 graph in both, and its output would
    dominate the maximum and hide the routed experts' graph."""
    from flash_moe_hip.backend import HipExpertBackend
    from flash_moe_hip.moe_layer import run_moe_layer

    layer, host, shared = make_layer(91, E, H, I, TYPES, scale=0.002)
    rng = np.random.default_rng(92)
    W = (rng.standard_normal((H, E)) * 0.05).astype(np.float32)

    class Router:
        top_k = K

        def route(self, x):
            return oracle_mod.route(x, W, K)

    backend = HipExpertBackend({5: layer})
    try:
        assert backend.fp16_graph == 1
        b = backend if via == "fused" else ProtocolOnly(backend)
        for i in range(3):
            x = (rng.standard_normal(H) * 0.05).astype(np.float32)
            print(f"FP16-graph run_moe_layer via {via} token {i}", flush=True)
            got = run_moe_layer(5, x, Router(), b, H, I)
            ids, ws = oracle_mod.route(x, W, K)
            want16 = oracle_layer(oracle_mod, layer, host, shared, x, ids, ws, fp16=1)
            want32 = oracle_layer(oracle_mod, layer, host, shared, x, ids, ws, fp16=0)
            err = oracle_mod.max_relative_error(got, want16)
            err32 = oracle_mod.max_relative_error(got, want32)
            print(f"  max rel err {err:.3e} against the FP16 graph, {err32:.3e} against the FP32 graph", flush=True)
            assert err <= 5e-4
            assert err < err32
    finally:
        backend.close()
