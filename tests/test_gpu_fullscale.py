"""Parity at the benchmark shapes, every token against the oracle.

* Decode layer, 1 token per call: hidden 2048, 256 experts x intermediate 512,
  top-8 + shared, gate/up Q4_K, down Q6_K, router FP32 ~ N(0, 0.02); 8 tokens,
  each as its own call (host routing) and through the routed decode (routing
  on the device); the integer-digit path's error is also held to <= 1e-4.
* Batched decode: 16 tokens in one call, every matrix Q3_K, top-8 of N(0,1)
  logits (experts overlap across tokens); the decode kernels and the grouped
  prefill kernels.
* Decode in the reference model's type mixes (Q3_K; Q4_K/Q6_K; Q4_K/Q8_0 with
  the Q6_K shared expert): single tokens and 16-token calls, FP32 and FP16
  graphs, and the generic kernels beside the integer-digit ones.
* Prefill: a 128-token BF16 prompt, Q4_K/Q6_K, top-8 of N(0,1) logits over 256
  experts (~252 distinct experts, ~4 tokens each, ~262 partly filled tiles).

The oracle is the reference's run_moe_layer / run_moe_sequence arithmetic over
moe_quant_expert (moe_layer.py:39-195, moe_quant_dot.cpp:171-214).
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, E, I, K = 2048, 256, 512, 8
TOL = 1e-3          # the north star's bar
DIGIT_TOL = 1e-4    # the integer-digit decode kernels (measured ~5e-5)
PREFILL_TOL = 1e-4  # exact MFMA operands: only the summation order differs


def _host_layer(layer):
    host = {r: layer.tensors[r].cpu().numpy() for r in ("gate", "up", "down")}
    shared = layer.host_shared()
    gi = layer.shared.gate_inp.cpu().numpy()
    return host, shared, gi


def _oracle_tokens(oracle_mod, layer, host, shared, gi, X, ids, ws):
    """Oracle layer output for every token (threads: the oracle releases the GIL)."""
    types = layer.types

    def expert(e):
        return {r: host[r][e * layer.expert_bytes(r):(e + 1) * layer.expert_bytes(r)] for r in host}

    def one(t):
        x = np.asarray(X[t], np.float32)
        outs = [oracle_mod.expert_forward(expert(int(e)), types, x, H, I, 0) for e in ids[t]]
        gate = oracle_mod._sigmoid(np.float32(x @ gi).reshape(()))
        sh = (gate * oracle_mod.expert_forward(shared, layer.shared.types, x, H, I, 0)).astype(np.float32)
        return oracle_mod.combine(outs, [float(v) for v in ws[t]], sh)

    with ThreadPoolExecutor(8) as pool:
        return list(pool.map(one, range(len(X))))


def _topk(rng, T, k=K):
    logits = rng.standard_normal((T, E))
    ids = np.argsort(-logits, axis=1)[:, :k]
    sel = np.take_along_axis(logits, ids, 1)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    return ids.astype(np.int32), (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


@pytest.fixture(scope="module")
def decode_layer(hip):
    from flash_moe_hip.layer_store import ExpertLayer

    types = {"gate": 12, "up": 12, "down": 14}
    layer = ExpertLayer.synthetic(types, E, H, I, seed=1001, shared_types=types, shared_intermediate=I,
                                  gate_inp=True, device="cuda")
    return (layer, *_host_layer(layer))


def test_decode_layer_full_scale(decode_layer, oracle_mod, hip):
    import torch

    from flash_moe_hip.moe_gpu import MoeRunner
    from flash_moe_hip.router import ExpertRouter

    layer, host, shared, gi = decode_layer
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((H, E)) * 0.02).astype(np.float32)
    router = ExpertRouter(H, E, top_k=K, gate_weights=W, gate_dtype=np.float32)
    X = rng.standard_normal((8, H)).astype(np.float32)
    ids, ws = router.route_batch(X)
    want = _oracle_tokens(oracle_mod, layer, host, shared, gi, X, ids, ws)
    runner = MoeRunner()
    worst = 0.0
    for t in range(8):   # the benchmark's unit: one token per call
        print(f"full-scale decode token {t}", flush=True)
        y = runner.decode(layer, torch.from_numpy(X[t:t + 1]).cuda(), torch.from_numpy(ids[t:t + 1]).cuda(),
                          torch.from_numpy(ws[t:t + 1]).cuda())
        got, rc = runner.fetch(y)
        assert rc == 0
        err = oracle_mod.max_relative_error(got[0], want[t])
        worst = max(worst, err)
        assert err <= DIGIT_TOL, (t, err)
    print(f"  decode max rel err over 8 tokens: {worst:.3e}", flush=True)
    # the same tokens routed on the device in one call
    layer.router_weights = W
    y, rid, rw = runner.decode_routed(layer, torch.from_numpy(X).cuda(), K)
    got, rc = runner.fetch(y)
    assert rc == 0
    assert np.array_equal(rid.cpu().numpy(), ids)
    np.testing.assert_allclose(rw.cpu().numpy(), ws, rtol=0, atol=2e-6)
    for t in range(8):
        assert oracle_mod.max_relative_error(got[t], want[t]) <= DIGIT_TOL, t


def test_fp16_graph_decode_full_scale(oracle_mod, hip):
    """The decode layer in the FP16 graph (the reference's production mode) at
    the benchmark shape: 256 experts, top-8 + shared, Q4_K/Q6_K, 8 tokens each as
    its own call, scales of the reference's FP16-graph check (d ~ 0.002, x ~
    0.05), against the oracle's FP16 graph (routed) and FP32 shared expert."""
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    types = {"gate": 12, "up": 12, "down": 14}
    layer = ExpertLayer.synthetic(types, E, H, I, seed=1002, shared_types=types, shared_intermediate=I,
                                  gate_inp=True, scale=0.002, device="cuda")
    host, shared, gi = _host_layer(layer)
    rng = np.random.default_rng(2)
    X = (rng.standard_normal((8, H)) * 0.05).astype(np.float32)
    ids, ws = _topk(rng, 8)
    runner = MoeRunner()

    def expert(e):
        return {r: host[r][e * layer.expert_bytes(r):(e + 1) * layer.expert_bytes(r)] for r in host}

    worst = 0.0
    for t in range(8):
        print(f"full-scale FP16-graph decode token {t}", flush=True)
        got, rc = runner.fetch(runner.decode(layer, torch.from_numpy(X[t:t + 1]).cuda(),
                                             torch.from_numpy(ids[t:t + 1]).cuda(),
                                             torch.from_numpy(ws[t:t + 1]).cuda(), fp16_graph=1))
        assert rc == 0
        outs = [oracle_mod.expert_forward(expert(int(e)), types, X[t], H, I, 1) for e in ids[t]]
        gate = oracle_mod._sigmoid(np.float32(X[t] @ gi).reshape(()))
        sh = (gate * oracle_mod.expert_forward(shared, types, X[t], H, I, 0)).astype(np.float32)
        want = oracle_mod.combine(outs, [float(v) for v in ws[t]], sh)
        worst = max(worst, oracle_mod.max_relative_error(got[0], want))
    print(f"  FP16-graph decode max rel err over 8 tokens: {worst:.3e}", flush=True)
    assert worst <= 1e-3
    del layer
    torch.cuda.empty_cache()


def test_batched_decode_full_scale(oracle_mod, hip):
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    types = {"gate": 11, "up": 11, "down": 11}
    layer = ExpertLayer.synthetic(types, E, H, I, seed=7000, shared_types=types, shared_intermediate=I,
                                  gate_inp=True, device="cuda")
    host, shared, gi = _host_layer(layer)
    rng = np.random.default_rng(4)
    T = 16
    X = rng.standard_normal((T, H)).astype(np.float32)
    ids, ws = _topk(rng, T)
    print(f"batched decode: {len(np.unique(ids))} distinct experts", flush=True)
    want = _oracle_tokens(oracle_mod, layer, host, shared, gi, X, ids, ws)
    runner = MoeRunner()
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (X, ids, ws))
    for name, call in (("decode", runner.decode), ("prefill", runner.prefill)):
        print(f"batched {name}", flush=True)
        got, rc = runner.fetch(call(layer, xd, idd, wd))
        assert rc == 0
        tol = DIGIT_TOL if name == "decode" else PREFILL_TOL
        errs = [oracle_mod.max_relative_error(got[t], want[t]) for t in range(T)]
        print(f"  {name}: max rel err {max(errs):.3e}", flush=True)
        assert max(errs) <= tol, (name, int(np.argmax(errs)), max(errs))
    del layer
    torch.cuda.empty_cache()


def test_prefill_full_scale(oracle_mod, hip):
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    types = {"gate": 12, "up": 12, "down": 14}
    layer = ExpertLayer.synthetic(types, E, H, I, seed=9000, shared_types=types, shared_intermediate=I,
                                  gate_inp=True, device="cuda")
    host, shared, gi = _host_layer(layer)
    rng = np.random.default_rng(5)
    T = 128
    xb = torch.randn((T, H), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    X = xb.float().numpy()
    ids, ws = _topk(rng, T)
    print(f"prefill: {len(np.unique(ids))} distinct experts", flush=True)
    want = _oracle_tokens(oracle_mod, layer, host, shared, gi, X, ids, ws)
    runner = MoeRunner()
    got, rc = runner.fetch(runner.prefill(layer, xb.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda()))
    assert rc == 0
    errs = [oracle_mod.max_relative_error(got[t], want[t]) for t in range(T)]
    print(f"  prefill max rel err over {T} tokens: {max(errs):.3e}", flush=True)
    assert max(errs) <= PREFILL_TOL, (int(np.argmax(errs)), max(errs))
    del layer
    torch.cuda.empty_cache()


# The reference model's MoE layers (docs/PHASE0_FINDINGS.md:60-69): a Q6_K
# shared expert in every layer, beside Q3_K routed matrices (layers 5-34),
# Q4_K gate/up with a Q6_K down (layers 1-4, 35-39) or a Q8_0 down (layer 0).
REAL_MIXES = {
    "L5-34": {"gate": 11, "up": 11, "down": 11},
    "L1-4": {"gate": 12, "up": 12, "down": 14},
    "L0": {"gate": 12, "up": 12, "down": 8},
}


@pytest.mark.parametrize("mix", list(REAL_MIXES))
def test_prefill_real_model_mix_full_scale(oracle_mod, hip, mix):
    """A 128-token BF16 prompt through one layer of the reference model's type
    mix at full size (256 experts, hidden 2048, intermediate 512, top-8 + the
    Q6_K shared expert): the shared expert runs inside the grouped kernels
    (no decode-kernel fallback), every token within 1e-4 of the oracle's
    run_moe_sequence arithmetic (moe_layer.py:110-195, shared_expert.py:200-219)."""
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    types = REAL_MIXES[mix]
    q6 = {"gate": 14, "up": 14, "down": 14}
    layer = ExpertLayer.synthetic(types, E, H, I, seed=9100 + len(mix), shared_types=q6, shared_intermediate=I,
                                  gate_inp=True, device="cuda")
    assert MoeRunner.prefill_supported(layer) and MoeRunner._shared_in_prefill(layer)
    host, shared, gi = _host_layer(layer)
    rng = np.random.default_rng(6 + len(mix))
    T = 128
    xb = torch.randn((T, H), generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    X = xb.float().numpy()
    ids, ws = _topk(rng, T)
    print(f"prefill {mix} {types} + Q6_K shared: {len(np.unique(ids))} distinct experts", flush=True)
    want = _oracle_tokens(oracle_mod, layer, host, shared, gi, X, ids, ws)
    runner = MoeRunner()
    got, rc = runner.fetch(runner.prefill(layer, xb.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda()))
    assert rc == 0
    errs = [oracle_mod.max_relative_error(got[t], want[t]) for t in range(T)]
    print(f"  prefill {mix} max rel err over {T} tokens: {max(errs):.3e}", flush=True)
    assert max(errs) <= PREFILL_TOL, (int(np.argmax(errs)), max(errs))
    del layer
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fp16", [0, 1], ids=["fp32-graph", "fp16-graph"])
@pytest.mark.parametrize("mix", list(REAL_MIXES))
def test_decode_real_model_mix_full_scale(oracle_mod, hip, mix, fp16):
    """The decode layer in the reference model's type mixes at full size (256
    experts, hidden 2048, intermediate 512, top-8 + the Q6_K shared expert):
    four tokens each as its own call (kernel A with the shared item on two
    waves and the shared expert's own item code) and 16 tokens in one call
    (two items a wave), both graphs (the FP16 graph at its check scales, d ~
    0.002, x ~ 0.05), every token against the oracle: routed experts in the
    call's graph, the shared expert in the FP32 graph as the reference runs it."""
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    types = REAL_MIXES[mix]
    q6 = {"gate": 14, "up": 14, "down": 14}
    kw = {"scale": 0.002} if fp16 else {}
    layer = ExpertLayer.synthetic(types, E, H, I, seed=9200 + len(mix) + 10 * fp16, shared_types=q6,
                                  shared_intermediate=I, gate_inp=True, device="cuda", **kw)
    host, shared, gi = _host_layer(layer)
    rng = np.random.default_rng(60 + len(mix) + fp16)
    X = (rng.standard_normal((20, H)) * (0.05 if fp16 else 1.0)).astype(np.float32)
    ids, ws = _topk(rng, 20)

    def expert(e):
        return {r: host[r][e * layer.expert_bytes(r):(e + 1) * layer.expert_bytes(r)] for r in host}

    def want(t):
        outs = [oracle_mod.expert_forward(expert(int(e)), types, X[t], H, I, fp16) for e in ids[t]]
        gate = oracle_mod._sigmoid(np.float32(X[t] @ gi).reshape(()))
        sh = (gate * oracle_mod.expert_forward(shared, q6, X[t], H, I, 0)).astype(np.float32)
        return oracle_mod.combine(outs, [float(v) for v in ws[t]], sh)

    with ThreadPoolExecutor(8) as pool:
        wants = list(pool.map(want, range(20)))
    runner = MoeRunner()
    # the digit error of a 16-column run (<= 1.6e-5 of its max per value), in the
    # hidden vector and again in the SwiGLU product, reaches ~1.2e-4 of the output
    # on the Q4_K/Q6_K mix's tokens here (the same bound the 32-expert tests hold)
    tol = TOL if fp16 else 2 * DIGIT_TOL
    worst = 0.0
    for t in range(4):
        print(f"full-scale decode {mix} fp16={fp16} token {t}", flush=True)
        got, rc = runner.fetch(runner.decode(layer, torch.from_numpy(X[t:t + 1]).cuda(),
                                             torch.from_numpy(ids[t:t + 1]).cuda(),
                                             torch.from_numpy(ws[t:t + 1]).cuda(), fp16_graph=fp16))
        assert rc == 0
        worst = max(worst, oracle_mod.max_relative_error(got[0], wants[t]))
    print(f"full-scale decode {mix} fp16={fp16}: 16 tokens in one call", flush=True)
    got, rc = runner.fetch(runner.decode(layer, torch.from_numpy(X[4:]).cuda(), torch.from_numpy(ids[4:]).cuda(),
                                         torch.from_numpy(ws[4:]).cuda(), fp16_graph=fp16))
    assert rc == 0
    for t in range(16):
        worst = max(worst, oracle_mod.max_relative_error(got[t], wants[4 + t]))
    print(f"  decode {mix} fp16={fp16} max rel err over 20 tokens: {worst:.3e}", flush=True)
    assert worst <= tol
    if not fp16:
        # the generic kernels (FP32 activations, no digits) on the same 16 tokens:
        # the FP32 reference arithmetic up to summation order
        old = hip.mqh_set_decode_path(1)
        try:
            gen, rc = runner.fetch(runner.decode(layer, torch.from_numpy(X[4:]).cuda(),
                                                 torch.from_numpy(ids[4:]).cuda(), torch.from_numpy(ws[4:]).cuda()))
        finally:
            hip.mqh_set_decode_path(old)
        assert rc == 0
        gen_err = max(oracle_mod.max_relative_error(gen[t], wants[4 + t]) for t in range(16))
        print(f"  generic kernels {mix}: max rel err {gen_err:.3e}", flush=True)
        assert gen_err <= 1e-5
    del layer
    torch.cuda.empty_cache()
