"""The 112-byte Q3_K resident form (type 111, ``ExpertLayer.aligned_q3k``).

The same blocks, each in a 16-byte-aligned slot, must decode to outputs
bit-identical to the GGUF-layout layer's (the kernels read the same bytes at
other addresses), in both graphs and at 1, 4 and 16 tokens, with Q3_K or Q6_K
shared experts.  Every path that does not read the form (generic kernels,
routed and prefill entry points, a shared expert left in GGUF layout) must
refuse it rather than misread it.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E, H, I, K = 256, 2048, 512, 8


def _layer(types, shared_types, seed, fp16):
    import torch
    from flash_moe_hip.layer_store import ExpertLayer

    kw = dict(scale=0.002) if fp16 else {}
    return ExpertLayer.synthetic(types, E, H, I, seed=seed, shared_types=shared_types, shared_intermediate=I,
                                 gate_inp=True, device=torch.device("cuda", 0), **kw)


def _inputs(T, seed, fp16):
    import torch

    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32) * (0.05 if fp16 else 1.0)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.dirichlet(np.ones(K), size=T).astype(np.float32)
    return (torch.from_numpy(v).cuda() for v in (x, ids, w))


Q3 = {"gate": 11, "up": 11, "down": 11}
Q6 = {"gate": 14, "up": 14, "down": 14}


@pytest.mark.parametrize("fp16", [0, 1])
@pytest.mark.parametrize("T", [1, 4, 16])
@pytest.mark.parametrize("shared", ["q3k", "q6k"])
def test_aligned_q3k_bit_identical(fp16, T, shared):
    import torch
    from flash_moe_hip.moe_gpu import MoeRunner

    print(f"aligned Q3_K decode: T={T} fp16={fp16} shared={shared}", flush=True)
    layer = _layer(Q3, Q3 if shared == "q3k" else Q6, seed=40 + T, fp16=fp16)
    al = layer.aligned_q3k()
    assert al.types == {"gate": 111, "up": 111, "down": 111}
    assert al.tensors["gate"].numel() == layer.tensors["gate"].numel() // 110 * 112
    x, ids, w = _inputs(T, 7 + T, fp16)
    r = MoeRunner(torch.device("cuda", 0))
    y0 = r.decode(layer, x, ids, w, fp16_graph=fp16)
    y1 = r.decode(al, x, ids, w, fp16_graph=fp16)
    torch.cuda.synchronize()
    assert r.status() == 0
    assert torch.isfinite(y0).all()
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))


def test_aligned_q3k_refused_outside_fast_decode(hip):
    import torch
    from flash_moe_hip.layer_store import ExpertLayer, SharedWeights
    from flash_moe_hip.moe_gpu import MoeRunner

    print("aligned Q3_K refusals", flush=True)
    layer = _layer(Q3, Q3, seed=3, fp16=0)
    al = layer.aligned_q3k()
    x, ids, w = _inputs(2, 5, 0)
    r = MoeRunner(torch.device("cuda", 0))
    # the generic kernels read GGUF blocks only
    old = hip.mqh_set_decode_path(1)
    try:
        with pytest.raises(RuntimeError, match="status"):
            r.decode(al, x, ids, w)
    finally:
        hip.mqh_set_decode_path(old)
    # routed experts in the aligned form beside a shared expert left in GGUF layout
    s = layer.shared
    mixed = ExpertLayer(al.tensors["gate"], al.tensors["up"], al.tensors["down"], al.types, E, H, I,
                        SharedWeights(s.gate, s.up, s.down, types=s.types, intermediate=s.intermediate,
                                      gate_inp=s.gate_inp))
    with pytest.raises(RuntimeError, match="status"):
        r.decode(mixed, x, ids, w)
    # the routed-decode entry point and the prefill kernels take GGUF blocks only
    with pytest.raises(RuntimeError, match="status"):
        r.decode_routed(al, x, K, router_w=torch.zeros((E, H), dtype=torch.float32, device="cuda"))
    assert not MoeRunner.prefill_supported(al)
    torch.cuda.synchronize()
    # the GGUF-layout layer still decodes after the refusals
    y = r.decode(layer, x, ids, w)
    torch.cuda.synchronize()
    assert r.status() == 0 and torch.isfinite(y).all()
