"""MoE layer entry points with the reference's signatures (``src/flash_moe/moe_layer.py``).

``run_moe_layer`` (moe_layer.py:39-107) and ``run_moe_sequence``
(moe_layer.py:110-195) compute, per token,

    sum_k fl32(w_k) * E_{id_k}(x)   (FP32, top-k order)   +  shared(x)

With a backend that offers the fused entry points (``HipExpertBackend``) the
router runs on the host exactly as in the reference, and all routed experts of
all tokens plus the shared expert (when it is this library's ``SharedExpert``
on the same backend) go to the GPU in one fused call.  Any other backend is
driven through the plain ``forward``/``forward_batch`` protocol with the same
combine arithmetic.
"""
from __future__ import annotations

from typing import Any

import numpy as np

from .key import ExpertKey
from .shared_expert import SharedExpert


def _fused_shared(backend, shared_expert) -> bool:
    return isinstance(shared_expert, SharedExpert) and shared_expert.backend is backend


def run_moe_layer(layer: int, activation, router, backend: Any, hidden_size: int, intermediate_size: int,
                  shared_expert: Any = None) -> np.ndarray:
    expert_ids, weights = router.route(activation)
    fused = getattr(backend, "moe_layer", None)
    if fused is not None and backend.has_layer(layer):
        inside = _fused_shared(backend, shared_expert)
        combined = fused(layer, activation, expert_ids, weights, include_shared=inside)
        if shared_expert is not None and not inside:
            shared_out = shared_expert.forward(layer, activation)
            if shared_out is not None:
                combined = combined + shared_out
        return combined

    combined = np.zeros(hidden_size, dtype=np.float32)
    for expert_id, weight in zip(expert_ids, weights):
        out = backend.forward(ExpertKey(layer, expert_id), activation, hidden_size, intermediate_size)
        combined += weight * np.asarray(out, dtype=np.float32)
    if shared_expert is not None:
        shared_out = shared_expert.forward(layer, activation)
        if shared_out is not None:
            combined = combined + shared_out
    return combined


def run_moe_sequence(layer: int, activations: np.ndarray, router, backend: Any, hidden_size: int,
                     intermediate_size: int, shared_expert: Any = None) -> np.ndarray:
    if activations.ndim != 2 or activations.shape[1] != hidden_size:
        raise ValueError(f"MoE activations must have shape (tokens, {hidden_size}), got {activations.shape}")
    T = activations.shape[0]
    fused = getattr(backend, "moe_tokens", None)
    if fused is not None and backend.has_layer(layer):
        ids, ws = router.route_batch(activations) if hasattr(router, "route_batch") else _route_all(router, activations)
        inside = _fused_shared(backend, shared_expert)
        result = fused(layer, activations, ids, ws, include_shared=inside)
        if shared_expert is not None and not inside:
            shared_out = shared_expert.forward_batch(layer, activations)
            if shared_out is not None:
                result = result + shared_out
        return result

    # generic backend: bucket tokens by expert (moe_layer.py:135-173)
    routed, grouped = [], {}
    for t, x in enumerate(activations):
        ids, ws = router.route(x)
        routed.append(list(zip(ids, ws)))
        for slot, (e, w) in enumerate(zip(ids, ws)):
            grouped.setdefault(e, []).append((t, slot))
    top_k = max(len(r) for r in routed) if routed else 0
    outs = np.empty((T, top_k, hidden_size), np.float32)
    for e, routes in grouped.items():
        tok = [t for t, _ in routes]
        y = backend.forward_batch(ExpertKey(layer, e), activations[tok], hidden_size, intermediate_size)
        for i, (t, slot) in enumerate(routes):
            outs[t, slot] = y[i]
    result = np.zeros((T, hidden_size), np.float32)
    for t, r in enumerate(routed):
        for slot, (_, w) in enumerate(r):
            result[t] += w * outs[t, slot]
    if shared_expert is not None:
        shared_out = shared_expert.forward_batch(layer, activations)
        if shared_out is not None:
            result += shared_out
    return result


def _route_all(router, activations):
    ids, ws = zip(*(router.route(x) for x in activations))
    return np.asarray(ids, np.int32), np.asarray(ws, np.float32)
