"""MoE layer entry points with the reference's signatures (``src/flash_moe/moe_layer.py``).

``run_moe_layer`` (moe_layer.py:39-107) and ``run_moe_sequence``
(moe_layer.py:110-195) compute, per token,

    sum_k fl32(w_k) * E_{id_k}(x)   (FP32, top-k order)   +  shared(x)

Two ways through:

* Fused: a backend that offers ``moe_layer`` / ``moe_tokens``
  (``HipExpertBackend``) gets every routed expert of every token, plus the
  shared expert when it is this package's ``SharedExpert`` over the same
  backend, in one call (two kernels for decode, the grouped GEMM for a
  prompt).  The router runs on the host exactly as in the reference.
* Protocol: any other backend is driven the way the reference drives it --
  ``forward`` per routed expert, fanned out on the backend's
  ``_moe_executor`` (or a pool of its own) and summed in top-k order; for a
  sequence, tokens bucketed per expert, ``forward`` for an expert with one
  token and ``forward_batch`` for more, and the shared expert per token or,
  for 16..128 tokens with a ``SharedExpert``, batched.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from typing import Any

import numpy as np

from .key import ExpertKey
from .shared_expert import SharedExpert

BATCH_SHARED_TOKENS = (16, 128)   # run_moe_sequence batches the shared expert in this range
PREFETCH_LOOKAHEAD = 8


def _fused_shared(backend, shared_expert) -> bool:
    return isinstance(shared_expert, SharedExpert) and shared_expert.backend is backend


def _prefetch(backend, keys) -> None:
    prefetch = getattr(backend, "prefetch_weights", None)
    store = getattr(backend, "store", None)
    if prefetch is not None:
        prefetch(keys)
    elif store is not None and hasattr(store, "prefetch_many"):
        store.prefetch_many(keys)


def _add_shared(combined, layer, activation, shared_expert):
    if shared_expert is not None:
        shared_out = shared_expert.forward(layer, activation)
        if shared_out is not None:
            combined = combined + shared_out
    return combined


def run_moe_layer(layer: int, activation, router, backend: Any, hidden_size: int, intermediate_size: int,
                  shared_expert: Any = None) -> np.ndarray:
    expert_ids, weights = router.route(activation)
    fused = getattr(backend, "moe_layer", None)
    if fused is not None and backend.has_layer(layer):
        inside = _fused_shared(backend, shared_expert)
        combined = fused(layer, activation, expert_ids, weights, include_shared=inside)
        return combined if inside else _add_shared(combined, layer, activation, shared_expert)

    keys = [ExpertKey(layer, int(e)) for e in expert_ids]
    _prefetch(backend, keys)
    combined = np.zeros(hidden_size, dtype=np.float32)
    if len(keys) == 1:
        out = backend.forward(keys[0], activation, hidden_size, intermediate_size)
        combined += weights[0] * np.asarray(out, dtype=np.float32)
    else:
        executor = getattr(backend, "_moe_executor", None)
        own = executor is None
        if own:
            executor = ThreadPoolExecutor(max_workers=len(keys))
        try:
            futures = [executor.submit(backend.forward, key, activation, hidden_size, intermediate_size)
                       for key in keys]
            try:
                for future, weight in zip(futures, weights):
                    combined += weight * np.asarray(future.result(), dtype=np.float32)
            finally:
                for future in futures:   # no worker may still run when an error propagates
                    try:
                        future.result()
                    except Exception:
                        pass
        finally:
            if own:
                executor.shutdown(wait=True)
    return _add_shared(combined, layer, activation, shared_expert)


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

    forward_batch = getattr(backend, "forward_batch", None)
    if forward_batch is None:
        return np.stack([run_moe_layer(layer, x, router, backend, hidden_size, intermediate_size, shared_expert)
                         for x in activations])

    # bucket (token, slot) by expert in first-seen order (moe_layer.py:135-173)
    routed: list[list[float]] = [[] for _ in range(T)]
    grouped: dict[ExpertKey, list[tuple[int, int]]] = {}
    for t, x in enumerate(activations):
        ids, ws = router.route(x)
        for slot, (e, w) in enumerate(zip(ids, ws)):
            routed[t].append(w)
            grouped.setdefault(ExpertKey(layer, int(e)), []).append((t, slot))
    keys = list(grouped)
    top_k = max((len(r) for r in routed), default=0)
    outs = np.empty((T, top_k, hidden_size), np.float32)
    _prefetch(backend, keys[:PREFETCH_LOOKAHEAD])
    for i, key in enumerate(keys):
        routes = grouped[key]
        tok = [t for t, _ in routes]
        if len(routes) == 1:
            y = np.asarray([backend.forward(key, activations[tok[0]], hidden_size, intermediate_size)])
        else:
            y = forward_batch(key, activations[tok], hidden_size, intermediate_size)
        for j, (t, slot) in enumerate(routes):
            outs[t, slot] = y[j]
        _prefetch(backend, keys[i + 1:i + 1 + PREFETCH_LOOKAHEAD])

    lo, hi = BATCH_SHARED_TOKENS
    batch_shared = lo <= T <= hi and isinstance(shared_expert, SharedExpert)
    result = np.zeros((T, hidden_size), np.float32)
    for t, ws in enumerate(routed):
        for slot, w in enumerate(ws):
            result[t] += w * outs[t, slot]
        if shared_expert is not None and not batch_shared:
            shared_out = shared_expert.forward(layer, activations[t])
            if shared_out is not None:
                result[t] += shared_out
    if batch_shared:
        shared_out = shared_expert.forward_batch(layer, activations)
        if shared_out is not None:
            result += shared_out
    return result


def _route_all(router, activations):
    ids, ws = zip(*(router.route(x) for x in activations))
    return np.asarray(ids, np.int32), np.asarray(ws, np.float32)
