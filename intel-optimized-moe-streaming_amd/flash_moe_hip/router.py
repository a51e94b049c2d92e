"""MoE router with the reference's semantics (``src/flash_moe/router.py``).

``ExpertRouter.route(x)`` returns ``(ids, weights)``: ids are the top-k
experts by FP32 score ``x @ W`` in descending order (NumPy argsort, last k,
reversed; router.py:151-156), weights the float64 softmax over the selected
scores (router.py:157-170), which equals the softmax over all experts
renormalised over the selection.  Gate weights are stored rounded to
``gate_dtype`` (FP16 by default) and promoted to FP32 once (router.py:39-59).

``route_batch`` returns the device-ready int32/FP32 arrays for a batch of
tokens, in the layout the fused kernels read.  ``from_gguf_tensor`` and
``routers_from_gguf`` build the per-layer routers from
``blk.N.ffn_gate_inp.weight`` (router.py:93-140, 180-210): the tensor map of
``GGUFFile.tensor_map()`` or of the ``gguf`` package's reader.
"""
from __future__ import annotations

import numpy as np


class ExpertRouter:
    def __init__(self, hidden_size: int, num_experts: int, top_k: int = 2,
                 gate_weights: np.ndarray | None = None, gate_dtype=np.float16) -> None:
        if top_k < 1:
            raise ValueError(f"top_k must be at least 1, got {top_k}")
        if num_experts < 1:
            raise ValueError(f"num_experts must be at least 1, got {num_experts}")
        if gate_weights is None:
            raise ValueError("ExpertRouter requires the layer's ffn_gate_inp weights")
        self.hidden_size = hidden_size
        self.num_experts = num_experts
        self.top_k = min(top_k, num_experts)
        self.gate_dtype = np.dtype(gate_dtype)
        w = np.asarray(gate_weights, dtype=self.gate_dtype)
        if w.shape != (hidden_size, num_experts):
            if w.shape == (num_experts, hidden_size):   # GGUF (n_expert, n_embd) order
                w = w.T
            else:
                raise ValueError(f"gate weight shape {w.shape} is neither ({hidden_size}, {num_experts}) "
                                 f"nor ({num_experts}, {hidden_size})")
        if not np.isfinite(w.astype(np.float32)).all():
            raise ValueError("gate weights contain NaN or Inf")
        self.gate_weights = np.ascontiguousarray(w, dtype=np.float32)

    @classmethod
    def from_gguf_tensor(cls, tensor, hidden_size: int, num_experts: int, top_k: int,
                         gate_dtype=np.float16) -> "ExpertRouter":
        """The layer's router from ``ffn_gate_inp.weight``: ``tensor.shape`` in
        ggml order (hidden first), so the stored matrix is (experts, hidden)
        and is transposed by the constructor."""
        shape = tuple(int(s) for s in reversed(tensor.shape))
        if shape not in ((num_experts, hidden_size), (hidden_size, num_experts)):
            raise ValueError(f"ffn_gate_inp shape {shape} does not match {num_experts} experts x "
                             f"{hidden_size} hidden")
        gate = np.asarray(tensor.data)
        if gate.size != num_experts * hidden_size:
            raise ValueError(f"ffn_gate_inp has {gate.size} elements, expected {num_experts * hidden_size}")
        return cls(hidden_size=hidden_size, num_experts=num_experts, top_k=top_k,
                   gate_weights=gate.reshape(shape).astype(gate_dtype, copy=False), gate_dtype=gate_dtype)

    def scores(self, activation) -> np.ndarray:
        x = np.asarray(activation, dtype=np.float32).reshape(-1)
        if x.size != self.hidden_size:
            raise ValueError(f"activation has {x.size} elements, expected {self.hidden_size}")
        return (x @ self.gate_weights).astype(np.float32)

    def route(self, activation) -> tuple[list[int], list[float]]:
        scores = self.scores(activation)
        idx = np.argsort(scores)[-self.top_k:][::-1].astype(np.int64).tolist()
        sel = scores[idx].astype(np.float64)
        e = np.exp(sel - np.max(sel))
        total = e.sum()
        if not np.isfinite(total) or total <= 0.0:
            w = np.full(len(idx), 1.0 / len(idx))
        else:
            w = e / total
        return idx, [float(v) for v in w]

    def route_batch(self, activations) -> tuple[np.ndarray, np.ndarray]:
        """int32 ids [T, k] and FP32 weights [T, k] for every row of ``activations``."""
        X = np.asarray(activations, dtype=np.float32).reshape(-1, self.hidden_size)
        ids = np.empty((X.shape[0], self.top_k), np.int32)
        ws = np.empty((X.shape[0], self.top_k), np.float32)
        for t, x in enumerate(X):
            i, w = self.route(x)
            ids[t] = i
            ws[t] = w
        return ids, ws


def softmax_all_experts(scores: np.ndarray) -> np.ndarray:
    s = np.asarray(scores, dtype=np.float64)
    e = np.exp(s - s.max())
    return e / e.sum()


def routers_from_gguf(tmap: dict, num_layers: int, hidden_size: int, num_experts: int, top_k: int,
                      arch: str = "qwen35moe", gate_dtype=np.float16) -> dict[int, ExpertRouter]:
    """{layer: ExpertRouter} from every ``blk.N.ffn_gate_inp.weight`` of the
    tensor map; a layer without one raises KeyError (router.py:180-210)."""
    routers: dict[int, ExpertRouter] = {}
    missing: list[int] = []
    for layer in range(num_layers):
        t = tmap.get(f"blk.{layer}.ffn_gate_inp.weight")
        if t is None:
            missing.append(layer)
            continue
        routers[layer] = ExpertRouter.from_gguf_tensor(t, hidden_size, num_experts, top_k, gate_dtype=gate_dtype)
    if missing:
        raise KeyError(f"ffn_gate_inp.weight is missing for layers {missing}: the experts to run cannot be chosen")
    return routers


def synthetic_router(hidden_size: int, num_experts: int, top_k: int, seed: int = 0,
                     layer: int | None = None) -> ExpertRouter:
    """Deterministic random router for tests and benchmarks; each layer gets
    seed + 1000 * layer (router.py:213-229)."""
    rng = np.random.default_rng(seed if layer is None else seed + 1000 * layer)
    gate = rng.standard_normal((hidden_size, num_experts)).astype(np.float16)
    return ExpertRouter(hidden_size, num_experts, top_k=top_k, gate_weights=gate)
