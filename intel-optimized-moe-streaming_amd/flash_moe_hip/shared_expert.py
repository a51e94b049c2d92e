"""Shared expert on the GPU (drop-in for ``SharedExpert``, src/flash_moe/shared_expert.py).

``forward(layer, x)`` and ``forward_batch(layer, X)`` return
``sigmoid(x . gate_inp) * W_down (silu(W_gate x) * (W_up x))`` in FP32
(shared_expert.py:200-251), or ``None`` for a layer without a shared expert.
The weights are the layer's quantized ``*_shexp`` tensors resident in HBM and
decoded exactly in the kernel; the reference instead promotes an FP16
dequantization to FP32 (shared_expert.py:141-149), a difference of at most
one FP16 rounding per weight.
"""
from __future__ import annotations

import numpy as np

from .backend import HipExpertBackend


class SharedExpert:
    def __init__(self, backend: HipExpertBackend):
        self.backend = backend
        self.hidden_size = next(iter(backend.layers.values())).hidden if backend.layers else 0

    def has(self, layer: int) -> bool:
        L = self.backend.layers.get(layer)
        return L is not None and L.shared is not None

    def forward(self, layer: int, activation) -> np.ndarray | None:
        if not self.has(layer):
            return None
        x = np.asarray(activation, dtype=np.float32).reshape(-1)
        if x.size != self.backend.layers[layer].hidden:
            raise ValueError(f"activation has {x.size} elements, expected {self.backend.layers[layer].hidden}")
        return self.backend.shared_forward(layer, x).reshape(-1)

    def forward_batch(self, layer: int, activations) -> np.ndarray | None:
        if not self.has(layer):
            return None
        x = np.ascontiguousarray(activations, dtype=np.float32)
        H = self.backend.layers[layer].hidden
        if x.ndim != 2 or x.shape[1] != H:
            raise ValueError(f"shared activations must have shape (tokens, {H})")
        return self.backend.shared_forward(layer, x)
