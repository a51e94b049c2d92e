"""Expert backend whose weights stay resident in HBM.

``HipExpertBackend`` speaks the duck-typed protocol the reference's MoE layer
uses (``src/flash_moe/moe_layer.py:62-67,76,125,147-149``; implemented there
by ``OpenVINOExpertBackend``, ``src/flash_moe/backend_ov.py:357-431``):

  forward(key, activation, hidden, inter)         one expert, one token
  forward_batch(key, activations, hidden, inter)  one expert, many tokens
  prefetch_weights(keys), begin_decode(), begin_prefill(), store, _moe_executor

plus two fused entry points that ``flash_moe_hip.moe_layer`` prefers:

  moe_layer(layer, activation, ids, weights)      every routed expert + shared, one launch
  moe_tokens(layer, activations, ids, weights)    the same for a batch of tokens

All arithmetic runs in the HIP kernels; results come back as NumPy FP32 like
the reference backend's.
"""
from __future__ import annotations

import numpy as np

from . import _lib
from .layer_store import ExpertLayer
from .moe_gpu import MoeRunner


class HipExpertBackend:
    def __init__(self, layers: dict[int, ExpertLayer], fp16_graph: int = 0, device=None):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("HipExpertBackend needs a HIP GPU")
        self.layers = dict(layers)
        self.fp16_graph = int(fp16_graph)
        self.runner = MoeRunner(device)
        self.device = self.runner.device
        # Weights are resident: there is no store to read or prefetch from,
        # and no worker pool (one launch covers all experts of a token).
        self.store = None
        self._moe_executor = None
        self._native_enabled = False

    # ------------------------------------------------------------ protocol
    def has_layer(self, layer: int) -> bool:
        return layer in self.layers

    def _get(self, layer: int, hidden_size: int, intermediate_size: int) -> ExpertLayer:
        L = self.layers.get(layer)
        if L is None:
            raise KeyError(f"layer {layer} is not resident")
        if (hidden_size, intermediate_size) != (L.hidden, L.intermediate):
            raise ValueError(f"layer {layer} is {L.hidden}x{L.intermediate}, "
                             f"called with {hidden_size}x{intermediate_size}")
        return L

    def prefetch_weights(self, keys):
        return None

    def begin_decode(self):
        self._native_enabled = True

    def begin_prefill(self):
        self._native_enabled = False

    def close(self):
        pass

    def _x(self, activations, hidden):
        import torch

        x = np.ascontiguousarray(activations, dtype=np.float32).reshape(-1, hidden)
        return torch.from_numpy(x).to(self.device)

    def _finish(self, y, what: str) -> np.ndarray:
        out = y.cpu().numpy()          # synchronizes the stream
        rc = self.runner.status()
        if rc:
            raise RuntimeError(f"{what} failed with status {rc} ({_lib.STATUS_TEXT.get(rc, 'unknown')})")
        return out

    def _run(self, layer: ExpertLayer, x, ids: np.ndarray | None, weights: np.ndarray | None,
             include_shared: bool, fp16_graph: int):
        import torch

        tid = tw = None
        if ids is not None:
            tid = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).to(self.device)
            tw = torch.from_numpy(np.ascontiguousarray(weights, dtype=np.float32)).to(self.device)
        return self.runner.decode(layer, x, tid, tw, fp16_graph=fp16_graph, use_shared=include_shared)

    def forward(self, key, activation, hidden_size: int, intermediate_size: int) -> np.ndarray:
        L = self._get(key.layer, hidden_size, intermediate_size)
        y = self._run(L, self._x(activation, hidden_size), np.array([[key.expert]]), np.ones((1, 1)),
                      False, self.fp16_graph)
        return self._finish(y, "native expert").reshape(hidden_size)

    def forward_batch(self, key, activations, hidden_size: int, intermediate_size: int) -> np.ndarray:
        x = np.ascontiguousarray(activations, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != hidden_size:
            raise ValueError(f"expert activations must have shape (tokens, {hidden_size}), got {x.shape}")
        if x.shape[0] == 0:
            return np.empty((0, hidden_size), dtype=np.float32)
        L = self._get(key.layer, hidden_size, intermediate_size)
        T = x.shape[0]
        y = self._run(L, self._x(x, hidden_size), np.full((T, 1), key.expert), np.ones((T, 1)),
                      False, self.fp16_graph)
        return self._finish(y, "native expert batch")

    # --------------------------------------------------------------- fused
    def moe_layer(self, layer: int, activation, expert_ids, weights, include_shared: bool = True) -> np.ndarray:
        L = self.layers[layer]
        y = self._run(L, self._x(activation, L.hidden), np.asarray(expert_ids).reshape(1, -1),
                      np.asarray(weights, dtype=np.float32).reshape(1, -1), include_shared, self.fp16_graph)
        return self._finish(y, "fused MoE layer").reshape(L.hidden)

    def moe_tokens(self, layer: int, activations, ids, weights, include_shared: bool = True) -> np.ndarray:
        """A prompt's tokens through the layer (run_moe_sequence): the grouped
        prefill kernels when they cover the layer (FP32 graph, more than one
        token), else the fused decode kernels."""
        import torch

        L = self.layers[layer]
        x = self._x(activations, L.hidden)
        if self.fp16_graph == 0 and x.shape[0] > 1 and self.runner.prefill_supported(L):
            tid = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).to(self.device)
            tw = torch.from_numpy(np.ascontiguousarray(weights, dtype=np.float32)).to(self.device)
            y = self.runner.prefill(L, x, tid, tw, use_shared=include_shared)
        else:
            y = self._run(L, x, ids, weights, include_shared, self.fp16_graph)
        return self._finish(y, "fused MoE tokens")

    def shared_forward(self, layer: int, activations) -> np.ndarray | None:
        L = self.layers.get(layer)
        if L is None or L.shared is None:
            return None
        y = self._run(L, self._x(activations, L.hidden), None, None, True, 0)
        return self._finish(y, "shared expert")
