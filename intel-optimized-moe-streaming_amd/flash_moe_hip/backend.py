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

Numerics.  The reference's decode calls its native expert in the FP16 graph
(``native_expert.py:33-34``, reached through ``backend_ov.py:373-377``), so
``fp16_graph`` defaults to 1: ``forward``, ``forward_batch`` and ``moe_layer``
round to FP16 at the points of ``moe_quant_dot.cpp:189-211`` (the shared
expert runs the FP32 graph, as the reference's NumPy shared expert does).
``fp16_graph=0`` gives the FP32 graph.  ``moe_tokens`` (the prompt path) runs
the grouped prefill kernels whenever they cover the layer, in either setting:
the reference's prompt path is its OpenVINO expert graph
(``backend_ov.py:210-237, 407-431``), not the native FP16 graph, and the
prefill kernels' exact FP16 products with FP32 accumulation stay within 1e-4
of the FP32 graph.

All arithmetic runs in the HIP kernels; results come back as NumPy FP32 like
the reference backend's.  Each call stages its inputs through the calling
thread's pinned host buffer (one host-to-device copy, no allocation) and
returns after one synchronisation, which also reads the kernels' fault
flags.  The calls are thread-safe: the reference runs ``forward`` for a
token's experts on the backend's ``_moe_executor`` (``moe_layer.py:74-94``),
and every worker thread has a workspace and pinned buffers of its own.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import _lib
from .layer_store import ExpertLayer
from .moe_gpu import MoeRunner


class HipExpertBackend:
    def __init__(self, layers: dict[int, ExpertLayer], fp16_graph: int = 1, device=None, expert_workers: int = 4):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("HipExpertBackend needs a HIP GPU")
        self.layers = dict(layers)
        self.fp16_graph = int(fp16_graph)
        self.runner = MoeRunner(device)
        self.device = self.runner.device
        # Weights are resident: there is no store to read or prefetch from.
        # The bounded worker pool the reference's run_moe_layer fans forward()
        # out on (backend_ov.py:160); the fused entry points do not use it.
        self.store = None
        self._moe_executor = ThreadPoolExecutor(max_workers=max(1, int(expert_workers)))
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
        self._moe_executor.shutdown(wait=True)

    def _stage(self, activations, hidden: int, ids=None, weights=None):
        """x [T, hidden] FP32 and the optional ids [T, k] int32 / weights [T, k]
        FP32 on the device, through one pinned host buffer and one copy."""
        import torch

        x = np.asarray(activations, dtype=np.float32).reshape(-1, hidden)
        T = x.shape[0]
        k = 0 if ids is None else int(np.asarray(ids).reshape(T, -1).shape[1])
        if not k:
            (xd,) = self.runner.upload([x])
            return xd.view(torch.float32).view(T, hidden), None, None
        xd, idd, wd = self.runner.upload([x, np.asarray(ids, dtype=np.int64).reshape(T, k).astype(np.int32),
                                          np.asarray(weights, dtype=np.float32).reshape(T, k)])
        return (xd.view(torch.float32).view(T, hidden), idd.view(torch.int32).view(T, k),
                wd.view(torch.float32).view(T, k))

    def _finish(self, y, what: str) -> np.ndarray:
        out, rc = self.runner.fetch(y)
        if rc:
            raise RuntimeError(f"{what} failed with status {rc} ({_lib.STATUS_TEXT.get(rc, 'unknown')})")
        return out

    def _decode(self, layer: ExpertLayer, activations, ids, weights, include_shared: bool, fp16_graph: int):
        x, tid, tw = self._stage(activations, layer.hidden, ids, weights)
        return self.runner.decode(layer, x, tid, tw, fp16_graph=fp16_graph, use_shared=include_shared)

    def forward(self, key, activation, hidden_size: int, intermediate_size: int) -> np.ndarray:
        L = self._get(key.layer, hidden_size, intermediate_size)
        y = self._decode(L, activation, [[key.expert]], [[1.0]], False, self.fp16_graph)
        return self._finish(y, "native expert").reshape(hidden_size)

    def forward_batch(self, key, activations, hidden_size: int, intermediate_size: int) -> np.ndarray:
        x = np.ascontiguousarray(activations, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != hidden_size:
            raise ValueError(f"expert activations must have shape (tokens, {hidden_size}), got {x.shape}")
        if x.shape[0] == 0:
            return np.empty((0, hidden_size), dtype=np.float32)
        L = self._get(key.layer, hidden_size, intermediate_size)
        T = x.shape[0]
        y = self._decode(L, x, np.full((T, 1), key.expert), np.ones((T, 1)), False, self.fp16_graph)
        return self._finish(y, "native expert batch")

    # --------------------------------------------------------------- fused
    def moe_layer(self, layer: int, activation, expert_ids, weights, include_shared: bool = True) -> np.ndarray:
        L = self.layers[layer]
        y = self._decode(L, activation, np.asarray(expert_ids).reshape(1, -1),
                         np.asarray(weights, dtype=np.float32).reshape(1, -1), include_shared, self.fp16_graph)
        return self._finish(y, "fused MoE layer").reshape(L.hidden)

    def moe_tokens(self, layer: int, activations, ids, weights, include_shared: bool = True) -> np.ndarray:
        """A prompt's tokens through the layer (run_moe_sequence): the grouped
        prefill kernels when they cover the layer (more than one token, any
        ``fp16_graph``), else the fused decode kernels in the backend's graph."""
        L = self.layers[layer]
        x, tid, tw = self._stage(activations, L.hidden, ids, weights)
        if x.shape[0] > 1 and self.runner.prefill_supported(L):
            y = self.runner.prefill(L, x, tid, tw, use_shared=include_shared)
        else:
            y = self.runner.decode(L, x, tid, tw, fp16_graph=self.fp16_graph, use_shared=include_shared)
        return self._finish(y, "fused MoE tokens")

    def shared_forward(self, layer: int, activations) -> np.ndarray | None:
        L = self.layers.get(layer)
        if L is None or L.shared is None:
            return None
        y = self._decode(L, activations, None, None, True, 0)
        return self._finish(y, "shared expert")
