"""Shared expert on the GPU (drop-in for ``SharedExpert``, src/flash_moe/shared_expert.py).

``SharedExpert(gguf_path, num_layers, hidden_size, intermediate_size,
dequant_fn=None, reader=None)`` loads every layer's ``ffn_{gate,up,down}_shexp``
and ``ffn_gate_inp_shexp`` tensors, as the reference does
(shared_expert.py:121-155), but keeps the three matrices QUANTIZED in HBM:
the kernels decode them exactly on the fly, so ``dequant_fn`` is accepted and
not needed.  A layer without the three matrices raises KeyError, as in the
reference.  ``SharedExpert.from_backend(backend)`` uses the shared experts a
``HipExpertBackend`` already holds; ``flash_moe_hip.moe_layer`` then runs the
shared expert inside the same fused launch as the routed experts.

``forward(layer, x)`` and ``forward_batch(layer, X)`` return
``sigmoid(x . gate_inp) * W_down (silu(W_gate x) * (W_up x))`` in FP32
(shared_expert.py:200-251), or ``None`` for a layer without a shared expert.
The reference instead multiplies FP32 copies of FP16-dequantized weights
(shared_expert.py:141-149): the two differ by at most one FP16 rounding per
weight.  ``gate_inp`` is stored as the reference stores it: rounded to FP16,
then promoted to FP32 (shared_expert.py:147, 173).

The three matrices must be in a quantized type the kernels decode (Q3_K,
Q4_K, Q5_K, Q6_K, Q8_0, IQ4_NL).  The reference also accepts F32/F16 shared
matrices (shared_expert.py:165-173); this class rejects them in the
constructor with a ``ValueError`` naming the tensor.
"""
from __future__ import annotations

import os

import numpy as np

from .layer_store import SharedWeights, _to_device_bytes
from .quant_types import DEVICE_TYPES, name_of, tensor_bytes

SHARED_ROLES = {
    "gate_inp": "ffn_gate_inp_shexp.weight",
    "gate": "ffn_gate_shexp.weight",
    "up": "ffn_up_shexp.weight",
    "down": "ffn_down_shexp.weight",
}


def shared_expert_present(tensor_map: dict, layer: int) -> bool:
    """True when the layer has the three SwiGLU matrices (gate_inp alone is not enough)."""
    return all(f"blk.{layer}.{SHARED_ROLES[r]}" in tensor_map for r in ("gate", "up", "down"))


def _reader_tensors(gguf_path, reader) -> dict:
    """name -> tensor with ``data`` and ``tensor_type`` (this package's
    GGUFFile, or any reader exposing ``tensors`` as the ``gguf`` package does)."""
    from .gguf_file import GGUFFile

    if reader is None:
        reader = GGUFFile(os.fspath(gguf_path))
    if isinstance(reader, GGUFFile):
        return reader.tensor_map()
    return {t.name: t for t in reader.tensors}


def _quantized_bytes(tensor, name: str, shape: tuple[int, int]) -> np.ndarray:
    """The raw block bytes of a quantized shared matrix of (rows, cols) =
    ``shape``; a type the kernels do not decode (F32, F16, ...) or a byte count
    that does not fit the shape raises ``ValueError`` here rather than at the
    first forward."""
    t = int(tensor.tensor_type)
    if t not in DEVICE_TYPES:
        raise ValueError(f"{name}: ggml type {name_of(t)} is not a quantized type the shared-expert kernels "
                         f"decode (Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, IQ4_NL)")
    data = np.asarray(tensor.data)
    if data.dtype != np.uint8:
        raise ValueError(f"{name}: expected the raw block bytes (uint8), got {data.dtype}")
    raw = np.ascontiguousarray(data).reshape(-1)
    want = tensor_bytes(t, *shape)
    if raw.size != want:
        raise ValueError(f"{name}: {raw.size} bytes, expected {want} for {name_of(t)} {shape}")
    return raw


class SharedExpert:
    def __init__(self, gguf_path, num_layers: int, hidden_size: int, intermediate_size: int,
                 dequant_fn=None, reader=None, *, device=None):
        import torch

        from .moe_gpu import MoeRunner

        self.hidden_size = int(hidden_size)
        self.intermediate_size = int(intermediate_size)
        self.backend = None
        self.runner = MoeRunner(device)
        dev = self.runner.device
        tmap = _reader_tensors(gguf_path, reader)
        self.layers: dict[int, SharedWeights] = {}
        self.missing: list[int] = []
        for layer in range(int(num_layers)):
            if not shared_expert_present(tmap, layer):
                self.missing.append(layer)
                continue
            ts = {r: tmap[f"blk.{layer}.{SHARED_ROLES[r]}"] for r in ("gate", "up", "down")}
            inter = int(ts["gate"].shape[1])   # ggml order: (hidden, intermediate)
            gi = tmap.get(f"blk.{layer}.{SHARED_ROLES['gate_inp']}")
            gate_inp = None
            if gi is not None:
                g16 = np.asarray(gi.data, dtype=np.float32).reshape(-1).astype(np.float16)
                gate_inp = torch.from_numpy(g16.astype(np.float32)).to(dev)
            mats = {r: _quantized_bytes(ts[r], f"blk.{layer}.{SHARED_ROLES[r]}",
                                        (inter, self.hidden_size) if r != "down" else (self.hidden_size, inter))
                    for r in ("gate", "up", "down")}
            self.layers[layer] = SharedWeights(
                *(_to_device_bytes(mats[r], dev) for r in ("gate", "up", "down")),
                types={r: int(ts[r].tensor_type) for r in ("gate", "up", "down")},
                intermediate=inter, gate_inp=gate_inp)
        if self.missing:
            raise KeyError(f"shared expert missing in layers {self.missing}: without its weights every "
                           f"token's output is wrong, not approximate")

    @classmethod
    def from_backend(cls, backend) -> "SharedExpert":
        """The shared experts a HipExpertBackend's resident layers already hold."""
        self = cls.__new__(cls)
        first = next(iter(backend.layers.values()), None)
        self.hidden_size = first.hidden if first is not None else 0
        self.intermediate_size = first.shared.intermediate if first is not None and first.shared else 0
        self.backend = backend
        self.runner = backend.runner
        self.layers = {l: L.shared for l, L in backend.layers.items() if L.shared is not None}
        self.missing = []
        return self

    def has(self, layer: int) -> bool:
        return layer in self.layers

    def _run(self, layer: int, x: np.ndarray) -> np.ndarray:
        import torch

        sh = self.layers[layer]
        x = np.ascontiguousarray(x, dtype=np.float32)
        (xd,) = self.runner.upload([x], slot="shared")
        xd = xd.view(torch.float32).view(x.shape)
        y = self.runner.decode_shared(sh, self.hidden_size, xd)
        out, rc = self.runner.fetch(y)
        if rc:
            from . import _lib

            raise RuntimeError(f"shared expert failed with status {rc} ({_lib.STATUS_TEXT.get(rc, 'unknown')})")
        return out

    def forward(self, layer: int, activation) -> np.ndarray | None:
        if not self.has(layer):
            return None
        x = np.asarray(activation, dtype=np.float32).reshape(-1)
        if x.size != self.hidden_size:
            raise ValueError(f"activation has {x.size} elements, expected {self.hidden_size}")
        return self._run(layer, x.reshape(1, -1)).reshape(-1)

    def forward_batch(self, layer: int, activations) -> np.ndarray | None:
        if not self.has(layer):
            return None
        x = np.ascontiguousarray(activations, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != self.hidden_size:
            raise ValueError(f"shared activations must have shape (tokens, {self.hidden_size})")
        return self._run(layer, x)
