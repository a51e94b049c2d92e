"""Drop-in for ``src/flash_moe/native_expert.py`` backed by the gfx950 library.

``NativeExpert`` keeps the reference class's constructor, ``function``
attribute (the ``moe_quant_expert`` export with the same argtypes),
``forward(tensors, kinds, activation, hidden, intermediate)`` contract and
error behaviour (``ValueError`` on a shape mismatch before the call,
``RuntimeError("native expert failed with status N")`` on a nonzero status;
native_expert.py:13-37).  The work runs on the GPU: the quantized bytes are
staged into HBM by the library and decoded there.

``NativeDelta`` (``NativeExpert.delta``) is the DeltaNet decode recurrence
with the reference class's ``forward(state, q, k, v, beta, gate)`` contract
(native_expert.py:76-97) over the library's ``moe_delta_heads``; ``DeltaState``
keeps a layer's recurrent state resident in HBM across decode steps
(``mqh_delta_heads``).

``load_native_expert(mode, library, device, tensor_types)`` keeps the
reference's auto/native/openvino contract (native_expert.py:40-75) with the
device check moved from AVX2/FMA/F16C CPU support to a gfx950 GPU.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import _lib
from .quant_types import SUPPORTED_TYPES

GPU_DEVICE_NAMES = ("GPU", "HIP", "CUDA", "gfx950")


class NativeExpert:
    """One token through one quantized SwiGLU expert on the GPU."""

    def __init__(self, path: Path | str | None = None, fp16_graph: int = 1):
        self.library = _lib.load(path)
        self.function = self.library.moe_quant_expert
        self.function.argtypes = [C.c_int, C.c_void_p, C.c_int64] * 3 + [
            C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int,
        ]
        self.function.restype = C.c_int
        # The reference always runs the FP16 graph (native_expert.py:33-34).
        self.fp16_graph = int(fp16_graph)
        # the DeltaNet recurrence export, found the way the reference probes it
        # (native_expert.py:21)
        self.delta = NativeDelta(self.library) if hasattr(self.library, "moe_delta_heads") else None

    def forward(self, tensors, kinds, activation, hidden, intermediate):
        arrays = [np.frombuffer(tensors[name], np.uint8) if isinstance(tensors[name], (bytes, bytearray))
                  else np.ascontiguousarray(tensors[name], dtype=np.uint8).reshape(-1)
                  for name in ("gate", "up", "down")]
        args = []
        for name, raw in zip(("gate", "up", "down"), arrays):
            args.extend((kinds[name], raw.ctypes.data, raw.nbytes))
        x = np.ascontiguousarray(activation, dtype=np.float32).reshape(-1)
        if x.size != hidden:
            raise ValueError("native expert activation shape mismatch")
        out = np.empty(hidden, np.float32)
        code = self.function(*args, x.ctypes.data, hidden, intermediate, out.ctypes.data, self.fp16_graph)
        if code:
            raise RuntimeError(f"native expert failed with status {code}")
        return out


class NativeDelta:
    """All-head FP32 state update (one DeltaNet decode step) on the GPU; host
    arrays in and out, the state updated in place."""

    def __init__(self, library):
        self.library = library
        self.function = library.moe_delta_heads
        self.function.argtypes = [C.c_void_p] * 7 + [C.c_int] * 3
        self.function.restype = C.c_int

    def forward(self, state, q, k, v, beta, gate):
        if state.dtype != np.float32 or not state.flags.c_contiguous:
            raise ValueError("DeltaNet state must be contiguous FP32")
        nv, dv, dk = state.shape
        arrays = [np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, beta, gate)]
        shapes = [(nv, dk), (nv, dk), (nv, dv), (nv,), (nv,)]
        if any(a.shape != shape for a, shape in zip(arrays, shapes)):
            raise ValueError("DeltaNet native input shape mismatch")
        out = np.empty((nv, dv), np.float32)
        code = self.function(state.ctypes.data, *[a.ctypes.data for a in arrays], out.ctypes.data, nv, dk, dv)
        if code:
            raise RuntimeError(f"native DeltaNet failed with status {code}")
        return out


class DeltaState:
    """One recurrent layer's state [heads, value_dim, key_dim] FP32 resident in
    HBM; ``step`` runs one decode step (mqh_delta_heads) on CUDA tensors and
    returns the [heads, value_dim] output, enqueued on the current stream."""

    def __init__(self, heads: int, value_dim: int, key_dim: int, device="cuda", state=None):
        import torch

        self.lib = _lib.load()
        self.shape = (int(heads), int(value_dim), int(key_dim))
        if state is None:
            self.state = torch.zeros(self.shape, dtype=torch.float32, device=device)
        else:
            self.state = torch.as_tensor(state, dtype=torch.float32).to(device).contiguous()
            if tuple(self.state.shape) != self.shape:
                raise ValueError("DeltaNet state shape mismatch")
        self._flags = torch.zeros(64, dtype=torch.int32, device=self.state.device)

    def reset(self):
        self.state.zero_()

    def step(self, q, k, v, beta, gate, out=None, stream=None):
        import torch

        nv, dv, dk = self.shape
        args = [q, k, v, beta, gate]
        shapes = [(nv, dk), (nv, dk), (nv, dv), (nv,), (nv,)]
        for a, shp in zip(args, shapes):
            if a.dtype != torch.float32 or not a.is_contiguous() or tuple(a.shape) != shp:
                raise ValueError(f"DeltaNet inputs must be contiguous FP32 of shapes {shapes}")
        if out is None:
            out = torch.empty((nv, dv), dtype=torch.float32, device=self.state.device)
        if stream is None:
            stream = torch.cuda.current_stream(self.state.device)
        rc = self.lib.mqh_delta_heads(self.state.data_ptr(), *[a.data_ptr() for a in args], out.data_ptr(),
                                      nv, dk, dv, self._flags.data_ptr(), stream.cuda_stream)
        _lib.check(rc, "mqh_delta_heads")
        return out

    def status(self, stream=None) -> int:
        """Synchronizes; -4 if an output was not finite since the last call."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.state.device)
        return int(self.lib.mqh_status(self._flags.data_ptr(), stream.cuda_stream))


def gpu_arch() -> str | None:
    """gcnArchName of device 0, or None when no HIP GPU is visible."""
    try:
        import torch
    except ImportError:
        return None
    if not torch.cuda.is_available():
        return None
    return str(getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")).split(":")[0]


def load_native_expert(mode, library, device, tensor_types):
    if mode not in ("auto", "native", "openvino"):
        raise ValueError("native_decode must be auto, native, or openvino")
    if mode == "openvino":
        return None
    reason = None
    arch = gpu_arch()
    if str(device) not in GPU_DEVICE_NAMES:
        reason = "native experts require --device GPU (a gfx950 HIP device)"
    elif arch is None:
        reason = "no HIP GPU is visible"
    elif arch != "gfx950":
        reason = f"the kernels are built for gfx950, found {arch}"
    elif not tensor_types or any(
        kinds.get(name) not in SUPPORTED_TYPES
        for kinds in tensor_types.values() for name in ("gate", "up", "down")
    ):
        reason = "expert quantization is unsupported"
    if reason is None:
        try:
            result = NativeExpert(library)
        except (OSError, AttributeError, _lib.NativeLibraryError) as error:
            reason = f"kernel unavailable ({error})"
        else:
            print("[Experts] native quantized decode on gfx950")
            return result
    if mode == "native":
        raise RuntimeError(reason)
    print(f"[Experts] OpenVINO decode: {reason}")
    return None
