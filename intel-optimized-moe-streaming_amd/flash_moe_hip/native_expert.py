"""Drop-in for ``src/flash_moe/native_expert.py`` backed by the gfx950 library.

``NativeExpert`` keeps the reference class's constructor, ``function``
attribute (the ``moe_quant_expert`` export with the same argtypes),
``forward(tensors, kinds, activation, hidden, intermediate)`` contract and
error behaviour (``ValueError`` on a shape mismatch before the call,
``RuntimeError("native expert failed with status N")`` on a nonzero status;
native_expert.py:13-37).  The work runs on the GPU: the quantized bytes are
staged into HBM by the library and decoded there.

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
        # moe_delta_heads (DeltaNet recurrence) is not part of this library.
        self.delta = None

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
