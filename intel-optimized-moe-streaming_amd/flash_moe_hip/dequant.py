"""Dequantization entry points (drop-in for the reference's dequant helpers).

Host API, same names and meaning as the reference:
  * ``dequant_to_f16(raw, ggml_type, n_elements, out=None)``
    (``src/run_q4k_f16_openvino.py:62-85``) -- FP16 decode, optionally into a
    caller buffer; the reference falls back to gguf when its DLL fails, this
    one raises (there is no CPU fallback).
  * ``dequantize`` / ``dequantize_to`` (``src/flash_moe/dequant.py:86-180``).
  * ``GGML_BLOCK_INFO``, ``name_of``, ``is_aligned``, ``max_relative_error``
    (``src/flash_moe/dequant.py:30-50,74-83,198-202``).

``dequantize_iq4_nl(raw, rows, cols)`` is the reference's IQ4_NL library call
(``dequantize_iq4_nl_avx2``, ``run_native_int4_openvino.py:94-99``): its
16-entry table (``cpp/fast_dequant.cpp:4-9``), not gguf's.

Device API: ``dequant_device`` decodes a uint8 CUDA tensor already in HBM
(the five types above and IQ4_NL).
"""
from __future__ import annotations

import numpy as np

from . import _lib
from .quant_types import GGML_BLOCK_INFO, block_info, name_of

__all__ = ["GGML_BLOCK_INFO", "name_of", "is_aligned", "dequant_to_f16", "dequantize", "dequantize_to",
           "dequantize_iq4_nl", "dequant_device", "max_relative_error"]


def is_aligned(ggml_type: int, nbytes: int) -> bool:
    info = GGML_BLOCK_INFO.get(name_of(ggml_type))
    if info is None:
        return False
    return nbytes % info[1] == 0


def _as_bytes(raw) -> np.ndarray:
    if isinstance(raw, (bytes, bytearray, memoryview)):
        return np.frombuffer(raw, dtype=np.uint8)
    return np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)


def _host_dequant(raw, ggml_type: int, n_elements: int, out: np.ndarray, want_f16: int) -> np.ndarray:
    lib = _lib.load()
    if not lib.dequant_k_supported(int(ggml_type)):
        _lib.check(-1, f"dequant_k(type {ggml_type})")
    src = _as_bytes(raw)
    bs, pb = block_info(ggml_type)
    if n_elements % bs or src.nbytes < n_elements // bs * pb:
        raise ValueError(f"{src.nbytes} bytes cannot hold {n_elements} {name_of(ggml_type)} values")
    rc = lib.dequant_k(int(ggml_type), src.ctypes.data, out.ctypes.data, int(n_elements), want_f16)
    _lib.check(rc, "dequant_k")
    return out


def dequant_to_f16(raw, ggml_type: int, n_elements: int, out: np.ndarray | None = None) -> np.ndarray:
    """FP16 decode of ``n_elements`` values; ``out`` is reused when it is a
    writeable float16 array of the right size, else a new array is returned."""
    if out is not None and (out.dtype != np.float16 or out.size != n_elements or not out.flags.writeable
                            or not out.flags.c_contiguous):
        out = None
    if out is None:
        out = np.empty(n_elements, dtype=np.float16)
    return _host_dequant(raw, ggml_type, n_elements, out, 1)


def dequantize(raw, ggml_type: int, shape: tuple[int, ...] | None = None) -> np.ndarray:
    """FP32 decode of a whole buffer of blocks."""
    data = _as_bytes(raw)
    if data.size == 0:
        raise ValueError("empty buffer passed to dequantize")
    if not is_aligned(ggml_type, data.nbytes):
        raise ValueError(f"{data.nbytes} bytes is not a whole number of {name_of(ggml_type)} blocks")
    bs, pb = block_info(ggml_type)
    out = _host_dequant(data, ggml_type, data.nbytes // pb * bs, np.empty(data.nbytes // pb * bs, np.float32), 0)
    return out.reshape(*shape) if shape is not None else out


def dequantize_to(raw, ggml_type: int, dtype: str = "f16", shape: tuple[int, ...] | None = None) -> np.ndarray:
    if dtype == "f32":
        return dequantize(raw, ggml_type, shape)
    if dtype != "f16":
        raise ValueError(f"unsupported dtype {dtype!r}, expected f32 or f16")
    data = _as_bytes(raw)
    if data.size == 0:
        raise ValueError("empty buffer passed to dequantize_to")
    if not is_aligned(ggml_type, data.nbytes):
        raise ValueError(f"{data.nbytes} bytes is not a whole number of {name_of(ggml_type)} blocks")
    bs, pb = block_info(ggml_type)
    out = dequant_to_f16(data, ggml_type, data.nbytes // pb * bs)
    return out.reshape(*shape) if shape is not None else out


def dequantize_iq4_nl(raw, rows: int, cols: int) -> np.ndarray:
    """[rows x cols] FP32 from rows * (cols // 32) IQ4_NL blocks (18 bytes each)."""
    src = _as_bytes(raw)
    if rows <= 0 or cols <= 0 or cols % 32 or src.nbytes < rows * (cols // 32) * 18:
        raise ValueError(f"{src.nbytes} bytes cannot hold [{rows} x {cols}] IQ4_NL values")
    dst = np.empty((rows, cols), dtype=np.float32)
    _lib.load().dequantize_iq4_nl_avx2(src.ctypes.data, dst.ctypes.data, int(rows), int(cols))
    return dst


def dequant_device(src, ggml_type: int, n_elements: int | None = None, dtype=None, out=None, stream=None):
    """Decode a uint8 CUDA tensor of blocks into FP16 (default) or FP32 on the GPU."""
    import torch

    bs, pb = block_info(ggml_type)
    if src.dtype != torch.uint8 or not src.is_cuda or not src.is_contiguous():
        raise ValueError("src must be a contiguous uint8 CUDA tensor")
    if n_elements is None:
        n_elements = src.numel() // pb * bs
    if n_elements % bs or src.numel() < n_elements // bs * pb:
        raise ValueError(f"{src.numel()} bytes cannot hold {n_elements} {name_of(ggml_type)} values")
    dtype = dtype or torch.float16
    if dtype not in (torch.float16, torch.float32):
        raise ValueError("dtype must be torch.float16 or torch.float32")
    if out is None:
        out = torch.empty(n_elements, dtype=dtype, device=src.device)
    elif out.dtype != dtype or out.numel() != n_elements or not out.is_contiguous():
        raise ValueError("out has the wrong dtype, size or layout")
    if stream is None:
        stream = torch.cuda.current_stream(src.device)
    rc = _lib.load().mqh_dequant(int(ggml_type), src.data_ptr(), out.data_ptr(), int(n_elements),
                                 1 if dtype == torch.float16 else 0, stream.cuda_stream)
    _lib.check(rc, "mqh_dequant")
    return out


def max_relative_error(actual: np.ndarray, reference: np.ndarray) -> float:
    scale = float(np.abs(reference).max())
    if scale == 0.0:
        return float(np.abs(actual).max())
    return float(np.abs(np.asarray(actual).astype(np.float64) - reference).max() / scale)
