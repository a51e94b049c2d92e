"""GGUF files: metadata, tensor table, zero-copy tensor bytes, and MoE layers straight into HBM.

The reference opens the model through the ``gguf`` package and slices each
layer's stacked expert tensors by offset (``src/run_q4k_f16_openvino.py:88-133``:
expert e of ``blk.{L}.ffn_{gate,up,down}_exps.weight`` is the byte range
``data_offset + e * (n_bytes // 256)``), reading the per-layer ggml types from
the same tensors (``src/run_q4k_f16_openvino.py:136-155``,
``src/flash_moe/model.py:372-383``).  This module reads the file format itself
(no third-party reader), maps the file, and hands the stacked tensors to
``ExpertLayer`` unchanged, so expert e's bytes in HBM are exactly the GGUF
slice the reference reads.

File layout (GGUF versions 2 and 3, little-endian):
  magic b"GGUF", u32 version, u64 tensor count, u64 metadata count;
  metadata entries: key (string), u32 value type, value;
  tensor infos: name (string), u32 n_dims, u64 dims[n_dims] (dims[0] is the
  innermost: the row length), u32 ggml type, u64 offset from the data section;
  the data section starts at the next multiple of ``general.alignment``
  (default 32) after the tensor infos.
A string is a u64 byte count and UTF-8 bytes; an array is a u32 element type,
a u64 count and the elements.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass

import numpy as np

from .quant_types import GGML_BLOCK_INFO

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types
T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, T_UINT64, T_INT64, \
    T_FLOAT64 = range(13)
_SCALAR = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I", T_INT32: "<i",
           T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q", T_FLOAT64: "<d"}

# ggml tensor type ids (ggml.h) -> names in GGML_BLOCK_INFO
GGML_TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 10: "Q2_K",
                   11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 16: "IQ2_XXS", 18: "IQ3_XXS",
                   19: "IQ1_S", 20: "IQ4_NL", 23: "IQ4_XS", 30: "BF16"}


class GGUFError(ValueError):
    pass


@dataclass(frozen=True)
class GGUFTensor:
    name: str
    dims: tuple          # ggml order: dims[0] is the row length
    ggml_type: int
    offset: int          # absolute byte offset in the file
    n_bytes: int | None  # None for a type whose block geometry is not known here

    @property
    def shape(self) -> tuple:
        """NumPy (row-major) shape: the dims reversed."""
        return tuple(reversed(self.dims))

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n


@dataclass(frozen=True)
class ReaderTensor:
    """A tensor as the ``gguf`` package's reader presents it, the form the
    reference's callers take (``router.py:93-140`` reads ``shape`` and
    ``data``; ``shared_expert.py:65-94`` also ``data_offset``, ``n_bytes`` and
    ``tensor_type``): ``shape`` in ggml order (row length first), ``data`` a
    zero-copy NumPy view in row-major order -- typed for F32/F16, the raw
    bytes ``[rows, row_bytes]`` for quantized types."""
    name: str
    shape: tuple
    tensor_type: int
    data_offset: int
    n_bytes: int
    data: np.ndarray


def tensor_nbytes(ggml_type: int, dims) -> int | None:
    name = GGML_TYPE_NAMES.get(int(ggml_type))
    if name is None:
        return None
    bs, pb = GGML_BLOCK_INFO[name]
    if int(dims[0]) % bs:
        raise GGUFError(f"row length {dims[0]} is not a multiple of the {name} block ({bs})")
    n = 1
    for d in dims:
        n *= int(d)
    return n // bs * pb


class _Cursor:
    def __init__(self, buf: memoryview, pos: int = 0):
        self.buf, self.pos = buf, pos

    def take(self, n: int) -> memoryview:
        if self.pos + n > len(self.buf):
            raise GGUFError("truncated file")
        v = self.buf[self.pos:self.pos + n]
        self.pos += n
        return v

    def scalar(self, vtype: int):
        fmt = _SCALAR[vtype]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(T_UINT64)
        return bytes(self.take(n)).decode("utf-8")

    def value(self, vtype: int):
        if vtype in _SCALAR:
            return self.scalar(vtype)
        if vtype == T_STRING:
            return self.string()
        if vtype == T_ARRAY:
            etype = self.scalar(T_UINT32)
            count = self.scalar(T_UINT64)
            if etype in _SCALAR:   # one bulk read for numeric arrays
                fmt = _SCALAR[etype]
                size = struct.calcsize(fmt)
                return np.frombuffer(bytes(self.take(size * count)), dtype=np.dtype(fmt)).tolist()
            return [self.value(etype) for _ in range(count)]
        raise GGUFError(f"unknown metadata value type {vtype}")


class GGUFFile:
    """A GGUF file mapped read-only.  ``metadata`` maps keys to Python values,
    ``tensors`` names to ``GGUFTensor``; ``raw(name)`` is a zero-copy uint8
    view of a tensor's bytes."""

    def __init__(self, path: str | os.PathLike):
        self.path = os.fspath(path)
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        cur = _Cursor(memoryview(self._map))
        if bytes(cur.take(4)) != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: not a GGUF file")
        self.version = cur.scalar(T_UINT32)
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path}: GGUF version {self.version} is not supported (2 or 3)")
        n_tensors = cur.scalar(T_UINT64)
        n_kv = cur.scalar(T_UINT64)
        self.metadata: dict = {}
        for _ in range(n_kv):
            key = cur.string()
            self.metadata[key] = cur.value(cur.scalar(T_UINT32))
        infos = []
        for _ in range(n_tensors):
            name = cur.string()
            n_dims = cur.scalar(T_UINT32)
            dims = tuple(cur.scalar(T_UINT64) for _ in range(n_dims))
            ggml_type = cur.scalar(T_UINT32)
            rel = cur.scalar(T_UINT64)
            infos.append((name, dims, ggml_type, rel))
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GGUFError(f"general.alignment {self.alignment} is not a power of two")
        self.data_offset = (cur.pos + self.alignment - 1) // self.alignment * self.alignment
        self.tensors: dict[str, GGUFTensor] = {}
        for name, dims, ggml_type, rel in infos:
            if rel % self.alignment:
                raise GGUFError(f"{name}: offset {rel} is not aligned to {self.alignment}")
            nb = tensor_nbytes(ggml_type, dims)
            t = GGUFTensor(name, dims, int(ggml_type), self.data_offset + int(rel), nb)
            if nb is not None and t.offset + nb > len(self._map):
                raise GGUFError(f"{name}: data runs past the end of the file")
            self.tensors[name] = t

    def raw(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        if t.n_bytes is None:
            raise GGUFError(f"{name}: ggml type {t.ggml_type} has no known block size")
        return self._map[t.offset:t.offset + t.n_bytes]

    def float_array(self, name: str) -> np.ndarray:
        """An F32, F16 or BF16 tensor as FP32, in NumPy shape."""
        t = self.tensors[name]
        raw = self.raw(name)
        if t.ggml_type == 0:
            a = raw.view(np.float32)
        elif t.ggml_type == 1:
            a = raw.view(np.float16).astype(np.float32)
        elif t.ggml_type == 30:
            a = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        else:
            raise GGUFError(f"{name}: ggml type {t.ggml_type} is not a float type")
        return np.asarray(a).reshape(t.shape)

    def reader_tensor(self, name: str) -> ReaderTensor:
        t = self.tensors[name]
        raw = self.raw(name)
        if t.ggml_type in (0, 1):
            data = raw.view(np.float32 if t.ggml_type == 0 else np.float16).reshape(t.shape)
        else:
            rows = t.n_elements // int(t.dims[0])
            data = raw.reshape(rows, -1)
        return ReaderTensor(name, tuple(int(d) for d in t.dims), t.ggml_type, t.offset, int(t.n_bytes), data)

    def tensor_map(self) -> dict:
        """{name: ReaderTensor} for every tensor of a known type: the ``tmap``
        the reference's routers_from_gguf and SharedExpert read."""
        return {n: self.reader_tensor(n) for n, t in self.tensors.items() if t.n_bytes is not None}

    def expert_layers(self) -> dict[int, dict[str, int]]:
        """{layer: {role: ggml type}} of every layer with stacked expert
        tensors (the reference's expert_tensor_types)."""
        out: dict[int, dict[str, int]] = {}
        for name, t in self.tensors.items():
            parts = name.split(".")
            if len(parts) == 4 and parts[0] == "blk" and parts[3] == "weight" and parts[2].endswith("_exps"):
                role = parts[2][len("ffn_"):-len("_exps")]
                if role in ("gate", "up", "down"):
                    out.setdefault(int(parts[1]), {})[role] = t.ggml_type
        return dict(sorted(out.items()))


def layer_host_tensors(gf: GGUFFile, layer: int, gate_dtype=np.float16) -> dict:
    """The host-side pieces of one MoE layer: stacked expert bytes (zero-copy
    views), types and shape, the shared expert and the router weights when the
    file has them.  Raises if the three stacks disagree in shape.

    The two gate vectors carry the reference's storage rounding, so the device
    routes and gates exactly as the reference's host code does:
    ``ffn_gate_inp`` is rounded to ``gate_dtype`` (FP16, the default of
    ``routers_from_gguf``) and promoted to FP32 (src/flash_moe/router.py:51-59,
    99, 136; built with that default by model.py:219-222), and
    ``ffn_gate_inp_shexp`` is rounded to FP16 and promoted, as
    ``SharedExpert._load`` stores every F32/F16 tensor (shared_expert.py:147,
    173).  In FP16 storage a close pair of experts can swap
    (router.py:101-104), so the rounding is part of the routing result."""
    name = f"blk.{layer}.ffn_{{}}_exps.weight"
    ts = {r: gf.tensors[name.format(r)] for r in ("gate", "up", "down")}
    g, u, d = ts["gate"], ts["up"], ts["down"]
    if len(g.dims) != 3 or g.dims != u.dims or d.dims != (g.dims[1], g.dims[0], g.dims[2]):
        raise GGUFError(f"layer {layer}: expert stacks {g.dims} / {u.dims} / {d.dims} do not form a SwiGLU FFN")
    hidden, inter, n_experts = (int(v) for v in g.dims)
    out = {"tensors": {r: gf.raw(t.name) for r, t in ts.items()},
           "types": {r: t.ggml_type for r, t in ts.items()},
           "n_experts": n_experts, "hidden": hidden, "intermediate": inter,
           "shared": None, "router_weights": None}
    sh = f"blk.{layer}.ffn_{{}}_shexp.weight"
    if all(sh.format(r) in gf.tensors for r in ("gate", "up", "down")):
        st = {r: gf.tensors[sh.format(r)] for r in ("gate", "up", "down")}
        sh_inter = int(st["gate"].dims[1])
        gi_name = f"blk.{layer}.ffn_gate_inp_shexp.weight"
        gate_inp = None
        if gi_name in gf.tensors:
            gate_inp = gf.float_array(gi_name).reshape(-1).astype(np.float16).astype(np.float32)
        out["shared"] = {"gate": gf.raw(st["gate"].name), "up": gf.raw(st["up"].name),
                         "down": gf.raw(st["down"].name),
                         "types": {r: t.ggml_type for r, t in st.items()},
                         "intermediate": sh_inter, "gate_inp": gate_inp}
    router = f"blk.{layer}.ffn_gate_inp.weight"
    if router in gf.tensors:
        w = gf.float_array(router)            # NumPy shape (n_experts, hidden)
        w = w.astype(np.dtype(gate_dtype)).astype(np.float32)
        out["router_weights"] = np.ascontiguousarray(w.T)   # [hidden x n_experts]
    return out


def load_expert_layer(gf: GGUFFile, layer: int, device="cuda", gate_dtype=np.float16):
    """One MoE layer of the file resident in HBM (``ExpertLayer``), its router
    weights stored as ``gate_dtype`` (the ``ExpertRouter`` default: FP16)."""
    from .layer_store import ExpertLayer

    h = layer_host_tensors(gf, layer, gate_dtype=gate_dtype)
    return ExpertLayer.from_host(h["tensors"], h["types"], h["n_experts"], h["hidden"], h["intermediate"],
                                 shared=h["shared"], router_weights=h["router_weights"], device=device)
