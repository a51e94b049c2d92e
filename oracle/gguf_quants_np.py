"""Vectorised NumPy restatement of the ``gguf.quants`` block dequantizers.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference's dequantizers (``cpp/dequant_k.cpp``) were validated by their
author against the Python package ``gguf`` (``gguf>=0.6.0``, unpinned in
``requirements.txt:5``; a text copy of its ``quants.py`` is vendored at
``tools/_kquant_ref.txt``, truncated inside Q5_K).  ``gguf`` is not installed
here, so this module restates its published array formulation -- split the
block into fields, broadcast shifts over the packed bytes, reshape into
sub-blocks -- for Q8_0, Q3_K, Q4_K, Q5_K and Q6_K.  It shares no code and no
index tables with the C oracle, which computes each output's bit position in
closed form; the tests require the two to agree bit for bit.

Field layouts (bytes):
  Q8_0  34: d f16 | qs int8[32]                       (_kquant_ref.txt:378-402)
  Q3_K 110: hmask[32] | qs[64] | scales[12] | d f16    (_kquant_ref.txt:431-473)
  Q4_K 144: d f16 | dmin f16 | scales[12] | qs[128]    (_kquant_ref.txt:475-523)
  Q5_K 176: d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
  Q6_K 210: ql[128] | qh[64] | scales int8[16] | d f16
"""
from __future__ import annotations

import numpy as np

QK_K = 256


def _f16(col: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(col).view(np.float16).astype(np.float32)


def _shifts(*vals: int) -> np.ndarray:
    return np.array(vals, dtype=np.uint8)


def q8_0(blocks: np.ndarray) -> np.ndarray:
    d = _f16(blocks[:, :2])                                   # (n, 1)
    q = np.ascontiguousarray(blocks[:, 2:]).view(np.int8).astype(np.float32)
    return q * d


def scale_min_k4(scales: np.ndarray):
    """Eight 6-bit scales and eight 6-bit mins from the 12 packed bytes:
    rows a=bytes 0-3, b=bytes 4-7, c=bytes 8-11 (each 4 wide).
    sc[0:4] = a & 63; sc[4:8] = (c & 15) | ((a >> 6) << 4)
    mn[0:4] = b & 63; mn[4:8] = (c >> 4) | ((b >> 6) << 4)"""
    a, b, c = scales[:, 0:4], scales[:, 4:8], scales[:, 8:12]
    sc = np.concatenate([a & 63, (c & 15) | ((a >> 6) << 4)], axis=1)
    mn = np.concatenate([b & 63, (c >> 4) | ((b >> 6) << 4)], axis=1)
    return sc.astype(np.float32), mn.astype(np.float32)


def q4_k(blocks: np.ndarray) -> np.ndarray:
    n = blocks.shape[0]
    d, dmin = _f16(blocks[:, 0:2]), _f16(blocks[:, 2:4])
    sc, mn = scale_min_k4(blocks[:, 4:16])
    qs = blocks[:, 16:144].reshape(n, 4, 1, 32)               # 4 groups of 32 bytes
    q = ((qs >> _shifts(0, 4).reshape(1, 1, 2, 1)) & 15).reshape(n, 8, 32).astype(np.float32)
    scale = (d * sc).reshape(n, 8, 1)
    offset = (dmin * mn).reshape(n, 8, 1)
    return (scale * q - offset).reshape(n, QK_K)


def q5_k(blocks: np.ndarray) -> np.ndarray:
    n = blocks.shape[0]
    d, dmin = _f16(blocks[:, 0:2]), _f16(blocks[:, 2:4])
    sc, mn = scale_min_k4(blocks[:, 4:16])
    qh = blocks[:, 16:48].reshape(n, 1, 32)                   # bit s of qh[l] -> sub-block s
    qs = blocks[:, 48:176].reshape(n, 4, 1, 32)
    lo = ((qs >> _shifts(0, 4).reshape(1, 1, 2, 1)) & 15).reshape(n, 8, 32)
    hi = ((qh >> np.arange(8, dtype=np.uint8).reshape(1, 8, 1)) & 1).reshape(n, 8, 32)
    q = (lo | (hi << 4)).astype(np.float32)
    scale = (d * sc).reshape(n, 8, 1)
    offset = (dmin * mn).reshape(n, 8, 1)
    return (scale * q - offset).reshape(n, QK_K)


def q6_k(blocks: np.ndarray) -> np.ndarray:
    n = blocks.shape[0]
    ql = blocks[:, 0:128].reshape(n, 2, 1, 64)                # per 128-output half: 64 bytes
    qh = blocks[:, 128:192].reshape(n, 2, 1, 32)              # per half: 32 bytes
    sc = np.ascontiguousarray(blocks[:, 192:208]).view(np.int8).astype(np.float32)
    d = _f16(blocks[:, 208:210])
    lo = ((ql >> _shifts(0, 4).reshape(1, 1, 2, 1)) & 15).reshape(n, 8, 32)
    hi = ((qh >> _shifts(0, 2, 4, 6).reshape(1, 1, 4, 1)) & 3).reshape(n, 8, 32)
    q = ((lo | (hi << 4)).astype(np.int16) - 32).reshape(n, 16, 16).astype(np.float32)
    scale = (d * sc).reshape(n, 16, 1)
    return (scale * q).reshape(n, QK_K)


def q3_k(blocks: np.ndarray) -> np.ndarray:
    n = blocks.shape[0]
    hmask = blocks[:, 0:32].reshape(n, 1, 32)
    qs = blocks[:, 32:96].reshape(n, 2, 1, 32)
    packed = blocks[:, 96:108]
    d = _f16(blocks[:, 108:110])
    # 16 six-bit scales: low nibbles from bytes 0-7 (low nibble first, then the
    # high nibbles), two high bits from bytes 8-11 at shifts 0,2,4,6.
    low = (packed[:, 0:8].reshape(n, 1, 8) >> _shifts(0, 4).reshape(1, 2, 1)).reshape(n, 16) & 15
    high = (packed[:, 8:12].reshape(n, 1, 4) >> _shifts(0, 2, 4, 6).reshape(1, 4, 1)).reshape(n, 16) & 3
    sc = ((low | (high << 4)).astype(np.int16) - 32).astype(np.float32)
    lo2 = ((qs >> _shifts(0, 2, 4, 6).reshape(1, 1, 4, 1)) & 3).reshape(n, 16, 16)
    bit = ((hmask >> np.arange(8, dtype=np.uint8).reshape(1, 8, 1)) & 1).reshape(n, 16, 16)
    q = (lo2.astype(np.int16) - ((bit ^ 1).astype(np.int16) << 2)).astype(np.float32)
    scale = (d * sc).reshape(n, 16, 1)
    return (scale * q).reshape(n, QK_K)


DEQUANT = {8: (32, 34, q8_0), 11: (256, 110, q3_k), 12: (256, 144, q4_k),
           13: (256, 176, q5_k), 14: (256, 210, q6_k)}


def dequantize(raw, ggml_type: int) -> np.ndarray:
    bs, pb, fn = DEQUANT[int(ggml_type)]
    data = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    if data.size % pb:
        raise ValueError(f"{data.size} bytes is not a whole number of {pb}-byte blocks")
    with np.errstate(all="ignore"):
        return fn(data.reshape(-1, pb)).reshape(-1).astype(np.float32)
