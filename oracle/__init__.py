"""CPU oracle for the quantized-expert hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this package, and only to check results against (or,
for the baseline, as the thing timed on the host).  The HIP product path never imports
it and never falls back to it.

Contents
--------
* ``liboracle_kquant.so`` (built from ``kquant_oracle.c``, ``kquant_avx2.c`` and
  ``delta_oracle.c`` by ``Makefile``): a C restatement of the reference kernels
  ``cpp/dequant_k.cpp``, ``cpp/moe_quant_dot.cpp`` and ``cpp/moe_delta.cpp``.
  Wrapped here as :func:`dequant_k`, :func:`moe_quant_expert` and
  :func:`delta_heads` with the reference's argument meaning and status codes.
* ``_ref/libref_delta.so`` (``make ref``, only where the reference tree is
  present; never committed): the reference's own ``cpp/moe_delta.cpp`` compiled
  from its source, the second check of :func:`delta_heads` and the CPU baseline
  of the DeltaNet bench line (:func:`reference_delta_lib`).
* NumPy restatements of the Python semantics around the kernels:
  :func:`route` (``src/flash_moe/router.py:140-170``), :func:`combine`
  (``src/flash_moe/moe_layer.py:70-106``), :func:`shared_expert_forward`
  (``src/flash_moe/shared_expert.py:221-251``) and :func:`max_relative_error`
  (``src/flash_moe/dequant.py:198-202``).
* ``gguf_quants_np``: an independent vectorised restatement of the published
  ``gguf.quants`` dequantizers, used by the tests to pin the C restatement.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_kquant.so"
REF_DELTA_PATH = HERE / "_ref" / "libref_delta.so"
REFERENCE_TREE = Path("/root/reference")

BLOCK = {8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 20: (32, 18)}
IQ4_NL = 20

_lib = None


def build() -> Path:
    """Compile the C restatement (make -C oracle) and, where the reference tree
    is present, the reference's DeltaNet kernel into _ref/ (make ref)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if (REFERENCE_TREE / "cpp" / "moe_delta.cpp").is_file():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REFERENCE={REFERENCE_TREE}"], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is not built; run `make -C oracle`")
        L = C.CDLL(str(LIB_PATH))
        L.oracle_dequant_k.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int]
        L.oracle_dequant_k.restype = C.c_int
        L.oracle_dequant_k_supported.argtypes = [C.c_int]
        L.oracle_dequant_k_block_size.argtypes = [C.c_int]
        L.oracle_moe_quant_expert.argtypes = [C.c_int, C.c_void_p, C.c_int64] * 3 + [
            C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int]
        L.oracle_moe_quant_expert.restype = C.c_int
        L.oracle_moe_quant_expert_avx2.argtypes = L.oracle_moe_quant_expert.argtypes
        L.oracle_moe_quant_expert_avx2.restype = C.c_int
        L.oracle_f32_to_f16.argtypes = [C.c_float]
        L.oracle_f32_to_f16.restype = C.c_uint16
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_f16_to_f32.restype = C.c_float
        L.oracle_dequantize_iq4_nl.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.oracle_dequantize_iq4_nl.restype = None
        L.oracle_delta_heads.argtypes = [C.c_void_p] * 7 + [C.c_int] * 3
        L.oracle_delta_heads.restype = C.c_int
        L.oracle_f32_to_f16_array.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.oracle_f16_to_f32_array.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        _lib = L
    return _lib


def f32_to_f16_bits(values) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(v.size, np.uint16)
    lib().oracle_f32_to_f16_array(v.ctypes.data, out.ctypes.data, v.size)
    return out


def f16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    out = np.empty(b.size, np.float32)
    lib().oracle_f16_to_f32_array(b.ctypes.data, out.ctypes.data, b.size)
    return out


def dequant_k(ggml_type: int, raw, n: int, want_f16: bool = False):
    """(status, values) exactly as ``dequant_k`` (dequant_k.cpp:350-394)."""
    src = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8) if isinstance(raw, (bytes, bytearray))
                               else raw, dtype=np.uint8)
    out = np.zeros(max(int(n), 0), np.float16 if want_f16 else np.float32)
    rc = lib().oracle_dequant_k(int(ggml_type), src.ctypes.data, out.ctypes.data, int(n), int(bool(want_f16)))
    return rc, out


def dequantize_iq4_nl(raw, rows: int, cols: int) -> np.ndarray:
    """``dequantize_iq4_nl_cpp`` (cpp/fast_dequant.cpp:40-65): [rows x cols] FP32."""
    src = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    if src.size < rows * (cols // 32) * 18:
        raise ValueError("not enough IQ4_NL blocks")
    out = np.zeros((rows, cols), np.float32)
    lib().oracle_dequantize_iq4_nl(src.ctypes.data, out.ctypes.data, int(rows), int(cols))
    return out


def dequant(ggml_type: int, raw, n: int | None = None, want_f16: bool = False) -> np.ndarray:
    """Values of a flat run of blocks, FP32 or RN_f16 (IQ4_NL through the
    reference's IQ4_NL library semantics, the rest through dequant_k)."""
    src = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    bs, pb = BLOCK[int(ggml_type)]
    if n is None:
        n = src.size // pb * bs
    if int(ggml_type) == IQ4_NL:
        vals = dequantize_iq4_nl(src, n // 32, 32).reshape(-1)
        return f32_to_f16_bits(vals).view(np.float16) if want_f16 else vals
    rc, out = dequant_k(ggml_type, src, n, want_f16)
    if rc != 0:
        raise RuntimeError(f"oracle dequant_k failed with status {rc}")
    return out


def moe_quant_expert(tensors: dict, kinds: dict, x, hidden: int, intermediate: int,
                     fp16_graph: int = 0, avx2: bool = False, out=None):
    """(status, y) with the argument meaning of ``moe_quant_expert``
    (moe_quant_dot.cpp:171-214).  ``tensors`` maps gate/up/down to raw bytes.
    ``avx2`` runs the AVX2 row dot of ``kquant_avx2.c`` (the reference's
    direct Q3_K/Q6_K form, moe_quant_dot.cpp:23-169): the same result bit for
    bit, the CPU baseline of the bench.  ``out`` (FP32 [hidden], written in
    place) keeps the rows a -4 return leaves untouched; by default a zeroed
    array."""
    arrays = [np.ascontiguousarray(np.frombuffer(bytes(tensors[k]), np.uint8) if
                                   isinstance(tensors[k], (bytes, bytearray)) else tensors[k],
                                   dtype=np.uint8).reshape(-1) for k in ("gate", "up", "down")]
    args = []
    for name, raw in zip(("gate", "up", "down"), arrays):
        args.extend((int(kinds[name]), raw.ctypes.data, raw.nbytes))
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if out is None:
        out = np.zeros(hidden, np.float32)
    if out.dtype != np.float32 or out.size != hidden or not out.flags.c_contiguous:
        raise ValueError("out must be a contiguous FP32 array of hidden values")
    fn = lib().oracle_moe_quant_expert_avx2 if avx2 else lib().oracle_moe_quant_expert
    rc = fn(*args, xv.ctypes.data, int(hidden), int(intermediate), out.ctypes.data, int(fp16_graph))
    return rc, out


def expert_forward(tensors, kinds, x, hidden, intermediate, fp16_graph=0, avx2=False) -> np.ndarray:
    rc, y = moe_quant_expert(tensors, kinds, x, hidden, intermediate, fp16_graph, avx2)
    if rc != 0:
        raise RuntimeError(f"oracle expert failed with status {rc}")
    return y


# ------------------------------------------------------------ Python semantics

def _delta_call(fn, state: np.ndarray, q, k, v, beta, gate, out=None):
    if state.dtype != np.float32 or not state.flags.c_contiguous or state.ndim != 3:
        raise ValueError("state must be a contiguous FP32 [heads, value_dim, key_dim] array")
    nv, dv, dk = state.shape
    arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, beta, gate)]
    shapes = [(nv, dk), (nv, dk), (nv, dv), (nv,), (nv,)]
    if any(a.shape != s_ for a, s_ in zip(arrs, shapes)):
        raise ValueError("DeltaNet input shape mismatch")
    if out is None:
        out = np.zeros((nv, dv), np.float32)
    if out.dtype != np.float32 or out.shape != (nv, dv) or not out.flags.c_contiguous:
        raise ValueError("out must be a contiguous FP32 [heads, value_dim] array")
    rc = fn(state.ctypes.data, *[a.ctypes.data for a in arrs], out.ctypes.data, nv, dk, dv)
    return rc, out


def delta_heads(state: np.ndarray, q, k, v, beta, gate, out=None):
    """``moe_delta_heads`` (cpp/moe_delta.cpp:18-69): one delta-rule step of every
    head, ``state`` [heads, value_dim, key_dim] FP32 updated in place.  Returns
    (status, output [heads, value_dim]); ``out``, when given, is written in
    place (the rows a -2 return leaves untouched keep their values)."""
    return _delta_call(lib().oracle_delta_heads, state, q, k, v, beta, gate, out)


def reference_delta_lib():
    """The reference's moe_delta_heads built from its source (oracle/_ref), or None."""
    if not REF_DELTA_PATH.exists():
        return None
    L = C.CDLL(str(REF_DELTA_PATH))
    L.moe_delta_heads.argtypes = [C.c_void_p] * 7 + [C.c_int] * 3
    L.moe_delta_heads.restype = C.c_int
    return L


def reference_delta_heads(state: np.ndarray, q, k, v, beta, gate, out=None):
    """Like :func:`delta_heads`, through the reference's own compiled kernel."""
    L = reference_delta_lib()
    if L is None:
        raise FileNotFoundError(f"{REF_DELTA_PATH} is not built (make -C oracle ref)")
    return _delta_call(L.moe_delta_heads, state, q, k, v, beta, gate, out)


def delta_step_numpy(S: np.ndarray, q, k, v, beta: float, gate: float) -> np.ndarray:
    """The closed form of one head's step (gated_deltanet.py:264-298, arXiv
    2412.06464 eq. 10) in float64: S <- exp(gate) S; S <- S + beta (v - S k) k^T;
    out = S q.  Updates S (float64) in place and returns out."""
    S *= np.exp(gate)
    S += np.outer(beta * (v - S @ k), k)
    return S @ q


def route(x, router_w: np.ndarray, top_k: int):
    """``ExpertRouter.route`` (router.py:140-170): FP32 scores ``x @ W`` with W
    shaped (hidden, experts); top-k by descending argsort; float64 softmax over
    the selected k; uniform weights if the softmax is not finite."""
    xv = np.asarray(x, dtype=np.float32).reshape(-1)
    scores = (xv @ np.asarray(router_w, dtype=np.float32)).astype(np.float32)
    idx = np.argsort(scores)[-top_k:][::-1].astype(np.int64).tolist()
    sel = scores[idx].astype(np.float64)
    e = np.exp(sel - np.max(sel))
    total = e.sum()
    if not np.isfinite(total) or total <= 0.0:
        w = np.full(len(idx), 1.0 / len(idx))
    else:
        w = e / total
    return idx, [float(v) for v in w]


def combine(expert_outputs, weights, shared_out=None) -> np.ndarray:
    """Weighted sum of ``run_moe_layer`` (moe_layer.py:70-106): FP32 accumulator,
    ``combined += w_k * y_k`` in top-k order with the Python-float weight cast to
    FP32 (NumPy 2 scalar promotion), then ``+ shared``."""
    width = np.asarray(expert_outputs[0] if len(expert_outputs) else shared_out).shape[-1]
    combined = np.zeros(width, dtype=np.float32)
    for y, w in zip(expert_outputs, weights):
        # route() hands out Python floats (router.py:170): a weak scalar, so the
        # product is taken in FP32
        combined += float(w) * np.asarray(y, dtype=np.float32)
    if shared_out is not None:
        combined = combined + shared_out
    return combined


def _sigmoid(x: np.ndarray) -> np.ndarray:
    """Stable sigmoid of shared_expert.py:55-62."""
    x = np.asarray(x)
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-x[pos]))
    e = np.exp(x[~pos])
    out[~pos] = e / (1.0 + e)
    return out


def shared_expert_forward(x, w_gate, w_up, w_down, gate_inp=None) -> np.ndarray:
    """``SharedExpert.forward`` (shared_expert.py:221-251) on weights that were
    FP16-dequantized and promoted to FP32 (shared_expert.py:141-149):
    ``sigmoid(x . g_inp) * (W_d (silu(W_g x) * (W_u x)))``.  With ``gate_inp``
    None the sigmoid scale is omitted."""
    xv = np.asarray(x, dtype=np.float32).reshape(-1)
    g = xv @ np.asarray(w_gate, dtype=np.float32).T
    act = (g * _sigmoid(g)) * (xv @ np.asarray(w_up, dtype=np.float32).T)
    out = act @ np.asarray(w_down, dtype=np.float32).T
    if gate_inp is None:
        return out.astype(np.float32)
    gate = _sigmoid((xv @ np.asarray(gate_inp, dtype=np.float32)).reshape(()))
    return (gate * out).astype(np.float32)


def max_relative_error(actual: np.ndarray, reference: np.ndarray) -> float:
    """The reference's parity metric (dequant.py:198-202): max|a-r| / max|r|."""
    reference = np.asarray(reference)
    scale = float(np.abs(reference).max())
    if scale == 0.0:
        return float(np.abs(actual).max())
    return float(np.abs(np.asarray(actual).astype(np.float64) - reference).max() / scale)
