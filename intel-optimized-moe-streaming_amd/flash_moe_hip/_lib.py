"""ctypes binding of libmoe_quant_hip.so (C ABI: include/moe_quant_hip.h).

There is no fallback: if the library is missing or cannot be loaded, every
entry point raises.  Build it with ``intel-optimized-moe-streaming_amd/build_hip.py``
(``__graft_entry__.build()`` does).
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

LIB_NAME = "libmoe_quant_hip.so"
DEFAULT_PATH = Path(__file__).resolve().parent / LIB_NAME

# Every symbol include/moe_quant_hip.h declares.
EXPORTS = (
    "dequant_k_supported",
    "dequant_k_block_size",
    "dequant_k",
    "moe_quant_expert",
    "moe_delta_heads",
    "mqh_delta_heads",
    "dequantize_iq4_nl_cpp",
    "dequantize_iq4_nl_avx2",
    "mqh_dequant",
    "mqh_moe_workspace_bytes",
    "mqh_moe_decode",
    "mqh_moe_decode_noalloc",
    "mqh_moe_decode_routed",
    "mqh_last_route_kernels",
    "mqh_moe_prefill_workspace_bytes",
    "mqh_moe_prefill",
    "mqh_set_decode_path",
    "mqh_last_decode_kernels",
    "mqh_last_decode_path",
    "mqh_read_floor",
    "mqh_route",
    "mqh_profile_next_decode",
    "mqh_workspace_init",
    "mqh_status",
)

STATUS_TEXT = {
    0: "ok",
    -1: "invalid argument",
    -2: "unsupported type or column count",
    -3: "byte count mismatch",
    -4: "non-finite output",
    -5: "HIP runtime failure",
    -6: "workspace too small",
    -9: "expert id out of range",
}

_P = C.c_void_p
_I = C.c_int
_I64 = C.c_int64

_lock = threading.Lock()
_libs: dict[str, C.CDLL] = {}


class NativeLibraryError(RuntimeError):
    pass


def _declare(lib: C.CDLL) -> C.CDLL:
    lib.dequant_k_supported.argtypes = [_I]
    lib.dequant_k_supported.restype = _I
    lib.dequant_k_block_size.argtypes = [_I]
    lib.dequant_k_block_size.restype = _I
    lib.dequant_k.argtypes = [_I, _P, _P, _I64, _I]
    lib.dequant_k.restype = _I
    lib.moe_quant_expert.argtypes = [_I, _P, _I64] * 3 + [_P, _I, _I, _P, _I]
    lib.moe_quant_expert.restype = _I
    lib.moe_delta_heads.argtypes = [_P] * 7 + [_I] * 3
    lib.moe_delta_heads.restype = _I
    lib.mqh_delta_heads.argtypes = [_P] * 7 + [_I] * 3 + [_P, _P]
    lib.mqh_delta_heads.restype = _I
    lib.dequantize_iq4_nl_cpp.argtypes = [_P, _P, _I, _I]
    lib.dequantize_iq4_nl_cpp.restype = None
    lib.dequantize_iq4_nl_avx2.argtypes = [_P, _P, _I, _I]
    lib.dequantize_iq4_nl_avx2.restype = None
    lib.mqh_dequant.argtypes = [_I, _P, _P, _I64, _I, _P]
    lib.mqh_dequant.restype = _I
    lib.mqh_moe_workspace_bytes.argtypes = [_I, _I, _I, _I]
    lib.mqh_moe_workspace_bytes.restype = _I64
    lib.mqh_moe_decode.argtypes = [
        _I, _P, _I, _P, _I, _P, _I, _I, _I,      # routed types/tensors, n_experts, hidden, inter
        _I, _P, _I, _P, _I, _P, _I, _P,          # shared types/tensors, sh_inter, sh_gate_inp
        _P, _I, _P, _P, _I,                      # x, n_tokens, ids, weights, top_k
        _P, _I, _P, _I64, _P,                    # y, fp16_graph, workspace, ws bytes, stream
    ]
    lib.mqh_moe_decode.restype = _I
    lib.mqh_moe_decode_noalloc.argtypes = [
        _I, _P, _I, _P, _I, _P, _I, _I, _I,      # routed types/tensors, n_experts, hidden, inter
        _I, _P, _I, _P, _I, _P, _I, _P,          # shared types/tensors, sh_inter, sh_gate_inp
        _P, _I, _P, _P, _I,                      # x, n_tokens, ids, weights, top_k
        _P, _I, _P, _P,                          # y, fp16_graph, flags, stream
    ]
    lib.mqh_moe_decode_noalloc.restype = _I
    lib.mqh_moe_decode_routed.argtypes = [
        _I, _P, _I, _P, _I, _P, _I, _I, _I,      # routed types/tensors, n_experts, hidden, inter
        _I, _P, _I, _P, _I, _P, _I, _P,          # shared types/tensors, sh_inter, sh_gate_inp
        _P, _I, _P, _I, _P, _P, _P,              # x, n_tokens, router weights, top_k, scores, ids, weights
        _P, _I, _P, _I64, _P,                    # y, fp16_graph, workspace, ws bytes, stream
    ]
    lib.mqh_moe_decode_routed.restype = _I
    lib.mqh_last_route_kernels.argtypes = []
    lib.mqh_last_route_kernels.restype = _I
    lib.mqh_moe_prefill_workspace_bytes.argtypes = [_I, _I, _I, _I, _I, _I]
    lib.mqh_moe_prefill_workspace_bytes.restype = _I64
    lib.mqh_moe_prefill.argtypes = [
        _I, _P, _I, _P, _I, _P, _I, _I, _I,      # routed types/tensors, n_experts, hidden, inter
        _I, _P, _I, _P, _I, _P, _I, _P,          # shared types/tensors, sh_inter, sh_gate_inp
        _P, _I, _I, _P, _P, _I,                  # x, x_bf16, n_tokens, ids, weights, top_k
        _P, _P, _I64, _P,                        # y, workspace, ws bytes, stream
    ]
    lib.mqh_moe_prefill.restype = _I
    lib.mqh_profile_next_decode.argtypes = [_P, _P, _P, _P]
    lib.mqh_profile_next_decode.restype = _I
    lib.mqh_set_decode_path.argtypes = [_I]
    lib.mqh_set_decode_path.restype = _I
    lib.mqh_last_decode_kernels.argtypes = []
    lib.mqh_last_decode_kernels.restype = _I
    lib.mqh_last_decode_path.argtypes = []
    lib.mqh_last_decode_path.restype = _I
    lib.mqh_read_floor.argtypes = [_P, C.c_int64, _P, _P, _P, _P]
    lib.mqh_read_floor.restype = _I
    lib.mqh_route.argtypes = [_P, _I, _I, _P, _I, _I, _P, _P, _P, _P]
    lib.mqh_route.restype = _I
    lib.mqh_workspace_init.argtypes = [_P, _I64, _P]
    lib.mqh_workspace_init.restype = _I
    lib.mqh_status.argtypes = [_P, _P]
    lib.mqh_status.restype = _I
    return lib


def library_path(path: str | os.PathLike | None = None) -> Path:
    if path is not None:
        return Path(path)
    env = os.environ.get("MQH_LIBRARY")
    return Path(env) if env else DEFAULT_PATH


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load (once) and return the HIP library; raise if it is unavailable."""
    p = library_path(path).resolve()
    key = str(p)
    with _lock:
        lib = _libs.get(key)
        if lib is None:
            if not p.exists():
                raise NativeLibraryError(
                    f"{p} is not built; run intel-optimized-moe-streaming_amd/build_hip.py")
            try:
                lib = _declare(C.CDLL(key))
            except (OSError, AttributeError) as err:
                raise NativeLibraryError(f"cannot load {p}: {err}") from err
            _libs[key] = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed with status {status} ({STATUS_TEXT.get(status, 'unknown')})")
