"""The C ABI library loads and exports what include/moe_quant_hip.h declares (CPU only).

Only host-side logic is called here: type queries and the argument validation
that returns before any HIP call (status codes of moe_quant_dot.cpp:181-188
and dequant_k.cpp:352-355).  No kernel runs.
"""
from __future__ import annotations

import ctypes as C
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "moe_quant_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:int|int64_t|void)\s+\**(\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    from flash_moe_hip import _lib

    return _lib.load()


def test_header_declares_the_binding_list():
    from flash_moe_hip import _lib

    assert sorted(declared_functions()) == sorted(_lib.EXPORTS)


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_type_queries(lib):
    expect = {8: 32, 11: 256, 12: 256, 13: 256, 14: 256}
    for t in range(0, 40):
        assert lib.dequant_k_supported(t) == (1 if t in expect else 0)
        assert lib.dequant_k_block_size(t) == expect.get(t, 0)


def test_dequant_k_rejects_bad_arguments(lib):
    buf = np.zeros(144, np.uint8)
    out = np.zeros(256, np.float32)
    assert lib.dequant_k(99, buf.ctypes.data, out.ctypes.data, 256, 0) == -1
    assert lib.dequant_k(12, None, out.ctypes.data, 256, 0) == -1
    assert lib.dequant_k(12, buf.ctypes.data, None, 256, 0) == -1
    assert lib.dequant_k(12, buf.ctypes.data, out.ctypes.data, 0, 0) == -1
    assert lib.dequant_k(12, buf.ctypes.data, out.ctypes.data, 257, 0) == -1


def test_moe_quant_expert_validation_codes(lib):
    H = I = 256
    g = np.zeros(I * 144, np.uint8)
    d = np.zeros(H * 210, np.uint8)
    x = np.zeros(H, np.float32)
    y = np.zeros(H, np.float32)

    def call(gt=12, gb=g.nbytes, ut=12, ub=g.nbytes, dt=14, db=d.nbytes, h=H, i=I, f16=0, gp=g, xp=x):
        return lib.moe_quant_expert(gt, None if gp is None else gp.ctypes.data, gb, ut, g.ctypes.data, ub,
                                    dt, d.ctypes.data, db, None if xp is None else xp.ctypes.data, h, i,
                                    y.ctypes.data, f16)

    assert call(gp=None) == -1
    assert call(xp=None) == -1
    assert call(h=0) == -1
    assert call(i=-1) == -1
    assert call(h=65537) == -1
    assert call(f16=2) == -1
    assert call(gt=999) == -2
    assert call(dt=7) == -2
    assert call(h=288) == -2            # 288 % 256
    assert call(gb=g.nbytes - 1) == -3
    assert call(db=d.nbytes + 210) == -3


def test_device_entry_validation(lib):
    assert lib.mqh_moe_workspace_bytes(0, 8, 512, 512) == -1
    assert lib.mqh_moe_workspace_bytes(1, 0, 512, 0) == -1
    ws = lib.mqh_moe_workspace_bytes(16, 8, 512, 512)
    assert ws >= 16 * 9 * 512 * 4 and ws % 256 == 0
    assert lib.mqh_moe_workspace_bytes(1, 0, 0, 512) > 0          # shared expert only
    assert lib.mqh_dequant(99, C.c_void_p(16), C.c_void_p(16), 256, 1, None) == -1
    assert lib.mqh_dequant(12, C.c_void_p(16), C.c_void_p(24), 256, 1, None) == -1   # dst not 16-B aligned
    args = [12, C.c_void_p(256), 12, C.c_void_p(256), 14, C.c_void_p(256), 256, 2048, 512,
            0, None, 0, None, 0, None, 0, None,
            C.c_void_p(256), 1, C.c_void_p(256), C.c_void_p(256), 8,
            C.c_void_p(256), 0, C.c_void_p(256), 1 << 20, None]
    bad_type = list(args)
    bad_type[0] = 99
    assert lib.mqh_moe_decode(*bad_type) == -2
    bad_k = list(args)
    bad_k[21] = 0                       # top_k 0 without a shared expert
    assert lib.mqh_moe_decode(*bad_k) == -1
    small_ws = list(args)
    small_ws[25] = 64
    assert lib.mqh_moe_decode(*small_ws) == -6


def test_route_validation(lib):
    p = C.c_void_p(256)
    ok = dict(x=p, t=1, h=2048, w=p, e=128, k=8, s=p, ids=p, wts=p)

    def call(**kw):
        a = {**ok, **kw}
        return lib.mqh_route(a["x"], a["t"], a["h"], a["w"], a["e"], a["k"], a["s"], a["ids"], a["wts"], None)

    assert call(x=None) == -1
    assert call(w=None) == -1
    assert call(s=None) == -1
    assert call(ids=None) == -1
    assert call(wts=None) == -1
    assert call(t=0) == -1
    assert call(h=0) == -1
    assert call(h=2046) == -1                 # rows are read 16 bytes at a time
    assert call(x=C.c_void_p(264)) == -1      # x not 16-byte aligned
    assert call(w=C.c_void_p(260)) == -1
    assert call(e=1025) == -1                 # at most 16 scores per lane
    assert call(k=0) == -1
    assert call(k=65) == -1                   # one selected score per lane
    assert call(e=4, k=5) == -1               # more slots than experts


def test_delta_heads_validation(lib):
    p = C.c_void_p(256)
    ok = dict(st=p, q=p, k=p, v=p, b=p, g=p, o=p, h=32, dk=128, dv=128)

    def call(fn, **kw):
        a = {**ok, **kw}
        args = [a["st"], a["q"], a["k"], a["v"], a["b"], a["g"], a["o"], a["h"], a["dk"], a["dv"]]
        return fn(*args) if fn is lib.moe_delta_heads else fn(*args, None, None)

    for fn in (lib.moe_delta_heads, lib.mqh_delta_heads):
        for key in ("st", "q", "k", "v", "b", "g", "o"):
            assert call(fn, **{key: None}) == -1
        for kw in (dict(h=0), dict(h=257), dict(dk=0), dict(dk=1025), dict(dv=0), dict(dv=1025)):
            assert call(fn, **kw) == -1          # moe_delta.cpp:21-24


def test_iq4_nl_stays_outside_the_reference_contracts(lib):
    # dequant_k and moe_quant_expert keep the reference's five types
    # (dequant_k.cpp:342-348); IQ4_NL has its own exports and the device paths
    assert lib.dequant_k_supported(20) == 0
    assert lib.dequant_k_block_size(20) == 0
    buf = np.zeros(18, np.uint8)
    out = np.zeros(32, np.float32)
    assert lib.dequant_k(20, buf.ctypes.data, out.ctypes.data, 32, 0) == -1
