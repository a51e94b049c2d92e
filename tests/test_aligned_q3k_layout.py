"""Host side of the 112-byte Q3_K resident form (type 111): block geometry, the
padding helper and the C header's type constant (no GPU)."""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest


def test_geometry():
    from flash_moe_hip.quant_types import DECODE_TYPES, DEVICE_TYPES, GGML_BLOCK_INFO, Q3_K_A112, block_info, tensor_bytes

    assert Q3_K_A112 == 111 and Q3_K_A112 in DECODE_TYPES and Q3_K_A112 not in DEVICE_TYPES
    assert block_info(111) == (256, 112) and block_info(11) == (256, 110)
    assert "Q3_K_A112" not in GGML_BLOCK_INFO   # not a GGUF type
    assert tensor_bytes(111, 512, 2048) == 512 * 8 * 112


def test_pad_blocks():
    import torch
    from flash_moe_hip.quant_types import pad_blocks

    rng = np.random.default_rng(1)
    raw = rng.integers(0, 256, 110 * 37, dtype=np.uint8)
    out = pad_blocks(torch.from_numpy(raw), 110, 112).numpy().reshape(37, 112)
    assert np.array_equal(out[:, :110], raw.reshape(37, 110))
    assert not out[:, 110:].any()
    with pytest.raises(ValueError):
        pad_blocks(torch.from_numpy(raw[:-1]), 110, 112)


def test_header_constant():
    text = (Path(__file__).resolve().parents[1] / "include" / "moe_quant_hip.h").read_text()
    m = re.search(r"#define\s+MQH_TYPE_Q3_K_A112\s+(\d+)", text)
    assert m and int(m.group(1)) == 111
