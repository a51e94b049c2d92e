"""GGML quantization type ids and block geometry.

Type ids and (values per block, bytes per block) are fixed by the GGUF format;
they are the same numbers as ``src/flash_moe/dequant.py:30-50`` (by name) and
``cpp/dequant_k.cpp:37-41,302-322`` (by id).
"""
from __future__ import annotations

GGML_TYPE_IDS: dict[str, int] = {"Q8_0": 8, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
IQ4_NL = 20
TYPE_NAMES: dict[int, str] = {**{v: k for k, v in GGML_TYPE_IDS.items()}, IQ4_NL: "IQ4_NL"}

# The types of the reference's native expert (native_expert.py:10 lists the
# same five): what NativeExpert / load_native_expert accept.
SUPPORTED_TYPES = frozenset(GGML_TYPE_IDS.values())
# What the device entry points decode: the five plus IQ4_NL (the reference's
# fast_dequant library, cpp/fast_dequant.cpp:40-65).
DEVICE_TYPES = SUPPORTED_TYPES | {IQ4_NL}

# A resident form of this library (not a GGUF type): Q3_K blocks byte for byte,
# each in a 112-byte slot (two zero bytes after the 110), so that every block
# starts on a 16-byte boundary.  Only the decode entry point takes it
# (``mqh_moe_decode`` on its fast kernels); ``pad_blocks`` makes it.
Q3_K_A112 = 111
RESIDENT_BLOCK_INFO: dict[str, tuple[int, int]] = {"Q3_K_A112": (256, 112)}
TYPE_NAMES[Q3_K_A112] = "Q3_K_A112"
# what a resident layer may hold
DECODE_TYPES = DEVICE_TYPES | {Q3_K_A112}

# name -> (block_size, bytes_per_block) for every GGUF type the reference names.
GGML_BLOCK_INFO: dict[str, tuple[int, int]] = {
    "F32": (1, 4),
    "F16": (1, 2),
    "BF16": (1, 2),
    "Q4_0": (32, 18),
    "Q4_1": (32, 20),
    "Q5_0": (32, 22),
    "Q5_1": (32, 24),
    "Q8_0": (32, 34),
    "Q2_K": (256, 84),
    "Q3_K": (256, 110),
    "Q4_K": (256, 144),
    "Q5_K": (256, 176),
    "Q6_K": (256, 210),
    "Q8_K": (256, 292),
    "IQ4_NL": (32, 18),
    "IQ4_XS": (256, 136),
    "IQ3_XXS": (256, 98),
    "IQ2_XXS": (256, 66),
    "IQ1_S": (256, 50),
}


def block_info(ggml_type: int) -> tuple[int, int]:
    """(values per block, bytes per block) of a supported type id."""
    name = TYPE_NAMES.get(int(ggml_type))
    if name is None:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    return RESIDENT_BLOCK_INFO.get(name) or GGML_BLOCK_INFO[name]


def pad_blocks(t, block_bytes: int, slot_bytes: int):
    """A flat uint8 tensor of whole blocks, each copied into a zero-padded slot."""
    import torch

    if t.numel() % block_bytes:
        raise ValueError(f"{t.numel()} bytes is not a whole number of {block_bytes}-byte blocks")
    v = t.reshape(-1, block_bytes)
    out = torch.zeros((v.shape[0], slot_bytes), dtype=torch.uint8, device=t.device)
    out[:, :block_bytes] = v
    return out.reshape(-1)


def name_of(ggml_type: int) -> str:
    return TYPE_NAMES.get(int(ggml_type), f"type_{int(ggml_type)}")


def tensor_bytes(ggml_type: int, rows: int, cols: int) -> int:
    bs, pb = block_info(ggml_type)
    if cols % bs:
        raise ValueError(f"{cols} columns is not a multiple of the {name_of(ggml_type)} block ({bs})")
    return rows * (cols // bs) * pb
