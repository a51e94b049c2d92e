"""Seeded synthetic GGUF expert tensors and activations.

The distributions are those of the benchmark workloads: every byte of a block
is uniform, except the FP16 super-block scales, which are ``|N(0,1)| * 0.01``
rounded to FP16, and the Q8_0 quants, which are uniform int8 in -127..127.
Uniform bytes are uniform over each type's legal bit ranges: Q4_K scales and
mins 0..63 (through the 6-bit unpacking), Q6_K int8 scales -128..127, Q3_K
signed 6-bit scales, 2/3/4/6-bit quants.

Two generators with the same distributions:
  * NumPy (``default_rng(seed)``) for parity cases, so the CPU oracle can
    regenerate identical bytes;
  * torch on the GPU for the multi-GB resident layer stacks of the benchmark.
"""
from __future__ import annotations

import numpy as np

from .quant_types import GGML_TYPE_IDS, block_info

# byte offsets of the FP16 scale fields per type: (d, dmin or None)
SCALE_FIELDS = {8: (0, None), 11: (108, None), 12: (0, 2), 13: (0, 2), 14: (208, None), 20: (0, None)}


def tensor_nbytes(ggml_type: int, rows: int, cols: int) -> int:
    bs, pb = block_info(ggml_type)
    if cols % bs:
        raise ValueError(f"cols={cols} is not a multiple of the block size {bs}")
    return rows * (cols // bs) * pb


def random_blocks(rng: np.random.Generator, ggml_type: int, n_blocks: int,
                  scale: float = 0.01) -> np.ndarray:
    """``n_blocks`` blocks of ``ggml_type`` as a (n_blocks, bytes_per_block) uint8 array."""
    ggml_type = int(ggml_type)
    _, pb = block_info(ggml_type)
    data = rng.integers(0, 256, size=(n_blocks, pb), dtype=np.uint8)
    if ggml_type == 8:
        data[:, 2:] = rng.integers(-127, 128, size=(n_blocks, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    d_off, m_off = SCALE_FIELDS[ggml_type]
    d = (np.abs(rng.standard_normal(n_blocks)) * scale).astype(np.float16)
    data[:, d_off:d_off + 2] = d.view(np.uint8).reshape(n_blocks, 2)
    if m_off is not None:
        m = (np.abs(rng.standard_normal(n_blocks)) * scale).astype(np.float16)
        data[:, m_off:m_off + 2] = m.view(np.uint8).reshape(n_blocks, 2)
    return data


def random_tensor(rng: np.random.Generator, ggml_type: int, rows: int, cols: int,
                  scale: float = 0.01) -> np.ndarray:
    """One [rows x cols] matrix as flat uint8 bytes, GGUF row-major block order."""
    bs, _ = block_info(ggml_type)
    return random_blocks(rng, ggml_type, rows * (cols // bs), scale).reshape(-1)


def random_expert(rng: np.random.Generator, kinds: dict, hidden: int, intermediate: int,
                  scale: float = 0.01) -> dict:
    """gate/up [intermediate x hidden], down [hidden x intermediate] raw bytes."""
    return {
        "gate": random_tensor(rng, kinds["gate"], intermediate, hidden, scale),
        "up": random_tensor(rng, kinds["up"], intermediate, hidden, scale),
        "down": random_tensor(rng, kinds["down"], hidden, intermediate, scale),
    }


def random_stack(rng: np.random.Generator, ggml_type: int, n_experts: int, rows: int, cols: int,
                 scale: float = 0.01) -> np.ndarray:
    """A stacked GGUF expert tensor: ``n_experts`` consecutive [rows x cols] slices."""
    return random_tensor(rng, ggml_type, n_experts * rows, cols, scale)


def config1_expert(seed: int = 0, hidden: int = 2048, intermediate: int = 512):
    """Single Q4_K expert, x ~ N(0,1) FP32 [hidden], seed 0."""
    rng = np.random.default_rng(seed)
    kinds = {"gate": 12, "up": 12, "down": 12}
    tensors = random_expert(rng, kinds, hidden, intermediate)
    x = rng.standard_normal(hidden).astype(np.float32)
    return tensors, kinds, x


# ------------------------------------------------------------------ torch/GPU

def torch_random_stack(ggml_type: int, n_experts: int, rows: int, cols: int, *,
                       generator, device, scale: float = 0.01):
    """Device-side generator with the distributions of :func:`random_stack`.

    Returns a flat uint8 CUDA tensor.  Bytes come from ``torch.randint`` under
    ``generator``; scale fields are overwritten with ``|N(0,1)|*scale`` in FP16.
    """
    import torch

    ggml_type = int(ggml_type)
    bs, pb = block_info(ggml_type)
    n_blocks = n_experts * rows * (cols // bs)
    data = torch.randint(0, 256, (n_blocks, pb), dtype=torch.uint8, device=device, generator=generator)
    if ggml_type == 8:
        q = torch.randint(-127, 128, (n_blocks, 32), dtype=torch.int16, device=device, generator=generator)
        data[:, 2:] = q.to(torch.int8).view(torch.uint8)
        del q
    d_off, m_off = SCALE_FIELDS[ggml_type]
    for off in (d_off, m_off):
        if off is None:
            continue
        d = (torch.randn(n_blocks, device=device, generator=generator).abs_() * scale).to(torch.float16)
        data[:, off:off + 2] = d.view(torch.uint8).view(n_blocks, 2)
        del d
    return data.view(-1)


__all__ = ["GGML_TYPE_IDS", "SCALE_FIELDS", "tensor_nbytes", "random_blocks", "random_tensor",
           "random_expert", "random_stack", "config1_expert", "torch_random_stack"]
