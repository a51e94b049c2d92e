"""The AVX2 row dot of the oracle (the bench's CPU baseline) against the scalar
oracle, bit for bit (CPU only).

The AVX2 form decodes Q3_K and Q6_K straight from their bit fields into one
8-lane accumulator, as the reference's quant_dot does
(cpp/moe_quant_dot.cpp:23-169); every other type goes through the block
decoder.  Both forms feed the same FP32 weights to the same per-lane FMA
sequence, so the expert outputs must be identical, not merely close: a wrong
shift, a flipped mask bit or a misplaced scale in the bit-field decoding
changes them.
"""
from __future__ import annotations

import numpy as np
import pytest

from test_oracle_expert import BLOCK, TRIPLES, kat_expert

KINDS = ("gate", "up", "down")


def _same(oracle_mod, tensors, kinds, x, hidden, inter, fp16_graph):
    rc0, y0 = oracle_mod.moe_quant_expert(tensors, kinds, x, hidden, inter, fp16_graph)
    rc1, y1 = oracle_mod.moe_quant_expert(tensors, kinds, x, hidden, inter, fp16_graph, avx2=True)
    assert rc0 == rc1
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32)), \
        (kinds, fp16_graph, int(np.argmax(y0.view(np.uint32) != y1.view(np.uint32))))
    return rc0, y0


@pytest.mark.parametrize("fp16_graph", [0, 1])
@pytest.mark.parametrize("triple", TRIPLES + [(14, 14, 14), (11, 14, 11)])
def test_avx2_expert_bit_identical(oracle_mod, triple, fp16_graph):
    rng = np.random.default_rng(100 + sum(triple) + fp16_graph)
    kinds = dict(zip(KINDS, triple))
    tensors = kat_expert(rng, triple)
    x = (rng.standard_normal(256) * (0.005 if fp16_graph else 1.0)).astype(np.float32)
    rc, y = _same(oracle_mod, tensors, kinds, x, 256, 256, fp16_graph)
    assert rc == 0 and np.abs(y).max() > 0


@pytest.mark.parametrize("kind", [11, 14])
@pytest.mark.parametrize("fill", [0x00, 0xFF, 0x55, 0xAA, 0x0F, 0xF0])
def test_avx2_bit_field_extremes(oracle_mod, kind, fill):
    """Every quant byte (low bits, high bits, mask) set to one pattern, scales
    random: the extreme quants -4/3 (Q3_K) and -32/31 (Q6_K) and every shift."""
    rng = np.random.default_rng(kind * 256 + fill)
    triple = (kind, kind, kind)
    tensors = kat_expert(rng, triple)
    _, size = BLOCK[kind]
    scale_at = 96 if kind == 11 else 192          # the 12 or 16 scale bytes precede d
    for name in KINDS:
        raw = tensors[name].reshape(-1, size)
        raw[:, :scale_at] = fill
    x = rng.standard_normal(256).astype(np.float32)
    for g in (0, 1):
        _same(oracle_mod, tensors, dict(zip(KINDS, triple)), x * (0.005 if g else 1.0), 256, 256, g)


def test_avx2_benchmark_shapes(oracle_mod):
    """The decode layer's expert (hidden 2048, intermediate 512, Q4_K/Q6_K) and
    the batched layer's all-Q3_K expert."""
    from flash_moe_hip.synthetic import config1_expert

    tensors, kinds, x = config1_expert(0)
    _same(oracle_mod, tensors, kinds, x, 2048, 512, 0)
    rng = np.random.default_rng(7)
    for triple in ((12, 12, 14), (11, 11, 11)):
        t = kat_expert(rng, triple, hidden=2048, inter=512)
        _same(oracle_mod, t, dict(zip(KINDS, triple)), rng.standard_normal(2048).astype(np.float32), 2048, 512, 0)
