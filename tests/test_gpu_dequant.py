"""GPU dequantization is bit-identical to the oracle (dequant_k contract).

Covers every type, FP32 and FP16 output, random blocks with the benchmark
distributions, edge blocks (zero/negative/subnormal/max scales, saturated
quant bytes), the host-pointer drop-in ``dequant_k`` and the device entry
``mqh_dequant``, and -- at the full standalone-dequant workload (256 experts x
gate/up/down of 512x2048) -- every value of every type.
"""
from __future__ import annotations

import numpy as np
import pytest

from test_oracle_pin import edge_blocks, random_blocks

pytestmark = pytest.mark.gpu

TYPES = [8, 11, 12, 13, 14]
BLOCK = {8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def _blocks(t, n=2048, seed=0):
    rng = np.random.default_rng(seed + t)
    from flash_moe_hip.synthetic import random_blocks as bench_blocks

    return np.concatenate([bench_blocks(rng, t, n), random_blocks(rng, t, 256), edge_blocks(t)]).reshape(-1)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("f16", [0, 1])
def test_host_dequant_k_bit_exact(hip, oracle_mod, t, f16):
    print(f"dequant_k type={t} f16={f16}", flush=True)
    data = _blocks(t)
    bs, pb = BLOCK[t]
    n = data.size // pb * bs
    out = np.zeros(n, np.uint16 if f16 else np.float32)
    assert hip.dequant_k(t, data.ctypes.data, out.ctypes.data, n, f16) == 0
    rc, want = oracle_mod.dequant_k(t, data, n, bool(f16))
    assert rc == 0
    got_bits = out.view(np.uint16) if f16 else out.view(np.uint32)
    want_bits = want.view(np.uint16) if f16 else want.view(np.uint32)
    bad = np.nonzero(got_bits != want_bits)[0]
    assert bad.size == 0, f"{bad.size} values differ, first at {bad[:5]}"
    assert hip.dequant_k(t, data.ctypes.data, out.ctypes.data, n + 1, f16) == -1


def test_package_dequant_helpers(hip, oracle_mod):
    from flash_moe_hip import dequant

    data = _blocks(12, 64)
    n = data.size // 144 * 256
    buf = np.empty(n, np.float16)
    got = dequant.dequant_to_f16(data.tobytes(), 12, n, out=buf)
    assert got is buf
    np.testing.assert_array_equal(got.view(np.uint16), oracle_mod.dequant(12, data, want_f16=True).view(np.uint16))
    np.testing.assert_array_equal(dequant.dequantize(data, 12).view(np.uint32),
                                  oracle_mod.dequant(12, data).view(np.uint32))
    with pytest.raises(RuntimeError):
        dequant.dequant_to_f16(data.tobytes(), 99, n)


@pytest.mark.parametrize("t", TYPES)
def test_device_dequant_bit_exact(hip, oracle_mod, t):
    import torch

    from flash_moe_hip.dequant import dequant_device

    print(f"mqh_dequant type={t}", flush=True)
    data = _blocks(t, 4096, seed=9)
    src = torch.from_numpy(data).cuda()
    for dtype, view in ((torch.float16, np.uint16), (torch.float32, np.uint32)):
        got = dequant_device(src, t, dtype=dtype).cpu().numpy().view(view)
        want = oracle_mod.dequant(t, data, want_f16=dtype == torch.float16).view(view)
        assert np.array_equal(got, want)


def _same_bits_or_nan(got, want, f16):
    """Bit equality, except that two NaNs match whatever their sign and payload."""
    ftype = np.float16 if f16 else np.float32
    nan = np.isnan(got.view(ftype)) & np.isnan(want.view(ftype))
    return np.nonzero((got != want) & ~nan)[0]


@pytest.mark.parametrize("t", TYPES)
def test_chunked_path_edge_blocks(hip, oracle_mod, t):
    """Edge blocks (zero, signed-zero, subnormal, max, infinite and NaN scales;
    saturated and patterned quant bytes) tiled into whole 4096-value chunks, so
    every one of them goes through the LDS-staged kernel, at both alignments a
    block can start on inside a chunk; FP16 and FP32 against the oracle."""
    import torch

    from flash_moe_hip.dequant import dequant_device
    from test_oracle_pin import D_OFF

    bs, pb = BLOCK[t]
    edge = edge_blocks(t)
    extra = []
    for db in (0x7C00, 0xFC00, 0x7E00):   # +inf, -inf, NaN
        for f in (0x00, 0x55, 0xFF):
            blk = np.full(pb, f, np.uint8)
            blk[D_OFF[t]:D_OFF[t] + 2] = np.array([db], np.uint16).view(np.uint8)
            extra.append(blk)
    blocks = np.concatenate([edge, np.stack(extra)])
    per_chunk = 4096 // bs
    reps = -(-2 * per_chunk // len(blocks))
    # twice over, the second copy shifted by one block, so each edge block sits
    # at an even and at an odd block index (2-byte vs 4-byte aligned for Q3_K,
    # Q6_K, Q8_0)
    tiled = np.concatenate([np.tile(blocks, (reps, 1)), blocks[1:], blocks[:1]])
    tiled = tiled[: len(tiled) // per_chunk * per_chunk].reshape(-1)
    src = torch.from_numpy(tiled).cuda()
    print(f"chunked edge dequant type={t} blocks={tiled.size // pb}", flush=True)
    for dtype, view in ((torch.float16, np.uint16), (torch.float32, np.uint32)):
        f16 = dtype == torch.float16
        got = dequant_device(src, t, dtype=dtype).cpu().numpy().view(view)
        want = oracle_mod.dequant(t, tiled, want_f16=f16).view(view)
        bad = _same_bits_or_nan(got, want, f16)
        assert bad.size == 0, (str(dtype), bad.size, bad[:5])


@pytest.mark.parametrize("t", [11, 12, 14, 8])
def test_full_workload_every_value(hip, oracle_mod, t):
    """256 experts x (gate, up, down) = 768 matrices of 1,048,576 values, generated on
    the GPU, dequantized to FP16 on the GPU and compared value by value with the oracle."""
    import torch

    from flash_moe_hip.dequant import dequant_device
    from flash_moe_hip.synthetic import torch_random_stack

    g = torch.Generator(device="cuda")
    g.manual_seed(2024 + t)
    for role, (rows, cols) in (("gate", (512, 2048)), ("up", (512, 2048)), ("down", (2048, 512))):
        print(f"full dequant type={t} role={role}", flush=True)
        stack = torch_random_stack(t, 256, rows, cols, generator=g, device="cuda")
        out = dequant_device(stack, t)
        torch.cuda.synchronize()
        host_src = stack.cpu().numpy()
        got = out.cpu().numpy().view(np.uint16)
        want = oracle_mod.dequant(t, host_src, want_f16=True).view(np.uint16)
        bad = int(np.count_nonzero(got != want))
        assert bad == 0, f"{role}: {bad} of {got.size} values differ"
        del stack, out


def test_read_floor_kernel(hip):
    """The streaming-read reference kernel (a measurement aid): runs between
    its events on the given stream, rejects misaligned or ragged sizes, and
    leaves the source untouched."""
    import torch

    buf = torch.arange(1 << 20, dtype=torch.int32, device="cuda")
    before = buf.clone()
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    assert hip.mqh_read_floor(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(), None, None, stream) == 0
    stop.record()
    torch.cuda.synchronize()
    assert start.elapsed_time(stop) > 0.0
    assert torch.equal(buf, before)
    assert hip.mqh_read_floor(buf.data_ptr() + 4, 1 << 12, None, None, None, stream) == -1
    assert hip.mqh_read_floor(buf.data_ptr(), 1000, None, None, None, stream) == -1
    assert hip.mqh_read_floor(None, 1 << 12, None, None, None, stream) == -1


def _iq4nl_blocks(n, seed):
    from flash_moe_hip.synthetic import random_blocks as bench_blocks

    rng = np.random.default_rng(seed)
    b = bench_blocks(rng, 20, n)
    edge = np.zeros((6, 18), np.uint8)
    edge[:, 2:] = rng.integers(0, 256, size=(6, 16), dtype=np.uint8)
    for i, d in enumerate((0.0, -0.0, -1.5, 65504.0, 6e-8, 2.0 ** -14)):
        edge[i, 0:2] = np.array([d], np.float16).view(np.uint8)
    return np.concatenate([b, edge]).reshape(-1)


def test_device_dequant_iq4_nl_bit_exact(hip, oracle_mod):
    """IQ4_NL (type 20) through mqh_dequant, FP32 and FP16, against the oracle
    of the reference's IQ4_NL library (cpp/fast_dequant.cpp:40-65)."""
    import torch

    from flash_moe_hip.dequant import dequant_device

    data = _iq4nl_blocks(4096, 5)
    src = torch.from_numpy(data).cuda()
    for dtype, view in ((torch.float16, np.uint16), (torch.float32, np.uint32)):
        got = dequant_device(src, 20, dtype=dtype).cpu().numpy().view(view)
        want = oracle_mod.dequant(20, data, want_f16=dtype == torch.float16).view(view)
        assert np.array_equal(got, want)


def test_host_iq4_nl_exports(hip, oracle_mod):
    """dequantize_iq4_nl_cpp / _avx2 (host pointers, the reference signature):
    whole rows, and a column count that leaves a partial block whose output
    columns stay untouched."""
    from flash_moe_hip.dequant import dequantize_iq4_nl

    rng = np.random.default_rng(6)
    rows = 40
    for cols in (64, 512, 70):
        bpr = cols // 32
        raw = _iq4nl_blocks(rows * bpr - 6, 7 + cols)
        want = oracle_mod.dequantize_iq4_nl(raw, rows, cols)
        for fn in (hip.dequantize_iq4_nl_cpp, hip.dequantize_iq4_nl_avx2):
            dst = np.full((rows, cols), 7.0, np.float32)
            fn(raw.ctypes.data, dst.ctypes.data, rows, cols)
            np.testing.assert_array_equal(dst[:, :32 * bpr].view(np.uint32), want[:, :32 * bpr].view(np.uint32))
            assert np.all(dst[:, 32 * bpr:] == 7.0)
        if cols % 32 == 0:
            got = dequantize_iq4_nl(raw, rows, cols)
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    dst = np.full((2, 64), 3.0, np.float32)
    hip.dequantize_iq4_nl_avx2(None, dst.ctypes.data, 2, 64)        # nothing to run: dst untouched
    assert np.all(dst == 3.0)
