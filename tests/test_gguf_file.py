"""GGUF reader (flash_moe_hip.gguf_file) against files packed here byte by byte.

The packer below writes the GGUF layout with explicit struct formats (magic,
u32 version, u64 counts, typed metadata, tensor infos, aligned data section),
independently of the reader's code path.  The checks pin metadata decoding for
every value type, tensor offsets under the default and a custom alignment,
zero-copy tensor bytes, the float tensor views, the expert-layer slicing the
reference uses (``run_q4k_f16_openvino.py:112-122``: expert e = bytes
[e * n_bytes/E, (e+1) * n_bytes/E) of the stacked tensor), and the error paths.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

from flash_moe_hip.gguf_file import GGUFError, GGUFFile, layer_host_tensors

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
       I64: "<q", F64: "<d"}


def p_str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def p_val(vtype, v) -> bytes:
    if vtype == STR:
        return p_str(v)
    if vtype == ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(p_val(etype, x) for x in items)
    return struct.pack(FMT[vtype], v)


def pack_gguf(kvs, tensors, alignment=32, version=3) -> bytes:
    """kvs: [(key, vtype, value)]; tensors: [(name, dims, ggml_type, data bytes)]."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, vtype, value in kvs:
        head += p_str(key) + struct.pack("<I", vtype) + p_val(vtype, value)
    infos, data, offs = b"", b"", []
    for name, dims, gtype, blob in tensors:
        pad = (-len(data)) % alignment
        data += b"\0" * pad
        offs.append(len(data))
        data += blob
    for (name, dims, gtype, blob), off in zip(tensors, offs):
        infos += p_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", gtype, off)
    body = head + infos
    body += b"\0" * ((-len(body)) % alignment)
    return body + data


def write(tmp_path, blob, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    return p


def test_metadata_every_value_type(tmp_path):
    kvs = [("a.u8", U8, 200), ("a.i8", I8, -5), ("a.u16", U16, 60000), ("a.i16", I16, -30000),
           ("a.u32", U32, 4000000000), ("a.i32", I32, -2000000000), ("a.f32", F32, 1.5), ("a.bool", BOOL, True),
           ("a.str", STR, "qwen3 moe ü"), ("a.u64", U64, 2 ** 40 + 3), ("a.i64", I64, -2 ** 40),
           ("a.f64", F64, 0.1), ("a.arr_i32", ARR, (I32, [1, -2, 3])), ("a.arr_str", ARR, (STR, ["x", "yz"])),
           ("a.arr_arr", ARR, (ARR, [(U8, [1, 2]), (U8, [])]))]
    g = GGUFFile(write(tmp_path, pack_gguf(kvs, [])))
    m = g.metadata
    assert g.version == 3 and not g.tensors
    assert (m["a.u8"], m["a.i8"], m["a.u16"], m["a.i16"]) == (200, -5, 60000, -30000)
    assert (m["a.u32"], m["a.i32"], m["a.u64"], m["a.i64"]) == (4000000000, -2000000000, 2 ** 40 + 3, -2 ** 40)
    assert m["a.f32"] == 1.5 and m["a.f64"] == 0.1 and m["a.bool"] is True
    assert m["a.str"] == "qwen3 moe ü"
    assert m["a.arr_i32"] == [1, -2, 3] and m["a.arr_str"] == ["x", "yz"] and m["a.arr_arr"] == [[1, 2], []]


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_tensor_table_offsets_and_bytes(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)              # dims (5, 3)
    f16 = rng.standard_normal(7).astype(np.float16)                   # dims (7,)
    q4k = rng.integers(0, 256, 2 * 144, dtype=np.uint8)               # Q4_K [2 rows x 256]
    bf = rng.standard_normal(4).astype(np.float32)
    bf16 = (bf.view(np.uint32) >> 16).astype(np.uint16)               # truncated to BF16
    kvs = [("general.alignment", U32, alignment)] if alignment != 32 else []
    tensors = [("w.f32", (5, 3), 0, f32.tobytes()), ("w.f16", (7,), 1, f16.tobytes()),
               ("w.q4k", (256, 2), 12, q4k.tobytes()), ("w.bf16", (4,), 30, bf16.tobytes())]
    g = GGUFFile(write(tmp_path, pack_gguf(kvs, tensors, alignment)))
    assert g.alignment == alignment and g.data_offset % alignment == 0
    t = g.tensors["w.q4k"]
    assert t.dims == (256, 2) and t.shape == (2, 256) and t.ggml_type == 12 and t.n_bytes == 288
    assert t.offset % alignment == 0
    assert np.array_equal(g.raw("w.q4k"), q4k)
    assert np.array_equal(g.float_array("w.f32"), f32)
    assert np.array_equal(g.float_array("w.f16"), f16.astype(np.float32))
    assert np.array_equal(g.float_array("w.bf16"), (bf16.astype(np.uint32) << 16).view(np.float32))
    with pytest.raises(GGUFError):
        g.float_array("w.q4k")


def test_errors(tmp_path):
    with pytest.raises(GGUFError):
        GGUFFile(write(tmp_path, b"GGML" + b"\0" * 32, "bad_magic.gguf"))
    with pytest.raises(GGUFError):
        GGUFFile(write(tmp_path, pack_gguf([], [], version=4), "v4.gguf"))
    full = pack_gguf([("k", STR, "value")], [("w", (4,), 0, b"\0" * 16)])
    with pytest.raises(GGUFError):
        GGUFFile(write(tmp_path, full[:30], "trunc.gguf"))            # inside the metadata
    with pytest.raises(GGUFError):
        GGUFFile(write(tmp_path, full[:-4], "short.gguf"))            # data past the end
    with pytest.raises(GGUFError):                                     # Q4_K row not a whole block
        GGUFFile(write(tmp_path, pack_gguf([], [("w", (100,), 12, b"\0" * 144)]), "ragged.gguf"))


def moe_file(tmp_path, rng, E=4, H=256, I=512, types=(12, 12, 14), sh_types=(14, 14, 14), sh_I=256):
    from flash_moe_hip.synthetic import random_stack

    g, u, d = (random_stack(rng, t, E, *shape) for t, shape in zip(types, ((I, H), (I, H), (H, I))))
    sg, su, sd = (random_stack(rng, t, 1, *shape) for t, shape in zip(sh_types, ((sh_I, H), (sh_I, H), (H, sh_I))))
    gate_inp_sh = rng.standard_normal(H).astype(np.float32)
    router = rng.standard_normal((E, H)).astype(np.float16)          # GGUF dims (H, E), stored F16
    tensors = [("blk.3.ffn_gate_exps.weight", (H, I, E), types[0], g.tobytes()),
               ("blk.3.ffn_up_exps.weight", (H, I, E), types[1], u.tobytes()),
               ("blk.3.ffn_down_exps.weight", (I, H, E), types[2], d.tobytes()),
               ("blk.3.ffn_gate_shexp.weight", (H, sh_I), sh_types[0], sg.tobytes()),
               ("blk.3.ffn_up_shexp.weight", (H, sh_I), sh_types[1], su.tobytes()),
               ("blk.3.ffn_down_shexp.weight", (sh_I, H), sh_types[2], sd.tobytes()),
               ("blk.3.ffn_gate_inp_shexp.weight", (H,), 0, gate_inp_sh.tobytes()),
               ("blk.3.ffn_gate_inp.weight", (H, E), 1, router.tobytes()),
               ("blk.3.attn_norm.weight", (H,), 0, np.ones(H, np.float32).tobytes())]
    path = write(tmp_path, pack_gguf([("general.architecture", STR, "qwen3moe")], tensors))
    return path, {"gate": g, "up": u, "down": d, "sh": (sg, su, sd), "gate_inp_sh": gate_inp_sh, "router": router}


def test_expert_layer_slicing(tmp_path):
    rng = np.random.default_rng(7)
    path, want = moe_file(tmp_path, rng)
    gf = GGUFFile(path)
    assert gf.expert_layers() == {3: {"gate": 12, "up": 12, "down": 14}}
    h = layer_host_tensors(gf, 3)
    assert (h["n_experts"], h["hidden"], h["intermediate"]) == (4, 256, 512)
    assert h["types"] == {"gate": 12, "up": 12, "down": 14}
    per = {"gate": 512 * 144, "up": 512 * 144, "down": 256 * 2 * 210}
    for r in ("gate", "up", "down"):
        assert np.array_equal(h["tensors"][r], want[r])
        for e in range(4):   # expert e = the e-th n_bytes/E slice, as the reference slices it
            assert np.array_equal(h["tensors"][r][e * per[r]:(e + 1) * per[r]], want[r][e * per[r]:(e + 1) * per[r]])
    sh = h["shared"]
    assert sh["types"] == {"gate": 14, "up": 14, "down": 14} and sh["intermediate"] == 256
    assert all(np.array_equal(sh[r], w) for r, w in zip(("gate", "up", "down"), want["sh"]))
    assert np.array_equal(sh["gate_inp"], want["gate_inp_sh"])
    assert h["router_weights"].shape == (256, 4)
    assert np.array_equal(h["router_weights"], want["router"].astype(np.float32).T)


def test_mismatched_expert_stacks_rejected(tmp_path):
    rng = np.random.default_rng(8)
    from flash_moe_hip.synthetic import random_stack

    g = random_stack(rng, 12, 2, 256, 256)
    d = random_stack(rng, 12, 2, 256, 256)
    tensors = [("blk.0.ffn_gate_exps.weight", (256, 256, 2), 12, g.tobytes()),
               ("blk.0.ffn_up_exps.weight", (256, 256, 2), 12, g.tobytes()),
               ("blk.0.ffn_down_exps.weight", (256, 256, 1), 12, d[:d.size // 2].tobytes())]
    gf = GGUFFile(write(tmp_path, pack_gguf([], tensors)))
    with pytest.raises(GGUFError):
        layer_host_tensors(gf, 0)


@pytest.mark.gpu
def test_layer_from_gguf_decodes_like_the_oracle(tmp_path, oracle_mod, hip):
    """A layer read from a GGUF file with the reference model's tensor names and
    type mix (routed Q4_K gate/up and Q6_K down, shared expert Q6_K with its own
    intermediate size), uploaded to HBM, routed by its own ffn_gate_inp weights
    and decoded: equal to the oracle's layer within 1e-3."""
    import torch

    from flash_moe_hip.gguf_file import load_expert_layer
    from flash_moe_hip.moe_gpu import MoeRunner
    from flash_moe_hip.router import ExpertRouter
    from test_gpu_decode import TOL, oracle_layer

    rng = np.random.default_rng(11)
    path, want = moe_file(tmp_path, rng, E=8, H=512, I=256, sh_I=512)
    gf = GGUFFile(path)
    layer = load_expert_layer(gf, 3, device="cuda")
    assert layer.n_experts == 8 and layer.types == {"gate": 12, "up": 12, "down": 14}
    router = ExpertRouter(512, 8, top_k=4, gate_weights=layer.router_weights)
    host = {r: want[r] for r in ("gate", "up", "down")}
    shared = {"gate": want["sh"][0], "up": want["sh"][1], "down": want["sh"][2],
              "types": {"gate": 14, "up": 14, "down": 14}, "intermediate": 512, "gate_inp": want["gate_inp_sh"]}
    X = rng.standard_normal((3, 512)).astype(np.float32)
    ids, ws = router.route_batch(X)
    runner = MoeRunner()
    y = runner.decode(layer, torch.from_numpy(X).cuda(), torch.from_numpy(ids).cuda(),
                      torch.from_numpy(ws).cuda()).cpu().numpy()
    assert runner.status() == 0
    for t in range(3):
        ref = oracle_layer(oracle_mod, layer, host, shared, X[t], ids[t].tolist(), ws[t].tolist())
        err = oracle_mod.max_relative_error(y[t], ref)
        print(f"  gguf layer token {t}: max rel err {err:.3e}", flush=True)
        assert err <= TOL
