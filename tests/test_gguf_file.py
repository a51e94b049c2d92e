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
    # stored as the reference stores them: FP16-rounded, promoted to FP32
    assert np.array_equal(sh["gate_inp"], want["gate_inp_sh"].astype(np.float16).astype(np.float32))
    assert not np.array_equal(sh["gate_inp"], want["gate_inp_sh"])   # the file's F32 values do change
    assert h["router_weights"].shape == (256, 4)
    assert np.array_equal(h["router_weights"], want["router"].astype(np.float32).T)


def test_f32_router_gate_is_stored_as_the_router_stores_it(tmp_path):
    """An F32 ffn_gate_inp is rounded to the router's gate_dtype (FP16 by
    default, router.py:51-59, 99, 136) and promoted: the weights the device
    routes with equal ExpertRouter.from_gguf_tensor's gate_weights bit for bit,
    for the FP16 default and for gate_dtype=float32 (no rounding)."""
    from flash_moe_hip.router import ExpertRouter

    from flash_moe_hip.synthetic import random_stack

    rng = np.random.default_rng(9)
    E, H = 8, 256
    r32 = rng.standard_normal((E, H)).astype(np.float32) * 0.02
    w = random_stack(rng, 12, E, 256, H).tobytes()        # [256 x 256] Q4_K per expert, every role
    tensors = [("blk.1.ffn_gate_exps.weight", (H, 256, E), 12, w),
               ("blk.1.ffn_up_exps.weight", (H, 256, E), 12, w),
               ("blk.1.ffn_down_exps.weight", (256, H, E), 12, w),
               ("blk.1.ffn_gate_inp.weight", (H, E), 0, r32.tobytes())]
    gf = GGUFFile(write(tmp_path, pack_gguf([], tensors)))
    tm = gf.tensor_map()
    for dt in (np.float16, np.float32):
        h = layer_host_tensors(gf, 1, gate_dtype=dt)
        ref = ExpertRouter.from_gguf_tensor(tm["blk.1.ffn_gate_inp.weight"], H, E, 2, gate_dtype=dt)
        assert h["router_weights"].dtype == np.float32
        assert np.array_equal(h["router_weights"], ref.gate_weights)
    assert not np.array_equal(layer_host_tensors(gf, 1)["router_weights"], r32.T)


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
              "types": {"gate": 14, "up": 14, "down": 14}, "intermediate": 512,
              "gate_inp": want["gate_inp_sh"].astype(np.float16).astype(np.float32)}
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


def near_tie_file(tmp_path, rng, E=16, H=512, I=256, k=4, a=7, b=12, top=(2, 5, 9)):
    """A layer file whose F32 ffn_gate_inp ranks expert b above expert a for
    the returned token, while the same weights rounded to FP16 rank a above b;
    a and b sit at ranks k and k+1 (the k-1 experts of ``top`` score far
    above, the rest far below), so the two storages select different sets.

    The token has x[0] = x[1] = 4; a and b share every other weight, so
    s(b) - s(a) = 4 (2^-12 - 2^-13) > 0 in FP32, while FP16 rounds row a's
    1 + 2^-11 + 2^-14 up to 1 + 2^-10 and row b's 1 + 2^-12 and
    1 + 2^-11 - 2^-14 down to 1, so s16(a) - s16(b) = 4 * 2^-10 > 0."""
    from flash_moe_hip.synthetic import random_stack

    x = rng.standard_normal(H).astype(np.float32)
    x[0] = x[1] = 4.0
    W = (rng.standard_normal((E, H)) * 0.01).astype(np.float32)
    sgn = np.sign(x).astype(np.float32)
    for e in top:
        W[e] = 0.08 * sgn + (rng.standard_normal(H) * 0.005).astype(np.float32)
        W[e, :2] = 1.0
    base = 0.05 * sgn
    W[a], W[b] = base, base
    W[a, 0], W[a, 1] = 1.0, 1.0 + 2.0 ** -11 + 2.0 ** -14
    W[b, 0], W[b, 1] = 1.0 + 2.0 ** -12, 1.0 + 2.0 ** -11 - 2.0 ** -14
    g, u, d = (random_stack(rng, t, E, *shape) for t, shape in ((12, (I, H)), (12, (I, H)), (14, (H, I))))
    sg, su, sd = (random_stack(rng, 14, 1, *shape) for shape in ((I, H), (I, H), (H, I)))
    gi = (rng.standard_normal(H) * 0.02).astype(np.float32)
    tensors = [("blk.0.ffn_gate_exps.weight", (H, I, E), 12, g.tobytes()),
               ("blk.0.ffn_up_exps.weight", (H, I, E), 12, u.tobytes()),
               ("blk.0.ffn_down_exps.weight", (I, H, E), 14, d.tobytes()),
               ("blk.0.ffn_gate_shexp.weight", (H, I), 14, sg.tobytes()),
               ("blk.0.ffn_up_shexp.weight", (H, I), 14, su.tobytes()),
               ("blk.0.ffn_down_shexp.weight", (I, H), 14, sd.tobytes()),
               ("blk.0.ffn_gate_inp_shexp.weight", (H,), 0, gi.tobytes()),
               ("blk.0.ffn_gate_inp.weight", (H, E), 0, W.tobytes())]
    path = write(tmp_path, pack_gguf([], tensors), "near_tie.gguf")
    host = {"gate": g, "up": u, "down": d}
    shared = {"gate": sg, "up": su, "down": sd, "types": {"gate": 14, "up": 14, "down": 14}, "intermediate": I,
              "gate_inp": gi.astype(np.float16).astype(np.float32)}   # as SharedExpert._load stores it
    return path, x, W, host, shared


def test_near_tie_file_flips_under_fp16_storage(tmp_path):
    """The construction above does what it says, on the host: the FP32 and the
    FP16 router of the file choose different expert sets for the token."""
    from flash_moe_hip.router import routers_from_gguf

    path, x, W, _, _ = near_tie_file(tmp_path, np.random.default_rng(31))
    tm = GGUFFile(path).tensor_map()
    r16 = routers_from_gguf(tm, 1, 512, 16, 4)[0]
    r32 = routers_from_gguf(tm, 1, 512, 16, 4, gate_dtype=np.float32)[0]
    ids16, ids32 = r16.route(x)[0], r32.route(x)[0]
    assert ids16[:3] == ids32[:3] and set(ids16[:3]) == {2, 5, 9}
    assert ids16[3] == 7 and ids32[3] == 12


@pytest.mark.gpu
def test_device_routes_a_file_layer_as_the_reference_router(tmp_path, oracle_mod, hip):
    """A GGUF layer whose F32 router gate flips a near-tie under FP16 storage:
    the device router (mqh_moe_decode_routed over the uploaded gate) selects
    exactly the experts, in the order, of the reference's default
    ExpertRouter built by routers_from_gguf (FP16 storage), not those of the
    unrounded FP32 gate; outputs within 1e-3 of the oracle's layer."""
    import torch

    from flash_moe_hip.gguf_file import load_expert_layer
    from flash_moe_hip.moe_gpu import MoeRunner
    from flash_moe_hip.router import routers_from_gguf
    from test_gpu_decode import TOL, oracle_layer

    rng = np.random.default_rng(31)
    path, x, W, host, shared = near_tie_file(tmp_path, rng)
    gf = GGUFFile(path)
    layer = load_expert_layer(gf, 0, device="cuda")
    router = routers_from_gguf(gf.tensor_map(), 1, 512, 16, 4)[0]
    X = np.stack([x] + [rng.standard_normal(512).astype(np.float32) for _ in range(2)])
    runner = MoeRunner()
    print("near-tie GGUF layer: routed decode of 3 tokens", flush=True)
    y, ids, wts = runner.decode_routed(layer, torch.from_numpy(X).cuda(), 4)
    torch.cuda.synchronize()
    assert runner.status() == 0
    y, ids, wts = y.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    assert sorted(ids[0].tolist()[:3]) == [2, 5, 9] and ids[0, 3] == 7
    for t in range(3):
        r_ids, r_w = router.route(X[t])
        assert ids[t].tolist() == r_ids, f"token {t}: device {ids[t].tolist()} reference {r_ids}"
        # the scores here reach ~40 (one FP32 ulp = 3.8e-6): the device's
        # summation order moves them by a few ulps against NumPy's, and the
        # softmax weights by ~1e-5 of their value
        np.testing.assert_allclose(wts[t], r_w, rtol=5e-5, atol=2e-6)
        ref = oracle_layer(oracle_mod, layer, host, shared, X[t], r_ids, r_w)
        err = oracle_mod.max_relative_error(y[t], ref)
        print(f"  token {t}: ids {r_ids} max rel err {err:.3e}", flush=True)
        assert err <= TOL
    assert 12 not in ids[0].tolist()
