"""The GGUF reader of the C-ABI library (engine/src/gguf.rs) on synthetic
files: the reference's own parser tests (engine/tests/gguf_parse.rs), built
here with the same byte layout, plus the error cases gguf.rs rejects and the
engine's per-layer MoE tensor names (engine.rs:175-187)."""
import struct

import numpy as np
import pytest

import dsmoe
from dsmoe import gguf as G


class Builder:
    """engine/tests/gguf_parse.rs GgufBuilder: magic, version 3, counts
    inserted after them, tensor infos, data at the next 32-byte boundary."""

    def __init__(self, version=3, magic=0x46554747):
        self.buf = bytearray(struct.pack("<II", magic, version))

    def u32(self, v):
        self.buf += struct.pack("<I", v)

    def u64(self, v):
        self.buf += struct.pack("<Q", v)

    def s(self, v):
        self.u64(len(v))
        self.buf += v.encode()

    def finish_header(self, n_tensors, n_kv):
        self.buf[8:8] = struct.pack("<QQ", n_tensors, n_kv)

    def add_tensor(self, name, type_id, dims, offset):
        self.s(name)
        self.u32(len(dims))
        for d in dims:
            self.u64(d)
        self.u32(type_id)
        self.u64(offset)

    def align_data(self):
        self.buf += b"\0" * ((-len(self.buf)) % 32)
        return len(self.buf)


def parse(tmp_path, fn, name="t.gguf"):
    b = Builder()
    fn(b)
    p = tmp_path / name
    p.write_bytes(bytes(b.buf))
    return G.GgufFile(p)


def test_parse_single_f16_tensor(tmp_path):
    def fn(b):
        b.finish_header(1, 0)
        b.add_tensor("blk.0.ffn_gate_inp.weight", 1, [4096, 256], 0)
        b.align_data()
        b.buf += bytes(4096 * 256 * 2)
    g = parse(tmp_path, fn)
    ts = g.tensors
    assert len(ts) == 1
    t = ts[0].info()
    assert t == {"name": "blk.0.ffn_gate_inp.weight", "type": G.F16, "dims": [4096, 256], "offset": 0,
                 "bytes": 4096 * 256 * 2}


def test_parse_single_q8_0_tensor(tmp_path):
    def fn(b):
        b.finish_header(1, 0)
        b.add_tensor("blk.0.attn_kv.weight", 8, [4096, 512], 0)
        b.align_data()
        b.buf += bytes((4096 * 512 + 31) // 32 * 34)
    t = parse(tmp_path, fn).tensors[0].info()
    assert t["type"] == G.Q8_0 and t["dims"] == [4096, 512] and t["bytes"] == 4096 * 512 // 32 * 34


def test_parse_iq2_xxs_tensor(tmp_path):
    def fn(b):
        b.finish_header(1, 0)
        b.add_tensor("blk.0.ffn_gate_exps.weight", 16, [4096, 2048], 0)
        b.align_data()
        b.buf += bytes((4096 * 2048 + 255) // 256 * 66)
    t = parse(tmp_path, fn).tensors[0].info()
    assert t["type"] == G.IQ2_XXS and t["bytes"] == 4096 * 2048 // 256 * 66


def test_parse_multiple_tensors_with_offsets(tmp_path):
    def fn(b):
        b.finish_header(2, 0)
        b.add_tensor("tensor0", 1, [4, 8], 0)
        b.add_tensor("tensor1", 1, [8, 8], 64)
        b.align_data()
        b.buf += bytes(64 + 128)
    g = parse(tmp_path, fn)
    t0, t1 = g.tensors
    assert t0.offset == 0 and t1.offset == 64
    assert len(t0.array()) == 64 and len(t1.array()) == 128
    assert t1.data - t0.data == 64


def test_tensor_data_slice_contains_written_bytes(tmp_path):
    def fn(b):
        b.finish_header(1, 0)
        b.add_tensor("w", 1, [1, 4], 0)
        b.align_data()
        b.buf += bytes([0x00, 0x3C] * 4)  # four f16 1.0
    d = parse(tmp_path, fn).tensors[0].array()
    assert list(d) == [0x00, 0x3C] * 4
    assert np.all(d.view(np.float16) == 1.0)


def test_find_by_name(tmp_path):
    def fn(b):
        b.finish_header(2, 0)
        b.add_tensor("alpha", 0, [4], 0)
        b.add_tensor("beta", 0, [4], 16)
        b.align_data()
        b.buf += bytes(32)
    g = parse(tmp_path, fn)
    assert g.find("alpha") is not None and g.find("beta") is not None
    assert g.find("gamma") is None
    assert g.find("beta").offset == 16


def test_type_id_1_is_f16_not_q8_0(tmp_path):
    def fn(b):
        b.finish_header(1, 0)
        b.add_tensor("router", 1, [4096, 256], 0)
        b.align_data()
        b.buf += bytes(4096 * 256 * 2)
    assert parse(tmp_path, fn).tensors[0].type == G.F16


def test_metadata_is_walked_and_read(tmp_path):
    """Every metadata type gguf.rs skips, then the u32 and i32-array reads
    (read_kv_u32 / read_kv_i32_array, gguf.rs:118-188), and the data
    section at the 32-byte boundary after the tensor infos."""
    def fn(b):
        b.finish_header(1, 14)
        for key, vt, payload in [("a.u8", 0, b"\x01"), ("a.i8", 1, b"\xff"), ("a.u16", 2, b"\x01\x00"),
                                 ("a.i16", 3, b"\xff\xff"), ("a.f32", 6, struct.pack("<f", 1.5)),
                                 ("a.bool", 7, b"\x01"), ("a.u64", 10, struct.pack("<Q", 7)),
                                 ("a.i64", 11, struct.pack("<q", -7)), ("a.f64", 12, struct.pack("<d", 2.5)),
                                 ("a.str", 8, struct.pack("<Q", 3) + b"abc"),
                                 ("a.strs", 9, struct.pack("<IQ", 8, 2) + struct.pack("<Q", 1) + b"x"
                                  + struct.pack("<Q", 2) + b"yz"),
                                 ("n.layers", 4, struct.pack("<I", 43)),
                                 ("tid2eid", 9, struct.pack("<IQ", 5, 3) + struct.pack("<3i", 5, -1, 7)),
                                 ("a.i32", 5, struct.pack("<i", -3))]:
            b.s(key)
            b.u32(vt)
            b.buf += payload
        b.add_tensor("w", 0, [3], 0)
        b.align_data()
        b.buf += struct.pack("<3f", 1.0, 2.0, 3.0)
    g = parse(tmp_path, fn)
    assert g.read_kv_u32("n.layers") == 43
    assert g.read_kv_u32("a.i32") is None  # another type
    assert g.read_kv_u32("missing") is None
    assert g.read_kv_i32_array("tid2eid") == [5, -1, 7]
    assert g.read_kv_i32_array("a.strs") == []
    assert g.data_offset % 32 == 0
    assert list(g.tensors[0].array().view(np.float32)) == [1.0, 2.0, 3.0]


@pytest.mark.parametrize("case,msg", [("magic", "bad magic"), ("version", "unsupported GGUF version 4"),
                                      ("type", "unknown tensor type 2"), ("kv", "unknown GGUF metadata type 13"),
                                      ("short", "past the end"), ("trunc", "truncated"),
                                      ("dims", "beyond 64 bits"), ("offset", "past the end"),
                                      ("bytes", "past the end")])
def test_rejected_files(tmp_path, case, msg):
    b = Builder(version=4 if case == "version" else 3, magic=0x12345678 if case == "magic" else 0x46554747)
    if case == "kv":
        b.finish_header(0, 1)
        b.s("k")
        b.u32(13)
        b.buf += bytes(8)
    elif case == "trunc":
        b.finish_header(1, 0)
        b.s("w")
        b.u32(2)
        b.buf += bytes(4)  # dims cut short; the file ends inside the tensor info
        b.buf += bytes(16)
    elif case in ("dims", "offset", "bytes"):
        # a dims product past 2^64, an offset near 2^64, a byte size past 2^64
        # (2^62 f32 elements): each would wrap an unchecked end test
        b.finish_header(1, 0)
        dims = {"dims": [1 << 33, 1 << 32], "offset": [64], "bytes": [1 << 62]}[case]
        b.add_tensor("w", 0, dims, (1 << 64) - 64 if case == "offset" else 0)
        b.align_data()
        b.buf += bytes(256)
    else:
        b.finish_header(1, 0)
        b.add_tensor("w", 2 if case == "type" else 0, [64], 0)
        b.align_data()
        b.buf += bytes(64 if case == "short" else 256)
    p = tmp_path / "bad.gguf"
    p.write_bytes(bytes(b.buf))
    with pytest.raises(dsmoe.DsmoeError) as ei:
        G.GgufFile(p)
    assert msg in str(ei.value)


def test_moe_layer_round_trip(tmp_path):
    """A synthetic MoE layer written as GGUF (the engine's tensor names) and
    read back through dsmoe_gguf_moe_layer: every tensor's bytes equal."""
    from dsmoe import configs as C
    case = C.CASES["c1"]
    w = C.make_weights(case, device="cpu")
    tensors = G.moe_layer_tensors(case.cfg, w, layer=3)
    p = tmp_path / "layer.gguf"
    G.write(p, tensors, kv={"general.architecture": "deepseek4", "deepseek4.block_count": 43})
    with G.GgufFile(p) as g:
        assert g.read_kv_u32("deepseek4.block_count") == 43
        t = g.moe_layer(3)
        assert set(t) == {n for n in G.MOE_TENSORS[:8]}
        for name, ty, dims, data in tensors:
            got = t[name.split(".", 2)[2]]
            assert got.type == ty and list(got.dims[:got.n_dims]) == dims
            assert got.bytes == len(data)
            assert np.array_equal(got.array(), np.asarray(data, np.uint8))
        assert g.moe_layer(2) == {}


@pytest.mark.parametrize("fault", ["router_type", "expert_dims", "missing_shared"])
def test_layer_weights_checks_types_and_dims(tmp_path, fault):
    """layer_weights refuses a layer whose tensors do not have the type and
    dims the kernels read: a router written as F32, experts with another
    intermediate size, a missing shared expert tensor."""
    from dsmoe import configs as C
    case = C.CASES["c1"]
    cfg = case.cfg
    w = C.make_weights(case, device="cpu")
    tensors = G.moe_layer_tensors(cfg, w, layer=0)
    out = []
    for name, ty, dims, data in tensors:
        if fault == "router_type" and name.endswith("ffn_gate_inp.weight"):
            ty, data = G.F32, np.zeros(dims[0] * dims[1], np.float32).view(np.uint8)
        if fault == "expert_dims" and name.endswith("ffn_gate_exps.weight"):
            dims = [dims[0], dims[1] - 256, dims[2]]
            data = data[:len(data) * dims[1] // (dims[1] + 256)]
        if fault == "missing_shared" and name.endswith("ffn_down_shexp.weight"):
            continue
        out.append((name, ty, dims, data))
    p = tmp_path / "bad_layer.gguf"
    G.write(p, out)
    with G.GgufFile(p) as g:
        with pytest.raises(ValueError) as ei:
            G.layer_weights(g, 0, cfg, device="cpu")
    want = {"router_type": "ffn_gate_inp.weight: type 0", "expert_dims": "ffn_gate_exps.weight: type",
            "missing_shared": "ffn_down_shexp.weight: missing"}[fault]
    assert want in str(ei.value)
    G.write(p, tensors)
    with G.GgufFile(p) as g:
        lw = G.layer_weights(g, 0, cfg, device="cpu")
    assert lw.gate.numel() == w.gate.numel()
