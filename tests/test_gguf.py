"""GGUF directory parser (uq_gguf_*) on the CPU: the rules and error
categories of Shard::parse (frontier_gguf.rs:145-200) and its tests
(frontier_gguf.rs:238-262). The reference's fixture headers
(reference/q3-metadata.gguf, shard2/3-header.gguf) are not part of the
reference tree available here; its synthetic-directory cases are restated
exactly, and every other rule gets a constructed case."""
import struct

import numpy as np
import pytest

import uq
import gguf_writer as W

U64_MAX = (1 << 64) - 1


def err(prefix, logical):
    with pytest.raises(uq.GgufError) as e:
        uq.Gguf.parse(prefix, logical)
    assert e.value.status == uq.Error.FORMAT
    return e.value.gguf_error


def test_reference_malformed_ranges():
    # frontier_gguf.rs:255-262
    assert err(W.synthetic([0, 32], 32), 10000) == "Overlap"
    assert err(W.synthetic([1], 32), 10000) == "Alignment"
    assert err(W.synthetic([U64_MAX - 31], 32), U64_MAX) == "Overflow"
    assert err(W.synthetic([0], U64_MAX - 31), U64_MAX) == "Overflow"
    assert err(W.synthetic([0], 33), 10000) == "Shape"
    g = uq.Gguf.parse(W.synthetic([0, 96], 32), 10000)
    ts = g.tensors()
    assert [t["bytes"] for t in ts] == [68, 68]
    assert ts[1]["offset"] - ts[0]["offset"] == 96
    assert g.data_offset % 32 == 0 and ts[0]["offset"] == g.data_offset


def sample_file():
    meta = [("general.architecture", W.STRING, "qwen2"), ("a.u8", W.U8, 7), ("a.u16", W.U16, 700),
            ("a.u32", W.U32, 70000), ("a.u64", W.U64, 7 << 40), ("a.f32", W.F32, 1e-6), ("a.bool", W.BOOL, True),
            ("a.i64", W.I64, -5), ("a.f64", W.F64, 2.5),
            ("a.arr", W.ARRAY, (W.U32, [1, 2, 3])), ("a.strs", W.ARRAY, (W.STRING, ["x", "yy", "zzz"]))]
    q = np.arange(2 * 34, dtype=np.uint8).tobytes()
    f = np.arange(8, dtype=np.float32).tobytes()
    return W.write(meta, [("w", [32, 2], 8, q), ("v", [8], 0, f)])


def test_metadata_and_tensor_directory():
    data, dlen = sample_file()
    g = uq.Gguf.parse(data, len(data))
    assert g.string("general.architecture") == "qwen2"
    assert (g.u64("a.u8"), g.u64("a.u16"), g.u64("a.u32"), g.u64("a.u64")) == (7, 700, 70000, 7 << 40)
    assert g.f32("a.f32") == np.float32(1e-6)
    assert g.array("a.arr") == (W.U32, 3) and g.array("a.strs") == (W.STRING, 3)
    with pytest.raises(uq.UqError):
        g.u64("a.i64")          # Value::unsigned takes u8/u16/u32/u64 only
    with pytest.raises(uq.UqError):
        g.f32("a.f64")
    with pytest.raises(uq.UqError):
        g.u64("absent")
    assert g.data_offset == dlen
    ts = g.tensors()
    assert [t["name"] for t in ts] == ["w", "v"]
    assert ts[0] == {"name": "w", "kind": 8, "dims": [32, 2], "offset": dlen, "bytes": 68}
    assert ts[1] == {"name": "v", "kind": 0, "dims": [8], "offset": dlen + 96, "bytes": 32}
    assert g.find("v") == 1 and g.find("nope") == -1
    assert g.split() == (0, 1, 2)


def test_every_short_prefix_is_truncated():
    data, dlen = sample_file()
    for n in list(range(0, 40)) + list(range(40, dlen, 7)):
        assert err(data[:n], len(data)) in ("Truncated", "Magic") if n < 4 else err(data[:n], len(data)) == "Truncated"


def test_header_rules():
    data, _ = sample_file()
    bad = bytearray(data); bad[0] = ord("X")
    assert err(bytes(bad), len(data)) == "Magic"
    bad = bytearray(data); bad[4] = 2                      # frontier_gguf.rs:243-244
    assert err(bytes(bad), len(data)) == "Version"
    bad = bytearray(data); bad[8:16] = struct.pack("<Q", U64_MAX)   # frontier_gguf.rs:241-242
    assert err(bytes(bad), len(data)) == "Limit"
    assert err(W.directory([], [], n_kv=1025), 10000) == "Limit"
    assert err(W.directory([], [], n_tensors=4097), 10000) == "Limit"
    assert err(data, 100) == "TensorBounds"               # file shorter than the data section


def test_key_name_type_and_utf8_rules():
    assert err(W.directory([("k", W.U8, 1), ("k", W.U8, 2)], []), 10000) == "Duplicate"
    assert err(W.directory([("k" * 257, W.U8, 1)], []), 10000) == "Limit"
    assert err(W.directory([], [("t", [32], 8, 0), ("t", [32], 8, 64)]), 10000) == "Duplicate"
    assert err(W.directory([], [("t" * 257, [32], 8, 0)]), 10000) == "Limit"
    assert err(W.directory([], [("t", [], 8, 0)]), 10000) == "Shape"
    assert err(W.directory([], [("t", [32, 1, 1, 1, 1], 8, 0)]), 10000) == "Shape"
    assert err(W.directory([], [("t", [32, 0], 8, 0)]), 10000) == "Shape"
    assert err(W.directory([], [("t", [32], 99, 0)]), 10000) == "Type"
    unknown = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W.gstr("k") + struct.pack("<I", 13) + bytes(8)
    assert err(unknown, 10000) == "Type"
    nested = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W.gstr("k") + struct.pack("<I", W.ARRAY)
    nested += struct.pack("<IQ", W.ARRAY, 1) + struct.pack("<IQ", W.U8, 0)
    assert err(nested, 10000) == "Type"
    big = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W.gstr("k") + struct.pack("<IIQ", W.ARRAY, W.U8, 1000001)
    assert err(big, 10000) == "Limit"
    assert err(W.directory([("k", W.STRING, b"\xff\xfe")], []), 10000) == "Utf8"


def test_alignment_and_split_rules():
    ok = W.directory([("general.alignment", W.U32, 64)], [("t", [32], 8, 64)])
    g = uq.Gguf.parse(ok, 10000)
    assert g.data_offset % 64 == 0
    assert err(W.directory([("general.alignment", W.U32, 64)], [("t", [32], 8, 32)]), 10000) == "Alignment"
    assert err(W.directory([("general.alignment", W.U32, 48)], []), 10000) == "Alignment"
    assert err(W.directory([("general.alignment", W.U32, 8192)], []), 10000) == "Alignment"
    assert err(W.directory([("split.count", W.U16, 0)], []), 10000) == "Split"
    assert err(W.directory([("split.no", W.U16, 3), ("split.count", W.U16, 3)], []), 10000) == "Split"
    assert err(W.directory([("split.tensors.count", W.I32, -1)], []), 10000) == "Split"
    assert err(W.directory([("split.tensors.count", W.I32, 0)], [("t", [32], 8, 0)]), 10000) == "Split"
    g = uq.Gguf.parse(W.directory([("split.no", W.U16, 1), ("split.count", W.U16, 3),
                                   ("split.tensors.count", W.I32, 1224)], []), 10000)
    assert g.split() == (1, 3, 1224)


def test_row_bytes_of_reference_kinds():
    # frontier_core.rs:129-132: row_bytes(20,160)=90, (18,2560)=980, (23,640) -> Shape
    for kind, width, rb in ((20, 160, 90), (18, 2560, 980), (8, 1536, 1632), (14, 256, 210), (30, 3, 6),
                            (0, 5, 20), (11, 512, 220), (12, 256, 144)):
        g = uq.Gguf.parse(W.directory([], [("t", [width, 3], kind, 0)]), 1 << 20)
        assert g.tensors()[0]["bytes"] == 3 * rb
    assert err(W.directory([], [("t", [640], 23, 0)]), 1 << 20) == "Shape"


def test_qwen2_config_from_metadata(tmp_path):
    cfg = dict(layers=2, dim=256, hidden=512, heads=4, kv_heads=2, head_dim=64, vocab=1024, max_seq=128,
               eps=1e-6, theta=1e6)
    tensors = uq.synth_qwen2(cfg, 0x5EED0099)
    data, _ = W.qwen2_file(cfg, tensors)
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    g = uq.Gguf.open(str(p))
    got = g.qwen2_config(64)
    want = dict(cfg, max_seq=64)
    assert {k: got[k] for k in want if k not in ("eps", "theta")} == {k: v for k, v in want.items() if k not in ("eps", "theta")}
    assert got["eps"] == np.float32(1e-6) and got["theta"] == np.float32(1e6)
    assert g.qwen2_config(0)["max_seq"] == 128
    # tensor bytes in the file are the GGUF bytes that were written
    t = g.tensors()[g.find("blk.1.ffn_down.weight")]
    kind, n, rows, arr = tensors["blk.1.ffn_down.weight"]
    assert t["dims"] == [n, rows] and data[t["offset"]:t["offset"] + t["bytes"]] == arr.tobytes()
    bad = data.replace(b"qwen2", b"llama", 1)
    p.write_bytes(bad)
    with pytest.raises(uq.UqError):
        uq.Gguf.open(str(p)).qwen2_config(64)
