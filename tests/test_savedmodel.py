"""SavedModel I/O without TensorFlow (annc_amd/savedmodel.py): CRC-32C,
protobuf wire format, LevelDB-format tables, tensor bundles, the graph.

Pins: CRC-32C by its published check value and the iSCSI test vectors of
RFC 3720 appendix B.4; varints and fields by the examples of the protobuf
encoding guide; the rest by round trips and by the checks the readers make
(block and tensor checksums, footer magic).  TensorFlow itself is absent, so
agreement with files TensorFlow writes is not pinned by these tests."""
import os

import numpy as np
import pytest

from annc_amd import savedmodel as sm


def test_crc32c_published_vectors():
    assert sm.crc32c(b"123456789") == 0xE3069283              # CRC-32C check value
    assert sm.crc32c(bytes(32)) == 0x8A9136AA                 # RFC 3720 B.4
    assert sm.crc32c(b"\xff" * 32) == 0x62A8AB43
    assert sm.crc32c(bytes(range(32))) == 0x46DD794E
    assert sm.crc32c(bytes(range(31, -1, -1))) == 0x113FDB5C


@pytest.mark.parametrize("n", [0, 1, 4095, 4096, 5000, 3 * 1024 + 1, 70001])
def test_crc32c_chunked_equals_serial(n):
    data = np.random.default_rng(n).integers(0, 256, size=n, dtype=np.uint8).tobytes()
    assert sm.crc32c_fast(data) == sm.crc32c(data)
    # continuation: crc of a || b from crc of a
    assert sm.crc32c(data[n // 3:], sm.crc32c(data[:n // 3])) == sm.crc32c(data)


def test_crc_mask():
    for c in (0, 1, 0xDEADBEEF, 0xFFFFFFFF):
        assert sm.unmask_crc(sm.mask_crc(c)) == c
    assert sm.mask_crc(0) == 0xA282EAD8
    assert sm.mask_crc(1) == (1 << 17) + 0xA282EAD8


def test_varints_and_fields_from_the_protobuf_guide():
    assert sm.put_varint(1) == b"\x01"
    assert sm.put_varint(150) == b"\x96\x01"
    assert sm.put_varint(300) == b"\xac\x02"
    assert sm.put_varint(-1) == b"\xff" * 9 + b"\x01"     # int64 -1: ten bytes
    assert sm.as_int64(sm.get_varint(sm.put_varint(-2), 0)[0]) == -2
    # field 1 varint 150; field 2 string "testing"
    m = sm.Msg.parse(bytes.fromhex("089601"))
    assert m.fields == [(1, sm.VARINT, 150)]
    m = sm.Msg.parse(bytes.fromhex("120774657374696e67"))
    assert m.fields == [(2, sm.LEN, b"testing")]
    assert m.serialize() == bytes.fromhex("120774657374696e67")
    with pytest.raises(ValueError):
        sm.Msg.parse(bytes.fromhex("1207746573"))   # truncated


def test_attr_values():
    for v in ("kn4", 7, -3, True, False, 1.5, sm.DType("DT_FLOAT"), sm.DType("DT_RESOURCE")):
        back = sm.decode_attr(sm.encode_attr(v))
        assert back == v and type(back) is type(v)
    assert sm.Msg.parse(sm.encode_attr(sm.DType("DT_INT64"))).fields == [(6, sm.VARINT, 9)]
    raw = sm.Msg([(1, sm.LEN, sm.Msg([(3, sm.LEN, b"\x01\x02")]))]).serialize()  # list {i: [1, 2]}
    assert sm.decode_attr(raw) == sm.RawAttr(raw) and sm.encode_attr(sm.RawAttr(raw)) == raw


def test_node_round_trip_keeps_unknown_fields():
    node = sm.GraphNode("mm", "MatMul", ["a", "b:1", "^c"],
                        {"T": sm.DType("DT_FLOAT"), "transpose_b": False}, "/device:CPU:0",
                        [(6, sm.LEN, b"\x0a\x03xyz"), (99, sm.VARINT, 5)])
    back = sm.parse_node(sm.serialize_node(node))
    assert back == node


@pytest.mark.parametrize("block", [64, 1024, 1 << 20])
def test_table_round_trip(block):
    g = np.random.default_rng(block)
    items = [(b"", b"header")] + [
        (f"layer{i // 7}/w{i:04d}".encode(), g.bytes(int(g.integers(0, 40)))) for i in range(700)]
    buf = sm.write_table(reversed(items), block_size=block)
    assert buf[-8:] == (0xDB4775248B80FB57).to_bytes(8, "little")
    assert sm.read_table(buf) == sorted(items)


def test_table_checks():
    buf = bytearray(sm.write_table([(b"a", b"b"), (b"c", b"d")]))
    with pytest.raises(ValueError, match="checksum"):
        bad = bytearray(buf)
        bad[4] ^= 1  # inside the data block
        sm.read_table(bytes(bad))
    with pytest.raises(ValueError, match="magic"):
        sm.read_table(bytes(buf[:-1]) + b"\x00")
    with pytest.raises(ValueError, match="duplicate"):
        sm.write_table([(b"a", b"1"), (b"a", b"2")])


def test_bundle_round_trip_and_checks(tmp_path):
    g = np.random.default_rng(0)
    t = {"dense/kernel": g.standard_normal((1024, 512)).astype(np.float32)[:, ::2],
         "dense/bias": g.standard_normal(256).astype(np.float64),
         "step": np.array(7, np.int64), "ids": np.arange(-5, 5, dtype=np.int32),
         "empty": np.zeros((0, 3), np.float32), "flag": np.array([True, False]),
         "h": np.ones(3, np.float16)}
    prefix = str(tmp_path / "variables" / "variables")
    sm.write_bundle(prefix, t)
    back = sm.read_bundle(prefix)
    assert sorted(back) == sorted(t)
    for k, v in t.items():
        assert back[k].dtype == v.dtype and back[k].shape == v.shape, k
        np.testing.assert_array_equal(back[k], v)
    # header: one shard, little-endian, version producer 1
    entries = dict(sm.read_table(open(prefix + ".index", "rb").read()))
    h = sm.Msg.parse(entries[b""])
    assert h.get(1) == 1 and h.get(2, 0) == 0 and sm.Msg.parse(h.get(3)).get(1) == 1
    e = sm.Msg.parse(entries[b"dense/kernel"])
    assert e.get(1) == 1 and sm.shape_of(e.get(2)) == (1024, 256)
    assert e.get(5) == 1024 * 256 * 4
    data = bytearray(open(prefix + ".data-00000-of-00001", "rb").read())
    off = e.get(4, 0)
    assert sm.unmask_crc(e.get(6)) == sm.crc32c(bytes(data[off:off + e.get(5)]))
    data[off + 100] ^= 0x40
    open(prefix + ".data-00000-of-00001", "wb").write(bytes(data))
    with pytest.raises(ValueError, match="checksum"):
        sm.read_bundle(prefix)


def test_attr_unknown_datatype_round_trips():
    """DataType values without a name here (24: a float8 type, 101: a
    reference type) decode to DType("DT_<n>") and encode to the same bytes."""
    for v in (24, 101):
        raw = sm.Msg([(6, sm.VARINT, v)]).serialize()
        d = sm.decode_attr(raw)
        assert isinstance(d, sm.DType) and d == f"DT_{v}" and d.enum == v
        assert sm.encode_attr(d) == raw
    assert sm.DType("DT_FLOAT").enum == 1 and sm.DType("DT_RESOURCE").enum == 20
    with pytest.raises(ValueError):
        sm.DType("DT_NOT_A_TYPE")


def test_bundle_keeps_string_entries(tmp_path):
    """A DT_STRING entry (a TF1 lookup table's keys) reads as OpaqueTensor and
    is written back byte for byte, its proto fields kept, beside re-encoded
    numeric tensors."""
    prefix = str(tmp_path / "variables" / "variables")
    w = np.arange(12, dtype=np.float32).reshape(3, 4)
    sm.write_bundle(prefix, {"w": w})
    index = dict(sm.read_table(open(prefix + ".index", "rb").read()))
    data = open(prefix + ".data-00000-of-00001", "rb").read()
    # TF's string tensor layout: varint lengths, then the bytes; opaque here
    raw = bytes([3, 5]) + b"abc" + b"hello"
    off = len(data)
    entry = sm.Msg([(1, sm.VARINT, 7), (2, sm.LEN, sm.shape_proto((2,))), (4, sm.VARINT, off),
                    (5, sm.VARINT, len(raw)), (6, sm.FIXED32, sm.mask_crc(sm.crc32c(raw)))])
    index[b"table/keys"] = entry.serialize()
    open(prefix + ".index", "wb").write(sm.write_table(sorted(index.items())))
    open(prefix + ".data-00000-of-00001", "wb").write(data + raw)
    back = sm.read_bundle(prefix)
    keys = back["table/keys"]
    assert isinstance(keys, sm.OpaqueTensor) and keys.dtype == "DT_STRING"
    assert keys.shape == (2,) and keys.raw == raw
    np.testing.assert_array_equal(back["w"], w)
    out = str(tmp_path / "out" / "variables")
    sm.write_bundle(out, back)
    again = sm.read_bundle(out)
    assert again["table/keys"].raw == raw and again["table/keys"].shape == (2,)
    e = sm.Msg.parse(dict(sm.read_table(open(out + ".index", "rb").read()))[b"table/keys"])
    nums = [f[0] for f in e.fields]  # field order kept; offset 0 left out (proto3)
    assert nums == sorted(nums) and 6 in nums and e.get(1) == 7 and e.get(5) == len(raw)
    np.testing.assert_array_equal(again["w"], w)


def test_saved_model_graph_round_trip(tmp_path):
    nodes = [sm.GraphNode("x", "Placeholder", [], {"dtype": sm.DType("DT_FLOAT")}),
             sm.GraphNode("w", "VariableV2", [], {"dtype": sm.DType("DT_FLOAT")}),
             sm.GraphNode("w/read", "Identity", ["w"], {"T": sm.DType("DT_FLOAT")}),
             sm.GraphNode("mm", "MatMul", ["x", "w/read"], {"transpose_b": False})]
    model = sm.new_saved_model(nodes)
    # a second meta graph under another tag, before the serving one
    other = sm.Msg([(1, sm.LEN, sm.Msg([(4, sm.LEN, b"train")]))])
    model.saved.fields.insert(1, (2, sm.LEN, other))
    model.meta_index = 1
    sm.write_saved_model(str(tmp_path), model)
    back = sm.read_saved_model(str(tmp_path))
    assert back.meta_index == 1 and sm.meta_tags(back.meta) == ["serve"]
    assert back.nodes == nodes
    assert back.serialize() == open(tmp_path / "saved_model.pb", "rb").read()
    # an edit rewrites the serving graph only
    back.nodes[3].attrs["rhs_format"] = "x"
    sm.write_saved_model(str(tmp_path), back)
    again = sm.read_saved_model(str(tmp_path))
    assert again.nodes[3].attrs["rhs_format"] == "x"
    assert again.saved.all(2)[0] == other.serialize()
