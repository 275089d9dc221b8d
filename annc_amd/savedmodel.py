"""TensorFlow SavedModel I/O without TensorFlow: the graph (saved_model.pb)
and the variables (variables/variables.index + .data-00000-of-00001), enough
for annc-opt's passes to read a model, rewrite nodes and variables, and write
a model TensorFlow loads.

The reference tool goes through TensorFlow (python/annc/optimize/graph.py:
300-338 reads saved_model.pb, constant_folding.py:43-59 saves the variables
with tf.compat.v1.train.Saver).  Here the formats are handled directly:

  * Protocol-buffer wire format (varints, length-delimited fields, fixed32 /
    fixed64).  Messages are kept as ordered field lists, so the SavedModel,
    meta graph and graph fields around the nodes are written back byte for
    byte, and fields this module does not name survive a rewrite; the nodes
    themselves are re-encoded (attrs in key order, as TensorFlow writes them).  Field numbers follow TensorFlow's .proto files:
    SavedModel {1 schema version, 2 meta_graphs}; MetaGraphDef {1
    meta_info_def (4 tags), 2 graph_def, ...}; GraphDef {1 node, ...};
    NodeDef {1 name, 2 op, 3 input, 4 device, 5 attr map}; AttrValue {1
    list, 2 s, 3 i, 4 f, 5 b, 6 type, 7 shape, 8 tensor, ...}.
  * The tensor bundle: a LevelDB-format table (the sstable of
    tensorflow/core/lib/io/table*.cc, LevelDB's doc/table_format.md: data
    blocks of prefix-compressed entries with restart points, a trailer of
    compression type and masked CRC-32C per block, an index block, an empty
    metaindex block and a 48-byte footer ending in the magic
    0xdb4775248b80fb57) mapping "" to a BundleHeaderProto {1 num_shards, 2
    endianness, 3 version} and each tensor name to a BundleEntryProto {1
    dtype, 2 shape, 3 shard_id, 4 offset, 5 size, 6 masked crc32c of the
    bytes}; the tensor bytes sit in the data shard at those offsets.
  * CRC-32C (Castagnoli, reflected polynomial 0x82F63B78) and LevelDB's
    mask, ((crc >> 15) | (crc << 17)) + 0xa282ead8.

Variables are looked up by node name, the key tf.compat.v1.train.Saver gives
a graph variable; numeric dtypes only.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field
from typing import Dict, Iterable, List, Optional, Tuple, Union

import numpy as np

# ---------------------------------------------------------------------------
# CRC-32C
# ---------------------------------------------------------------------------
_CRC_POLY = 0x82F63B78
_CRC_TABLE = []
for _b in range(256):
    _c = _b
    for _ in range(8):
        _c = (_c >> 1) ^ (_CRC_POLY if _c & 1 else 0)
    _CRC_TABLE.append(_c)
_CRC_NP = np.array(_CRC_TABLE, dtype=np.uint32)
_MASK_DELTA = 0xA282EAD8


def crc32c(data: bytes, crc: int = 0) -> int:
    """CRC-32C of `data` (continuing from `crc`)."""
    c = crc ^ 0xFFFFFFFF
    tab = _CRC_TABLE
    for b in memoryview(bytes(data)):
        c = tab[(c ^ b) & 0xFF] ^ (c >> 8)
    return c ^ 0xFFFFFFFF


_CHUNK = 1024
_SHIFT: List[int] = []  # register after _CHUNK zero bytes, from each one-bit register


def _zero_shift_table() -> List[int]:
    if not _SHIFT:
        for bit in range(32):
            c = 1 << bit
            for _ in range(_CHUNK):
                c = _CRC_TABLE[c & 0xFF] ^ (c >> 8)
            _SHIFT.append(c)
    return _SHIFT


def crc32c_fast(data: bytes) -> int:
    """crc32c() of large buffers.  The byte update is linear over GF(2) in
    the register and the byte, so the register after chunk B from start x is
    crc(B from 0) xor crc(zeros from x): the chunks' own CRCs are computed
    together by numpy (one table lookup per byte column), then chained with
    the zero-shift map of a chunk, built from its 32 one-bit images."""
    data = bytes(data)
    nchunk = len(data) // _CHUNK
    if nchunk < 4:
        return crc32c(data)
    cols = np.frombuffer(data, dtype=np.uint8)[:nchunk * _CHUNK].reshape(nchunk, _CHUNK)
    reg = np.zeros(nchunk, dtype=np.uint32)
    for j in range(_CHUNK):
        reg = _CRC_NP[(reg ^ cols[:, j]) & 0xFF] ^ (reg >> 8)
    shift = _zero_shift_table()
    c = 0xFFFFFFFF
    for r in reg.tolist():
        s, x = 0, c
        while x:
            low = x & -x
            s ^= shift[low.bit_length() - 1]
            x ^= low
        c = s ^ r
    return crc32c(data[nchunk * _CHUNK:], c ^ 0xFFFFFFFF)


def mask_crc(crc: int) -> int:
    """LevelDB's stored form of a CRC (so a CRC of data holding CRCs differs)."""
    return ((((crc >> 15) | (crc << 17)) & 0xFFFFFFFF) + _MASK_DELTA) & 0xFFFFFFFF


def unmask_crc(masked: int) -> int:
    rot = (masked - _MASK_DELTA) & 0xFFFFFFFF
    return ((rot >> 17) | (rot << 15)) & 0xFFFFFFFF


# ---------------------------------------------------------------------------
# Protocol-buffer wire format
# ---------------------------------------------------------------------------
VARINT, FIXED64, LEN, FIXED32 = 0, 1, 2, 5


def put_varint(v: int) -> bytes:
    if v < 0:
        v &= (1 << 64) - 1  # negative int64: ten-byte two's complement
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def get_varint(buf: bytes, pos: int) -> Tuple[int, int]:
    shift = result = 0
    while True:
        if pos >= len(buf):
            raise ValueError("truncated varint")
        b = buf[pos]
        pos += 1
        result |= (b & 0x7F) << shift
        if not b & 0x80:
            return result, pos
        shift += 7
        if shift > 63:
            raise ValueError("varint too long")


def as_int64(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


@dataclass
class Msg:
    """A message as its ordered (field number, wire type, value) list; LEN
    values are bytes (sub-messages are parsed on demand)."""
    fields: List[Tuple[int, int, object]] = field(default_factory=list)

    @staticmethod
    def parse(buf: bytes) -> "Msg":
        out, pos, n = [], 0, len(buf)
        while pos < n:
            key, pos = get_varint(buf, pos)
            num, wt = key >> 3, key & 7
            if wt == VARINT:
                v, pos = get_varint(buf, pos)
            elif wt == FIXED64:
                v = struct.unpack_from("<Q", buf, pos)[0]
                pos += 8
            elif wt == FIXED32:
                v = struct.unpack_from("<I", buf, pos)[0]
                pos += 4
            elif wt == LEN:
                ln, pos = get_varint(buf, pos)
                if pos + ln > n:
                    raise ValueError("truncated length-delimited field")
                v = bytes(buf[pos:pos + ln])
                pos += ln
            else:
                raise ValueError(f"unsupported wire type {wt}")
            out.append((num, wt, v))
        return Msg(out)

    def serialize(self) -> bytes:
        out = bytearray()
        for num, wt, v in self.fields:
            out += put_varint((num << 3) | wt)
            if wt == VARINT:
                out += put_varint(int(v))
            elif wt == FIXED64:
                out += struct.pack("<Q", int(v))
            elif wt == FIXED32:
                out += struct.pack("<I", int(v))
            else:
                b = v.serialize() if isinstance(v, Msg) else bytes(v)
                out += put_varint(len(b)) + b
        return bytes(out)

    def get(self, num: int, default=None):
        for n, _, v in self.fields:
            if n == num:
                return v
        return default

    def all(self, num: int) -> list:
        return [v for n, _, v in self.fields if n == num]

    def add(self, num: int, wt: int, v) -> None:
        self.fields.append((num, wt, v))


# ---------------------------------------------------------------------------
# DataType (types.proto) and numpy
# ---------------------------------------------------------------------------
DTYPES = {
    "DT_INVALID": 0, "DT_FLOAT": 1, "DT_DOUBLE": 2, "DT_INT32": 3, "DT_UINT8": 4,
    "DT_INT16": 5, "DT_INT8": 6, "DT_STRING": 7, "DT_COMPLEX64": 8, "DT_INT64": 9,
    "DT_BOOL": 10, "DT_QINT8": 11, "DT_QUINT8": 12, "DT_QINT32": 13, "DT_BFLOAT16": 14,
    "DT_QINT16": 15, "DT_QUINT16": 16, "DT_UINT16": 17, "DT_COMPLEX128": 18,
    "DT_HALF": 19, "DT_RESOURCE": 20, "DT_VARIANT": 21, "DT_UINT32": 22, "DT_UINT64": 23,
}
DTYPE_NAMES = {v: k for k, v in DTYPES.items()}
_NP_OF = {1: np.float32, 2: np.float64, 3: np.int32, 4: np.uint8, 5: np.int16, 6: np.int8,
          9: np.int64, 10: np.bool_, 17: np.uint16, 19: np.float16, 22: np.uint32,
          23: np.uint64}
_DT_OF = {np.dtype(v): k for k, v in _NP_OF.items()}


class DType(str):
    """A `type` attr value ("DT_FLOAT"), kept apart from string attrs.
    `enum` is its DataType number, kept for values this module has no name
    for (float8, int4, the reference types 101+), which then round-trip as
    "DT_<number>"."""

    def __new__(cls, name: str, enum: Optional[int] = None):
        obj = super().__new__(cls, name)
        if enum is None:
            if name in DTYPES:
                enum = DTYPES[name]
            elif name.startswith("DT_") and name[3:].isdigit():
                enum = int(name[3:])
            else:
                raise ValueError(f"unknown DataType {name!r}")
        obj.enum = int(enum)
        return obj


@dataclass
class RawAttr:
    """An AttrValue this module does not interpret, kept as its bytes."""
    data: bytes


def decode_attr(buf: bytes):
    """AttrValue -> str (s), int (i), float (f), bool (b), DType (type), or
    RawAttr for lists, shapes, tensors, functions and placeholders."""
    m = Msg.parse(buf)
    if len(m.fields) == 1:
        num, wt, v = m.fields[0]
        if num == 2 and wt == LEN:
            try:
                return bytes(v).decode("utf-8")
            except UnicodeDecodeError:
                return RawAttr(buf)
        if num == 3 and wt == VARINT:
            return as_int64(v)
        if num == 4 and wt == FIXED32:
            return struct.unpack("<f", struct.pack("<I", v))[0]
        if num == 5 and wt == VARINT:
            return bool(v)
        if num == 6 and wt == VARINT:
            return DType(DTYPE_NAMES.get(v, f"DT_{v}"), v)
    return RawAttr(buf)


def encode_attr(value) -> bytes:
    m = Msg()
    if isinstance(value, RawAttr):
        return value.data
    if isinstance(value, DType):
        m.add(6, VARINT, value.enum)
    elif isinstance(value, bool):
        m.add(5, VARINT, int(value))
    elif isinstance(value, int):
        m.add(3, VARINT, value)
    elif isinstance(value, float):
        m.add(4, FIXED32, struct.unpack("<I", struct.pack("<f", value))[0])
    elif isinstance(value, str):
        m.add(2, LEN, value.encode("utf-8"))
    else:
        raise TypeError(f"cannot encode attr value {value!r}")
    return m.serialize()


def shape_proto(shape: Iterable[int]) -> Msg:
    """TensorShapeProto {2: Dim {1: size}}."""
    m = Msg()
    for d in shape:
        m.add(2, LEN, Msg([(1, VARINT, int(d))]))
    return m


def shape_of(buf: bytes) -> Tuple[int, ...]:
    m = Msg.parse(buf)
    if m.get(3):
        raise ValueError("unknown-rank shape")
    return tuple(as_int64(Msg.parse(d).get(1, 0)) for d in m.all(2))


# ---------------------------------------------------------------------------
# GraphDef nodes
# ---------------------------------------------------------------------------
@dataclass
class GraphNode:
    name: str
    op: str
    inputs: List[str]
    attrs: Dict[str, object]
    device: str = ""
    extra: List[Tuple[int, int, object]] = field(default_factory=list)  # other NodeDef fields


def parse_node(buf: bytes) -> GraphNode:
    m = Msg.parse(buf)
    name = op = device = ""
    inputs: List[str] = []
    attrs: Dict[str, object] = {}
    extra = []
    for num, wt, v in m.fields:
        if num == 1:
            name = v.decode()
        elif num == 2:
            op = v.decode()
        elif num == 3:
            inputs.append(v.decode())
        elif num == 4:
            device = v.decode()
        elif num == 5:
            entry = Msg.parse(v)
            attrs[entry.get(1, b"").decode()] = decode_attr(entry.get(2, b""))
        else:
            extra.append((num, wt, v))
    return GraphNode(name, op, inputs, attrs, device, extra)


def serialize_node(node: GraphNode) -> bytes:
    m = Msg()
    m.add(1, LEN, node.name.encode())
    m.add(2, LEN, node.op.encode())
    for inp in node.inputs:
        m.add(3, LEN, inp.encode())
    if node.device:
        m.add(4, LEN, node.device.encode())
    for key in sorted(node.attrs):  # TensorFlow writes its attr map sorted by key
        m.add(5, LEN, Msg([(1, LEN, key.encode()), (2, LEN, encode_attr(node.attrs[key]))]))
    for f in node.extra:
        m.add(*f)
    return m.serialize()


@dataclass
class SavedModelGraph:
    """saved_model.pb with the graph of one meta graph unpacked into nodes."""
    saved: Msg
    meta_index: int  # which meta_graphs entry (field 2) holds the graph
    meta: Msg
    graph: Msg
    nodes: List[GraphNode]

    def serialize(self) -> bytes:
        graph = Msg([f for f in self.graph.fields if f[0] != 1])
        node_fields = [(1, LEN, serialize_node(n)) for n in self.nodes]
        graph.fields = node_fields + graph.fields  # nodes first, as TensorFlow writes them
        meta = Msg([(n, wt, graph if n == 2 else v) for n, wt, v in self.meta.fields])
        if meta.get(2) is None:
            meta.add(2, LEN, graph)
        out, k = Msg(), 0
        for n, wt, v in self.saved.fields:
            if n == 2:
                out.add(n, wt, meta if k == self.meta_index else v)
                k += 1
            else:
                out.add(n, wt, v)
        return out.serialize()


def meta_tags(meta: Msg) -> List[str]:
    info = meta.get(1)
    return [t.decode() for t in Msg.parse(info).all(4)] if info is not None else []


def read_saved_model(path: str, tag: str = "serve") -> SavedModelGraph:
    """The graph of the meta graph tagged `tag` (the first one if none is)."""
    with open(os.path.join(path, "saved_model.pb"), "rb") as f:
        saved = Msg.parse(f.read())
    metas = saved.all(2)
    if not metas:
        raise ValueError(f"{path}: saved_model.pb holds no meta graph")
    parsed = [Msg.parse(m) for m in metas]
    idx = next((i for i, m in enumerate(parsed) if tag in meta_tags(m)), 0)
    meta = parsed[idx]
    gbuf = meta.get(2)
    graph = Msg.parse(gbuf) if gbuf is not None else Msg()
    nodes = [parse_node(b) for b in graph.all(1)]
    return SavedModelGraph(saved, idx, meta, graph, nodes)


def write_saved_model(path: str, model: SavedModelGraph) -> None:
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "saved_model.pb"), "wb") as f:
        f.write(model.serialize())


def new_saved_model(nodes: List[GraphNode], tags: Tuple[str, ...] = ("serve",),
                    producer: int = 1286) -> SavedModelGraph:
    """A one-meta-graph SavedModel around `nodes` (GraphDef versions
    {1 producer})."""
    graph = Msg([(4, LEN, Msg([(1, VARINT, producer)]))])
    info = Msg([(4, LEN, t.encode()) for t in tags])
    meta = Msg([(1, LEN, info), (2, LEN, graph)])
    saved = Msg([(1, VARINT, 1), (2, LEN, meta)])
    return SavedModelGraph(saved, 0, meta, graph, list(nodes))


# ---------------------------------------------------------------------------
# LevelDB-format table
# ---------------------------------------------------------------------------
TABLE_MAGIC = 0xDB4775248B80FB57
FOOTER_LEN = 48
BLOCK_TRAILER = 5
RESTART_INTERVAL = 16


def _block(entries: List[Tuple[bytes, bytes]]) -> bytes:
    out = bytearray()
    restarts = []
    prev = b""
    for i, (k, v) in enumerate(entries):
        if i % RESTART_INTERVAL == 0:
            restarts.append(len(out))
            shared = 0
        else:
            shared = 0
            lim = min(len(prev), len(k))
            while shared < lim and prev[shared] == k[shared]:
                shared += 1
        out += put_varint(shared) + put_varint(len(k) - shared) + put_varint(len(v))
        out += k[shared:] + v
        prev = k
    if not restarts:
        restarts = [0]
    for r in restarts:
        out += struct.pack("<I", r)
    out += struct.pack("<I", len(restarts))
    return bytes(out)


def _handle(offset: int, size: int) -> bytes:
    return put_varint(offset) + put_varint(size)


def write_table(items: Iterable[Tuple[bytes, bytes]], block_size: int = 4096) -> bytes:
    """Keys must be unique; they are written in bytewise order."""
    items = sorted(items, key=lambda kv: kv[0])
    for a, b in zip(items, items[1:]):
        if a[0] == b[0]:
            raise ValueError(f"duplicate key {a[0]!r}")
    out = bytearray()
    index: List[Tuple[bytes, bytes]] = []

    def emit(block: bytes) -> Tuple[int, int]:
        off = len(out)
        out.extend(block)
        trailer_type = b"\x00"  # no compression
        out.extend(trailer_type)
        out.extend(struct.pack("<I", mask_crc(crc32c(block + trailer_type))))
        return off, len(block)

    cur: List[Tuple[bytes, bytes]] = []
    size = 0
    for k, v in items:
        cur.append((k, v))
        size += len(k) + len(v) + 8
        if size >= block_size:
            off, ln = emit(_block(cur))
            index.append((cur[-1][0], _handle(off, ln)))  # the block's last key separates it
            cur, size = [], 0
    if cur:
        off, ln = emit(_block(cur))
        index.append((cur[-1][0], _handle(off, ln)))
    meta_off, meta_len = emit(_block([]))
    idx_off, idx_len = emit(_block(index))
    footer = _handle(meta_off, meta_len) + _handle(idx_off, idx_len)
    footer += b"\x00" * (40 - len(footer)) + struct.pack("<Q", TABLE_MAGIC)
    out.extend(footer)
    return bytes(out)


def _read_block(buf: bytes, handle: bytes, pos: int = 0, verify: bool = True) -> bytes:
    off, pos = get_varint(handle, pos)
    size, pos = get_varint(handle, pos)
    block = buf[off:off + size]
    if verify:
        kind = buf[off + size:off + size + 1]
        crc = struct.unpack_from("<I", buf, off + size + 1)[0]
        if kind != b"\x00":
            raise ValueError("compressed table blocks are not supported")
        if unmask_crc(crc) != crc32c(bytes(block) + kind):
            raise ValueError("table block checksum mismatch")
    return bytes(block)


def _block_entries(block: bytes) -> List[Tuple[bytes, bytes]]:
    if len(block) < 4:
        raise ValueError("table block too short")
    nrest = struct.unpack_from("<I", block, len(block) - 4)[0]
    end = len(block) - 4 - 4 * nrest
    out, pos, prev = [], 0, b""
    while pos < end:
        shared, pos = get_varint(block, pos)
        unshared, pos = get_varint(block, pos)
        vlen, pos = get_varint(block, pos)
        key = prev[:shared] + block[pos:pos + unshared]
        pos += unshared
        out.append((key, block[pos:pos + vlen]))
        pos += vlen
        prev = key
    return out


def read_table(buf: bytes) -> List[Tuple[bytes, bytes]]:
    if len(buf) < FOOTER_LEN or struct.unpack_from("<Q", buf, len(buf) - 8)[0] != TABLE_MAGIC:
        raise ValueError("not a table file (bad footer magic)")
    footer = buf[len(buf) - FOOTER_LEN:]
    _, pos = get_varint(footer, 0)
    _, pos = get_varint(footer, pos)  # metaindex handle (unused)
    index = _block_entries(_read_block(buf, footer, pos))
    out = []
    for _, handle in index:
        out.extend(_block_entries(_read_block(buf, handle)))
    return out


# ---------------------------------------------------------------------------
# Tensor bundle (variables/variables.index + .data-00000-of-00001)
# ---------------------------------------------------------------------------
def bundle_paths(prefix: str) -> Tuple[str, str]:
    return prefix + ".index", prefix + ".data-00000-of-00001"


@dataclass
class OpaqueTensor:
    """A bundle entry this module does not decode (strings, resources,
    quantized types): its BundleEntryProto and data bytes, written back
    unchanged.  `dtype` is the DataType name, `shape` the dims."""
    entry: bytes
    raw: bytes
    dtype: str
    shape: Tuple[int, ...]

    @property
    def ndim(self) -> int:
        return len(self.shape)


def read_bundle(prefix: str) -> Dict[str, Union[np.ndarray, OpaqueTensor]]:
    """name -> array of every numeric tensor of a one-shard little-endian
    bundle (checksums verified); other tensors (DT_STRING lookup-table keys
    of TF1 checkpoints and the like) come back as OpaqueTensor."""
    index_path, data_path = bundle_paths(prefix)
    with open(index_path, "rb") as f:
        entries = read_table(f.read())
    header = dict(entries).get(b"")
    if header is None:
        raise ValueError(f"{index_path}: no bundle header")
    h = Msg.parse(header)
    if h.get(1, 1) != 1:
        raise ValueError("only one-shard bundles are supported")
    if h.get(2, 0) != 0:
        raise ValueError("only little-endian bundles are supported")
    data = open(data_path, "rb").read() if os.path.exists(data_path) else b""
    out: Dict[str, np.ndarray] = {}
    for key, val in entries:
        if key == b"":
            continue
        e = Msg.parse(val)
        dt = e.get(1, 0)
        if e.all(7):
            raise ValueError(f"{key.decode()}: sliced tensors are not supported")
        shape = shape_of(e.get(2, b""))
        off, size = e.get(4, 0), e.get(5, 0)
        raw = data[off:off + size]
        if len(raw) != size:
            raise ValueError(f"{key.decode()}: data shard too short")
        crc = e.get(6)
        if crc is not None and unmask_crc(crc) != crc32c_fast(raw):
            raise ValueError(f"{key.decode()}: tensor checksum mismatch")
        if dt not in _NP_OF:
            out[key.decode()] = OpaqueTensor(bytes(val), bytes(raw),
                                             DTYPE_NAMES.get(dt, f"DT_{dt}"), shape)
            continue
        arr = np.frombuffer(raw, dtype=_NP_OF[dt]).reshape(shape)
        out[key.decode()] = arr.copy()
    return out


def write_bundle(prefix: str, tensors: Dict[str, Union[np.ndarray, OpaqueTensor]]) -> None:
    """One shard, tensors in key order, each at the next offset of the data
    shard; OpaqueTensor entries keep their proto and bytes, with the new
    offset and size."""
    index_path, data_path = bundle_paths(prefix)
    os.makedirs(os.path.dirname(index_path) or ".", exist_ok=True)
    data = bytearray()
    items = []
    for name in sorted(tensors):
        t = tensors[name]
        if isinstance(t, OpaqueTensor):
            fields = Msg.parse(t.entry).fields
            off = len(data)
            data += t.raw
            place = []  # offset (4) and size (5) in field order; proto3 omits zeros
            if off:
                place.append((4, VARINT, off))
            if t.raw:
                place.append((5, VARINT, len(t.raw)))
            e = Msg([f for f in fields if f[0] < 4] + place + [f for f in fields if f[0] > 5])
            items.append((name.encode(), e.serialize()))
            continue
        arr = np.asarray(t)  # (ascontiguousarray would make a scalar 1-D)
        if not arr.flags.c_contiguous:
            arr = arr.copy(order="C")
        if arr.dtype not in _DT_OF:
            raise ValueError(f"{name}: dtype {arr.dtype} is not supported")
        raw = arr.astype(arr.dtype.newbyteorder("<"), copy=False).tobytes()
        off = len(data)
        data += raw
        e = Msg([(1, VARINT, _DT_OF[arr.dtype]), (2, LEN, shape_proto(arr.shape))])
        if off:  # proto3 leaves zero scalars out
            e.add(4, VARINT, off)
        if raw:
            e.add(5, VARINT, len(raw))
        e.add(6, FIXED32, mask_crc(crc32c_fast(raw)))
        items.append((name.encode(), e.serialize()))
    # {1 num_shards: 1, 3 version {1 producer: 1}} (endianness LITTLE = 0 omitted)
    header = Msg([(1, VARINT, 1), (3, LEN, Msg([(1, VARINT, 1)]))])
    items.append((b"", header.serialize()))
    with open(index_path, "wb") as f:
        f.write(write_table(items))
    with open(data_path, "wb") as f:
        f.write(bytes(data))


def variables_prefix(model_dir: str) -> str:
    return os.path.join(model_dir, "variables", "variables")


def has_saved_model(path: str) -> bool:
    return os.path.exists(os.path.join(path, "saved_model.pb"))


def read_variables(model_dir: str) -> Dict[str, np.ndarray]:
    prefix = variables_prefix(model_dir)
    if not os.path.exists(bundle_paths(prefix)[0]):
        return {}
    return read_bundle(prefix)


def write_variables(model_dir: str, tensors: Dict[str, np.ndarray]) -> None:
    write_bundle(variables_prefix(model_dir), tensors)


def find_node(nodes: List[GraphNode], name: str) -> Optional[GraphNode]:
    for n in nodes:
        if n.name == name:
            return n
    return None
