"""annc-opt: the offline model rewriter: the `layout_matmul` pass and the
hash-bucket embedding passes `embed_hash_bucket` / `lookup_embedding_hash` /
`dnn_sparse` / `dnn_hash_bucket` / `linear_sparse`.

Command line, as python/annc/main.py:14-68 (`annc-opt -I <in> -O <out> passes...`):

    python -m annc_amd.annc_opt -I <input model dir> -O <output model dir> \
        embed_hash_bucket layout_matmul

Passes run in the order given, except that layout_matmul always runs last.

A model is a TensorFlow SavedModel directory (saved_model.pb and
variables/variables.{index,data-00000-of-00001}), read and written by
`annc_amd.savedmodel` without TensorFlow: the graph of the "serve" meta
graph, and the variables by node name (the key tf.compat.v1.train.Saver,
which the reference saves with, gives a graph variable; a VarHandleOp is
also found under its shared_name).  The output directory gets saved_model.pb
with the rewritten graph, the variables with the packed weights, and
everything else of the input (assets, ...) except the now stale
saved_model.pbtxt, fingerprint.pb and old variables.  (The reference writes
the new graph as saved_model.pbtxt beside an unchanged copy of
saved_model.pb, graph.py:312-338, which TensorFlow, preferring the .pb,
does not load.)

A directory without saved_model.pb is read in this build's plain form, for
hand-written tests: graph.json ({"nodes": [{"name", "op", "inputs",
"attrs"}]}) and variables.safetensors (one array per variable node).

`layout_matmul` (constant_folding.py:11-98) pre-packs constant MatMul weights
for `__layout_matmul`: every MatMul whose rhs resolves through Identity /
ReadVariableOp to a variable, carries no `rhs_format` attr yet, and has no
operand dimension below 12, gets its rhs variable re-ordered in place (same
shape, same element count) and the attr `rhs_format` set.  The packed order
is this library's MFMA-fragment format (`annc_layout_matmul_rhs_format()`,
"mfma_f32_32x32x2_k16") instead of kpgemm's "kn4", so a weight packed by the
reference is never read as the new format by mistake.  Like the reference,
the pass always runs last.

`embed_hash_bucket` (rec_embedding.py:490-785) replaces each TF feature-column
subgraph of an embedding_column over a hash-bucket categorical column (the
SparseFillEmptyRows / Unique / gather / SparseSegmentSum-or-Mean chain, about
45 nodes) by one KPFusedEmbeddingWithHashBucket node with inputs (the string
tensor, the embedding weight) and attrs num_buckets, combiner (0 sum, 1 mean)
and T_weight.  `lookup_embedding_hash` emits KPLookupEmbeddingByHash for the
same subgraph.

`dnn_sparse` and `linear_sparse` (rec_embedding.py:6-86, 794-891) replace a
hash-bucket column's sparse-id subgraph (ExpandDims ... SparseFillEmptyRows,
20 to 26 nodes) by one KPFusedSparseEmbedding (the strings in; the
SparseFillEmptyRows' indices, values and empty-row indicator and the dense
shape out).  `dnn_hash_bucket` (rec_embedding.py:88-211) replaces the column
through its SparseSegmentMean and reshapes (43 nodes) by one
KPFusedDnnEmbeddingWithHashBucket (strings and embedding weight in).  The
remaining pattern passes of the reference (embed, softmax) emit ops outside
this library and are refused.

Differences from the reference, each deliberate:
  * lhs variables are not packed: the reference's "k4m4" lhs packing has no
    consumer (no custom call reads a packed lhs); the reference's rule that a
    too-small variable lhs skips the whole node is kept.
  * only rank-2 rhs variables are packed: `__layout_matmul` is a rank-2 call,
    and a packed rank-3 BatchMatMul weight would be read row-major by
    `__batch_matmul`.
  * MatMuls with transpose_b / adj_y are left alone: the packed format
    describes an untransposed [k, n] operand (the reference packs them as
    if they were [k, n]).
  * weights already packed by the reference (`rhs_format: "kn4"`) are
    converted: unpacked with the kn4 order (data_pack.py:24-149, restated in
    `kn4_permutation`) and re-packed into the MFMA format.
  * an embedding subgraph is fused only if nothing outside it reads a node
    the rewrite removes (other than the outputs the fused node takes over);
    the reference removes them regardless, leaving dangling inputs.  Users
    are taken from the graph as it stands before each match, and every
    anchor (SparseFillEmptyRows, or ExpandDims for the sparse passes) is
    visited (the reference walks its node list while editing it).
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import sys
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import savedmodel

VECTOR_LEN = 12                     # constant_folding.py:12 (__vector_len__)
KN4_TILING = ((0, 352), (1, 128))   # constant_folding.py:94-95 (generate_tiling)
REF_RHS_FORMAT = "kn4"

MATMUL_OPS = frozenset(["MatMul", "BatchMatMul", "BatchMatMulV2", "BatchMatMulV3"])
PASS_THROUGH_OPS = frozenset(["Identity", "ReadVariableOp"])
VARIABLE_OPS = frozenset(["VarHandleOp", "VariableV2", "Variable"])
# Pattern passes of the reference (rec_embedding.py) this build implements,
# and the ones it does not (their fused ops are not part of this library)
EMBEDDING_PASSES = ("embed_hash_bucket", "lookup_embedding_hash")
SPARSE_PASSES = ("dnn_sparse", "dnn_hash_bucket", "linear_sparse")
UNSUPPORTED_PASSES = ("embed", "softmax")


def mfma_rhs_format() -> str:
    from . import _lib
    return _lib.lib().annc_layout_matmul_rhs_format().decode()


# ---------------------------------------------------------------------------
# kpgemm "kn4" order (reader for weights packed by the reference)
# ---------------------------------------------------------------------------
def _tile_bounds(dim: int, tile: int, vec: int) -> List[tuple]:
    """[start, end) of each tile along one axis (data_pack.py:49-79): tiles of
    `tile`, except that a remainder is absorbed by re-splitting the last two
    tiles evenly at a multiple of `vec`."""
    num = -(-dim // tile)
    out = []
    for i in range(num):
        start, end = i * tile, (i + 1) * tile
        if dim < tile:
            end = dim
        elif dim % tile and i >= num - 2:
            res = dim - (num - 2) * tile        # both branches measure the same span
            docker = (res // 2) // vec * vec
            if res - docker > docker + 1:
                docker += vec
            split = (num - 2) * tile + docker
            start, end = (start, split) if i == num - 2 else (split, dim)
        out.append((start, end))
    return out


def _panel_widths(n: int, vec: int = VECTOR_LEN) -> List[int]:
    """Panel widths along N inside a block (data_pack.py:129-149, vec 12):
    12-wide panels, then tails of 4, 2, 1."""
    widths = [vec] * (n // vec)
    rest = n % vec
    small = 4
    while small:
        while rest >= small:
            widths.append(small)
            rest -= small
        small //= 2
    return widths


def kn4_permutation(k: int, n: int) -> np.ndarray:
    """perm[i] = row-major index (k*n + n) of the weight element stored at
    position i of the reference's kn4 packing of a [k, n] weight: blocks in
    K-major order (K tiles of 352, then N tiles of 128 within each), each
    block cut into N panels flattened row-major [k_block, width]
    (data_pack.py:36-41, 94-100, 118-127)."""
    idx = np.arange(k * n, dtype=np.int64).reshape(k, n)
    parts = []
    for k0, k1 in _tile_bounds(k, KN4_TILING[0][1], VECTOR_LEN):
        for n0, n1 in _tile_bounds(n, KN4_TILING[1][1], VECTOR_LEN):
            loc = n0
            for w in _panel_widths(n1 - n0):
                parts.append(idx[k0:k1, loc:loc + w].reshape(-1))
                loc += w
    perm = np.concatenate(parts) if parts else np.zeros(0, np.int64)
    return perm


def pack_kn4(w: np.ndarray) -> np.ndarray:
    k, n = w.shape
    return np.ascontiguousarray(w).reshape(-1)[kn4_permutation(k, n)].reshape(k, n)


def unpack_kn4(packed: np.ndarray, k: int, n: int) -> np.ndarray:
    out = np.empty(k * n, dtype=packed.dtype)
    out[kn4_permutation(k, n)] = np.ascontiguousarray(packed).reshape(-1)
    return out.reshape(k, n)


# ---------------------------------------------------------------------------
# Model directory
# ---------------------------------------------------------------------------
@dataclass
class Node:
    name: str
    op: str
    inputs: List[str] = field(default_factory=list)
    attrs: Dict[str, object] = field(default_factory=dict)


@dataclass
class Model:
    nodes: List[Node]
    variables: Dict[str, np.ndarray]
    saved: Optional[savedmodel.SavedModelGraph] = None  # set for a SavedModel directory

    def node(self, name: str) -> Optional[Node]:
        base = name.split(":")[0].lstrip("^")
        for nd in self.nodes:
            if nd.name == base:
                return nd
        return None


def load_model(path: str) -> Model:
    if savedmodel.has_saved_model(path):
        saved = savedmodel.read_saved_model(path)
        nodes = [Node(g.name, g.op, list(g.inputs), dict(g.attrs)) for g in saved.nodes]
        return Model(nodes, savedmodel.read_variables(path), saved)
    from safetensors.numpy import load_file
    with open(os.path.join(path, "graph.json")) as f:
        spec = json.load(f)
    nodes = [Node(n["name"], n["op"], list(n.get("inputs", [])), dict(n.get("attrs", {})))
             for n in spec["nodes"]]
    var_path = os.path.join(path, "variables.safetensors")
    variables = load_file(var_path) if os.path.exists(var_path) else {}
    return Model(nodes, dict(variables))


# input entries a SavedModel output does not copy: rewritten, or stale after the rewrite
_SAVED_MODEL_OWN = ("saved_model.pb", "saved_model.pbtxt", "fingerprint.pb", "variables")


def _save_saved_model(model: Model, path: str, source: Optional[str]) -> None:
    old = {g.name: g for g in model.saved.nodes}
    nodes = []
    for n in model.nodes:
        g = old.get(n.name)
        nodes.append(savedmodel.GraphNode(n.name, n.op, list(n.inputs), dict(n.attrs),
                                          g.device if g else "", list(g.extra) if g else []))
    model.saved.nodes = nodes
    os.makedirs(path, exist_ok=True)
    savedmodel.write_saved_model(path, model.saved)
    savedmodel.write_variables(path, model.variables)
    if source and os.path.abspath(source) != os.path.abspath(path):
        for entry in os.listdir(source):
            if entry in _SAVED_MODEL_OWN:
                continue
            src, dst = os.path.join(source, entry), os.path.join(path, entry)
            if os.path.isdir(src):
                shutil.copytree(src, dst, dirs_exist_ok=True)
            else:
                shutil.copy2(src, dst)


def save_model(model: Model, path: str, source: Optional[str] = None) -> None:
    if model.saved is not None:
        _save_saved_model(model, path, source)
        return
    from safetensors.numpy import save_file
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "graph.json"), "w") as f:
        json.dump({"nodes": [{"name": n.name, "op": n.op, "inputs": n.inputs, "attrs": n.attrs}
                             for n in model.nodes]}, f, indent=1)
    save_file({k: np.ascontiguousarray(v) for k, v in model.variables.items()},
              os.path.join(path, "variables.safetensors"))
    if source and os.path.abspath(source) != os.path.abspath(path):
        # anything else the model carries (assets, metadata) travels unchanged
        for entry in os.listdir(source):
            if entry in ("graph.json", "variables.safetensors"):
                continue
            src = os.path.join(source, entry)
            dst = os.path.join(path, entry)
            if os.path.isdir(src):
                shutil.copytree(src, dst, dirs_exist_ok=True)
            else:
                shutil.copy2(src, dst)


# ---------------------------------------------------------------------------
# layout_matmul
# ---------------------------------------------------------------------------
def _variable_operand(model: Model, name: str) -> Optional[str]:
    """The key of the variable a MatMul operand reads, through Identity /
    ReadVariableOp (constant_folding.py:65-75): its node name, or a
    VarHandleOp's shared_name when only that names a stored variable."""
    nd = model.node(name)
    seen = set()
    while nd is not None and nd.name not in seen:
        seen.add(nd.name)
        if nd.op in VARIABLE_OPS:
            shared = nd.attrs.get("shared_name")
            if nd.name not in model.variables and isinstance(shared, str) and \
                    shared in model.variables:
                return shared
            return nd.name
        if nd.op in PASS_THROUGH_OPS and nd.inputs:
            nd = model.node(nd.inputs[0])
            continue
        return None
    return None


def _too_small(arr: np.ndarray) -> bool:
    """constant_folding.py:61-63: any of the first two dims below 12."""
    return arr.ndim < 2 or arr.shape[0] < VECTOR_LEN or arr.shape[1] < VECTOR_LEN


def pack_rhs(w: np.ndarray) -> np.ndarray:
    """Row-major float32 [k, n] -> the MFMA-fragment order, same shape."""
    from .device import pack_weight_host
    k, n = w.shape
    return pack_weight_host(np.ascontiguousarray(w, dtype=np.float32)).reshape(k, n)


def layout_matmul(model: Model) -> List[str]:
    """Pack every eligible MatMul rhs variable in place; returns the names of
    the packed (or converted) variables."""
    fmt = mfma_rhs_format()
    done: List[str] = []
    for nd in model.nodes:
        if nd.op not in MATMUL_OPS or len(nd.inputs) < 2:
            continue
        lhs = _variable_operand(model, nd.inputs[0])
        if lhs is not None and "lhs_format" not in nd.attrs and lhs in model.variables:
            if _too_small(model.variables[lhs]):
                continue  # the reference skips the whole node here
        rhs = _variable_operand(model, nd.inputs[1])
        if rhs is None or rhs not in model.variables:
            continue
        w = model.variables[rhs]
        if not isinstance(w, np.ndarray) or w.ndim != 2 or _too_small(w):
            continue  # (a bundle entry of a type the packer cannot read stays as it is)
        if nd.attrs.get("transpose_b") or nd.attrs.get("adj_y"):
            continue  # the packed format describes an untransposed [k, n] operand
        current = nd.attrs.get("rhs_format")
        if current == fmt:
            continue
        if current == REF_RHS_FORMAT:
            w = unpack_kn4(w, *w.shape)
        elif current is not None:
            raise ValueError(f"{nd.name}: unknown rhs_format {current!r}")
        model.variables[rhs] = pack_rhs(w)
        nd.attrs["rhs_format"] = fmt
        done.append(rhs)
    return done


# ---------------------------------------------------------------------------
# embed_hash_bucket / lookup_embedding_hash
# ---------------------------------------------------------------------------
# The TF feature-column lowering of embedding_column(categorical_column_with_
# hash_bucket(...)) that EmbeddingWithHashBucketPatternRewriter
# (rec_embedding.py:490-785) replaces by one fused op.  A pattern is a list of
# steps over named pattern variables, anchored at the SparseFillEmptyRows
# node "sfer":
#   ("in",  v, [(op, w), ...], count)  operands of v, by position
#   ("out", v, [(op, w), ...], count)  users of v, in graph order
# Entry i must have type `op` (None: any).  `w` names the variable it is: a
# new name binds it, a bound name must be the same node, None checks the type
# only.  `count` (or None) is the exact number of operands / users.
_SEGMENT_SUM_PATTERN = [
    ("in", "sfer", [("GatherV2", "g0"), ("GatherV2", "g1"), ("Identity", "id0")], None),
    ("in", "g0", [("SparseReshape", "sr0"), ("Reshape", "rs0")], None),
    ("in", "g1", [("Identity", "id1"), ("Reshape", "rs0")], None),
    ("in", "id0", [("SparseReshape", "sr0")], None),
    ("in", "rs0", [("Where", "wh0")], None),
    ("in", "wh0", [("GreaterEqual", "ge0")], None),
    ("in", "ge0", [("Identity", "id1")], None),
    ("in", "id1", [("Identity", "id2")], None),
    ("in", "id2", [("StringToHashBucketFast", "hash")], None),
    ("in", "sr0", [("SparseReshape", "sr1"), ("SparseReshape", None), ("Pack", "pk0")], None),
    ("in", "pk0", [("Prod", "pr0"), ("GatherV2", "g2")], None),
    ("in", "pr0", [("Slice", "sl0")], None),
    ("in", "sl0", [("SparseReshape", "sr1")], None),
    ("in", "g2", [("SparseReshape", "sr1")], None),
    ("in", "sr1", [("Where", "wh1"), ("Shape", "sh0"), ("Cast", "c0")], None),
    ("in", "c0", [("Pack", "pk1")], None),
    ("in", "pk1", [("StridedSlice", "ss0")], None),
    ("in", "ss0", [(None, "c1")], None),
    ("in", "c1", [("Shape", "sh0")], None),
    ("in", "wh1", [("NotEqual", "ne")], None),
    ("in", "ne", [("ExpandDims", "ed")], None),
    ("in", "hash", [("GatherNd", "gnd")], None),
    ("in", "gnd", [("ExpandDims", "ed"), ("Where", "wh1")], None),
    ("out", "sfer", [("StridedSlice", "ss1"), ("Unique", "uq"), ("Reshape", "rs1")], 3),
    ("out", "uq", [("ResourceGather", "gather"), ("SparseSegmentSum", "seg")], 2),
    ("out", "gather", [("Identity", "id3")], None),
    ("out", "id3", [("Identity", "id4")], None),
    ("out", "id4", [("SparseSegmentSum", "seg")], None),
    ("out", "ss1", [("Cast", "c2")], None),
    ("out", "c2", [("SparseSegmentSum", "seg")], None),
    ("out", "seg", [("Shape", "sh1"), ("ZerosLike", "zl"), ("Select", "sel")], None),
    ("out", "sh1", [("StridedSlice", "ss2")], None),
    ("out", "ss2", [("Pack", "pk2")], None),
    ("out", "pk2", [("Tile", "tl")], None),
    ("out", "rs1", [("Tile", "tl")], None),
    ("out", "tl", [("Select", "sel")], None),
    ("out", "zl", [("Select", "sel")], None),
    ("out", "sel", [("Shape", "sh2"), ("Reshape", "result")], None),
    ("out", "sh2", [("Slice", "sl1")], None),
    ("out", "sl1", [("ConcatV2", "cc")], None),
    ("out", "sr1", [("Slice", None), ("GatherV2", None), ("SparseReshape", None),
                    ("SparseReshape", None), ("Cast", "c3")], None),
    ("out", "c3", [("Slice", "sl2")], None),
    ("out", "sl2", [("ConcatV2", "cc")], None),
    ("out", "cc", [("Reshape", "result")], None),
]

_SEGMENT_MEAN_PATTERN = [
    ("in", "sfer", [("GatherV2", "g0"), ("GatherV2", "g1"), ("Identity", "id0")], None),
    ("in", "g0", [("SparseReshape", "sr0"), ("Reshape", "rs0")], None),
    ("in", "g1", [("Identity", "id1"), ("Reshape", "rs0")], None),
    ("in", "id0", [("SparseReshape", "sr0")], None),
    ("in", "rs0", [("Where", "wh0")], None),
    ("in", "wh0", [("GreaterEqual", "ge0")], None),
    ("in", "ge0", [("Identity", "id1")], None),
    ("in", "id1", [("StringToHashBucketFast", "hash")], None),
    ("in", "sr0", [("Where", "wh1"), ("Shape", "sh0"), ("Pack", "pk0")], None),
    ("in", "pk0", [("Prod", "pr0"), ("GatherV2", "g2")], None),
    ("in", "pr0", [("Slice", "sl0")], None),
    ("in", "sl0", [("Shape", "sh0")], None),
    ("in", "g2", [("Shape", "sh0")], None),
    ("in", "sh0", [("ExpandDims", "ed")], None),
    ("in", "hash", [("GatherNd", "gnd")], None),
    ("in", "gnd", [("ExpandDims", "ed"), ("Where", "wh1")], None),
    ("in", "wh1", [("NotEqual", "ne")], None),
    ("in", "ne", [("ExpandDims", "ed")], None),
    ("out", "sfer", [("StridedSlice", "ss1"), ("Unique", "uq"), ("Reshape", "rs1")], 3),
    ("out", "uq", [("GatherV2", "gather"), ("SparseSegmentMean", "seg")], None),
    ("out", "gather", [("Identity", "id3")], None),
    ("out", "id3", [("SparseSegmentMean", "seg")], None),
    ("out", "ss1", [("Cast", "c2")], None),
    ("out", "c2", [("SparseSegmentMean", "seg")], None),
    ("out", "seg", [("Shape", "sh1"), ("ZerosLike", "zl"), ("Select", "sel")], None),
    ("out", "sh1", [("StridedSlice", "ss2")], None),
    ("out", "ss2", [("Pack", "pk1")], None),
    ("out", "pk1", [("Tile", "tl")], None),
    ("out", "rs1", [("Tile", "tl")], None),
    ("out", "tl", [("Select", "sel")], None),
    ("out", "zl", [("Select", "sel")], None),
    ("out", "sel", [("Shape", "sh2"), ("Reshape", "rs2")], None),
    ("out", "sh2", [("Slice", "sl1")], None),
    ("out", "sl1", [("ConcatV2", "cc")], None),
    ("out", "sh0", [("Slice", None), ("GatherV2", None), ("SparseReshape", None),
                    ("Cast", "c3")], None),
    ("out", "c3", [("Slice", "sl2")], None),
    ("out", "sl2", [("ConcatV2", "cc")], None),
    ("out", "cc", [("Reshape", "rs2")], None),
    ("out", "rs2", [("Shape", "sh3"), ("Reshape", "result")], None),
    ("out", "sh3", [("StridedSlice", "ss3")], None),
    ("out", "ss3", [("Pack", "pk2")], None),
    ("out", "pk2", [("Reshape", "result")], None),
]

# pass -> (fused op type, name suffix); rec_embedding.py:490-492, 787-789
_EMBEDDING_FUSED_OPS = {
    "embed_hash_bucket": ("KPFusedEmbeddingWithHashBucket", "/rec_embed_kp_bucket"),
    "lookup_embedding_hash": ("KPLookupEmbeddingByHash", "/rec_embed_kp_hash"),
}


def _input_node(inp: str) -> str:
    return inp.split(":")[0]


class _GraphIndex:
    """Data operands (node, output index) and users of every node; a user
    appears once per data input it takes from the node, in graph order, and
    control inputs ("^name") are neither."""

    def __init__(self, model: Model):
        self.by_name = {n.name: n for n in model.nodes}
        self.users: Dict[str, List[Node]] = {n.name: [] for n in model.nodes}
        for n in model.nodes:
            for inp in n.inputs:
                if not inp.startswith("^") and _input_node(inp) in self.users:
                    self.users[_input_node(inp)].append(n)

    def operands(self, node: Node) -> List[Optional[Node]]:
        return [self.by_name.get(_input_node(i)) for i in node.inputs if not i.startswith("^")]


def _match(index: _GraphIndex, anchor: Node, pattern,
           anchor_var: str = "sfer") -> Optional[Dict[str, Node]]:
    bound = {anchor_var: anchor}
    for kind, var, entries, count in pattern:
        node = bound[var]
        seq = index.operands(node) if kind == "in" else index.users[node.name]
        if count is not None and len(seq) != count:
            return None
        if len(entries) > len(seq):
            return None
        for (op, name), cand in zip(entries, seq):
            if cand is None or (op is not None and cand.op != op):
                return None
            if name is None:
                continue
            if name in bound:
                if bound[name] is not cand:
                    return None
            else:
                bound[name] = cand
    return bound


def _rewrite_embedding(model: Model, anchor: Node, bound: Dict[str, Node], mean: bool,
                       op: str, suffix: str) -> Node:
    """Replace the matched subgraph by one fused node: inputs (the string
    tensor ExpandDims reads, the embedding weight the gather reads); attrs
    the hash node's (num_buckets), combiner 0 / T_weight resource for
    SparseSegmentSum, combiner 1 / T_weight float for SparseSegmentMean
    (rec_embedding.py:614-621, 749-756)."""
    ed, gather, result, hash_node = bound["ed"], bound["gather"], bound["result"], bound["hash"]
    attrs = {k: v for k, v in hash_node.attrs.items() if k != "_output_shapes"}
    attrs["combiner"] = 1 if mean else 0
    attrs["T_weight"] = savedmodel.DType("DT_FLOAT" if mean else "DT_RESOURCE")
    if "_output_shapes" in result.attrs:
        attrs["_output_shapes"] = result.attrs["_output_shapes"]
    fused = Node(anchor.name + suffix, op, [ed.inputs[0], gather.inputs[0]], attrs)
    gone = {n.name for n in bound.values()}
    for n in model.nodes:
        if n.name in gone:
            continue
        for i, inp in enumerate(n.inputs):
            if inp in (result.name, result.name + ":0"):
                n.inputs[i] = fused.name
            elif inp == "^" + result.name:
                n.inputs[i] = "^" + fused.name
    at = model.nodes.index(anchor)
    model.nodes.insert(at + 1, fused)
    model.nodes[:] = [n for n in model.nodes if n.name not in gone]
    return fused


def embedding_with_hash_bucket(model: Model, pass_name: str = "embed_hash_bucket") -> List[str]:
    """EmbeddingWithHashBucketPatternRewriter / LookupEmbeddingWithHash-
    PatternRewriter (rec_embedding.py:490-792): every SparseFillEmptyRows at
    the centre of a hash-bucket embedding_column subgraph (segment sum or
    segment mean) becomes one fused node.  Returns the fused node names.

    A match is rewritten only when no node outside it reads a node it
    removes (other than through the result, which the fused node replaces);
    the reference removes the nodes regardless."""
    op, suffix = _EMBEDDING_FUSED_OPS[pass_name]
    made: List[str] = []
    anchors = [n.name for n in model.nodes if n.op == "SparseFillEmptyRows"]
    for name in anchors:
        index = _GraphIndex(model)
        anchor = index.by_name.get(name)
        if anchor is None:
            continue
        mean = False
        bound = _match(index, anchor, _SEGMENT_SUM_PATTERN)
        if bound is None:
            bound = _match(index, anchor, _SEGMENT_MEAN_PATTERN)
            mean = True
        if bound is None:
            continue
        gone = {n.name for n in bound.values()}
        inner = gone - {bound["result"].name}
        escapes = any(u.name not in gone for v in inner for u in index.users[v])
        escapes = escapes or any(i.startswith("^") and i[1:] in inner
                                 for n in model.nodes if n.name not in gone for i in n.inputs)
        if escapes:
            continue
        made.append(_rewrite_embedding(model, anchor, bound, mean, op, suffix).name)
    return made


# ---------------------------------------------------------------------------
# dnn_sparse / linear_sparse -> KPFusedSparseEmbedding and dnn_hash_bucket ->
# KPFusedDnnEmbeddingWithHashBucket (rec_embedding.py:6-211, 794-891): the
# same step lists as above, anchored at the ExpandDims ("ed") that reads the
# string placeholder.  Steps with a None name check the type only, as the
# reference's unnamed checks do.
# ---------------------------------------------------------------------------
_DNN_FRONT = [  # rec_embedding.py:9-53 (and 91-135)
    ("in", "ed", [("Placeholder", "ph"), ("Const", "ed_dim")], None),
    ("out", "ed", [("NotEqual", "ne"), ("GatherNd", "gnd"), ("Shape", "sh")], 3),
    ("out", "ne", [("Where", "wh")], 1),
    ("out", "wh", [("GatherNd", "gnd"), ("SparseReshape", "sr")], None),
    ("out", "gnd", [("StringToHashBucketFast", "hash")], 1),
    ("out", "hash", [("Identity", "id")], 1),
    ("out", "id", [("GreaterEqual", "ge"), ("GatherV2", "gv")], 2),
    ("out", "ge", [("Where", "wh2")], 1),
    ("out", "wh2", [("Reshape", "rs")], 1),
    ("out", "rs", [("GatherV2", "gv1"), ("GatherV2", "gv")], 2),
    ("out", "sh", [("Slice", "sl"), ("GatherV2", "gv3"), ("SparseReshape", "sr"),
                   ("Cast", None)], 4),
    ("out", "sl", [("Prod", "pr")], 1),
    ("out", "pr", [("Pack", "pk")], 1),
    ("out", "gv3", [("Pack", "pk")], 1),
    ("out", "pk", [("SparseReshape", "sr")], 1),
    ("out", "sr", [("GatherV2", "gv1"), ("Identity", "id2")], 2),
    ("out", "id2", [("SparseFillEmptyRows", "sfer")], 1),
    ("out", "gv", [("SparseFillEmptyRows", None)], 1),
    ("out", "gv1", [("SparseFillEmptyRows", None)], 1),
]

_DNN_SPARSE_PATTERN = _DNN_FRONT

_DNN_HASH_BUCKET_PATTERN = _DNN_FRONT + [  # rec_embedding.py:137-172
    ("out", "sfer", [("StridedSlice", "ss"), ("Unique", "uq"), ("Reshape", "rsh")], 3),
    ("out", "rsh", [("Tile", None)], 1),
    ("out", "uq", [("GatherV2", "gv4"), ("SparseSegmentMean", "ssm")], 2),
    ("out", "gv4", [("Identity", "id3")], 1),
    ("out", "id3", [("SparseSegmentMean", None)], 1),
    ("out", "ss", [("Cast", "cst")], 1),
    ("out", "cst", [("SparseSegmentMean", None)], 1),
    ("out", "ssm", [("Shape", "sh2"), ("ZerosLike", "zl"), ("Select", "sel")], 3),
    ("out", "zl", [("Select", None)], 1),
    ("out", "sh2", [("StridedSlice", "ss2")], 1),
    ("out", "ss2", [("Pack", "pk2")], 1),
    ("out", "pk2", [("Tile", "tl")], 1),
    ("out", "tl", [("Select", None)], 1),
    ("out", "sel", [("Shape", "sh3"), ("Reshape", "rs2")], 2),
    ("out", "sh3", [("Slice", "sl2")], 1),
    ("out", "sl2", [("ConcatV2", None)], 1),
    ("out", "sh", [(None, None), (None, None), (None, None), ("Cast", "cst2")], 4),
    ("out", "cst2", [("Slice", "sl3")], 1),
    ("out", "sl3", [("ConcatV2", "cc")], 1),
    ("out", "cc", [("Reshape", None)], 1),
    ("out", "rs2", [("Shape", "sh4"), ("Reshape", "rs3")], 2),
    ("out", "sh4", [("StridedSlice", "ss3")], 1),
    ("out", "ss3", [("Pack", "pk3")], 1),
    ("out", "pk3", [("Reshape", None)], 1),
]

_LINEAR_SPARSE_PATTERN = [  # rec_embedding.py:797-855
    ("in", "ed", [("Placeholder", "ph"), ("Const", "ed_dim")], None),
    ("out", "ed", [("NotEqual", "ne"), ("GatherNd", "gnd"), ("Shape", "sh")], 3),
    ("out", "ne", [("Where", "wh")], 1),
    ("out", "wh", [("GatherNd", "gnd"), ("SparseReshape", "sr")], None),
    ("out", "gnd", [("StringToHashBucketFast", "hash")], 1),
    ("out", "hash", [("Identity", "id")], 1),
    ("out", "id", [("Identity", "id2")], 1),
    ("out", "id2", [("GreaterEqual", "ge"), ("GatherV2", "gv")], 2),
    ("out", "ge", [("Where", "wh2")], 1),
    ("out", "wh2", [("Reshape", "rs")], 1),
    ("out", "rs", [("GatherV2", "gv1"), ("GatherV2", "gv")], 2),
    ("out", "sh", [("Cast", "c0"), ("SparseReshape", "sr")], 2),
    ("out", "c0", [("StridedSlice", "ss0")], 1),
    ("out", "ss0", [("Pack", "pk0")], 1),
    ("out", "pk0", [("Cast", "c1")], 1),
    ("out", "c1", [("SparseReshape", "sr")], 1),
    ("out", "sr", [("Slice", "sl"), ("GatherV2", "gvb"), ("SparseReshape", "sr2"),
                   ("SparseReshape", None), ("Cast", None)], 5),
    ("out", "sl", [("Prod", "pr")], 1),
    ("out", "pr", [("Pack", "pk1")], 1),
    ("out", "gvb", [("Pack", "pk1")], 1),
    ("out", "sr2", [("GatherV2", "gv1"), ("Identity", "id3")], 2),
    ("out", "id3", [("SparseFillEmptyRows", "sfer")], 1),
    ("out", "gv1", [("SparseFillEmptyRows", "sfer")], 1),
    ("out", "gv", [("SparseFillEmptyRows", "sfer")], 1),
]


def _shape_entries(attr) -> list:
    """Entries of an `_output_shapes` attr: shape lists in the plain form,
    TensorShapeProto bytes in a SavedModel (AttrValue.list.shape)."""
    if isinstance(attr, savedmodel.RawAttr):
        lst = savedmodel.Msg.parse(attr.data).get(1)
        return savedmodel.Msg.parse(lst).all(7) if lst is not None else []
    return list(attr or [])


def _shapes_like(entries: list, like):
    """An `_output_shapes` attr of `entries`, in the form of `like`."""
    if isinstance(like, savedmodel.RawAttr):
        lst = savedmodel.Msg([(7, savedmodel.LEN, e) for e in entries])
        return savedmodel.RawAttr(savedmodel.Msg([(1, savedmodel.LEN, lst)]).serialize())
    return entries


def _tensor(node: Node, index: int) -> str:
    return node.name if index == 0 else f"{node.name}:{index}"


def _fuse(model: Model, index: _GraphIndex, bound: Dict[str, Node], keep: Sequence[str],
          op: str, name: str, inputs: List[str], attrs: Dict[str, object],
          outputs: Sequence[Tuple[Node, int]], after: Node) -> Optional[Node]:
    """Replace the bound nodes (less `keep`) by one node of type `op` whose
    output j stands for tensor outputs[j]: every reader of that tensor
    outside the match reads output j instead (replace_all_users_with,
    rewriter.py:82-88).  Returns None, changing nothing, when a node outside
    the match reads any other output of a removed node, or names one as a
    control input (the reference removes the nodes regardless)."""
    gone = {bound[v].name for v in bound if v not in keep}
    remap = {(node.name, k): j for j, (node, k) in enumerate(outputs)}
    for n in model.nodes:
        if n.name in gone:
            continue
        for inp in n.inputs:
            if inp.startswith("^"):
                if inp[1:] in gone:
                    return None
                continue
            src, _, k = inp.partition(":")
            if src in gone and (src, int(k or 0)) not in remap:
                return None
    fused = Node(name, op, list(inputs), attrs)
    for n in model.nodes:
        if n.name in gone:
            continue
        for i, inp in enumerate(n.inputs):
            src, _, k = inp.partition(":")
            j = remap.get((src, int(k or 0))) if not inp.startswith("^") else None
            if j is not None:
                n.inputs[i] = _tensor(fused, j)
    at = model.nodes.index(after)
    model.nodes.insert(at + 1, fused)
    model.nodes[:] = [n for n in model.nodes if n.name not in gone]
    return fused


def sparse_embedding_passes(model: Model, pass_name: str) -> List[str]:
    """DnnSparseEmbeddingPatternRewriter, DnnEmbeddingWithHashBucket-
    PatternRewriter and LinearSparseEmbeddingPatternRewriter
    (rec_embedding.py:6-211, 794-891): every ExpandDims at the root of such a
    hash-bucket column becomes one KPFusedSparseEmbedding (outputs: the
    SparseFillEmptyRows' indices, values and empty-row indicator, then the
    dense shape) or KPFusedDnnEmbeddingWithHashBucket (inputs: the strings
    and the embedding weight; output: the column's [batch, dim] result),
    with the hash node's attrs (num_buckets).  Returns the fused node names."""
    pattern = {"dnn_sparse": _DNN_SPARSE_PATTERN, "dnn_hash_bucket": _DNN_HASH_BUCKET_PATTERN,
               "linear_sparse": _LINEAR_SPARSE_PATTERN}[pass_name]
    made: List[str] = []
    for anchor_name in [n.name for n in model.nodes if n.op == "ExpandDims"]:
        index = _GraphIndex(model)
        ed = index.by_name.get(anchor_name)
        if ed is None:
            continue
        b = _match(index, ed, pattern, "ed")
        if b is None:
            continue
        sfer, hash_node = b["sfer"], b["hash"]
        attrs = {k: v for k, v in hash_node.attrs.items() if k != "_output_shapes"}
        if pass_name == "dnn_hash_bucket":
            # rec_embedding.py:186-196
            outputs = [(b["rs3"], 0)]
            shapes = _shape_entries(b["rs3"].attrs.get("_output_shapes"))[:1]
            like = b["rs3"].attrs.get("_output_shapes")
            op, suffix = "KPFusedDnnEmbeddingWithHashBucket", "/rec_embed_kp_dnn_bucket"
            inputs = [ed.inputs[0], b["gv4"].inputs[0]]
        else:
            # rec_embedding.py:57-72 (dense shape: the Shape node's output) and
            # 863-877 (the SparseReshape's output 1)
            tail = (b["sh"], 0) if pass_name == "dnn_sparse" else (b["sr"], 1)
            outputs = [(sfer, 0), (sfer, 1), (sfer, 2), tail]
            like = sfer.attrs.get("_output_shapes")
            shapes = (_shape_entries(like)[:3] +
                      _shape_entries(tail[0].attrs.get("_output_shapes"))[tail[1]:tail[1] + 1])
            op, suffix = "KPFusedSparseEmbedding", "/rec_embed_kp_sparse"
            inputs = [ed.inputs[0]]
        if like is not None:
            attrs["_output_shapes"] = _shapes_like(shapes, like)
        fused = _fuse(model, index, b, ("ph",), op, sfer.name + suffix, inputs, attrs, outputs,
                      after=ed)
        if fused is not None:
            made.append(fused.name)
    return made


def optimize(input_path: str, output_path: str, passes: Sequence[str]) -> List[str]:
    """main.opt (main.py:43-68): load, run the passes in the order given with
    layout_matmul moved last, save.  Returns the variables layout_matmul
    packed."""
    passes = list(passes)
    for p in passes:
        if p in UNSUPPORTED_PASSES:
            raise TypeError(f"Pass '{p}' emits a fused op this build does not implement")
        if p != "layout_matmul" and p not in EMBEDDING_PASSES + SPARSE_PASSES:
            raise TypeError(f"Pass '{p}' not found")
    if "layout_matmul" in passes:
        passes = [p for p in passes if p != "layout_matmul"] + ["layout_matmul"]
    model = load_model(input_path)
    packed: List[str] = []
    for p in passes:
        if p == "layout_matmul":
            packed = layout_matmul(model)
        elif p in SPARSE_PASSES:
            sparse_embedding_passes(model, p)
        else:
            embedding_with_hash_bucket(model, p)
    save_model(model, output_path, source=input_path)
    return packed


def parse_args(argv=None):
    parser = argparse.ArgumentParser("ANNC-Model-Optimizer")
    parser.add_argument("-I", "--input", required=True, help="Input model path")
    parser.add_argument("-O", "--output", required=True, help="Output model path")
    parser.add_argument("passes", nargs="+",
                        help="opt: " + ", ".join(repr(p) for p in EMBEDDING_PASSES + SPARSE_PASSES)
                             + ", 'layout_matmul'")
    return parser.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    packed = optimize(args.input, args.output, args.passes)
    for name in packed:
        print(f"layout_matmul: packed {name}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
