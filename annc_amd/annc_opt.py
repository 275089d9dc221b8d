"""annc-opt: the offline model rewriter, `layout_matmul` pass.

Command line, as python/annc/main.py:14-68 (`annc-opt -I <in> -O <out> passes...`):

    python -m annc_amd.annc_opt -I <input model dir> -O <output model dir> layout_matmul

The reference rewrites a TensorFlow SavedModel.  TensorFlow is not part of
this build, so a model here is a directory holding

    graph.json              {"nodes": [{"name", "op", "inputs": [...], "attrs": {...}}]}
    variables.safetensors   one float32 array per variable node, keyed by node name

with TensorFlow's op names (MatMul, BatchMatMul, Identity, ReadVariableOp,
VarHandleOp, VariableV2, Variable) and the operand order of the graph.

`layout_matmul` (constant_folding.py:11-98) pre-packs constant MatMul weights
for `__layout_matmul`: every MatMul whose rhs resolves through Identity /
ReadVariableOp to a variable, carries no `rhs_format` attr yet, and has no
operand dimension below 12, gets its rhs variable re-ordered in place (same
shape, same element count) and the attr `rhs_format` set.  The packed order
is this library's MFMA-fragment format (`annc_layout_matmul_rhs_format()`,
"mfma_f32_32x32x2_k16") instead of kpgemm's "kn4", so a weight packed by the
reference is never read as the new format by mistake.  Like the reference,
the pass always runs last.

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
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import sys
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

VECTOR_LEN = 12                     # constant_folding.py:12 (__vector_len__)
KN4_TILING = ((0, 352), (1, 128))   # constant_folding.py:94-95 (generate_tiling)
REF_RHS_FORMAT = "kn4"

MATMUL_OPS = frozenset(["MatMul", "BatchMatMul", "BatchMatMulV2", "BatchMatMulV3"])
PASS_THROUGH_OPS = frozenset(["Identity", "ReadVariableOp"])
VARIABLE_OPS = frozenset(["VarHandleOp", "VariableV2", "Variable"])
# TensorFlow graph pattern rewrites of the reference (rec_embedding.py); they
# match TF subgraphs that this build's model format does not describe
TF_PATTERN_PASSES = ("lookup_embedding_hash", "dnn_sparse", "dnn_hash_bucket", "embed",
                     "embed_hash_bucket", "linear_sparse", "softmax")


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

    def node(self, name: str) -> Optional[Node]:
        base = name.split(":")[0].lstrip("^")
        for nd in self.nodes:
            if nd.name == base:
                return nd
        return None


def load_model(path: str) -> Model:
    from safetensors.numpy import load_file
    with open(os.path.join(path, "graph.json")) as f:
        spec = json.load(f)
    nodes = [Node(n["name"], n["op"], list(n.get("inputs", [])), dict(n.get("attrs", {})))
             for n in spec["nodes"]]
    var_path = os.path.join(path, "variables.safetensors")
    variables = load_file(var_path) if os.path.exists(var_path) else {}
    return Model(nodes, dict(variables))


def save_model(model: Model, path: str, source: Optional[str] = None) -> None:
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
    """The variable a MatMul operand reads, through Identity / ReadVariableOp
    (constant_folding.py:65-75)."""
    nd = model.node(name)
    seen = set()
    while nd is not None and nd.name not in seen:
        seen.add(nd.name)
        if nd.op in VARIABLE_OPS:
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
        if w.ndim != 2 or _too_small(w):
            continue
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


def optimize(input_path: str, output_path: str, passes: Sequence[str]) -> List[str]:
    """main.opt (main.py:43-68): load, run the passes (layout_matmul last),
    save.  Returns the variables layout_matmul packed."""
    passes = list(passes)
    for p in passes:
        if p in TF_PATTERN_PASSES:
            raise TypeError(f"Pass '{p}' rewrites TensorFlow subgraphs; this build's model "
                            f"format carries the fused ops directly")
        if p != "layout_matmul":
            raise TypeError(f"Pass '{p}' not found")
    model = load_model(input_path)
    packed: List[str] = []
    if "layout_matmul" in passes:
        packed = layout_matmul(model)
    save_model(model, output_path, source=input_path)
    return packed


def parse_args(argv=None):
    parser = argparse.ArgumentParser("ANNC-Model-Optimizer")
    parser.add_argument("-I", "--input", required=True, help="Input model path")
    parser.add_argument("-O", "--output", required=True, help="Output model path")
    parser.add_argument("passes", nargs="+",
                        help="opt: 'layout_matmul' (the TF pattern passes "
                             + ", ".join(repr(p) for p in TF_PATTERN_PASSES)
                             + " apply to TensorFlow graphs only)")
    return parser.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    packed = optimize(args.input, args.output, args.passes)
    for name in packed:
        print(f"layout_matmul: packed {name}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
