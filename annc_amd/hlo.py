"""Which HLO fragments ANNC turns into fusions and custom calls.

Binding of ``annc_hlo_rewrite_instruction``, the library's restatement of
ANNC's KDnnRewriter selection (annc/service/cpu/kdnn_rewriter.cc:8-69,
gemm_rewriter.cc:13-134, graph_opt.cc:8-129) under the process-wide
ANNC_FLAGS set.  A :class:`Fragment` collects instructions in program order
(their index order is the users() order the patterns walk);
:func:`rewrite` reports the first rewriter that fires on one instruction.

:func:`dense_layer` builds the fragment XLA emits for
``act(x @ W + b)``: dot -> add(broadcast(b)) -> maximum(broadcast(0)) for
ReLU, the shape the GEMM patterns match.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Sequence

from . import _lib

MAX_RANK = 8
MAX_OPERANDS = 8
MAX_FUSED = 16

OPCODES = {
    "other": 0, "parameter": 1, "constant": 2, "dot": 3, "add": 4, "maximum": 5,
    "multiply": 6, "select": 7, "broadcast": 8, "gather": 9, "convert": 10, "and": 11,
    "compare": 12, "divide": 13, "reshape": 14, "reduce": 15, "slice": 16,
    "reduce-window": 17,
}
DTYPES = {"other": 0, "pred": 1, "s32": 2, "s64": 3, "f32": 4}


class _Node(ctypes.Structure):
    _fields_ = [("opcode", ctypes.c_int32), ("dtype", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("num_operands", ctypes.c_int32), ("dims", ctypes.c_int64 * MAX_RANK),
                ("minor_to_major", ctypes.c_int32 * MAX_RANK),
                ("operands", ctypes.c_int32 * MAX_OPERANDS),
                ("has_control_deps", ctypes.c_int32)]


class _Rewrite(ctypes.Structure):
    _fields_ = [("matched", ctypes.c_int32), ("target", ctypes.c_char * 32),
                ("custom_call", ctypes.c_int32), ("benefit", ctypes.c_int32),
                ("num_fused", ctypes.c_int32), ("fused", ctypes.c_int32 * MAX_FUSED),
                ("num_operands", ctypes.c_int32),
                ("operands", ctypes.c_int32 * (2 * MAX_OPERANDS)),
                ("num_shape_infos", ctypes.c_int32),
                ("shape_info_of", ctypes.c_int32 * (2 * MAX_OPERANDS))]


@dataclass
class Instr:
    opcode: str
    shape: tuple
    dtype: str = "f32"
    operands: tuple = ()
    minor_to_major: tuple | None = None  # None: row-major
    control_deps: bool = False


@dataclass
class Rewrite:
    target: str
    custom_call: bool
    benefit: int
    fused: list
    operands: list          # instruction indices; "slice_starts" / "slice_limits" constants
    shape_infos: list       # instruction index per s64[2*rank] shape-info operand


@dataclass
class Fragment:
    instrs: list = field(default_factory=list)

    def add(self, opcode: str, shape: Sequence[int], dtype: str = "f32",
            operands: Sequence[int] = (), minor_to_major: Sequence[int] | None = None,
            control_deps: bool = False) -> int:
        if opcode not in OPCODES:
            raise ValueError(f"unknown opcode {opcode!r}")
        if len(shape) > MAX_RANK or len(operands) > MAX_OPERANDS:
            raise ValueError("rank or operand count too large")
        self.instrs.append(Instr(opcode, tuple(int(d) for d in shape), dtype, tuple(operands),
                                 None if minor_to_major is None else tuple(minor_to_major),
                                 control_deps))
        return len(self.instrs) - 1

    def _nodes(self):
        arr = (_Node * len(self.instrs))()
        for i, ins in enumerate(self.instrs):
            nd = arr[i]
            nd.opcode = OPCODES[ins.opcode]
            nd.dtype = DTYPES.get(ins.dtype, 0)
            nd.rank = len(ins.shape)
            nd.num_operands = len(ins.operands)
            for d, v in enumerate(ins.shape):
                nd.dims[d] = v
            m2m = ins.minor_to_major or tuple(range(len(ins.shape) - 1, -1, -1))
            for d, v in enumerate(m2m):
                nd.minor_to_major[d] = v
            for k, o in enumerate(ins.operands):
                nd.operands[k] = o
            nd.has_control_deps = 1 if ins.control_deps else 0
        return arr


def rewrite(fragment: Fragment, instr: int) -> Rewrite | None:
    """The rewriter ANNC's visitor would apply to instruction `instr`
    (None when none fires), under the current ANNC_FLAGS."""
    nodes = fragment._nodes()
    out = _Rewrite()
    _lib.check(_lib.lib().annc_hlo_rewrite_instruction(ctypes.addressof(nodes),
                                                       len(fragment.instrs), instr,
                                                       ctypes.addressof(out)))
    if not out.matched:
        return None
    names = {-1: "slice_starts", -2: "slice_limits"}
    return Rewrite(out.target.decode(), bool(out.custom_call), out.benefit,
                   list(out.fused[:out.num_fused]),
                   [names.get(o, o) for o in out.operands[:out.num_operands]],
                   list(out.shape_info_of[:out.num_shape_infos]))


def dense_layer(m: int, k: int, n: int, activation: str = "relu", weight_parameter: bool = True,
                bias: bool = True, fragment: Fragment | None = None, x: int | None = None):
    """Append the HLO of act(x @ W + b) for x f32[m, k], W f32[k, n].

    Returns (fragment, dot index, output index).  ReLU is
    maximum(add, broadcast(0)); sigmoid is a logistic-like `other` user.
    """
    f = fragment or Fragment()
    if x is None:
        x = f.add("parameter", (m, k))
    w = f.add("parameter" if weight_parameter else "constant", (k, n))
    dot = f.add("dot", (m, n), operands=(x, w))
    h = dot
    if bias:
        b = f.add("parameter", (n,))
        bb = f.add("broadcast", (m, n), operands=(b,))
        h = f.add("add", (m, n), operands=(dot, bb))
    if activation == "relu":
        z = f.add("constant", (), operands=())
        zb = f.add("broadcast", (m, n), operands=(z,))
        h = f.add("maximum", (m, n), operands=(h, zb))
    elif activation == "sigmoid":
        h = f.add("other", (m, n), operands=(h,))
    return f, dot, h
