"""Invoke the XLA-CPU custom-call targets the way XLA's emitted code does.

XLA passes `void* out, const void** in`, where the operand list is the
fusion operands followed by one shape-info constant per fused parameter
(annc/service/hlo_util.h:14-33: s64[2*rank] = dims..., minor_to_major...).
These helpers build that list for numpy (host) or torch CUDA arrays and look
the target up through annc_custom_call_target(), i.e. by registered name.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import ptr

# Operand order of every target (gemm_rewriter.cc:136-281, graph_opt.cc:100-107).
TARGETS = ("__matmul", "__batch_matmul", "__matmul_add", "__matmul_add_relu", "__reduce_mean",
           "__pooling", "__layout_matmul")

_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p)


def shape_info(shape: Sequence[int]) -> np.ndarray:
    """get_param_info of a row-major (dim-0-major) operand."""
    rank = len(shape)
    return np.asarray(list(shape) + list(range(rank - 1, -1, -1)), dtype=np.int64)


def registered_targets() -> list[str]:
    names: list[str] = []
    cb_t = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_void_p)

    def cb(name, fn, user):
        names.append(name.decode())

    cb_c = cb_t(cb)
    _lib.lib().annc_register_custom_call_targets(ctypes.cast(cb_c, ctypes.c_void_p), None)
    return names


def call(target: str, out, operands: Sequence) -> None:
    """Run `target(out, in)` with `operands` in XLA operand order."""
    addr = _lib.lib().annc_custom_call_target(target.encode())
    if not addr:
        raise KeyError(f"unknown custom-call target {target!r}")
    arr = (ctypes.c_void_p * len(operands))(*[ptr(o) for o in operands])
    _FN(addr)(ptr(out), ctypes.addressof(arr))
    err = _lib.last_error()
    if err:
        raise _lib.AnncError(_lib.INTERNAL, f"{target}: {err}")


def _shape(x):
    return tuple(int(d) for d in x.shape)


def matmul(a, b, out):
    call("__matmul", out, [a, b, shape_info(_shape(a)), shape_info(_shape(b))])


def matmul_add(e, a, b, out):
    call("__matmul_add", out, [e, a, b, shape_info(_shape(e)), shape_info(_shape(a)),
                               shape_info(_shape(b))])


def matmul_add_relu(z, e, a, b, out):
    call("__matmul_add_relu", out, [z, e, a, b, shape_info(_shape(z)), shape_info(_shape(e)),
                                    shape_info(_shape(a)), shape_info(_shape(b))])


def batch_matmul(a, b, out):
    call("__batch_matmul", out, [a, b, shape_info(_shape(a)), shape_info(_shape(b))])


def layout_matmul(a, b_packed, k: int, n: int, out):
    call("__layout_matmul", out, [a, b_packed, shape_info(_shape(a)), shape_info((k, n))])


def reduce_mean(x, out, axis: float = 0.0):
    """__reduce_mean on x of shape (m, n): out (n values) gets, for each i,
    the mean of |x| over the i-th run of m consecutive values of x."""
    call("__reduce_mean", out, [np.asarray([axis], dtype=np.float32), x, shape_info((1,)),
                                shape_info(_shape(x))])


def pooling(ids, gathered, slice_starts, slice_limits, out):
    ss = np.asarray(slice_starts, dtype=np.int64)
    sl = np.asarray(slice_limits, dtype=np.int64)
    call("__pooling", out, [ids, gathered, ss, sl, shape_info(_shape(ids)),
                            shape_info(_shape(gathered))])
