"""ctypes binding of libannc_hip.so (the C-ABI declared in include/annc_hip.h).

The library is built in-tree (``make -C annc_amd/csrc``); importing a
function that needs it raises ``LibraryNotBuilt`` when the shared object is
missing.  There is no CPU fallback: every compute entry point runs the
gfx950 kernels.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libannc_hip.so")

# TensorFlow error codes used by the C-ABI.
OK = 0
INVALID_ARGUMENT = 3
RESOURCE_EXHAUSTED = 8
INTERNAL = 13

EPI_NONE = 0
EPI_RELU = 1
EPI_SIGMOID = 2
COMBINER_SUM = 0
COMBINER_MEAN = 1


class LibraryNotBuilt(ImportError):
    pass


class AnncError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code
        self.message = message


class InvalidArgumentError(AnncError):
    pass


_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_cp = ctypes.c_char_p

# name -> (restype, argtypes)
_PROTOTYPES = {
    "annc_hip_last_error": (_cp, []),
    "annc_hip_version": (_cp, []),
    "annc_hip_stream_status": (_i32, [_c_void_p]),
    "annc_flag_enabled": (_i32, [_cp]),
    "annc_flags_reset": (None, [_cp]),
    "annc_flags_dump": (_i64, [_c_void_p, _i64]),
    "__matmul": (None, [_c_void_p, _c_void_p]),
    "__matmul_add": (None, [_c_void_p, _c_void_p]),
    "__matmul_add_relu": (None, [_c_void_p, _c_void_p]),
    "__batch_matmul": (None, [_c_void_p, _c_void_p]),
    "__layout_matmul": (None, [_c_void_p, _c_void_p]),
    "__pooling": (None, [_c_void_p, _c_void_p]),
    "__reduce_mean": (None, [_c_void_p, _c_void_p]),
    "annc_custom_call_target": (_c_void_p, [_cp]),
    "annc_register_custom_call_targets": (_i32, [_c_void_p, _c_void_p]),
    "annc_layout_matmul_rhs_format": (_cp, []),
    "annc_layout_matmul_pack_rhs": (_i32, [_i64, _i64, _c_void_p, _c_void_p]),
    "annc_layout_matmul_unpack_rhs": (_i32, [_i64, _i64, _c_void_p, _c_void_p]),
    "annc_hip_layout_matmul_pack_rhs": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "annc_hip_gemm": (_i32, [_c_void_p, _i64, _i64, _i64, _i64,
                             _c_void_p, _i64, _i64,
                             _c_void_p, _i64, _i64, _i32,
                             _c_void_p, _i64, _i64,
                             _c_void_p, _i32,
                             _c_void_p, _i64, _i64]),
    "annc_hip_dense_score": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64,
                                    _c_void_p, _c_void_p, _i32,
                                    _c_void_p, _c_void_p, _i32,
                                    _c_void_p, _i64, _c_void_p, _i64]),
    "annc_hip_embedding_bag": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i32,
                                      _c_void_p, _i64, _i32, _c_void_p, _i64]),
    "annc_hip_segment_reduce": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i32,
                                       _c_void_p, _i64, _i64, _i32, _i64, _c_void_p, _i32]),
    "annc_hip_segment_reduce_noalloc": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p,
                                               _i32, _c_void_p, _i64, _i64, _i32, _i64,
                                               _c_void_p, _i32, _c_void_p]),
    "annc_hip_sparse_embedding2": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i32,
                                          _i64, _i64, _c_void_p]),
    "annc_hip_pooling": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                _c_void_p, _c_void_p, _c_void_p]),
    "annc_hip_fingerprint64": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _c_void_p]),
    "annc_hip_hash_bucket_strings": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32,
                                            _c_void_p]),
    "annc_hip_hash_bucket_int64": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "annc_hip_hashed_embedding_bags": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p,
                                              _c_void_p, _c_void_p, _c_void_p, _i32, _c_void_p,
                                              _i64, _c_void_p]),
    "annc_hip_unique_gather": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
                                      _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "annc_kp_fused_gather": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _i32, _c_void_p,
                                    _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "annc_kp_fused_batch_matmul_add_sigmoid": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p,
                                                      _i32, _c_void_p, _c_void_p, _i32,
                                                      _c_void_p, _c_void_p]),
    "annc_kp_fused_sparse_segment_reduce": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _i32,
                                                   _i64, _c_void_p, _i32, _c_void_p, _c_void_p,
                                                   _i64, _c_void_p, _i64, _i32, _c_void_p,
                                                   _c_void_p, _c_void_p]),
    "annc_kp_fused_sparse_segment_reduce_nonzero": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p,
                                                           _i32, _i64, _c_void_p, _i32,
                                                           _c_void_p, _c_void_p, _i64, _i32,
                                                           _c_void_p, _c_void_p, _c_void_p,
                                                           _c_void_p]),
    "annc_kp_fused_embedding_with_hash_bucket": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p,
                                                        _i64, _i64, _i64, _i32, _c_void_p]),
    "annc_kp_fused_dnn_embedding_with_hash_bucket": (_i32, [_c_void_p, _c_void_p, _i64,
                                                            _c_void_p, _i64, _i64, _i64,
                                                            _c_void_p]),
    "annc_kp_fused_linear_embedding_with_hash_bucket": (_i32, [_c_void_p, _c_void_p, _i64,
                                                               _c_void_p, _i64, _i64, _i64,
                                                               _c_void_p]),
    "annc_kp_fused_sparse_embedding": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p,
                                              _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "annc_hlo_rewrite_instruction": (_i32, [_c_void_p, _i64, _i32, _c_void_p]),
}

_lock = threading.Lock()
_lib = None


def exported_names():
    return list(_PROTOTYPES)


def lib() -> ctypes.CDLL:
    """The loaded library (raises LibraryNotBuilt when absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise LibraryNotBuilt(
                f"{LIB_PATH} is missing: build it with `make -C annc_amd/csrc` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().annc_hip_last_error().decode()


def check(code: int) -> None:
    """Raise the matching AnncError for a non-zero C-ABI status."""
    if code == OK:
        return
    msg = last_error()
    if code == INVALID_ARGUMENT:
        raise InvalidArgumentError(code, msg)
    raise AnncError(code, msg)


def ptr(x) -> int | None:
    """Raw address of a torch tensor, numpy array, ctypes buffer or int."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    dp = getattr(x, "data_ptr", None)
    if dp is not None:
        return dp()
    iface = getattr(x, "__array_interface__", None)
    if iface is not None:
        return iface["data"][0]
    return ctypes.addressof(x)


def stream_ptr(stream=None) -> int | None:
    """HIP stream handle: explicit torch stream, else torch's current stream."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream
