"""ctypes binding of oracle/libannc_oracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of ANNC's hot path that the GPU library is checked
against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg import this module; the product package (annc_amd) never does.
"""
from __future__ import annotations

import ctypes
import glob
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libannc_oracle.so")
REF_FLAGS_PATH = os.path.join(HERE, "_ref", "libref_flags.so")

_v = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float

_PROTO = {
    "ora_fingerprint64": (_u64, [ctypes.c_char_p, ctypes.c_size_t]),
    "ora_fingerprint64_batch": (None, [_v, _v, _i64, _i32, _v]),
    "ora_format_int64": (_i32, [_i64, ctypes.c_char_p]),
    "ora_hash_bucket_strings": (None, [_v, _v, _i64, _i64, _i32, _v]),
    "ora_hash_bucket_int64": (None, [_v, _i64, _i64, _v]),
    "ora_segment_reduce": (None, [_v, _i64, _i64, _v, _i32, _v, _i64, _i64, _i32, _i64, _v]),
    "ora_embedding_bag": (None, [_v, _i64, _i64, _v, _i32, _v, _i64, _i32, _v, _i64, _i32]),
    "ora_segment_reduce_nonzero": (_i64, [_v, _i64, _i64, _v, _i32, _v, _i64, _i64, _i32, _i32,
                                          _v, _v, _v, _i64]),
    "ora_pooling": (None, [_v, _v, _i64, _i64, _i64, _v, _v, _v]),
    "ora_reduce_mean": (None, [_v, _i64, _i64, _v]),
    "ora_sparse_embedding2": (None, [_v, _i64, _i64, _v, _i32, _i64, _i64, _v]),
    "ora_fused_gather": (_i64, [_v, _i64, _i64, _v, _i64, _i64, _v, _v, _v]),
    "ora_batch_matmul_add_sigmoid": (None, [_v, _v, _i32, _v, _v, _i64, _i64, _i64, _i64, _v]),
    "ora_embedding_with_hash_bucket": (None, [_v, _v, _i64, _v, _i64, _i64, _v]),
    "ora_dnn_embedding_with_hash_bucket": (None, [_v, _v, _i64, _v, _i64, _i64, _i64, _v]),
    "ora_sparse_embedding": (None, [_v, _v, _i64, _i64, _v, _v, _v, _v, _v]),
    "ora_hashed_embedding_bags": (None, [_i64, _i64, _i64, _v, _v, _v, _v, _i32, _v, _i64, _v,
                                         _i32]),
    "ora_blas_load": (_i32, [ctypes.c_char_p]),
    "ora_blas_config": (ctypes.c_char_p, []),
    "ora_blas_set_threads": (None, [_i32]),
    "ora_sgemm": (_i32, [_i64, _i64, _i64, _f32, _v, _i64, _v, _i64, _f32, _v, _i64]),
    "ora_matmul": (_i32, [_i64, _i64, _i64, _v, _v, _v]),
    "ora_matmul_add": (_i32, [_i64, _i64, _i64, _v, _v, _v, _v]),
    "ora_matmul_add_relu": (_i32, [_i64, _i64, _i64, _v, _v, _v, _v]),
    "ora_batch_matmul": (_i32, [_i64, _i64, _i64, _i64, _v, _v, _v]),
    "ora_dense_layer": (_i32, [_i64, _i64, _i64, _v, _i64, _v, _v, _i32, _v]),
}

_lib = None


def build() -> None:
    """Compile the oracle (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def openblas_path() -> str | None:
    import numpy

    libs = glob.glob(os.path.join(os.path.dirname(numpy.__file__), "..", "numpy.libs",
                                  "libscipy_openblas64_*.so"))
    return os.path.abspath(libs[0]) if libs else None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _PROTO.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        path = openblas_path()
        if path is None or h.ora_blas_load(path.encode()) != 0:
            raise RuntimeError("OpenBLAS (numpy's scipy_openblas64_) not found for the oracle")
        _lib = h
    return _lib


def blas_config() -> str:
    return lib().ora_blas_config().decode()


def set_threads(n: int) -> None:
    lib().ora_blas_set_threads(int(n))


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- hashing
def fingerprint64(s: bytes) -> int:
    return int(lib().ora_fingerprint64(s, len(s)))


def format_int64(v: int) -> bytes:
    buf = ctypes.create_string_buffer(32)
    n = lib().ora_format_int64(int(v), buf)
    return buf.raw[:n]


def pack_strings(strings):
    enc = [s.encode() if isinstance(s, str) else bytes(s) for s in strings]
    offsets = np.zeros(len(enc) + 1, dtype=np.int64)
    if enc:
        np.cumsum([len(s) for s in enc], out=offsets[1:])
    blob = np.frombuffer(b"".join(enc) + b"\0", dtype=np.uint8).copy()
    return blob, offsets


def fingerprint64_batch(strings, nul_terminated=False) -> np.ndarray:
    blob, off = pack_strings(strings)
    out = np.empty(len(off) - 1, dtype=np.uint64)
    lib().ora_fingerprint64_batch(_p(blob), _p(off), len(off) - 1, int(nul_terminated), _p(out))
    return out


def hash_bucket_strings(strings, num_buckets, nul_terminated=False) -> np.ndarray:
    blob, off = pack_strings(strings)
    out = np.empty(len(off) - 1, dtype=np.int64)
    lib().ora_hash_bucket_strings(_p(blob), _p(off), len(off) - 1, int(num_buckets),
                                  int(nul_terminated), _p(out))
    return out


def hash_bucket_int64(ids, num_buckets) -> np.ndarray:
    ids = _c(ids, np.int64)
    out = np.empty_like(ids)
    lib().ora_hash_bucket_int64(_p(ids), ids.size, int(num_buckets), _p(out))
    return out


# ---------------------------------------------------------------- segments
def segment_reduce(data, indices, seg, batch, combiner) -> np.ndarray:
    data = _c(data, np.float32)
    idx64 = indices.dtype == np.int64
    indices = _c(indices, np.int64 if idx64 else np.int32)
    seg = _c(seg, np.int64)
    out = np.empty((batch, data.shape[1]), dtype=np.float32)
    lib().ora_segment_reduce(_p(data), data.shape[0], data.shape[1], _p(indices), int(idx64),
                             _p(seg), 1, indices.size, int(combiner), int(batch), _p(out))
    return out


def segment_reduce_nonzero(data, indices, seg, combiner):
    """KPFusedSparseSegmentReduceNonzero: (output_shape int32, output_indices
    int32 [nnz, 1 or 2], output_nonzero float32 [nnz]); data 1-D or 2-D."""
    data = _c(data, np.float32)
    one_d = data.ndim == 1
    data2 = data.reshape(data.shape[0], -1) if data.size else data.reshape(data.shape[0], 1)
    idx64 = indices.dtype == np.int64
    indices = _c(indices, np.int64 if idx64 else np.int32)
    seg = _c(seg, np.int64)
    n, dim = indices.size, data2.shape[1]
    width = 1 if one_d else 2
    shape = np.zeros(2, np.int32)
    cap = max(n * dim, 1)
    idx = np.empty(cap * width, np.int32)
    val = np.empty(cap, np.float32)
    nz = lib().ora_segment_reduce_nonzero(_p(data2), data2.shape[0], dim, _p(indices), int(idx64), _p(seg), 1, n, int(combiner),
           int(one_d), _p(shape), _p(idx), _p(val), cap)
    return (shape[:1 if one_d else 2].copy(), idx[:nz * width].reshape(nz, width).copy(),
            val[:nz].copy())


def embedding_bag(table, ids, offsets, combiner, threads=1) -> np.ndarray:
    idx64 = ids.dtype == np.int64
    ids = _c(ids, np.int64 if idx64 else np.int32)
    offsets = _c(offsets, np.int64)
    nb = offsets.size - 1
    out = np.empty((nb, table.shape[1]), dtype=np.float32)
    lib().ora_embedding_bag(_p(table), table.shape[0], table.shape[1], _p(ids), int(idx64),
                            _p(offsets), nb, int(combiner), _p(out), table.shape[1], int(threads))
    return out


def reduce_mean(x) -> np.ndarray:
    """__reduce_mean on x [m, n]: n means of |x| over runs of m values."""
    x = _c(x, np.float32)
    m, n = x.shape
    out = np.empty(n, dtype=np.float32)
    lib().ora_reduce_mean(_p(x), m, n, _p(out))
    return out


def pooling(ids, gathered, ss, sl) -> np.ndarray:
    ids = _c(ids, np.int64)
    gathered = _c(gathered, np.float32)
    m, k = ids.shape
    n = gathered.shape[2]
    ss = _c(ss, np.int64)
    sl = _c(sl, np.int64)
    out = np.empty((m, n), dtype=np.float32)
    lib().ora_pooling(_p(ids), _p(gathered), m, k, n, _p(ss), _p(sl), _p(out))
    return out


def fused_gather(table, keys2d, col):
    """KPFusedGather: (unique int64[U], indices int32[N], rows [U, D]); raises
    IndexError for a unique key outside the table."""
    table = _c(table, np.float32)
    keys2d = _c(keys2d, np.int64)
    n, c = keys2d.shape
    uniq = np.empty(max(n, 1), np.int64)
    idx = np.empty(n, np.int32)
    out = np.empty((max(n, 1), table.shape[1]), np.float32)
    u = lib().ora_fused_gather(_p(table), table.shape[0], table.shape[1],
                               keys2d.ctypes.data + 8 * col, c, n, _p(uniq), _p(idx), _p(out))
    if u < 0:
        raise IndexError("idx out of table range")
    return uniq[:u].copy(), idx, out[:u].copy()


def batch_matmul_add_sigmoid(lhs, rhs, bias) -> np.ndarray:
    lhs = _c(lhs, np.float32)
    rhs = _c(rhs, np.float32)
    bias = _c(bias, np.float32)
    b, m, k = lhs.shape
    n = rhs.shape[-1]
    bd = np.ones(3, np.int64)
    if bias.ndim:
        bd[3 - bias.ndim:] = bias.shape
    out = np.empty((b, m, n), np.float32)
    lib().ora_batch_matmul_add_sigmoid(_p(lhs), _p(rhs), int(rhs.ndim == 3), _p(bias), _p(bd),
                                       b, m, k, n, _p(out))
    return out


def sparse_embedding2(table, ids, fallback=0) -> np.ndarray:
    table = _c(table, np.float32)
    idx64 = ids.dtype == np.int64
    ids = _c(ids, np.int64 if idx64 else np.int32)
    out = np.empty((ids.size, table.shape[1]), dtype=np.float32)
    lib().ora_sparse_embedding2(_p(table), table.shape[0], table.shape[1], _p(ids), int(idx64),
                                ids.size, int(fallback), _p(out))
    return out


def embedding_with_hash_bucket(strings, weight, num_buckets) -> np.ndarray:
    blob, off = pack_strings(strings)
    weight = _c(weight, np.float32)
    out = np.empty((len(off) - 1, weight.shape[1]), dtype=np.float32)
    lib().ora_embedding_with_hash_bucket(_p(blob), _p(off), len(off) - 1, _p(weight),
                                         weight.shape[1], int(num_buckets), _p(out))
    return out


def dnn_embedding_with_hash_bucket(strings, weight, num_buckets) -> np.ndarray:
    blob, off = pack_strings(strings)
    weight = _c(weight, np.float32)
    out = np.empty((len(off) - 1, weight.shape[1]), dtype=np.float32)
    lib().ora_dnn_embedding_with_hash_bucket(_p(blob), _p(off), len(off) - 1, _p(weight),
                                             weight.shape[0], weight.shape[1], int(num_buckets),
                                             _p(out))
    return out


def sparse_embedding(strings, num_buckets):
    blob, off = pack_strings(strings)
    n = len(off) - 1
    idx = np.empty((n, 2), dtype=np.int64)
    vals = np.empty(max(n, 1), dtype=np.int64)
    empty = np.empty(max(n, 1), dtype=np.uint8)
    shape = np.empty(2, dtype=np.int64)
    nv = np.zeros(1, dtype=np.int64)
    lib().ora_sparse_embedding(_p(blob), _p(off), n, int(num_buckets), _p(idx), _p(vals),
                               _p(empty), _p(shape), _p(nv))
    v = int(nv[0])
    return idx, vals[:v].copy(), empty[:v].astype(bool), shape


def hashed_embedding_bags(tables, num_buckets, ids, offsets, batch, combiner, threads=1,
                          with_buckets=False):
    nf = len(tables)
    dim = tables[0].shape[1]
    tptr = np.asarray([t.ctypes.data for t in tables], dtype=np.uint64)
    nb = np.asarray([num_buckets] * nf if np.isscalar(num_buckets) else num_buckets,
                    dtype=np.int64)
    ids = _c(ids, np.int64)
    offsets = _c(offsets, np.int64)
    out = np.empty((batch, nf * dim), dtype=np.float32)
    buckets = np.empty(ids.size, dtype=np.int64) if with_buckets else None
    lib().ora_hashed_embedding_bags(nf, batch, dim, _p(tptr), _p(nb), _p(ids), _p(offsets),
                                    int(combiner), _p(out), nf * dim, _p(buckets), int(threads))
    return (out, buckets) if with_buckets else out


# ---------------------------------------------------------------- GEMM
def matmul(a, b) -> np.ndarray:
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty((a.shape[0], b.shape[1]), dtype=np.float32)
    assert lib().ora_matmul(a.shape[0], b.shape[1], a.shape[1], _p(a), _p(b), _p(out)) == 0
    return out


def matmul_add(e, a, b) -> np.ndarray:
    a, b, e = _c(a, np.float32), _c(b, np.float32), _c(e, np.float32)
    out = np.empty((a.shape[0], b.shape[1]), dtype=np.float32)
    assert lib().ora_matmul_add(a.shape[0], b.shape[1], a.shape[1], _p(e), _p(a), _p(b),
                                _p(out)) == 0
    return out


def matmul_add_relu(e, a, b) -> np.ndarray:
    a, b, e = _c(a, np.float32), _c(b, np.float32), _c(e, np.float32)
    out = np.empty((a.shape[0], b.shape[1]), dtype=np.float32)
    assert lib().ora_matmul_add_relu(a.shape[0], b.shape[1], a.shape[1], _p(e), _p(a), _p(b),
                                     _p(out)) == 0
    return out


def batch_matmul(a, b) -> np.ndarray:
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty((a.shape[0], a.shape[1], b.shape[2]), dtype=np.float32)
    assert lib().ora_batch_matmul(a.shape[0], a.shape[1], b.shape[2], a.shape[2], _p(a), _p(b),
                                  _p(out)) == 0
    return out


def dense_layer(a, w, bias, act, lda=None) -> np.ndarray:
    """sgemm then bias and activation loops (act: 0 none, 1 relu, 2 sigmoid)."""
    w = _c(w, np.float32)
    m = a.shape[0]
    k, n = w.shape
    if lda is None:
        a = _c(a, np.float32)
        lda = k
    out = np.empty((m, n), dtype=np.float32)
    b = None if bias is None else _c(bias, np.float32)
    assert lib().ora_dense_layer(m, n, k, _p(a), lda, _p(w), _p(b), int(act), _p(out)) == 0
    return out


def mlp_tower(x, weights, biases) -> np.ndarray:
    h = x
    for i, (w, b) in enumerate(zip(weights, biases)):
        h = dense_layer(h, w, b, 2 if i == len(weights) - 1 else 1)
    return h


# ---------------------------------------------------------------- reference flags
_ref_flags = None


def ref_flag_enabled(flags: str, name: str) -> bool | None:
    """The reference's own parser (oracle/_ref), or None when not built."""
    global _ref_flags
    if _ref_flags is None:
        if not os.path.exists(REF_FLAGS_PATH):
            return None
        h = ctypes.CDLL(REF_FLAGS_PATH)
        h.ref_flag_enabled.restype = _i32
        h.ref_flag_enabled.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
        _ref_flags = h
    return bool(_ref_flags.ref_flag_enabled(flags.encode(), name.encode()))
