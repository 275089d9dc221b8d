"""Python mirror of ANNC's TensorFlow custom ops on the gfx950 library.

TensorFlow is not installed, so each REGISTER_OP is a function with the same
inputs, attributes and error messages; arrays may be numpy (host memory, as
TF CPU tensors) or torch CUDA tensors.  Invalid inputs raise
``InvalidArgumentError`` carrying the reference's OP_REQUIRES text.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np

from . import _lib
from ._lib import InvalidArgumentError, check, ptr

__all__ = [
    "kp_fused_sparse_segment_reduce",
    "kp_fused_embedding_with_hash_bucket",
    "kp_fused_dnn_embedding_with_hash_bucket",
    "kp_fused_linear_embedding_with_hash_bucket",
    "kp_fused_sparse_embedding",
    "kp_fused_gather",
    "kp_fused_batch_matmul_add_sigmoid",
    "InvalidArgumentError",
]


def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


def _dims(x) -> np.ndarray:
    return np.asarray(tuple(x.shape), dtype=np.int64)


def _empty_like_kind(ref, shape, np_dtype):
    if _is_torch(ref):
        import torch

        tdt = {np.float32: torch.float32, np.int32: torch.int32, np.int64: torch.int64}[np_dtype]
        return torch.empty(shape, dtype=tdt, device=ref.device)
    return np.empty(shape, dtype=np_dtype)


def _as_host_i32(x) -> np.ndarray:
    if _is_torch(x):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


def _contig(x):
    if _is_torch(x):
        return x.contiguous()
    return np.ascontiguousarray(x)


def kp_fused_sparse_segment_reduce(data, indices, slice_input, begin, begin_1, combiner: int = 1):
    """KPFusedSparseSegmentReduce
    (annc/tensorflow/ops/embedding_fused_ops.cc:29-39,
     annc/tensorflow/kernels/embedding_fused_sparse_segment_reduce.cc:27-164).

    Returns (output [max_seg+1, D] float32, slice_output int32 scalar).
    """
    lib = _lib.lib()
    data = _contig(data)
    indices = _contig(indices)
    slice_input = _contig(slice_input)
    begin_h = _as_host_i32(begin).reshape(-1)
    begin1_h = _as_host_i32(begin_1).reshape(-1)
    idx64 = str(indices.dtype).endswith("int64")
    if not idx64 and not str(indices.dtype).endswith("int32"):
        raise TypeError("indices must be int32 or int64 (attr Tidx)")
    ddims = _dims(data)
    sdims = _dims(slice_input)
    num_indices = int(indices.shape[0]) if len(indices.shape) else 0
    rows = np.zeros(1, dtype=np.int64)
    args = (ptr(data), len(data.shape), ptr(ddims), ptr(indices), 1 if idx64 else 0, num_indices,
            ptr(slice_input), len(slice_input.shape), ptr(sdims), ptr(begin_h), begin_h.size,
            ptr(begin1_h), begin1_h.size, int(combiner), ptr(rows))
    check(lib.annc_kp_fused_sparse_segment_reduce(*args, None, None))
    batch = int(rows[0])
    dim = int(ddims[1])
    out = _empty_like_kind(data, (batch, dim), np.float32)
    slice_out = np.zeros(1, dtype=np.int32)
    check(lib.annc_kp_fused_sparse_segment_reduce(*args, ptr(out), ptr(slice_out)))
    return out, np.int32(slice_out[0])


def kp_fused_sparse_segment_reduce_nonzero(data, indices, slice_input, begin, combiner: int = 1):
    """KPFusedSparseSegmentReduceNonzero
    (annc/tensorflow/ops/embedding_fused_ops.cc:41-51,
     annc/tensorflow/kernels/embedding_fused_sparse_segment_reduce_nonzero.cc:39-372).

    Returns (output_shape int32 [1] or [2], output_indices int32 [nnz, 1]
    (1-D data) or [nnz, 2] (2-D data), output_nonzero float32 [nnz]): the
    segment reductions' values != 0, segments in order of first appearance.
    """
    lib = _lib.lib()
    data = _contig(data)
    indices = _contig(indices)
    slice_input = _contig(slice_input)
    begin_h = _as_host_i32(begin).reshape(-1)
    idx64 = str(indices.dtype).endswith("int64")
    if not idx64 and not str(indices.dtype).endswith("int32"):
        raise TypeError("indices must be int32 or int64 (attr Tidx)")
    ddims = _dims(data)
    sdims = _dims(slice_input)
    num_indices = int(indices.shape[0]) if len(indices.shape) else 0
    shape = np.zeros(2, dtype=np.int32)
    nnz = np.zeros(1, dtype=np.int64)
    args = (ptr(data), len(data.shape), ptr(ddims), ptr(indices), 1 if idx64 else 0, num_indices,
            ptr(slice_input), len(slice_input.shape), ptr(sdims), ptr(begin_h), begin_h.size,
            int(combiner), ptr(shape), ptr(nnz))
    check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(*args, None, None))
    count = int(nnz[0])
    width = 1 if len(data.shape) == 1 else 2
    out_idx = _empty_like_kind(data, (count, width), np.int32)
    out_val = _empty_like_kind(data, (count,), np.float32)
    if count:
        check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(*args, ptr(out_idx), ptr(out_val)))
    return shape[:width].copy(), out_idx, out_val


def kp_fused_gather(data, slice_input, begin):
    """KPFusedGather (annc/tensorflow/ops/embedding_fused_ops.cc:114-121,
    annc/tensorflow/kernels/embedding_fused_gather.cc:26-85).

    Returns (out_shape int64[U]: the distinct keys of column begin[1] in order
    of first occurrence, out_indices int32[N], out_data float32[U, D]), as
    host arrays for a host table and device tensors for a device one.
    Errors raise AnncError (code 13, errors::Internal) with the reference text.
    """
    lib = _lib.lib()
    data = _contig(data)
    slice_input = _contig(slice_input)
    begin_h = _as_host_i32(begin).reshape(-1)
    ddims = _dims(data)
    sdims = _dims(slice_input)
    nu = np.zeros(1, dtype=np.int64)
    args = (ptr(data), len(data.shape), ptr(ddims), ptr(slice_input), len(slice_input.shape),
            ptr(sdims), ptr(begin_h), begin_h.size, ptr(nu))
    n = int(sdims[0]) if sdims.size else 0
    dim = int(ddims[1]) if ddims.size == 2 else 0
    # outputs sized for every key being distinct, trimmed to U afterwards;
    # device tables give device outputs (no copy through pageable memory)
    uniq = _empty_like_kind(data, (max(n, 1),), np.int64)
    idx = _empty_like_kind(data, (n,), np.int32)
    out = _empty_like_kind(data, (max(n, 1), dim), np.float32)
    check(lib.annc_kp_fused_gather(*args, ptr(uniq), ptr(idx), ptr(out)))
    u = int(nu[0])
    return (uniq[:u].copy() if isinstance(uniq, np.ndarray) else uniq[:u]), idx, out[:u]


def kp_fused_batch_matmul_add_sigmoid(lhs, rhs, bias):
    """KPFusedBatchMatMulAddSigmoid (annc/tensorflow/ops/embedding_fused_ops.cc:134-139,
    annc/tensorflow/kernels/fused_batchmatmul_add_sigmoid.cc):
    sigmoid(bias + lhs @ rhs) -> float32 [batch, m, n]."""
    lib = _lib.lib()
    lhs, rhs, bias = _contig(lhs), _contig(rhs), _contig(bias)
    ld, rd, bd = _dims(lhs), _dims(rhs), _dims(bias)
    if len(lhs.shape) == 3 and len(rhs.shape) in (2, 3):
        n = int(rd[-1])
        shape = (int(ld[0]), int(ld[1]), n)
    else:
        shape = (0,)
    out = _empty_like_kind(lhs, shape, np.float32)
    check(lib.annc_kp_fused_batch_matmul_add_sigmoid(
        ptr(lhs), len(lhs.shape), ptr(ld), ptr(rhs), len(rhs.shape), ptr(rd), ptr(bias),
        len(bias.shape), ptr(bd) if bd.size else None, ptr(out)))
    return out


def _pack_strings(strings: Sequence[bytes | str]):
    enc = [s.encode() if isinstance(s, str) else bytes(s) for s in strings]
    offsets = np.zeros(len(enc) + 1, dtype=np.int64)
    if enc:
        np.cumsum([len(s) for s in enc], out=offsets[1:])
    blob = np.frombuffer(b"".join(enc) + b"\0", dtype=np.uint8).copy()
    return blob, offsets


def _dense_hash_op(fn_name, strings, weight, num_buckets, *extra):
    if num_buckets < 1:
        raise InvalidArgumentError(_lib.INVALID_ARGUMENT, "num_buckets must be >= 1")
    blob, offsets = _pack_strings(strings)
    weight = _contig(weight)
    rows, dim = int(weight.shape[0]), int(weight.shape[1])
    out = _empty_like_kind(weight, (len(offsets) - 1, dim), np.float32)
    fn = getattr(_lib.lib(), fn_name)
    check(fn(ptr(blob), ptr(offsets), len(offsets) - 1, ptr(weight), rows, dim, int(num_buckets),
             *extra, ptr(out)))
    return out


def kp_fused_embedding_with_hash_bucket(strings, weight, num_buckets: int, combiner: int = 0):
    """KPFusedEmbeddingWithHashBucket
    (python/tensorflow/kernels/fused_embedding_with_hash_bucket.cc:15-83)."""
    return _dense_hash_op("annc_kp_fused_embedding_with_hash_bucket", strings, weight,
                          num_buckets, int(combiner))


def kp_fused_dnn_embedding_with_hash_bucket(strings, weight, num_buckets: int):
    """KPFusedDnnEmbeddingWithHashBucket (fused_dnn_embedding_with_hash_bucket.cc:10-62)."""
    return _dense_hash_op("annc_kp_fused_dnn_embedding_with_hash_bucket", strings, weight,
                          num_buckets)


def kp_fused_linear_embedding_with_hash_bucket(strings, weight, num_buckets: int):
    """KPFusedLinearEmbeddingWithHashBucket (fused_linear_embdedding_with_hash_bucket.cc:13-72)."""
    return _dense_hash_op("annc_kp_fused_linear_embedding_with_hash_bucket", strings, weight,
                          num_buckets)


def kp_fused_sparse_embedding(strings, num_buckets: int):
    """KPFusedSparseEmbedding (fused_sparse_embedding.cc:10-87).

    Returns (indices int64[n,2], values int64[v], empty_row_indicator bool[v],
    dense_shape int64[2]).
    """
    if num_buckets < 1:
        raise InvalidArgumentError(_lib.INVALID_ARGUMENT, "num_buckets must be >= 1")
    blob, offsets = _pack_strings(strings)
    n = len(offsets) - 1
    indices = np.empty((n, 2), dtype=np.int64)
    values = np.empty(max(n, 1), dtype=np.int64)
    empty = np.empty(max(n, 1), dtype=np.uint8)
    shape = np.empty(2, dtype=np.int64)
    nv = np.zeros(1, dtype=np.int64)
    check(_lib.lib().annc_kp_fused_sparse_embedding(ptr(blob), ptr(offsets), n, int(num_buckets),
                                                    ptr(indices), ptr(values), ptr(empty),
                                                    ptr(shape), ptr(nv)))
    v = int(nv[0])
    return indices, values[:v].copy(), empty[:v].astype(bool), shape
