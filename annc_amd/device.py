"""Device-pointer entry points on torch tensors (all operands on one GPU).

Thin wrappers over the asynchronous C-ABI functions of include/annc_hip.h:
they check shapes, dtypes and placement on the host, then enqueue the
gfx950 kernels on torch's current stream (or the stream passed in).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch

from . import _lib
from ._lib import check, ptr, stream_ptr


def _require_cuda(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError("device entry points take CUDA (HIP) torch tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all operands must live on the same GPU")
    return dev


def _row_major_2d(t: torch.Tensor, name: str):
    if t.dim() < 2 or t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit stride in its last dimension")
    return t.stride(-2)


@dataclass
class PackedWeight:
    """A [k, n] weight in layout_matmul (MFMA fragment) order."""

    data: torch.Tensor  # k*n float32 elements, 16-byte aligned
    k: int
    n: int
    rhs_format: str = "mfma_f32_32x32x2_k16"


def pack_weight(w: torch.Tensor, stream=None) -> PackedWeight:
    """Pre-pack a row-major [k, n] float32 weight on the GPU."""
    _require_cuda(w)
    if w.dtype != torch.float32 or w.dim() != 2:
        raise ValueError("pack_weight takes a 2-D float32 tensor")
    w = w.contiguous()
    k, n = w.shape
    out = torch.empty(k * n, dtype=torch.float32, device=w.device)
    check(_lib.lib().annc_hip_layout_matmul_pack_rhs(stream_ptr(stream), k, n, ptr(w), ptr(out)))
    return PackedWeight(out, k, n)


def pack_weight_host(w: np.ndarray) -> np.ndarray:
    """Pre-pack on the host (the annc-opt step); returns k*n float32."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    k, n = w.shape
    out = np.empty(k * n, dtype=np.float32)
    check(_lib.lib().annc_layout_matmul_pack_rhs(k, n, ptr(w), ptr(out)))
    return out


def unpack_weight_host(packed: np.ndarray, k: int, n: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.float32).reshape(-1)
    out = np.empty((k, n), dtype=np.float32)
    check(_lib.lib().annc_layout_matmul_unpack_rhs(k, n, ptr(packed), ptr(out)))
    return out


def gemm(a: torch.Tensor, b, *, addend: torch.Tensor | None = None,
         bias: torch.Tensor | None = None, epilogue: int = _lib.EPI_NONE,
         out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """out = epi(a @ b (+ addend) (+ bias)) on fp32 MFMA.

    a: [M, K] or [batch, M, K]; b: [K, N], [batch, K, N] or PackedWeight.
    """
    packed = isinstance(b, PackedWeight)
    bt = b.data if packed else b
    _require_cuda(a, bt, addend, bias, out)
    if a.dtype != torch.float32 or bt.dtype != torch.float32:
        raise ValueError("gemm is float32")
    batched = a.dim() == 3
    batch = a.shape[0] if batched else 1
    m, k = a.shape[-2], a.shape[-1]
    lda = _row_major_2d(a, "a")
    stride_a = a.stride(0) if batched else 0
    if packed:
        if b.k != k:
            raise ValueError(f"packed weight has k={b.k}, a has k={k}")
        n, ldb, stride_b = b.n, b.n, 0
        if batched:
            raise ValueError("packed weights are 2-D")
    else:
        if bt.shape[-2] != k:
            raise ValueError("inner dimensions differ")
        n = bt.shape[-1]
        ldb = _row_major_2d(bt, "b")
        stride_b = bt.stride(0) if bt.dim() == 3 else 0
    if out is None:
        out = torch.empty((batch, m, n) if batched else (m, n), dtype=torch.float32, device=a.device)
    ldc = _row_major_2d(out, "out")
    stride_c = out.stride(0) if batched else 0
    lde, stride_e = 0, 0
    if addend is not None:
        lde = _row_major_2d(addend, "addend")
        stride_e = addend.stride(0) if addend.dim() == 3 else 0
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != n or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous [n] vector")
    check(_lib.lib().annc_hip_gemm(stream_ptr(stream), batch, m, n, k, ptr(a), lda, stride_a,
                                   ptr(bt), ldb, stride_b, 1 if packed else 0,
                                   ptr(addend), lde, stride_e, ptr(bias), epilogue,
                                   ptr(out), ldc, stride_c))
    return out


DENSE_SCORE_WIDTHS = (64, 128, 256)
DENSE_SCORE_MAX_K = 2048


def dense_score_fits(k: int, n: int) -> bool:
    """Whether annc_hip_dense_score takes a hidden layer of shape [k, n]."""
    return n in DENSE_SCORE_WIDTHS and n <= k <= DENSE_SCORE_MAX_K and k % n == 0


def dense_score(a: torch.Tensor, weight: PackedWeight, score_weight: torch.Tensor, *,
                bias: torch.Tensor | None = None, epilogue: int = _lib.EPI_RELU,
                score_bias: torch.Tensor | None = None, score_epilogue: int = _lib.EPI_SIGMOID,
                hidden: torch.Tensor | None = None, out: torch.Tensor | None = None,
                stream=None) -> torch.Tensor:
    """Tower tail in one kernel: out = score_epi(epi(a @ W + bias) @ w + score_bias).

    a: [M, K] (rows 16-byte aligned); weight: packed [K, N] with N in
    DENSE_SCORE_WIDTHS and K a multiple of N; score_weight: N floats (a
    [N, 1] weight).  `hidden` ([M, N]) receives epi(a @ W + bias) when given.
    Returns out, [M, 1]."""
    if not isinstance(weight, PackedWeight):
        raise ValueError("dense_score takes a packed weight")
    _require_cuda(a, weight.data, score_weight, bias, score_bias, hidden, out)
    if a.dtype != torch.float32 or a.dim() != 2:
        raise ValueError("a must be a 2-D float32 tensor")
    m, k = a.shape
    n = weight.n
    if weight.k != k:
        raise ValueError(f"packed weight has k={weight.k}, a has k={k}")
    if not dense_score_fits(k, n):
        raise ValueError(f"dense_score takes n in {DENSE_SCORE_WIDTHS} and k a multiple of n "
                         f"up to {DENSE_SCORE_MAX_K}, not k={k}, n={n}")
    lda = _row_major_2d(a, "a")
    sw = score_weight.reshape(-1)
    if sw.numel() != n or not sw.is_contiguous() or sw.dtype != torch.float32:
        raise ValueError("score_weight must hold n contiguous float32 values")
    for name, v, size in (("bias", bias, n), ("score_bias", score_bias, 1)):
        if v is not None and (v.numel() != size or not v.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous vector of {size}")
    ldh = 0
    if hidden is not None:
        if tuple(hidden.shape) != (m, n):
            raise ValueError("hidden must be [m, n]")
        ldh = _row_major_2d(hidden, "hidden")
    if out is None:
        out = torch.empty((m, 1), dtype=torch.float32, device=a.device)
    if out.dim() != 2 or tuple(out.shape) != (m, 1):
        raise ValueError("out must be [m, 1]")
    ldo = out.stride(0)
    check(_lib.lib().annc_hip_dense_score(stream_ptr(stream), m, n, k, ptr(a), lda,
                                          ptr(weight.data), ptr(bias), epilogue,
                                          ptr(sw), ptr(score_bias), score_epilogue,
                                          ptr(hidden), ldh, ptr(out), ldo))
    return out


def embedding_bag(table: torch.Tensor, ids: torch.Tensor, offsets: torch.Tensor,
                  combiner: int = _lib.COMBINER_SUM, out: torch.Tensor | None = None,
                  stream=None) -> torch.Tensor:
    """CSR embedding bag with KPFusedSparseSegmentReduce arithmetic."""
    _require_cuda(table, ids, offsets, out)
    if table.dtype != torch.float32 or table.dim() != 2 or not table.is_contiguous():
        raise ValueError("table must be a contiguous [rows, dim] float32 tensor")
    if ids.dtype not in (torch.int32, torch.int64) or not ids.is_contiguous():
        raise ValueError("ids must be contiguous int32 or int64")
    if offsets.dtype != torch.int64 or not offsets.is_contiguous():
        raise ValueError("offsets must be contiguous int64")
    rows, dim = table.shape
    nbags = offsets.numel() - 1
    if out is None:
        out = torch.empty((nbags, dim), dtype=torch.float32, device=table.device)
    ldo = _row_major_2d(out, "out")
    if ids.numel() == 0:
        # no ids (a null data pointer, which the C entry rejects): offsets
        # consistent with them leave every bag empty, i.e. 0 under both
        # combiners
        return out.zero_()
    check(_lib.lib().annc_hip_embedding_bag(stream_ptr(stream), ptr(table), rows, dim, ptr(ids),
                                            1 if ids.dtype == torch.int64 else 0, ptr(offsets),
                                            nbags, combiner, ptr(out), ldo))
    return out


def segment_reduce(data: torch.Tensor, indices: torch.Tensor, segment_ids: torch.Tensor,
                   batch: int, combiner: int = _lib.COMBINER_SUM, sorted_ids: bool = False,
                   stream=None) -> torch.Tensor:
    """Segment sum/mean into [batch, dim] (index order per segment).
    sorted_ids=True promises non-decreasing segment ids (skips the sort)."""
    _require_cuda(data, indices, segment_ids)
    rows, dim = data.shape
    # (torch may give an empty or one-element view any stride, 0 included)
    seg_stride = max(segment_ids.stride(0), 1)
    out = torch.empty((batch, dim), dtype=torch.float32, device=data.device)
    check(_lib.lib().annc_hip_segment_reduce(stream_ptr(stream), ptr(data.contiguous()), rows, dim,
                                             ptr(indices), 1 if indices.dtype == torch.int64 else 0,
                                             ptr(segment_ids), seg_stride, indices.numel(),
                                             combiner, batch, ptr(out), 1 if sorted_ids else 0))
    return out


def unique_gather(table: torch.Tensor, keys: torch.Tensor, col: int = 0, stream=None):
    """KPFusedGather engine on device tensors: keys [N, C] (or [N]) int64,
    column `col`.  Returns (unique int64[U], indices int32[N], rows [U, dim])
    -- U is read back, which synchronises the stream."""
    _require_cuda(table, keys)
    if keys.dtype != torch.int64:
        raise ValueError("keys must be int64")
    k2 = keys if keys.dim() == 2 else keys.reshape(-1, 1)
    if k2.stride(-1) != 1:
        k2 = k2.contiguous()
    if not 0 <= col < k2.shape[1]:
        raise ValueError("col outside the key columns")
    rows, dim = table.shape
    n = k2.shape[0]
    nu = torch.empty(1, dtype=torch.int64, device=table.device)  # always written
    uniq = torch.empty(max(n, 1), dtype=torch.int64, device=table.device)
    idx = torch.empty(n, dtype=torch.int32, device=table.device)
    out = torch.empty((max(n, 1), dim), dtype=torch.float32, device=table.device)
    check(_lib.lib().annc_hip_unique_gather(stream_ptr(stream), ptr(table.contiguous()), rows, dim,
                                            ptr(k2) + 8 * col if n else None, k2.stride(0), n,
                                            ptr(nu), ptr(uniq), ptr(idx), ptr(out)))
    u = int(nu.item())
    return uniq[:u], idx, out[:u]


def sparse_embedding2(table: torch.Tensor, ids: torch.Tensor, fallback_row: int = 0,
                      out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Masked gather: out[i] = table[ids[i]] if 0 <= ids[i] < rows else 0."""
    _require_cuda(table, ids, out)
    rows, dim = table.shape
    if out is None:
        out = torch.empty((ids.numel(), dim), dtype=torch.float32, device=table.device)
    elif out.shape != (ids.numel(), dim) or not out.is_contiguous():
        raise ValueError("out must be a contiguous [ids.numel(), dim] tensor")
    check(_lib.lib().annc_hip_sparse_embedding2(stream_ptr(stream), ptr(table.contiguous()), rows,
                                                dim, ptr(ids.contiguous()),
                                                1 if ids.dtype == torch.int64 else 0, ids.numel(),
                                                fallback_row, ptr(out)))
    return out


def pooling(ids: torch.Tensor, gathered: torch.Tensor, slice_starts: Sequence[int],
            slice_limits: Sequence[int], stream=None) -> torch.Tensor:
    """__pooling on device tensors: ids [m,k] int64, gathered [m,k,n]."""
    _require_cuda(ids, gathered)
    m, k = ids.shape
    n = gathered.shape[2]
    ss = np.asarray(slice_starts, dtype=np.int64)
    sl = np.asarray(slice_limits, dtype=np.int64)
    for d, size in enumerate((m, k, n)):
        if not (0 <= ss[d] <= sl[d] <= size):
            raise ValueError("slice outside the operand")
    out = torch.empty((m, n), dtype=torch.float32, device=ids.device)
    check(_lib.lib().annc_hip_pooling(stream_ptr(stream), ptr(ids.contiguous()),
                                      ptr(gathered.contiguous()), m, k, n, ptr(ss), ptr(sl),
                                      ptr(out)))
    return out


def strings_to_device(strings: Sequence[bytes | str], device) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack strings into (bytes uint8, offsets int64[n+1]) device tensors."""
    enc = [s.encode() if isinstance(s, str) else bytes(s) for s in strings]
    offsets = np.zeros(len(enc) + 1, dtype=np.int64)
    np.cumsum([len(s) for s in enc], out=offsets[1:])
    blob = np.frombuffer(b"".join(enc) or b"\0", dtype=np.uint8)
    return (torch.from_numpy(blob.copy()).to(device), torch.from_numpy(offsets).to(device))


def fingerprint64(data: torch.Tensor, offsets: torch.Tensor, nul_terminated: bool = False,
                  stream=None) -> torch.Tensor:
    _require_cuda(data, offsets)
    n = offsets.numel() - 1
    out = torch.empty(n, dtype=torch.int64, device=data.device)
    check(_lib.lib().annc_hip_fingerprint64(stream_ptr(stream), ptr(data), ptr(offsets), n,
                                            1 if nul_terminated else 0, ptr(out)))
    return out


def hash_bucket_strings(data: torch.Tensor, offsets: torch.Tensor, num_buckets: int,
                        nul_terminated: bool = False, stream=None) -> torch.Tensor:
    _require_cuda(data, offsets)
    n = offsets.numel() - 1
    out = torch.empty(n, dtype=torch.int64, device=data.device)
    check(_lib.lib().annc_hip_hash_bucket_strings(stream_ptr(stream), ptr(data), ptr(offsets), n,
                                                  num_buckets, 1 if nul_terminated else 0,
                                                  ptr(out)))
    return out


def hash_bucket_int64(ids: torch.Tensor, num_buckets: int, stream=None) -> torch.Tensor:
    _require_cuda(ids)
    if ids.dtype != torch.int64 or not ids.is_contiguous():
        raise ValueError("ids must be contiguous int64")
    out = torch.empty_like(ids)
    check(_lib.lib().annc_hip_hash_bucket_int64(stream_ptr(stream), ptr(ids), ids.numel(),
                                                num_buckets, ptr(out)))
    return out


def hashed_embedding_bags(tables: Sequence[torch.Tensor], num_buckets: Sequence[int],
                          ids: torch.Tensor, offsets: torch.Tensor, batch: int,
                          combiner: int = _lib.COMBINER_MEAN, out: torch.Tensor | None = None,
                          buckets_out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Multi-field hash -> bucket -> gather -> pool into out[batch, F*dim].

    ids: all fields' raw int64 ids, field-major; offsets: int64[F*batch+1].
    `out` may be a column slice of a wider row-major buffer.
    """
    _require_cuda(ids, offsets, out, buckets_out, *tables)
    nf = len(tables)
    dim = tables[0].shape[1]
    for t in tables:
        if t.dim() != 2 or t.shape[1] != dim or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("tables must be contiguous float32 [rows, dim] with one dim")
    if offsets.numel() != nf * batch + 1:
        raise ValueError("offsets must hold num_fields*batch+1 entries")
    if out is None:
        out = torch.empty((batch, nf * dim), dtype=torch.float32, device=ids.device)
    ldo = _row_major_2d(out, "out")
    if ids.numel() == 0 and nf * batch > 0:
        # no ids (a null data pointer, which the C entry rejects): every bag
        # is empty, 0 under both combiners
        return out.zero_()
    tptrs = (ctypes_array_u64([t.data_ptr() for t in tables]))
    rows = np.asarray([t.shape[0] for t in tables], dtype=np.int64)
    nb = np.asarray(list(num_buckets), dtype=np.int64)
    check(_lib.lib().annc_hip_hashed_embedding_bags(stream_ptr(stream), nf, batch, dim,
                                                    ptr(tptrs), ptr(rows), ptr(nb), ptr(ids),
                                                    ptr(offsets), combiner, ptr(out), ldo,
                                                    ptr(buckets_out)))
    return out


def ctypes_array_u64(values: Sequence[int]) -> np.ndarray:
    return np.asarray(values, dtype=np.uint64)


def stream_status(stream=None) -> None:
    """Synchronise the stream and raise if a kernel met an out-of-range id."""
    check(_lib.lib().annc_hip_stream_status(stream_ptr(stream)))
