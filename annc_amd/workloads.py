"""Seeded synthetic inputs for the five benchmark configurations.

All draws use numpy's PCG64 generator; the order of draws within each
function is fixed so a seed pins every array.  Zipf ids are drawn with
``Generator.zipf(alpha) - 1`` and values >= the table size are re-drawn until
none remain (a truncated Zipf over [0, rows)).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def truncated_zipf(g: np.random.Generator, alpha: float, high: int, size: int) -> np.ndarray:
    out = g.zipf(alpha, size=size) - 1
    bad = out >= high
    while bad.any():
        out[bad] = g.zipf(alpha, size=int(bad.sum())) - 1
        bad = out >= high
    return out.astype(np.int64)


def glorot_uniform(g: np.random.Generator, fan_in: int, fan_out: int) -> np.ndarray:
    lim = np.sqrt(6.0 / (fan_in + fan_out))
    return g.uniform(-lim, lim, size=(fan_in, fan_out)).astype(np.float32)


# --------------------------------------------------------------------------
# Config 1: single __matmul_add_relu, A[512x256] B[256x256] bias[256]
# --------------------------------------------------------------------------
@dataclass
class MatmulAddReluInputs:
    a: np.ndarray
    b: np.ndarray
    bias: np.ndarray
    e: np.ndarray  # bias broadcast to [m, n], the materialised XLA addend
    z: np.ndarray  # broadcast zero operand of max()


def config1(seed: int = 0, m: int = 512, k: int = 256, n: int = 256) -> MatmulAddReluInputs:
    g = rng(seed)
    a = g.standard_normal((m, k), dtype=np.float32)
    b = g.uniform(-1.0 / 16, 1.0 / 16, size=(k, n)).astype(np.float32)
    bias = (g.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    e = np.ascontiguousarray(np.broadcast_to(bias, (m, n)))
    z = np.zeros((m, n), dtype=np.float32)
    return MatmulAddReluInputs(a, b, bias, e, z)


# --------------------------------------------------------------------------
# Config 2: layout_matmul MLP tower 1024 -> 512 -> 256 -> 1, batch 4096
# --------------------------------------------------------------------------
@dataclass
class TowerInputs:
    x: np.ndarray
    weights: list
    biases: list


def config2(seed: int = 0, batch: int = 4096, widths=(1024, 512, 256, 1)) -> TowerInputs:
    g = rng(seed)
    x = g.standard_normal((batch, widths[0]), dtype=np.float32)
    weights, biases = [], []
    for fi, fo in zip(widths[:-1], widths[1:]):
        weights.append(glorot_uniform(g, fi, fo))
        biases.append((g.standard_normal(fo, dtype=np.float32) * np.float32(0.01)).astype(np.float32))
    return TowerInputs(x, weights, biases)


# --------------------------------------------------------------------------
# Config 3: embedding bag, table [1e6 x 64], 4096 bags, Poisson(20) lengths
# --------------------------------------------------------------------------
@dataclass
class BagInputs:
    table: np.ndarray | None
    ids: np.ndarray
    offsets: np.ndarray


def bag_structure(g: np.random.Generator, rows: int, bags: int, mean_len: float = 20.0,
                  max_len: int = 100, alpha: float = 1.05):
    lens = np.clip(g.poisson(mean_len, size=bags), 1, max_len).astype(np.int64)
    offsets = np.zeros(bags + 1, dtype=np.int64)
    np.cumsum(lens, out=offsets[1:])
    ids = truncated_zipf(g, alpha, rows, int(offsets[-1]))
    return ids, offsets


def config3(seed: int = 0, rows: int = 1_000_000, dim: int = 64, bags: int = 4096,
            with_table: bool = True) -> BagInputs:
    g = rng(seed)
    ids, offsets = bag_structure(g, rows, bags)
    table = None
    if with_table:
        table = (g.standard_normal((rows, dim), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    return BagInputs(table, ids, offsets)


# --------------------------------------------------------------------------
# Config 4: 26 hashed fields, tables [1e5 x 16], 1-5 ids, batch 8192, mean
# --------------------------------------------------------------------------
@dataclass
class HashedInputs:
    tables: list
    ids: np.ndarray      # raw int64 ids, field-major
    offsets: np.ndarray  # int64[F*batch+1]
    num_buckets: int
    batch: int
    dim: int


def hashed_structure(g: np.random.Generator, fields: int, batch: int, lo: int = 1, hi: int = 5,
                     zipf_rows: int | None = None, alpha: float = 1.05):
    lens = g.integers(lo, hi + 1, size=fields * batch, dtype=np.int64)
    offsets = np.zeros(fields * batch + 1, dtype=np.int64)
    np.cumsum(lens, out=offsets[1:])
    nnz = int(offsets[-1])
    if zipf_rows is None:
        ids = g.integers(0, np.iinfo(np.int64).max, size=nnz, dtype=np.int64, endpoint=False)
    else:
        ids = truncated_zipf(g, alpha, zipf_rows, nnz)
    return ids, offsets


def config4(seed: int = 0, fields: int = 26, batch: int = 8192, dim: int = 16,
            rows: int = 100_000) -> HashedInputs:
    g = rng(seed)
    ids, offsets = hashed_structure(g, fields, batch)
    tables = [(g.standard_normal((rows, dim), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
              for _ in range(fields)]
    return HashedInputs(tables, ids, offsets, rows, batch, dim)


# --------------------------------------------------------------------------
# Config 5: wide&deep graph, 26 fields dim 32 + 13 dense, MLP 1024-512-256-1
# --------------------------------------------------------------------------
@dataclass
class WideDeepInputs:
    hashed: HashedInputs
    dense: np.ndarray
    weights: list
    biases: list


def config5(seed: int = 0, fields: int = 26, batch: int = 4096, dim: int = 32,
            rows: int = 100_000, num_dense: int = 13, hidden=(1024, 512, 256)) -> WideDeepInputs:
    g = rng(seed)
    ids, offsets = hashed_structure(g, fields, batch, zipf_rows=rows)
    tables = [(g.standard_normal((rows, dim), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
              for _ in range(fields)]
    dense = g.lognormal(0.0, 1.0, size=(batch, num_dense)).astype(np.float32)
    widths = (fields * dim + num_dense,) + tuple(hidden) + (1,)
    weights, biases = [], []
    for fi, fo in zip(widths[:-1], widths[1:]):
        weights.append(glorot_uniform(g, fi, fo))
        biases.append((g.standard_normal(fo, dtype=np.float32) * np.float32(0.01)).astype(np.float32))
    return WideDeepInputs(HashedInputs(tables, ids, offsets, rows, batch, dim), dense, weights,
                          biases)
