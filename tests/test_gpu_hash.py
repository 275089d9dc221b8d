"""GPU parity: FarmHash Fingerprint64, hash buckets, hashed embedding ops.

Bucket ids and gather indices bit-exact; pooled rows bit-exact (same order)."""
import json
import os

import numpy as np
import pytest
import torch

from annc_amd import tf_ops, workloads
from annc_amd import device as dev
from oracle import ora
from tests.gpu_util import device, note, to_dev, to_host

pytestmark = pytest.mark.gpu
VECS = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "farmhash_fingerprint64_vectors.json")))


def _u64(x):
    return np.asarray(x).astype(np.int64).view(np.uint64)


def test_fingerprint_published_vectors_on_gpu():
    note("fingerprint published vectors")
    strs = []
    for v in VECS["vectors"]:
        if "input_repeat" in v:
            s, n = v["input_repeat"]
            strs.append((s * n).encode())
        else:
            strs.append(v["input"].encode())
    data, off = dev.strings_to_device(strs, device())
    got = _u64(to_host(dev.fingerprint64(data, off)))
    assert [int(x) for x in got] == [v["fingerprint"] for v in VECS["vectors"]]


def test_fingerprint_all_lengths_match_oracle():
    note("fingerprint lengths 0..300")
    g = workloads.rng(12)
    strs = [g.integers(0, 256, size=n, dtype=np.uint8).tobytes() for n in range(0, 301)]
    strs += [g.integers(0, 256, size=int(n), dtype=np.uint8).tobytes()
             for n in g.integers(0, 2000, size=200)]
    data, off = dev.strings_to_device(strs, device())
    got = _u64(to_host(dev.fingerprint64(data, off)))
    np.testing.assert_array_equal(got, ora.fingerprint64_batch(strs))
    gotn = _u64(to_host(dev.fingerprint64(data, off, nul_terminated=True)))
    np.testing.assert_array_equal(gotn, ora.fingerprint64_batch(strs, nul_terminated=True))


EDGE_IDS = [0, 1, -1, 9, 10, 11, 99, 100, 101, -9, -10, 999_999, 1_000_000, 12345678,
            99_999_999, 100_000_000, 100_000_001, 10**15, 10**16 - 1, 10**16, 10**16 + 1,
            10**17, 10**18, 2**63 - 1, -2**63, -2**63 + 1, -(10**18), 4_294_967_295,
            4_294_967_296, -4_294_967_296]
# every decimal length 1..19 at both ends, both signs
EDGE_IDS += sorted({s * v for k in range(19) for v in (10**k - 1, 10**k, 10**k + 1, 2 * 10**k)
                    for s in (1, -1) if -2**63 <= s * v < 2**63})


@pytest.mark.parametrize("num_buckets", [1, 2, 7, 10, 100_000, 2**31 - 1, 2**32 + 15,
                                         2**62 + 3, 2**63 - 1])
def test_hash_bucket_int64_bit_exact(num_buckets):
    note(f"hash bucket int64 nb={num_buckets}")
    g = workloads.rng(num_buckets % 997)
    ids = np.concatenate([np.asarray(EDGE_IDS, dtype=np.int64),
                          g.integers(-2**63, 2**63 - 1, size=20000, dtype=np.int64),
                          g.integers(0, 10**6, size=5000, dtype=np.int64)])
    got = to_host(dev.hash_bucket_int64(to_dev(ids), num_buckets))
    np.testing.assert_array_equal(got, ora.hash_bucket_int64(ids, num_buckets))


def test_hash_bucket_strings_bit_exact():
    note("hash bucket strings")
    strs = [str(i).encode() for i in range(-500, 500)] + [b"", b"hello", b"x" * 40, b"y" * 90]
    data, off = dev.strings_to_device(strs, device())
    got = to_host(dev.hash_bucket_strings(data, off, 1000))
    np.testing.assert_array_equal(got, ora.hash_bucket_strings(strs, 1000))
    v = VECS["hash_bucket_vectors"][0]
    d2, o2 = dev.strings_to_device(v["inputs"], device())
    assert to_host(dev.hash_bucket_strings(d2, o2, v["num_buckets"])).tolist() == v["buckets"]


def test_hashed_bags_config4_bit_exact():
    note("hashed bags config4")
    w = workloads.config4(seed=0)
    ref, ref_buckets = ora.hashed_embedding_bags(w.tables, w.num_buckets, w.ids, w.offsets,
                                                 w.batch, 1, threads=8, with_buckets=True)
    tables = [to_dev(t) for t in w.tables]
    buckets = to_dev(np.full(w.ids.size, -7, dtype=np.int64))
    out = dev.hashed_embedding_bags(tables, [w.num_buckets] * len(tables), to_dev(w.ids),
                                    to_dev(w.offsets), w.batch, 1, buckets_out=buckets)
    np.testing.assert_array_equal(to_host(buckets), ref_buckets)
    np.testing.assert_array_equal(to_host(out), ref)


@pytest.mark.parametrize("dim", [4, 16, 32, 64, 128, 264])
def test_hashed_bags_dims_sum(dim):
    note(f"hashed bags dim={dim}")
    g = workloads.rng(dim + 1)
    nf, batch, rows = 3, 257, 777
    ids, offsets = workloads.hashed_structure(g, nf, batch, lo=0, hi=9)
    tables = [g.standard_normal((rows, dim)).astype(np.float32) for _ in range(nf)]
    ref = ora.hashed_embedding_bags(tables, rows - 5, ids, offsets, batch, 0)
    out = dev.hashed_embedding_bags([to_dev(t) for t in tables], [rows - 5] * nf, to_dev(ids),
                                    to_dev(offsets), batch, 0)
    np.testing.assert_array_equal(to_host(out), ref)


@pytest.mark.parametrize("dim", [16, 32, 64])
def test_hashed_bags_long_bags_mean(dim):
    """Bags of 40-130 ids: a wave's run of bags spans several windows of
    staged row offsets, and single bags straddle window edges."""
    note(f"hashed bags long bags dim={dim}")
    g = workloads.rng(dim + 2)
    nf, batch, rows = 2, 67, 5000
    ids, offsets = workloads.hashed_structure(g, nf, batch, lo=40, hi=130)
    tables = [g.standard_normal((rows, dim)).astype(np.float32) for _ in range(nf)]
    ref, ref_buckets = ora.hashed_embedding_bags(tables, rows, ids, offsets, batch, 1,
                                                 with_buckets=True)
    buckets = to_dev(np.full(ids.size, -7, dtype=np.int64))
    out = dev.hashed_embedding_bags([to_dev(t) for t in tables], [rows] * nf, to_dev(ids),
                                    to_dev(offsets), batch, 1, buckets_out=buckets)
    np.testing.assert_array_equal(to_host(buckets), ref_buckets)
    np.testing.assert_array_equal(to_host(out), ref)


def test_tf_embedding_with_hash_bucket_ops():
    note("tf hash bucket ops")
    g = workloads.rng(5)
    weight = g.standard_normal((1000, 8)).astype(np.float32)
    strs = [str(int(v)).encode() for v in g.integers(-10**12, 10**12, size=3000)]
    strs[::97] = [b""] * len(strs[::97])
    strs[5] = b"ab\0cd"
    out = tf_ops.kp_fused_embedding_with_hash_bucket(strs, weight, 1000, combiner=1)
    np.testing.assert_array_equal(out, ora.embedding_with_hash_bucket(strs, weight, 1000))
    for fn in (tf_ops.kp_fused_dnn_embedding_with_hash_bucket,
               tf_ops.kp_fused_linear_embedding_with_hash_bucket):
        got = fn(strs, weight[:600], 1000)  # buckets >= rows stay zero
        np.testing.assert_array_equal(got, ora.dnn_embedding_with_hash_bucket(strs, weight[:600], 1000))


@pytest.mark.parametrize("count", [0, 2000, 4092, 50_000])
def test_tf_sparse_embedding(count):
    """KPFusedSparseEmbedding against the oracle, bucket-0 quirk included;
    the compaction scan over 4 ids, 2004, exactly one tile of 4096, and
    50,004 (13 tiles)."""
    note(f"tf sparse embedding, {count} ids")
    strs = [str(i).encode() for i in range(count)] + [b""] * 3 + [b"\0x"]
    got = tf_ops.kp_fused_sparse_embedding(strs, 7)
    ref = ora.sparse_embedding(strs, 7)
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("dim,combiner", [(4, 0), (8, 1), (12, 0), (16, 1)])
def test_hashed_bags_ragged_mixed_ids(dim, combiner):
    """Rows of at most 16 floats (the pipelined run kernel): empty and
    ragged bags, a padded output stride, ids of every decimal length and
    sign in one wave, fields whose runs straddle waves."""
    note(f"hashed bags ragged mixed dim={dim} combiner={combiner}")
    g = workloads.rng(100 + dim)
    nf, batch, rows = 5, 203, 3001
    lens = g.integers(0, 7, size=nf * batch)
    lens[::11] = 0
    lens[5] = 70    # a run of 64-128 positions (two hashed chunks)
    lens[40] = 140  # a run of more than 128 positions (synchronous path)
    lens[300] = 9   # a bag longer than one batch of row loads
    offsets = np.zeros(nf * batch + 1, dtype=np.int64)
    np.cumsum(lens, out=offsets[1:])
    nnz = int(offsets[-1])
    pool = np.asarray(EDGE_IDS, dtype=np.int64)
    ids = np.where(g.random(nnz) < 0.5, g.choice(pool, size=nnz),
                   g.integers(-2**63, 2**63 - 1, size=nnz, dtype=np.int64))
    tables = [g.standard_normal((rows, dim)).astype(np.float32) for _ in range(nf)]
    nbk = [rows - 7 * f for f in range(nf)]
    ldo = nf * dim + 4
    ref = np.stack([ora.hashed_embedding_bags([tables[f]], nbk[f], ids,
                                              offsets[f * batch:(f + 1) * batch + 1], batch,
                                              combiner) for f in range(nf)], axis=1)
    out_full = to_dev(np.full((batch, ldo), 7.0, dtype=np.float32))
    dev.hashed_embedding_bags([to_dev(t) for t in tables], nbk, to_dev(ids), to_dev(offsets),
                              batch, combiner, out=out_full[:, :nf * dim])
    got = to_host(out_full)
    np.testing.assert_array_equal(got[:, :nf * dim].reshape(batch, nf, dim), ref)
    np.testing.assert_array_equal(got[:, nf * dim:], 7.0)  # padding untouched


def test_hashed_bags_table_of_2gib():
    """A field table of exactly 2 GiB (2^25 rows x 16 floats) takes the
    64-bit-address kernel; buckets from the oracle's FarmHash, sums in index
    order."""
    rows, dim, batch = 1 << 25, 16, 512
    note("hashed bags 2 GiB table")
    r = ((torch.arange(rows, device=device(), dtype=torch.int64) % 1000) - 500).to(torch.float32)
    table = (r * torch.tensor(0.001, dtype=torch.float32, device=device()))[:, None] + \
        torch.arange(dim, device=device(), dtype=torch.float32)[None, :]
    del r
    g = workloads.rng(4096)
    ids, offsets = workloads.hashed_structure(g, 1, batch, lo=1, hi=6)
    buckets = ora.hash_bucket_int64(ids, rows)
    vals = (((buckets % 1000) - 500).astype(np.float32) * np.float32(0.001))[:, None] + \
        np.arange(dim, dtype=np.float32)[None, :]
    ref = np.zeros((batch, dim), dtype=np.float32)
    for b in range(batch):
        acc = np.zeros(dim, dtype=np.float32)
        for p in range(offsets[b], offsets[b + 1]):
            acc = acc + vals[p]
        n = offsets[b + 1] - offsets[b]
        ref[b] = acc * np.float32(1.0 / np.float32(n)) if n else acc
    got_b = to_dev(np.full(ids.size, -7, dtype=np.int64))
    out = dev.hashed_embedding_bags([table], [rows], to_dev(ids), to_dev(offsets), batch, 1,
                                    buckets_out=got_b)
    np.testing.assert_array_equal(to_host(got_b), buckets)
    np.testing.assert_array_equal(to_host(out), ref)
    del table
    torch.cuda.empty_cache()


@pytest.mark.parametrize("seed", range(10))
def test_hashed_bags_random_shapes_bit_exact(seed):
    """Seeded random multi-field shapes across the three hashed-bag kernels
    (dims up to 16, 17-64 and wider): 1-30 fields, ragged bags with a few
    over 128 positions, either combiner; bucket ids and sums bit-exact."""
    g = workloads.rng(9100 + seed)
    dim = int(g.choice([4, 8, 12, 16, 20, 32, 48, 64, 68, 128]))
    nf = int(g.integers(1, 31))
    batch = int(g.integers(1, 600))
    rows = int(g.integers(50, 20000))
    lens = g.integers(0, 6, size=nf * batch)
    longs = g.random(nf * batch) < 0.01
    lens[longs] = g.integers(60, 300, size=int(longs.sum()))
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    nnz = int(offsets[-1])
    ids = g.integers(-2**63, 2**63 - 1, size=nnz, dtype=np.int64)
    combiner = seed % 2
    nbk = [int(g.integers(1, rows + 1)) for _ in range(nf)]
    note(f"hashed random seed={seed}: dim={dim} fields={nf} batch={batch} rows={rows} "
         f"nnz={nnz} combiner={combiner}")
    tables = [g.standard_normal((rows, dim)).astype(np.float32) for _ in range(nf)]
    ref = np.stack([ora.hashed_embedding_bags([tables[f]], nbk[f], ids,
                                              offsets[f * batch:(f + 1) * batch + 1], batch,
                                              combiner) for f in range(nf)], axis=1)
    out = dev.hashed_embedding_bags([to_dev(t) for t in tables], nbk, to_dev(ids),
                                    to_dev(offsets), batch, combiner)
    np.testing.assert_array_equal(to_host(out).reshape(batch, nf, dim), ref)
