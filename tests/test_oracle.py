"""Pins the CPU oracle before it is trusted as the GPU checker (CPU only)."""
import json
import os

import numpy as np
import pytest

from oracle import ora

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


# ------------------------------------------------------------ FarmHash
def _vec_input(v):
    if "input_repeat" in v:
        s, n = v["input_repeat"]
        return (s * n).encode()
    return v["input"].encode()


@pytest.mark.parametrize("vec", _load("farmhash_fingerprint64_vectors.json")["vectors"],
                         ids=lambda v: v.get("input", str(v.get("input_repeat"))))
def test_fingerprint64_published_vectors(vec):
    assert ora.fingerprint64(_vec_input(vec)) == vec["fingerprint"]


def test_hash_bucket_published_vector():
    for v in _load("farmhash_fingerprint64_vectors.json")["hash_bucket_vectors"]:
        got = ora.hash_bucket_strings(v["inputs"], v["num_buckets"])
        assert got.tolist() == v["buckets"]


def test_fingerprint_batch_matches_scalar_and_nul_prefix():
    strs = [b"", b"x", b"hello world, farmhash", b"ab\0cd", b"z" * 70]
    fp = ora.fingerprint64_batch(strs)
    assert [int(x) for x in fp] == [ora.fingerprint64(s) for s in strs]
    # NUL-terminated hashing (tensorflow::Fingerprint64(const char*)) sees the prefix.
    fpn = ora.fingerprint64_batch(strs, nul_terminated=True)
    assert int(fpn[3]) == ora.fingerprint64(b"ab")
    assert int(fpn[4]) == ora.fingerprint64(b"z" * 70)


@pytest.mark.parametrize("v", [0, 1, -1, 9, 10, -10, 99999999, 100000000, 10**16 - 1, 10**16,
                               2**63 - 1, -2**63, 1234567890123456789, -987654321])
def test_format_int64_is_decimal(v):
    assert ora.format_int64(v) == str(v).encode()


def test_hash_bucket_int64_is_hash_of_decimal_text():
    g = np.random.Generator(np.random.PCG64(3))
    ids = g.integers(-2**63, 2**63 - 1, size=200, dtype=np.int64)
    got = ora.hash_bucket_int64(ids, 100_000)
    want = [ora.fingerprint64(str(int(v)).encode()) % 100_000 for v in ids]
    assert got.tolist() == want


def _gm_mod(n, d):
    """Granlund-Montgomery round-up reciprocal, as make_divisor/mod_invariant use it."""
    if d == 1:
        return 0
    l = (d - 1).bit_length()
    magic = (((1 << l) - d) << 64) // d + 1
    assert magic < 2**64
    t1 = (magic * n) >> 64
    q = (t1 + ((n - t1) >> 1)) >> (l - 1)
    return n - q * d


@pytest.mark.parametrize("d", [1, 2, 3, 7, 10, 100_000, 2**32 - 1, 2**32 + 15, 2**63 - 25, 2**63,
                               2**63 + 1, 2**64 - 1])
def test_invariant_divisor_mod(d):
    g = np.random.Generator(np.random.PCG64(d % 1000))
    ns = [0, 1, d - 1, d, d + 1, 2**64 - 1, 2**63, 2**63 - 1]
    ns += [int(x) for x in g.integers(0, 2**64 - 1, size=300, dtype=np.uint64)]
    for n in ns:
        n %= 2**64
        assert _gm_mod(n, d) == n % d


# ------------------------------------------------------------ segment reduce
def _brute_segment(data, indices, seg, batch, combiner):
    """float32 scalar loop: out[seg] += row, in index order; mean *= 1/count."""
    out = np.zeros((batch, data.shape[1]), dtype=np.float32)
    cnt = np.zeros(batch, dtype=np.int64)
    for i in range(len(indices)):
        s = int(seg[i])
        cnt[s] += 1
        for d in range(data.shape[1]):
            out[s, d] = np.float32(out[s, d] + data[indices[i], d])
    if combiner == 1:
        for s in range(batch):
            if cnt[s]:
                inv = np.float32(1.0) / np.float32(cnt[s])
                out[s] = (out[s] * inv).astype(np.float32)
    return out


@pytest.mark.parametrize("case", _load("segment_reduce_reference_gtest.json")["cases"],
                         ids=lambda c: c["name"])
def test_segment_reduce_reference_goldens(case):
    data = np.asarray(case["data"], dtype=np.float32)
    idx = np.asarray(case["indices"], dtype=np.int32)
    sl = np.asarray(case["slice_input"], dtype=np.int64)
    seg = sl[:, case["begin"][1]]
    batch = int(seg.max()) + 1
    out = ora.segment_reduce(data, idx, seg, batch, case["combiner"])
    np.testing.assert_array_equal(out, np.asarray(case["expected"], dtype=np.float32))


@pytest.mark.parametrize("combiner", [0, 1])
def test_segment_reduce_matches_brute_force(combiner):
    g = np.random.Generator(np.random.PCG64(7))
    data = g.standard_normal((50, 5)).astype(np.float32)
    n = 200
    indices = g.integers(0, 50, size=n).astype(np.int64)
    seg = g.integers(0, 30, size=n).astype(np.int64)  # unsorted on purpose
    out = ora.segment_reduce(data, indices, seg, 30, combiner)
    np.testing.assert_array_equal(out, _brute_segment(data, indices, seg, 30, combiner))


@pytest.mark.parametrize("combiner", [0, 1])
def test_embedding_bag_equals_segment_reduce(combiner):
    g = np.random.Generator(np.random.PCG64(11))
    table = g.standard_normal((1000, 12)).astype(np.float32)
    lens = g.integers(0, 9, size=64)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ids = g.integers(0, 1000, size=int(offsets[-1])).astype(np.int64)
    seg = np.repeat(np.arange(64), lens).astype(np.int64)
    a = ora.embedding_bag(table, ids, offsets, combiner)
    b = ora.segment_reduce(table, ids, seg, 64, combiner)
    np.testing.assert_array_equal(a, b)
    # thread count does not change the per-bag order
    np.testing.assert_array_equal(a, ora.embedding_bag(table, ids, offsets, combiner, threads=4))


# ------------------------------------------------------------ pooling / masked gather
def _brute_pooling(ids, g, ss, sl):
    m, k = ids.shape
    n = g.shape[2]
    out = np.zeros((m, n), dtype=np.float32)
    for i in range(m):
        red = np.float32(0)
        for j in range(k):
            red = np.float32(red + np.float32(ids[i, j] > 0))
        for p in range(n):
            s = np.float32(0)
            for j in range(k):
                take = (ss[0] <= i < sl[0]) and (ss[1] <= j < sl[1]) and (ss[2] <= p < sl[2]) \
                    and ids[i, j] > 0
                s = np.float32(s + (g[i, j, p] if take else np.float32(0)))
            out[i, p] = np.float32(0) if red == 0 else np.float32(s / red)
    return out


def test_pooling_matches_brute_force():
    g = np.random.Generator(np.random.PCG64(5))
    ids = g.integers(-3, 6, size=(6, 7)).astype(np.int64)
    ids[2] = 0  # a row without positive ids pools to 0
    gathered = g.standard_normal((6, 7, 5)).astype(np.float32)
    for ss, sl in [((0, 0, 0), (6, 7, 5)), ((1, 2, 1), (5, 6, 4))]:
        np.testing.assert_array_equal(ora.pooling(ids, gathered, ss, sl),
                                      _brute_pooling(ids, gathered, ss, sl))


def test_reduce_mean_is_the_mean_absolute_value_of_consecutive_runs():
    """__reduce_mean (reduce_rewriter.cc:31-46): cblas_sasum over n runs of m
    consecutive values, divided by m: the absolute values (not the values)
    of x viewed as [n, m], whatever x's [m, n] shape says."""
    g = np.random.Generator(np.random.PCG64(9))
    for m, n in [(7, 5), (1, 3), (64, 1), (300, 17)]:
        x = g.standard_normal((m, n)).astype(np.float32)
        want = np.abs(x.astype(np.float64)).reshape(n, m).sum(axis=1) / m
        np.testing.assert_allclose(ora.reduce_mean(x), want, rtol=2e-6)
        if m > 1 and n > 1:  # a plain mean of the values, or of x's columns, is not it
            assert not np.allclose(ora.reduce_mean(x), x.reshape(n, m).mean(axis=1), rtol=1e-3)
            assert not np.allclose(ora.reduce_mean(x), np.abs(x).mean(axis=0), rtol=1e-3)
    assert np.isnan(ora.reduce_mean(np.zeros((0, 2), np.float32))).all()  # 0 / 0


def test_sparse_embedding2_mask_semantics():
    table = np.arange(12, dtype=np.float32).reshape(4, 3) - 5.0
    ids = np.array([0, 3, -1, 4, 2], dtype=np.int64)
    out = ora.sparse_embedding2(table, ids, fallback=1)
    np.testing.assert_array_equal(out[0], table[0])
    np.testing.assert_array_equal(out[1], table[3])
    # invalid ids multiply the fallback row by 0.0: signed zeros of that row
    np.testing.assert_array_equal(out[2], table[1] * np.float32(0))
    assert np.signbit(out[2]).tolist() == np.signbit(table[1] * np.float32(0)).tolist()
    np.testing.assert_array_equal(out[4], table[2])


# ------------------------------------------------------------ hash-bucket ops
def test_embedding_with_hash_bucket_closed_form():
    g = np.random.Generator(np.random.PCG64(2))
    weight = g.standard_normal((50, 4)).astype(np.float32)
    strs = [b"alpha", b"", b"1234567890123456789", b"x"]
    out = ora.embedding_with_hash_bucket(strs, weight, 50)
    for i, s in enumerate(strs):
        want = np.zeros(4, np.float32) if not s else weight[ora.fingerprint64(s) % 50]
        np.testing.assert_array_equal(out[i], want)


def test_sparse_embedding_zero_bucket_quirk():
    # find a non-empty string whose bucket is 0 for num_buckets = 3
    zero = next(s for s in (str(i).encode() for i in range(1000))
                if ora.fingerprint64(s) % 3 == 0)
    nz = next(s for s in (str(i).encode() for i in range(1000))
              if ora.fingerprint64(s) % 3 != 0)
    idx, vals, empty, shape = ora.sparse_embedding([nz, b"", zero, nz], 3)
    assert shape.tolist() == [4, 1]
    assert idx.tolist() == [[0, 0], [1, 0], [2, 0], [3, 0]]
    b = ora.fingerprint64(nz) % 3
    assert vals.tolist() == [b, 0, b]  # the bucket-0 string adds no value
    assert empty.tolist() == [False, True, False]


def _dnn_expected(strs, weight, num_buckets):
    """KPFusedDnn/LinearEmbeddingWithHashBucket, from the pinned pieces
    (fused_dnn_embedding_with_hash_bucket.cc:33-44,
    fused_linear_embdedding_with_hash_bucket.cc:43-51): a string equal to ""
    gives zeros; otherwise Fingerprint64 of the text up to the first NUL
    (tensorflow::Fingerprint64(const char*)), modulo num_buckets as uint64,
    and the row only when that bucket is below the weight's rows."""
    rows, dim = weight.shape
    out = np.zeros((len(strs), dim), np.float32)
    for i, s in enumerate(strs):
        if s == b"":
            continue
        b = ora.fingerprint64(s.split(b"\0", 1)[0]) % num_buckets
        if b < rows:
            out[i] = weight[b]
    return out


def _dnn_strings():
    g = np.random.Generator(np.random.PCG64(21))
    strs = [b"", b"\0", b"\0tail", b"ab\0cd", b"abc", b"x" * 70, b"12345678901234567"]
    strs += [str(int(v)).encode() for v in g.integers(-2**63, 2**63 - 1, size=120, dtype=np.int64)]
    return strs


def test_dnn_embedding_with_hash_bucket_closed_form():
    """Buckets at or past the weight's rows (num_buckets 2x rows) give zero
    rows, the empty string gives zeros, and a string with a NUL hashes only
    its prefix ("\0tail" hashes as "", whose fingerprint is pinned)."""
    g = np.random.Generator(np.random.PCG64(22))
    weight = g.standard_normal((40, 6)).astype(np.float32)
    strs = _dnn_strings()
    want = _dnn_expected(strs, weight, 80)
    got = ora.dnn_embedding_with_hash_bucket(strs, weight, 80)
    np.testing.assert_array_equal(got, want)
    # the cases the checks above must tell apart are present
    past = [i for i, s in enumerate(strs) if s and
            ora.fingerprint64(s.split(b"\0", 1)[0]) % 80 >= 40]
    assert len(past) > 10 and not got[past].any()
    # every bucket inside the table: "\0" and "\0tail" are non-empty strings
    # whose hashed text is "" (Fingerprint64("") = k2, a pinned vector)
    k2 = 0x9AE16A3B2F90404F
    got40 = ora.dnn_embedding_with_hash_bucket(strs, weight, 40)
    np.testing.assert_array_equal(got40, _dnn_expected(strs, weight, 40))
    assert got40[1].tolist() == got40[2].tolist() == weight[k2 % 40].tolist()
    assert ora.fingerprint64(b"\0tail") % 40 != k2 % 40
    assert ora.fingerprint64(b"ab") % 40 != ora.fingerprint64(b"ab\0cd") % 40


def test_dnn_embedding_check_catches_whole_string_hash_and_missing_bound():
    """The closed form fails for an oracle that hashes the whole string
    (NUL included) or copies rows for buckets past the table (mistakes
    planted in the checker's inputs, on the CPU)."""
    g = np.random.Generator(np.random.PCG64(23))
    weight = g.standard_normal((40, 6)).astype(np.float32)
    strs = _dnn_strings()
    want = _dnn_expected(strs, weight, 80)
    whole = ora.embedding_with_hash_bucket(
        [s for s in strs], np.concatenate([weight, weight]), 80)  # whole-string hash, no bound
    assert not np.array_equal(whole, want)
    # bucket bound only: the rows past the table would be copied
    wide = np.concatenate([weight, g.standard_normal((40, 6)).astype(np.float32)])
    assert not np.array_equal(ora.dnn_embedding_with_hash_bucket(strs, wide, 80), want)


def _ragged_fields(seed, nf, batch, rows):
    g = np.random.Generator(np.random.PCG64(seed))
    tables = [g.standard_normal((rows[f], 5)).astype(np.float32) for f in range(nf)]
    lens = g.integers(0, 7, size=nf * batch)
    lens[:3] = [0, 1, 6]
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ids = g.integers(-2**63, 2**63 - 1, size=int(offsets[-1]), dtype=np.int64)
    return tables, ids, offsets


def _bags_by_field(tables, num_buckets, ids, offsets, batch, combiner):
    """Per field f: the pinned bucket ids (decimal text -> Fingerprint64 %
    buckets), then the pinned CSR embedding bag over field f's slice of the
    offsets, placed at columns [f*dim, (f+1)*dim) of the concatenated output."""
    nf = len(tables)
    dim = tables[0].shape[1]
    out = np.empty((batch, nf * dim), np.float32)
    for f in range(nf):
        off = offsets[f * batch:(f + 1) * batch + 1]
        lo, hi = int(off[0]), int(off[-1])
        buckets = ora.hash_bucket_int64(ids[lo:hi], num_buckets[f])
        out[:, f * dim:(f + 1) * dim] = ora.embedding_bag(tables[f], buckets, off - lo, combiner)
    return out


@pytest.mark.parametrize("combiner", [0, 1])
@pytest.mark.parametrize("threads", [1, 4])
def test_hashed_embedding_bags_is_per_field_composition(combiner, threads):
    """ora_hashed_embedding_bags (the checker of the multi-field hashed bags)
    equals, bit for bit, the per-field composition of the pinned
    hash_bucket_int64 and embedding_bag, on ragged bags (empty ones
    included) over fields with different tables and bucket counts; its
    bucket output equals the pinned bucket ids."""
    nf, batch = 4, 37
    nb = [101, 57, 1000, 3]
    tables, ids, offsets = _ragged_fields(40 + combiner, nf, batch, [101, 60, 1000, 3])
    got, buckets = ora.hashed_embedding_bags(tables, nb, ids, offsets, batch, combiner,
                                             threads=threads, with_buckets=True)
    np.testing.assert_array_equal(got, _bags_by_field(tables, nb, ids, offsets, batch, combiner))
    want_b = np.concatenate([ora.hash_bucket_int64(
        ids[offsets[f * batch]:offsets[(f + 1) * batch]], nb[f]) for f in range(nf)])
    np.testing.assert_array_equal(buckets, want_b)


def test_hashed_embedding_bags_check_catches_field_mixups():
    """The composition check fails for a field order swapped, a bucket count
    taken from the wrong field, or a mean where a sum is due (mistakes
    planted in the oracle's inputs, on the CPU)."""
    nf, batch = 3, 20
    nb = [101, 57, 1000]
    tables, ids, offsets = _ragged_fields(50, nf, batch, [101, 60, 1000])
    want = _bags_by_field(tables, nb, ids, offsets, batch, 0)
    swapped = [tables[1], tables[0], tables[2]]
    assert not np.array_equal(
        ora.hashed_embedding_bags(swapped, [57, 101, 1000], ids, offsets, batch, 0), want)
    assert not np.array_equal(
        ora.hashed_embedding_bags(tables, [101, 101, 1000], ids, offsets, batch, 0), want)
    assert not np.array_equal(
        ora.hashed_embedding_bags(tables, nb, ids, offsets, batch, 1), want)


# ------------------------------------------------------------ GEMM via OpenBLAS
def test_openblas_is_0_3_29():
    assert "0.3.29" in ora.blas_config()


@pytest.mark.parametrize("m,n,k", [(512, 256, 256), (37, 45, 19), (1, 7, 300)])
def test_gemm_oracle_against_float64(m, n, k):
    g = np.random.Generator(np.random.PCG64(m * n))
    a = g.standard_normal((m, k)).astype(np.float32)
    b = g.standard_normal((k, n)).astype(np.float32)
    e = g.standard_normal((m, n)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    bound = 1e-5 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)) + 1e-6
    assert np.all(np.abs(ora.matmul(a, b) - ref) <= bound)
    assert np.all(np.abs(ora.matmul_add(e, a, b) - (ref + e)) <= bound + 1e-6 * np.abs(e))
    r = ora.matmul_add_relu(e, a, b)
    assert np.all(r >= 0)
    assert np.all(np.abs(r - np.maximum(ref + e, 0)) <= bound + 1e-6 * np.abs(e))


def test_batch_matmul_oracle_is_loop():
    g = np.random.Generator(np.random.PCG64(9))
    a = g.standard_normal((3, 10, 8)).astype(np.float32)
    b = g.standard_normal((3, 8, 12)).astype(np.float32)
    out = ora.batch_matmul(a, b)
    for i in range(3):
        np.testing.assert_array_equal(out[i], ora.matmul(a[i], b[i]))


def test_dense_layer_relu_and_sigmoid():
    g = np.random.Generator(np.random.PCG64(4))
    a = g.standard_normal((20, 16)).astype(np.float32)
    w = g.standard_normal((16, 9)).astype(np.float32)
    bias = g.standard_normal(9).astype(np.float32)
    lin = ora.dense_layer(a, w, bias, 0)
    np.testing.assert_allclose(lin, a.astype(np.float64) @ w + bias, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(ora.dense_layer(a, w, bias, 1), np.where(lin < 0, 0, lin))
    np.testing.assert_allclose(ora.dense_layer(a, w, bias, 2), 1 / (1 + np.exp(-lin.astype(np.float64))),
                               rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------- KPFusedGather
NONZERO_GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                           "segment_reduce_nonzero_reference_gtest.json")))


@pytest.mark.parametrize("case", NONZERO_GOLD["cases"], ids=lambda c: c["name"])
def test_segment_reduce_nonzero_reference_goldens(case):
    """The reference's KPFusedSparseSegmentReduceNonzero goldens pin the
    segment reduction (index-order sums, mean = sum * (1/count), max_seg + 1
    rows): the oracle's dense result, listed as that op lists it, equals
    them exactly."""
    from tests.nonzero_util import case_inputs, check_case
    data, indices, _, seg = case_inputs(case)
    data2 = data.reshape(data.shape[0], -1)
    dense = ora.segment_reduce(data2, indices, seg, int(seg.max()) + 1, case["combiner"])
    check_case(case, dense)


@pytest.mark.parametrize("case", NONZERO_GOLD["cases"], ids=lambda c: c["name"])
def test_oracle_segment_reduce_nonzero_goldens(case):
    """ora_segment_reduce_nonzero reproduces the reference op's goldens."""
    from tests.nonzero_util import case_inputs
    data, indices, _, seg = case_inputs(case)
    shape, idx, val = ora.segment_reduce_nonzero(data, indices, seg, case["combiner"])
    assert shape.tolist() == case["expected_shape"]
    assert list(idx.shape) == case["expected_indices_shape"]
    assert idx.reshape(-1).tolist() == case["expected_indices"]
    np.testing.assert_array_equal(val, np.asarray(case["expected_values"], np.float32))


@pytest.mark.parametrize("one_d", [True, False])
@pytest.mark.parametrize("combiner", [0, 1])
def test_oracle_segment_reduce_nonzero_random(one_d, combiner):
    """On shuffled segment ids (first appearance differs from id order) and
    data with zeros, the op's listing equals the listing of
    ora_segment_reduce's dense result in first-appearance order."""
    from tests.nonzero_util import nonzero_coo
    g = np.random.default_rng(11 + combiner + 2 * one_d)
    n, rows, dim = 300, 50, 1 if one_d else 7
    data = g.integers(-2, 3, size=(rows, dim)).astype(np.float32)  # many exact zeros
    indices = g.integers(0, rows, size=n).astype(np.int32)
    seg = g.permutation(np.repeat(np.arange(40), 8)[:n]).astype(np.int64)
    dense = ora.segment_reduce(data, indices, seg, int(seg.max()) + 1, combiner)
    want = nonzero_coo(dense, seg, one_d)
    got = ora.segment_reduce_nonzero(data[:, 0] if one_d else data, indices, seg, combiner)
    for w, o in zip(want, got):
        np.testing.assert_array_equal(o, w)


def test_segment_reduce_nonzero_check_catches_a_wrong_reduction():
    """The check fails for a reduction that drops the first position (a
    mistake planted in the oracle's inputs, on the CPU)."""
    from tests.nonzero_util import case_inputs, check_case
    case = [c for c in NONZERO_GOLD["cases"] if c["name"] == "Test2DReduceSum"][0]
    data, indices, _, seg = case_inputs(case)
    dense = ora.segment_reduce(data, indices[1:], seg[1:], int(seg.max()) + 1, 0)
    with pytest.raises(AssertionError):
        check_case(case, dense)


GATHER_GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                          "fused_gather_reference_gtest.json")))


def test_fused_gather_reference_golden():
    c = GATHER_GOLD["cases"][0]
    data = np.asarray(c["data"], np.float32).reshape(c["data_shape"])
    keys = np.asarray(c["slice_input"], np.int64).reshape(c["slice_shape"])
    u, idx, rows = ora.fused_gather(data, keys, c["begin"][1])
    assert u.tolist() == c["expected_unique"]
    assert idx.tolist() == c["expected_indices"]
    assert rows.reshape(-1).tolist() == c["expected_data"]


@pytest.mark.parametrize("n,span", [(1, 1), (50, 5), (5000, 300), (20000, 10**9)])
def test_fused_gather_against_numpy_unique(n, span):
    """First-occurrence order: numpy.unique gives sorted keys with the index
    of each key's first occurrence; ordering the keys by that index is the
    reference's order, and the inverse map renumbered the same way is the
    per-row index."""
    g = np.random.default_rng(n)
    keys = g.integers(-span, span, size=(n, 3))
    table = g.standard_normal((4, 5)).astype(np.float32)
    keys[:, 1] = np.abs(keys[:, 1]) % 4
    u, idx, rows = ora.fused_gather(table, keys, 1)
    srt, first, inv = np.unique(keys[:, 1], return_index=True, return_inverse=True)
    order = np.argsort(first, kind="stable")
    rank = np.empty_like(order)
    rank[order] = np.arange(order.size)
    np.testing.assert_array_equal(u, srt[order])
    np.testing.assert_array_equal(idx, rank[inv.reshape(-1)])
    np.testing.assert_array_equal(rows, table[u])


def test_fused_gather_out_of_range_is_reported():
    with pytest.raises(IndexError):
        ora.fused_gather(np.zeros((2, 3), np.float32), np.array([[0], [2]], np.int64), 0)


# ---------------------------------------------------------------- KPFusedBatchMatMulAddSigmoid
BMS_GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "batch_matmul_add_sigmoid_reference_gtest.json")))


def make_range(shape, start_step):
    """MakeRange (fused_batchmatmul_add_sigmoid_test.cc:30-36): start + step*i in float32."""
    start, step = (np.float32(v) for v in start_step)
    size = int(np.prod(shape))
    return (start + step * np.arange(size, dtype=np.float32)).astype(np.float32).reshape(shape)


def bms_inputs(c):
    return (make_range(c["lhs_shape"], c["lhs_range"]), make_range(c["rhs_shape"], c["rhs_range"]),
            make_range(c["bias_shape"], c["bias_range"]))


@pytest.mark.parametrize("case", BMS_GOLD["cases"], ids=lambda c: c["name"])
def test_batch_matmul_add_sigmoid_oracle_closed_form(case):
    """Against float64 numpy (matmul, broadcasting, exp) at the reference
    test's own tolerance."""
    lhs, rhs, bias = bms_inputs(case)
    lin = np.matmul(lhs.astype(np.float64), rhs.astype(np.float64)) + bias.astype(np.float64)
    want = 1.0 / (1.0 + np.exp(-lin))
    got = ora.batch_matmul_add_sigmoid(lhs, rhs, bias)
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=0, atol=BMS_GOLD["tolerance"])
