"""GPU parity: embedding bags, segment reduction, masked gather, pooling.

Bit-exact against the CPU oracle (same summation order per dim)."""
import json
import os

import numpy as np
import pytest
import torch

from annc_amd import tf_ops, workloads, xla
from annc_amd import device as dev
from oracle import ora
from tests.gpu_util import device, note, to_dev, to_host

pytestmark = pytest.mark.gpu
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "segment_reduce_reference_gtest.json")))


@pytest.mark.parametrize("combiner", [0, 1])
@pytest.mark.parametrize("idx_dtype", [np.int64, np.int32])
def test_bag_config3_bit_exact(combiner, idx_dtype):
    note(f"bag config3 combiner={combiner} idx={idx_dtype.__name__}")
    w = workloads.config3(seed=0)
    ids = w.ids.astype(idx_dtype)
    ref = ora.embedding_bag(w.table, ids, w.offsets, combiner, threads=8)
    out = dev.embedding_bag(to_dev(w.table), to_dev(ids), to_dev(w.offsets), combiner)
    dev.stream_status()
    np.testing.assert_array_equal(to_host(out), ref)


@pytest.mark.parametrize("dim", [1, 3, 4, 8, 16, 20, 32, 64, 100, 128, 256, 260, 512])
def test_bag_dims_bit_exact(dim):
    note(f"bag dim={dim}")
    g = workloads.rng(dim)
    rows = 5000
    table = g.standard_normal((rows, dim)).astype(np.float32)
    lens = np.clip(g.poisson(9, size=300), 0, 40)
    lens[:5] = [0, 1, 40, 0, 8]  # empty, single, long bags
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ids = g.integers(0, rows, size=int(offsets[-1])).astype(np.int64)
    for combiner in (0, 1):
        ref = ora.embedding_bag(table, ids, offsets, combiner)
        out = dev.embedding_bag(to_dev(table), to_dev(ids), to_dev(offsets), combiner)
        np.testing.assert_array_equal(to_host(out), ref)


@pytest.mark.parametrize("seed", range(48))
def test_bag_random_configurations(seed):
    """Seeded random bags: dims of every lane-group width and the scalar
    path, 1 to 20000 bags of Poisson or heavy-tailed lengths (empty bags
    included), uniform or Zipf ids, int32 and int64 ids, both combiners, an
    output with padded rows; bit-exact against the sequential loop, the
    padding untouched."""
    g = np.random.default_rng(5000 + seed)
    dim = int(g.choice([1, 2, 3, 4, 6, 8, 12, 16, 20, 32, 60, 64, 100, 128, 256, 260, 512]))
    rows = min(int(g.integers(1, 200_000)), 20_000_000 // dim)
    nbags = int(g.choice([1, 5, 300, 4096, 20000]))
    lens = (g.poisson(g.choice([0.3, 3, 20, 200]), size=nbags) if seed % 3 else
            np.minimum(g.zipf(1.4, size=nbags) - 1, 2000))
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n = int(offsets[-1])
    ids = (g.integers(0, rows, size=n) if seed % 2 else
           np.minimum(g.zipf(1.2, size=n) - 1, rows - 1))
    ids = ids.astype(np.int64 if seed % 4 < 2 else np.int32)
    table = g.standard_normal((rows, dim)).astype(np.float32)
    pad = int(g.choice([0, 3]))
    note(f"bag random config seed={seed}: dim {dim} rows {rows} bags {nbags} ids {n} "
         f"{ids.dtype} pad {pad}")
    dt, di, do = to_dev(table), to_dev(ids), to_dev(offsets)
    for combiner in (0, 1):
        obuf = torch.full((nbags, dim + pad), float("nan"), device=device())
        dev.embedding_bag(dt, di, do, combiner, out=obuf[:, :dim])
        dev.stream_status()
        got = to_host(obuf)
        np.testing.assert_array_equal(got[:, :dim],
                                      ora.embedding_bag(table, ids, offsets, combiner, threads=8))
        assert np.isnan(got[:, dim:]).all()


def test_bag_strided_output_and_no_bags():
    note("bag strided output")
    g = workloads.rng(1)
    table = g.standard_normal((100, 16)).astype(np.float32)
    offsets = np.array([0, 3, 3, 7], dtype=np.int64)
    ids = g.integers(0, 100, size=7).astype(np.int64)
    wide = torch.full((3, 40), 7.0, device=device())
    dev.embedding_bag(to_dev(table), to_dev(ids), to_dev(offsets), 1, out=wide[:, 8:24])
    h = to_host(wide)
    np.testing.assert_array_equal(h[:, 8:24], ora.embedding_bag(table, ids, offsets, 1))
    assert (h[:, :8] == 7).all() and (h[:, 24:] == 7).all()
    empty = dev.embedding_bag(to_dev(table), to_dev(ids), to_dev(np.zeros(1, np.int64)), 0)
    assert empty.shape == (0, 16)


def test_empty_inputs_through_the_device_wrappers():
    """No ids, keys or strings: empty tensors (torch gives them null data
    pointers) through every device wrapper give empty results, or all-zero
    bags and segments, and leave no error on the stream."""
    note("empty inputs through the device wrappers")
    d = device()
    table = to_dev(np.arange(40, dtype=np.float32).reshape(10, 4))
    none64 = torch.empty(0, dtype=torch.int64, device=d)
    for combiner in (0, 1):
        out = dev.embedding_bag(table, none64, torch.zeros(3, dtype=torch.int64, device=d),
                                combiner)
        np.testing.assert_array_equal(to_host(out), np.zeros((2, 4), np.float32))
        out = dev.hashed_embedding_bags([table, table], [10, 7], none64,
                                        torch.zeros(2 * 3 + 1, dtype=torch.int64, device=d), 3,
                                        combiner)
        np.testing.assert_array_equal(to_host(out), np.zeros((3, 8), np.float32))
        out = dev.segment_reduce(table, none64, none64, 3, combiner)
        np.testing.assert_array_equal(to_host(out), np.zeros((3, 4), np.float32))
    assert dev.sparse_embedding2(table, none64).shape == (0, 4)
    assert dev.hash_bucket_int64(none64, 100).shape == (0,)
    u, idx, rows = dev.unique_gather(table, none64)
    assert u.shape == (0,) and idx.shape == (0,) and rows.shape == (0, 4)
    pooled = dev.pooling(torch.empty((0, 3), dtype=torch.int64, device=d),
                         torch.empty((0, 3, 4), dtype=torch.float32, device=d), [0, 0, 0],
                         [0, 3, 4])
    assert pooled.shape == (0, 4)
    data, offs = dev.strings_to_device([""], d)
    got = to_host(dev.fingerprint64(data, offs))
    np.testing.assert_array_equal(got.view(np.uint64), ora.fingerprint64_batch([b""]))
    dev.stream_status()


def test_bag_out_of_range_ids_flagged():
    note("bag out-of-range ids")
    table = np.ones((10, 8), dtype=np.float32)
    ids = np.array([1, 10, -1, 2], dtype=np.int64)
    offsets = np.array([0, 2, 4], dtype=np.int64)
    out = dev.embedding_bag(to_dev(table), to_dev(ids), to_dev(offsets), 0)
    with pytest.raises(Exception, match="out of range"):
        dev.stream_status()
    np.testing.assert_array_equal(to_host(out), np.ones((2, 8), np.float32))
    dev.stream_status()  # flag cleared


@pytest.mark.parametrize("case", GOLD["cases"], ids=lambda c: c["name"])
@pytest.mark.parametrize("where", ["host", "device"])
def test_tf_segment_reduce_reference_goldens(case, where):
    note(f"segment reduce golden {case['name']} {where}")
    data = np.asarray(case["data"], dtype=np.float32)
    idx = np.asarray(case["indices"], dtype=np.int32)
    sl = np.asarray(case["slice_input"], dtype=np.int64)
    begin = np.asarray(case["begin"], np.int32)
    begin1 = np.asarray(case["begin_1"], np.int32)
    if where == "device":
        data, idx, sl = to_dev(data), to_dev(idx), to_dev(sl)
    out, so = tf_ops.kp_fused_sparse_segment_reduce(data, idx, sl, begin, begin1, case["combiner"])
    out = to_host(out) if where == "device" else out
    np.testing.assert_array_equal(out, np.asarray(case["expected"], np.float32))
    assert int(so) == case["expected_slice_output"]


@pytest.mark.parametrize("sorted_segments", [True, False])
@pytest.mark.parametrize("combiner", [0, 1])
def test_tf_segment_reduce_random(sorted_segments, combiner):
    note(f"segment reduce random sorted={sorted_segments} combiner={combiner}")
    g = workloads.rng(21)
    rows, dim, n = 20000, 24, 50000
    data = g.standard_normal((rows, dim)).astype(np.float32)
    idx = g.integers(0, rows, size=n).astype(np.int64)
    seg = g.integers(0, 3000, size=n).astype(np.int64)
    if sorted_segments:
        seg.sort()
    slice_input = np.stack([np.zeros(n, np.int64), seg, seg * 7], axis=1)
    out, so = tf_ops.kp_fused_sparse_segment_reduce(data, idx, slice_input,
                                                    np.array([0, 1], np.int32),
                                                    np.array([0], np.int32), combiner)
    batch = int(seg.max()) + 1
    assert out.shape == (batch, dim) and int(so) == batch
    np.testing.assert_array_equal(out, ora.segment_reduce(data, idx, seg, batch, combiner))


def test_tf_segment_reduce_empty_indices():
    note("segment reduce empty")
    out, so = tf_ops.kp_fused_sparse_segment_reduce(
        np.ones((3, 4), np.float32), np.zeros(0, np.int32), np.zeros((0, 2), np.int64),
        np.array([0, 1], np.int32), np.array([1], np.int32), 1)
    np.testing.assert_array_equal(out, np.zeros((1, 4), np.float32))  # max_seg starts at 0
    assert int(so) == 4


SEG_ORDER_CASES = [
    ("reversed", 3000, 50000),
    ("one segment over 5 blocks of 1024 positions", 1, 5000),
    ("largest sort batch: 64 segments per filter workgroup", 16384, 70000),
    ("radix-sort batch", 16385, 70000),
    ("mostly empty segments", 10000, 100),
    ("ids outside [0, batch) dropped", 1000, 30000),
    ("ids outside [0, batch) dropped, radix sort", 20000, 30000),
    ("radix sort, 16 key bits exactly (2 passes), ids outside [0, batch) dropped", 2**16 - 1, 200_000),
    ("radix sort, 3 passes (18 key bits)", 2**17 + 5, 300_000),
    ("radix sort, 4 passes (25 key bits)", 2**24 + 3, 300_000),
    ("sorted", 4096, 81857),
    ("two-level sort, 128 blocks", 4096, 131072),
    ("two-level sort, last block partial", 4096, 131073),
    ("two-level sort, 5000 segments: 5 per one-wave range, 3 key bits", 5000, 90000),
    ("two-level sort past the one-wave ranges' 1 Mi positions", 4096, 1_200_000),
    ("counting sort: past the two-level sort's 4 Mi positions", 64, 4 * 2**20 + 1),
    ("counting sort, ids outside [0, batch) dropped", 2000, 4 * 2**20 + 3000),
    ("three segments: more entries per range than its list holds", 3, 100000),
    ("skewed: every other position in one segment", 4096, 120000),
]


@pytest.mark.parametrize("what,batch,n", SEG_ORDER_CASES)
@pytest.mark.parametrize("combiner", [0, 1])
def test_device_segment_reduce_orders(what, batch, n, combiner):
    """Every segment's rows are summed in position order whatever the order
    of the segment ids (up to 16384 segments: the two-level sort up to 4 Mi
    positions, the stable counting sort beyond; radix sort for more
    segments): bit-exact against the sequential loop."""
    note(f"device segment reduce: {what} (batch {batch}, n {n}, combiner {combiner})")
    g = workloads.rng(batch + n)
    data = g.standard_normal((2000, 8)).astype(np.float32)
    idx = g.integers(0, 2000, size=n).astype(np.int64)
    seg = g.integers(0, batch, size=n).astype(np.int64)
    if what.startswith("reversed"):
        seg = np.sort(seg)[::-1].copy()
    elif what.startswith("skewed"):
        seg[::2] = 17
    elif what.startswith("sorted"):
        seg.sort()
    keep = np.ones(n, bool)
    if what.startswith("ids outside") or "dropped" in what:
        bad = g.choice(n, size=n // 10, replace=False)
        seg[bad] = g.choice([-1, -7, batch, batch + 5, 2**40], size=bad.size)
        keep[bad] = False
    out = dev.segment_reduce(to_dev(data), to_dev(idx), to_dev(seg), batch, combiner)
    ref = ora.segment_reduce(data, idx[keep], seg[keep], batch, combiner)
    np.testing.assert_array_equal(to_host(out), ref)
    if what.startswith("sorted"):  # the caller's promise skips the sort: same bits
        out = dev.segment_reduce(to_dev(data), to_dev(idx), to_dev(seg), batch, combiner,
                                 sorted_ids=True)
        np.testing.assert_array_equal(to_host(out), ref)


def test_device_segment_reduce_radix_sort_long_scan():
    """Radix-sort path over 2^26 + 123 positions: 16,385 blocks of 4096, so
    the scan of the digit histograms (256 per block) spans 1025 tiles and
    its tile-totals step walks two totals per thread; bit-exact against the
    sequential loop."""
    n, batch = 2**26 + 123, 70_000
    note(f"device segment reduce: radix sort, long scan (batch {batch}, n {n})")
    g = workloads.rng(77)
    data = g.standard_normal((2000, 4)).astype(np.float32)
    idx = g.integers(0, 2000, size=n, dtype=np.int64)
    seg = g.integers(0, batch, size=n, dtype=np.int64)
    out = dev.segment_reduce(to_dev(data), to_dev(idx), to_dev(seg), batch, 1)
    np.testing.assert_array_equal(to_host(out), ora.segment_reduce(data, idx, seg, batch, 1))


SORTED_CHUNK = 160  # positions per workgroup of the sorted-id kernel


def _sorted_segments(what, g):
    """Non-decreasing segment ids for the sorted-id path, and the batch.
    The path cuts positions into chunks of SORTED_CHUNK (plus the closing
    position n) and reads one chunk ahead: the cases put boundaries on and
    around chunk edges, segments longer than the read-ahead, and runs of
    empty segments."""
    c = SORTED_CHUNK
    if what == "no positions":
        return np.zeros(0, np.int64), 5
    if what == "one position":
        return np.array([2], np.int64), 3
    sizes = {"n = chunk - 1": c - 1, "n = chunk": c, "n = chunk + 1": c + 1,
             "n = 2 * chunk - 1": 2 * c - 1, "n = 2 * chunk": 2 * c}
    if what in sizes:
        return np.sort(g.integers(0, 50, size=sizes[what])), 50
    if what == "empty segments at both ends":
        return np.sort(g.integers(10, 90, size=3000)), 100
    if what == "one segment over 30 chunks":
        return np.repeat(np.array([0, 1, 2, 4]), [3, 5000, 1, 700]), 6
    if what == "segments of one chunk, on chunk edges":
        return np.repeat(np.arange(40), c), 40
    if what == "segments of two chunks, on chunk edges":
        return np.repeat(np.arange(20), 2 * c), 21
    if what == "segments of a chunk -1 and +1 positions":
        return np.repeat(np.arange(30), np.tile([c - 1, c + 1], 15)), 30
    if what == "mostly empty segments":
        return np.sort(g.choice(100000, size=300, replace=False)), 100000
    if what == "ids outside [0, batch) at both ends":
        seg = np.concatenate([g.integers(-10, 1010, size=20000), [-2**40, -2, 2**40, 1000]])
        return np.sort(seg), 1000
    if what == "every id outside [0, batch)":
        return np.full(700, -5, np.int64), 10
    if what == "configs[2] shape":
        return np.sort(g.integers(0, 4096, size=81857)), 4096
    raise AssertionError(what)


SORTED_CASES = ["no positions", "one position", "n = chunk - 1", "n = chunk", "n = chunk + 1",
                "n = 2 * chunk - 1", "n = 2 * chunk", "empty segments at both ends",
                "one segment over 30 chunks", "segments of one chunk, on chunk edges",
                "segments of two chunks, on chunk edges",
                "segments of a chunk -1 and +1 positions", "mostly empty segments",
                "ids outside [0, batch) at both ends", "every id outside [0, batch)",
                "configs[2] shape"]


@pytest.mark.parametrize("what", SORTED_CASES)
@pytest.mark.parametrize("dim,idx64", [(16, True), (6, False), (300, True), (64, False)])
def test_device_segment_reduce_sorted_ids(what, dim, idx64):
    """The caller's promise of non-decreasing segment ids takes the one-launch
    path (segment boundaries found per chunk of positions, no offsets array):
    bit-exact against the sequential loop, both combiners, with the ids read
    in place from a column of a [n, 3] slice (stride 3) as the TF op passes
    them; dim 6 takes the scalar lane groups, 300 two column chunks."""
    note(f"device segment reduce sorted ids: {what} (dim {dim}, idx64 {idx64})")
    g = workloads.rng(len(what) * 131 + dim)
    seg, batch = _sorted_segments(what, g)
    seg = seg.astype(np.int64)
    n = seg.size
    assert (np.diff(seg) >= 0).all()
    rows = 900
    data = g.standard_normal((rows, dim)).astype(np.float32)
    idx = g.integers(0, rows, size=n).astype(np.int64 if idx64 else np.int32)
    keep = (seg >= 0) & (seg < batch)
    slice3 = np.stack([np.zeros(n, np.int64), seg, -seg], axis=1)
    seg_col = to_dev(slice3)[:, 1]
    assert n < 2 or seg_col.stride(0) == 3
    for combiner in (0, 1):
        out = dev.segment_reduce(to_dev(data), to_dev(idx), seg_col, batch, combiner,
                                 sorted_ids=True)
        ref = ora.segment_reduce(data, idx[keep], seg[keep], batch, combiner)
        np.testing.assert_array_equal(to_host(out), ref)


@pytest.mark.parametrize("dim", [4, 6, 12, 16, 32, 64, 128, 256, 300])
@pytest.mark.parametrize("idx64", [True, False])
def test_device_segment_reduce_any_order_dims(dim, idx64):
    """Unsorted segment ids at every lane-group width of the fused range
    kernels (G = 4..64 lanes a segment; dim 300 takes two column chunks;
    dim 6 is not a multiple of 4 and takes the sort with perm and the bag
    kernel), int32 and int64 indices, both combiners: bit-exact."""
    note(f"device segment reduce any order dim={dim} idx64={idx64}")
    g = workloads.rng(dim * 2 + idx64)
    rows, n, batch = 700, 9000, 1500
    data = g.standard_normal((rows, dim)).astype(np.float32)
    idx = g.integers(0, rows, size=n).astype(np.int64 if idx64 else np.int32)
    seg = g.integers(0, batch, size=n).astype(np.int64)
    for combiner in (0, 1):
        out = dev.segment_reduce(to_dev(data), to_dev(idx), to_dev(seg), batch, combiner)
        np.testing.assert_array_equal(to_host(out), ora.segment_reduce(data, idx, seg, batch,
                                                                       combiner))


@pytest.mark.parametrize("seed", range(64))
def test_device_segment_reduce_random_configurations(seed):
    """Seeded random configurations across both paths (sorted promise or
    not): dims of every lane-group width and the scalar path, int32 and
    int64 indices, Poisson or heavy-tailed segment lengths with empty
    segments, ids outside [0, batch), both combiners; bit-exact against the
    sequential loop."""
    g = np.random.default_rng(1000 + seed)
    dim = int(g.choice([1, 3, 4, 8, 12, 16, 20, 32, 64, 100, 128, 256, 260]))
    rows = int(g.integers(50, 3000))
    batch = int(g.choice([1, 7, 100, 1000, 5000]))
    lens = (g.poisson(g.choice([0.5, 3, 20]), size=batch) if seed % 3 else
            np.minimum(g.zipf(1.5, size=batch), 3000))
    seg = np.repeat(np.arange(batch, dtype=np.int64), lens)
    n = seg.size
    bad = g.random(n) < (0.05 if seed % 4 == 0 else 0.0)
    seg[bad] = g.choice([-3, -1, batch, batch + 9], size=int(bad.sum()))
    sorted_ids = bool(seed % 2)
    if sorted_ids:
        seg = np.sort(seg)
    else:
        seg = seg[g.permutation(n)]
    idx64 = bool(seed % 5 < 3)
    idx = g.integers(0, rows, size=n).astype(np.int64 if idx64 else np.int32)
    data = g.standard_normal((rows, dim)).astype(np.float32)
    keep = (seg >= 0) & (seg < batch)
    note(f"segment reduce random config seed={seed}: dim {dim} batch {batch} n {n} "
         f"sorted {sorted_ids} idx64 {idx64}")
    for combiner in (0, 1):
        out = dev.segment_reduce(to_dev(data), to_dev(idx), to_dev(seg), batch, combiner,
                                 sorted_ids=sorted_ids)
        np.testing.assert_array_equal(
            to_host(out), ora.segment_reduce(data, idx[keep], seg[keep], batch, combiner))


def test_device_segment_reduce_unsorted():
    note("device segment reduce")
    g = workloads.rng(8)
    data = g.standard_normal((500, 12)).astype(np.float32)
    idx = g.integers(0, 500, size=4000).astype(np.int32)
    seg = g.integers(0, 700, size=4000).astype(np.int64)
    out = dev.segment_reduce(to_dev(data), to_dev(idx), to_dev(seg), 700, 1)
    np.testing.assert_array_equal(to_host(out), ora.segment_reduce(data, idx, seg, 700, 1))


@pytest.mark.parametrize("dim", [16, 1, 3, 64, 300, 1028])
@pytest.mark.parametrize("idx_dtype", [np.int64, np.int32])
def test_sparse_embedding2_bit_exact(dim, idx_dtype):
    """dims divisible by 4 take the lane-group float4 kernel (1028: chunks of
    256 floats), the others the scalar one; masked ids multiply the fallback
    row by 0, so a NaN there stays NaN, as in the reference's mul."""
    note(f"sparse_embedding2 dim={dim} ids={np.dtype(idx_dtype).name}")
    g = workloads.rng(3 + dim)
    table = g.standard_normal((1000, dim)).astype(np.float32)
    table[0, 0] = np.nan   # the fallback row
    table[7, -1] = -0.0
    ids = g.integers(-50, 1050, size=3000).astype(idx_dtype)
    ids[:4] = [7, -1, 999, 1000]
    out = dev.sparse_embedding2(to_dev(table), to_dev(ids), fallback_row=0)
    got = to_host(out)
    ref = ora.sparse_embedding2(table, ids, 0)
    np.testing.assert_array_equal(got, ref)
    assert (np.signbit(got) == np.signbit(ref)).all()
    assert np.isnan(got[1, 0])


# slices as (starts, limits) for rows of k positions: all of it, an inner
# box, and a late start with every column
POOL_SLICES = {"full": lambda k, n: ((0, 0, 0), (64, k, n)),
               "inner": lambda k, n: ((3, 2, 1), (60, max(k - 5, 3), min(12, n))),
               "late_start": lambda k, n: ((0, min(4, k - 1), 0), (64, k, n))}


# k <= 16, 32 and 48 take the one-round kernel (R = 16, 32, 48; 48 is its
# edge), longer rows the multi-round one; n = 4, 8, 16, 64, 260 give lane
# groups of 1, 2, 4, 16 and 64 (260: two column chunks), n = 6 the scalar kernel
@pytest.mark.parametrize("k", [7, 30, 39, 48, 49, 100])
@pytest.mark.parametrize("n", [4, 8, 16, 64, 6, 260])
@pytest.mark.parametrize("slice_kind", list(POOL_SLICES))
def test_pooling_bit_exact(k, n, slice_kind):
    """n % 4 == 0 takes the lane-group kernels (masked positions are never
    read: NaNs there must not leak), other widths the scalar one."""
    ss, sl = POOL_SLICES[slice_kind](k, n)
    note(f"pooling k={k} n={n} {ss} {sl}")
    g = workloads.rng(4 + n + 7 * k)
    ids = g.integers(-2, 50, size=(64, k)).astype(np.int64)
    ids[5] = 0
    gathered = g.standard_normal((64, k, n)).astype(np.float32)
    gathered[ids <= 0] = np.nan
    ref = ora.pooling(ids, gathered, ss, sl)
    got = to_host(dev.pooling(to_dev(ids), to_dev(gathered), ss, sl))
    np.testing.assert_array_equal(got, ref)
    out = np.empty((64, n), np.float32)
    xla.pooling(ids, gathered, ss, sl, out)  # __pooling custom call on host buffers
    np.testing.assert_array_equal(out, ref)


NONZERO_GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                           "segment_reduce_nonzero_reference_gtest.json")))


@pytest.mark.parametrize("where", ["host", "device"])
@pytest.mark.parametrize("case", NONZERO_GOLD["cases"], ids=lambda c: c["name"])
def test_segment_reduce_nonzero_reference_goldens(case, where):
    """The reference's KPFusedSparseSegmentReduceNonzero goldens through the
    KPFusedSparseSegmentReduce entry (same reduction, dense output): listed
    as the nonzero op lists its output, the result equals the goldens."""
    from tests.nonzero_util import case_inputs, check_case
    note(f"nonzero golden {case['name']} ({where})")
    data, indices, slice_input, _ = case_inputs(case)
    data2 = np.ascontiguousarray(data.reshape(data.shape[0], -1))
    begin = np.asarray(case["begin"], np.int32)
    begin_1 = np.zeros(1, np.int32)
    if where == "device":
        data2, indices, slice_input = to_dev(data2), to_dev(indices), to_dev(slice_input)
    out, _ = tf_ops.kp_fused_sparse_segment_reduce(data2, indices, slice_input, begin, begin_1,
                                                   case["combiner"])
    check_case(case, to_host(out) if where == "device" else np.asarray(out))


@pytest.mark.parametrize("where", ["host", "device"])
@pytest.mark.parametrize("case", NONZERO_GOLD["cases"], ids=lambda c: c["name"])
def test_tf_segment_reduce_nonzero_reference_goldens(case, where):
    """KPFusedSparseSegmentReduceNonzero on the GPU reproduces the reference
    op's goldens exactly."""
    from tests.nonzero_util import case_inputs
    note(f"KPFusedSparseSegmentReduceNonzero golden {case['name']} ({where})")
    data, indices, slice_input, _ = case_inputs(case)
    if where == "device":
        data, indices, slice_input = to_dev(data), to_dev(indices), to_dev(slice_input)
    shape, idx, val = tf_ops.kp_fused_sparse_segment_reduce_nonzero(
        data, indices, slice_input, np.asarray(case["begin"], np.int32), case["combiner"])
    if where == "device":
        idx, val = to_host(idx), to_host(val)
    assert shape.tolist() == case["expected_shape"]
    assert list(idx.shape) == case["expected_indices_shape"]
    assert idx.reshape(-1).tolist() == case["expected_indices"]
    np.testing.assert_array_equal(val, np.asarray(case["expected_values"], np.float32))


@pytest.mark.parametrize("one_d", [True, False])
@pytest.mark.parametrize("combiner", [0, 1])
@pytest.mark.parametrize("idx64", [False, True])
def test_tf_segment_reduce_nonzero_random_bit_exact(one_d, combiner, idx64):
    """Shuffled segment ids (first appearance differs from id order), data
    with exact zeros and a NaN, 5000 positions: equal to the oracle."""
    note(f"KPFusedSparseSegmentReduceNonzero random one_d={one_d} comb={combiner} idx64={idx64}")
    g = workloads.rng(100 + 4 * one_d + 2 * combiner + idx64)
    n, rows, dim = 5000, 300, 1 if one_d else 20
    data = g.integers(-2, 3, size=(rows, dim)).astype(np.float32)
    data[7, 0] = np.nan
    indices = g.integers(0, rows, size=n).astype(np.int64 if idx64 else np.int32)
    seg = g.permutation(np.repeat(np.arange(700), 8)[:n]).astype(np.int64)
    slice_input = np.stack([np.zeros(n, np.int64), seg], axis=1)
    data_in = data[:, 0].copy() if one_d else data
    want = ora.segment_reduce_nonzero(data_in, indices, seg, combiner)
    shape, idx, val = tf_ops.kp_fused_sparse_segment_reduce_nonzero(
        to_dev(data_in), to_dev(indices), to_dev(slice_input), np.array([0, 1], np.int32), combiner)
    np.testing.assert_array_equal(shape, want[0])
    np.testing.assert_array_equal(to_host(idx), want[1])
    np.testing.assert_array_equal(to_host(val), want[2])


@pytest.mark.parametrize("case", ["normal", "negative_ids", "negative_small_range",
                                  "many_segments", "host_5000"])
def test_tf_segment_reduce_nonzero_order_sensitive(case):
    """Data from standard_normal, so the summation order shows in the bits:
    negative segment ids (INT64_MIN among them, listed as the reference's
    int32 cast lists them), more than 16384 first-appearance segments (the
    radix-sort path) and host-memory operands at 5000 positions; each equal
    to the oracle bit for bit.  Segment ids spanning a small range (negative
    ones included) take the directly indexed first-occurrence table, the
    others the hash table."""
    note(f"KPFusedSparseSegmentReduceNonzero order-sensitive {case}")
    g = workloads.rng({"normal": 31, "negative_ids": 32, "many_segments": 33,
                       "host_5000": 34, "negative_small_range": 36}[case])
    n, rows, dim, nseg = 6000, 400, 9, 900
    if case == "many_segments":
        n, nseg = 40000, 20000
    seg = g.permutation(np.arange(n) % nseg).astype(np.int64)
    if case == "negative_small_range":
        seg = seg - nseg // 2
    if case == "negative_ids":
        seg = seg - nseg // 2
        seg[seg == -7] = np.iinfo(np.int64).min
        seg[seg == 5] = -(2 ** 40)
    data = g.standard_normal((rows, dim)).astype(np.float32)
    indices = g.integers(0, rows, size=n).astype(np.int64)
    slice_input = np.stack([np.zeros(n, np.int64), seg, np.ones(n, np.int64)], axis=1)
    for combiner in (0, 1):
        want = ora.segment_reduce_nonzero(data, indices, seg, combiner)
        args = (data, indices, slice_input) if case == "host_5000" else \
            (to_dev(data), to_dev(indices), to_dev(slice_input))
        shape, idx, val = tf_ops.kp_fused_sparse_segment_reduce_nonzero(
            *args, np.array([0, 1], np.int32), combiner)
        if case != "host_5000":
            idx, val = to_host(idx), to_host(val)
        np.testing.assert_array_equal(shape, want[0])
        np.testing.assert_array_equal(idx, want[1])
        np.testing.assert_array_equal(val, want[2])


def _nonzero_args(data, indices, slice_input, rows, dim, n, combiner, shape, nnz, keep):
    """C-ABI arguments of annc_kp_fused_sparse_segment_reduce_nonzero (the
    host shape arrays are appended to `keep` so they outlive the call)."""
    from annc_amd import _lib
    ddims = np.array([rows, dim], np.int64)
    sdims = np.array([n, 2], np.int64)
    begin = np.array([0, 1], np.int32)
    keep += [ddims, sdims, begin]
    return (_lib.ptr(data), 2, _lib.ptr(ddims), _lib.ptr(indices), 0, n, _lib.ptr(slice_input),
            2, _lib.ptr(sdims), _lib.ptr(begin), 2, combiner, _lib.ptr(shape), _lib.ptr(nnz))


@pytest.mark.parametrize("between", [False, True])
def test_tf_segment_reduce_nonzero_short_phase2_buffer(between):
    """A phase-2 call whose buffers hold one value fewer than phase 1
    counted is refused with the count mismatch, and writes nothing past the
    buffers it was given (a guard word after them keeps its value; the write
    kernel stops at the buffer's end itself), with or without a phase 1 on
    other operands in between."""
    import ctypes
    from annc_amd import _lib
    note(f"KPFusedSparseSegmentReduceNonzero short phase-2 buffer (between={between})")
    g = workloads.rng(35)
    n, rows, dim = 500, 50, 4
    data = to_dev(g.standard_normal((rows, dim)).astype(np.float32))
    indices = to_dev(g.integers(0, rows, size=n).astype(np.int32))
    slice_input = to_dev(np.stack([np.zeros(n, np.int64),
                                   g.integers(0, 60, size=n).astype(np.int64)], axis=1))
    lib = _lib.lib()
    ddims = np.array([rows, dim], np.int64)
    sdims = np.array([n, 2], np.int64)
    begin = np.array([0, 1], np.int32)
    shape = np.zeros(2, np.int32)
    nnz = np.zeros(1, np.int64)
    args = (_lib.ptr(data), 2, _lib.ptr(ddims), _lib.ptr(indices), 0, n, _lib.ptr(slice_input),
            2, _lib.ptr(sdims), _lib.ptr(begin), 2, 0, _lib.ptr(shape), _lib.ptr(nnz))
    _lib.check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(*args, None, None))
    count = int(nnz[0])
    assert count > 1
    if between:  # phase 1 of other operands (the other combiner) in between
        keep, nnz2, shape2 = [], np.zeros(1, np.int64), np.zeros(2, np.int32)
        _lib.check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(
            *_nonzero_args(data, indices, slice_input, rows, dim, n, 1, shape2, nnz2, keep),
            None, None))
    short = count - 1
    guard = np.float32(123.5)
    out_idx = torch.full((short * 2 + 64,), -5, dtype=torch.int32, device=device())
    out_val = torch.full((short + 64,), float(guard), dtype=torch.float32, device=device())
    nnz[0] = short
    rc = lib.annc_kp_fused_sparse_segment_reduce_nonzero(*args, ctypes.c_void_p(out_idx.data_ptr()),
                                                         ctypes.c_void_p(out_val.data_ptr()))
    assert rc == 3
    assert "differs from the" in _lib.last_error()
    torch.cuda.synchronize()
    assert (to_host(out_idx)[short * 2:] == -5).all()
    assert (to_host(out_val)[short:] == guard).all()


def test_tf_segment_reduce_nonzero_phase2_after_other_operands():
    """Phase 1 on A, phase 1 on B, phase 2 on A, then phase 1 and 2 on B and
    phase 2 on B again: every phase 2 matches the oracle of its own
    operands."""
    from annc_amd import _lib
    note("KPFusedSparseSegmentReduceNonzero phase 2 after other operands")
    g = workloads.rng(36)
    n, rows, dim = 3000, 200, 8
    lib = _lib.lib()
    cases = []
    for seg_hi in (300, 40):
        data = g.standard_normal((rows, dim)).astype(np.float32)
        data[g.random((rows, dim)) < 0.3] = 0.0
        idx = g.integers(0, rows, size=n).astype(np.int32)
        seg = g.integers(0, seg_hi, size=n).astype(np.int64)
        sl = np.stack([np.zeros(n, np.int64), seg], axis=1)
        cases.append((data, idx, seg, to_dev(data), to_dev(idx), to_dev(sl)))
    keep, counts = [], []
    shape, nnz = np.zeros(2, np.int32), np.zeros(1, np.int64)
    for data, idx, seg, dd, di, ds in cases:  # phase 1 on A, then on B
        _lib.check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(
            *_nonzero_args(dd, di, ds, rows, dim, n, 0, shape, nnz, keep), None, None))
        counts.append(int(nnz[0]))
    for k in (0, 1, 1):  # phase 2 on A, phase 1 + 2 on B, phase 2 on B again
        data, idx, seg, dd, di, ds = cases[k]
        if k == 1:
            _lib.check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(
                *_nonzero_args(dd, di, ds, rows, dim, n, 0, shape, nnz, keep), None, None))
        want = ora.segment_reduce_nonzero(data, idx, seg, 0)
        out_idx = torch.full((counts[k], 2), -1, dtype=torch.int32, device=device())
        out_val = torch.full((counts[k],), -1.0, dtype=torch.float32, device=device())
        nnz[0] = counts[k]
        _lib.check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(
            *_nonzero_args(dd, di, ds, rows, dim, n, 0, shape, nnz, keep),
            _lib.ptr(out_idx), _lib.ptr(out_val)))
        assert int(nnz[0]) == counts[k] == want[1].shape[0]
        np.testing.assert_array_equal(shape, want[0])
        np.testing.assert_array_equal(to_host(out_idx), want[1])
        np.testing.assert_array_equal(to_host(out_val), want[2])


def test_tf_segment_reduce_nonzero_operands_changed_between_phases():
    """Phase 1, then the data and indices change in place (same addresses,
    shapes and nonzero count), then phase 2: phase 2 lists the new values."""
    from annc_amd import _lib
    note("KPFusedSparseSegmentReduceNonzero operands changed in place between phases")
    g = workloads.rng(37)
    n, rows, dim = 2000, 100, 4
    data = g.standard_normal((rows, dim)).astype(np.float32) + 3.0  # no zero sums
    idx = g.integers(0, rows, size=n).astype(np.int32)
    seg = g.integers(0, 50, size=n).astype(np.int64)
    dd, di = to_dev(data), to_dev(idx)
    ds = to_dev(np.stack([np.zeros(n, np.int64), seg], axis=1))
    lib, keep = _lib.lib(), []
    shape, nnz = np.zeros(2, np.int32), np.zeros(1, np.int64)
    _lib.check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(
        *_nonzero_args(dd, di, ds, rows, dim, n, 1, shape, nnz, keep), None, None))
    count = int(nnz[0])
    data2 = data * 2.0 + 1.0
    idx2 = idx[::-1].copy()
    dd.copy_(to_dev(data2))
    di.copy_(to_dev(idx2))
    want = ora.segment_reduce_nonzero(data2, idx2, seg, 1)
    assert want[1].shape[0] == count
    out_idx = torch.full((count, 2), -1, dtype=torch.int32, device=device())
    out_val = torch.full((count,), -1.0, dtype=torch.float32, device=device())
    _lib.check(lib.annc_kp_fused_sparse_segment_reduce_nonzero(
        *_nonzero_args(dd, di, ds, rows, dim, n, 1, shape, nnz, keep),
        _lib.ptr(out_idx), _lib.ptr(out_val)))
    np.testing.assert_array_equal(to_host(out_idx), want[1])
    np.testing.assert_array_equal(to_host(out_val), want[2])


def test_tf_segment_reduce_nonzero_index_out_of_range():
    note("KPFusedSparseSegmentReduceNonzero idx out of range")
    with pytest.raises(tf_ops.InvalidArgumentError, match="out of range"):
        tf_ops.kp_fused_sparse_segment_reduce_nonzero(
            np.ones((4, 2), np.float32), np.array([0, 9], np.int32),
            np.array([[0, 0], [0, 1]], np.int64), np.array([0, 1], np.int32), 0)


# ---------------------------------------------------------------- KPFusedGather
GATHER_GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                          "fused_gather_reference_gtest.json")))


@pytest.mark.parametrize("where", ["host", "device"])
def test_tf_fused_gather_reference_golden(where):
    note(f"KPFusedGather golden ({where})")
    c = GATHER_GOLD["cases"][0]
    data = np.asarray(c["data"], np.float32).reshape(c["data_shape"])
    keys = np.asarray(c["slice_input"], np.int64).reshape(c["slice_shape"])
    begin = np.asarray(c["begin"], np.int32)
    if where == "device":
        data, keys = to_dev(data), to_dev(keys)
    u, idx, rows = tf_ops.kp_fused_gather(data, keys, begin)
    idx = to_host(idx) if where == "device" else idx
    rows = to_host(rows) if where == "device" else rows
    assert u.tolist() == c["expected_unique"]
    assert np.asarray(idx).tolist() == c["expected_indices"]
    assert np.asarray(rows).reshape(-1).tolist() == c["expected_data"]


def test_tf_fused_gather_index_out_of_range():
    note("KPFusedGather idx out of table range")
    c = [e for e in GATHER_GOLD["error_cases"] if e.get("needs_gpu")][0]
    data = np.ones(c["data_shape"], np.float32)
    keys = np.asarray(c["slice_input"], np.int64).reshape(c["slice_shape"])
    with pytest.raises(Exception) as e:
        tf_ops.kp_fused_gather(data, keys, np.asarray(c["begin"], np.int32))
    assert c["message"] in str(e.value)
    # the status word is cleared again: a valid call right after succeeds
    ok = np.asarray([[0, 1], [1, 1]], np.int64)
    u, _, _ = tf_ops.kp_fused_gather(data, ok, np.asarray([0, 0], np.int32))
    assert u.tolist() == [0, 1]


@pytest.mark.parametrize("n,span,dim", [(1, 1, 8), (1000, 10, 12), (200_000, 50_000, 16),
                                        (131_072, 10**6, 64), (4097, 3, 1)])
def test_fused_gather_random_bit_exact(n, span, dim):
    note(f"KPFusedGather random n={n} span={span} dim={dim}")
    g = workloads.rng(n + span)
    rows = max(span, 1)
    table = g.standard_normal((rows, dim)).astype(np.float32)
    keys = g.integers(0, rows, size=(n, 2)).astype(np.int64)
    keys[:, 0] = -keys[:, 0]  # the other column is ignored
    ref_u, ref_idx, ref_rows = ora.fused_gather(table, keys, 1)
    u, idx, out = tf_ops.kp_fused_gather(table, keys, np.asarray([0, 1], np.int32))
    np.testing.assert_array_equal(u, ref_u)
    np.testing.assert_array_equal(idx, ref_idx)
    np.testing.assert_array_equal(out, ref_rows)
    # device API on a strided column view
    du, didx, drows = dev.unique_gather(to_dev(table), to_dev(keys), col=1)
    np.testing.assert_array_equal(to_host(du), ref_u)
    np.testing.assert_array_equal(to_host(didx), ref_idx)
    np.testing.assert_array_equal(to_host(drows), ref_rows)


def test_fused_gather_negative_and_huge_keys_group_correctly():
    note("KPFusedGather signed keys")
    keys = np.array([[5], [-(2**63)], [2**63 - 1], [5], [-1], [-(2**63)], [0]], np.int64)
    table = np.arange(6, dtype=np.float32).reshape(6, 1)
    # keys outside the table are an error, so compare the grouping on the
    # device API with a table-free dim of 0
    du, didx, _ = dev.unique_gather(to_dev(table[:, :0].copy()), to_dev(keys), col=0)
    assert to_host(du).tolist() == [5, -(2**63), 2**63 - 1, -1, 0]
    assert to_host(didx).tolist() == [0, 1, 2, 0, 3, 1, 4]


@pytest.mark.parametrize("n", [512 * 1024, 512 * 1024 + 4097, 2**24 + 3])
def test_fused_gather_beyond_the_lds_prefix(n):
    """Up to 2^19 keys (1024 blocks of 512 positions) the number workgroups
    form the prefix of the block counts in LDS; beyond, a separate launch
    forms it.  Checked against numpy.unique (first indices, inverse)."""
    note(f"KPFusedGather n={n} (block prefix in LDS / separate launch)")
    g = workloads.rng(n)
    rows, dim = 3_000_000, 4
    keys = g.integers(0, rows, size=n).astype(np.int64)
    keys[n // 3] = rows - 1
    u, first, inv = np.unique(keys, return_index=True, return_inverse=True)
    order = np.argsort(first, kind="stable")
    ref_u = u[order]
    number = np.empty(len(order), np.int64)
    number[order] = np.arange(len(order))
    ref_idx = number[inv.reshape(-1)].astype(np.int32)
    table = _formula_table_dev(rows, dim)
    du, didx, drows = dev.unique_gather(table, to_dev(keys[:, None].copy()), col=0)
    np.testing.assert_array_equal(to_host(du), ref_u)
    np.testing.assert_array_equal(to_host(didx), ref_idx)
    np.testing.assert_array_equal(to_host(drows), _formula_rows_host(ref_u, dim))


def _formula_table_dev(rows, dim):
    """[rows, dim] float32 on the device with value ((r % 1000) - 500) * 0.001 + c,
    exactly reproducible on the host for any row subset."""
    r = ((torch.arange(rows, device=device(), dtype=torch.int64) % 1000) - 500).to(torch.float32)
    c = torch.arange(dim, device=device(), dtype=torch.float32)
    return (r * torch.tensor(0.001, dtype=torch.float32, device=device()))[:, None] + c[None, :]


def _formula_rows_host(row_ids, dim):
    r = ((np.asarray(row_ids, dtype=np.int64) % 1000) - 500).astype(np.float32)
    return (r * np.float32(0.001))[:, None] + np.arange(dim, dtype=np.float32)[None, :]


@pytest.mark.parametrize("combiner", [0, 1])
def test_embedding_bag_table_over_2gib(combiner):
    """A table of 2.15 GB (the 64-bit address path): rows past byte 2^31
    gathered bit-exactly."""
    rows, dim = 8_400_000, 64  # 8_400_000 * 256 B > 2^31
    note(f"embedding bag 2.15 GB table combiner={combiner}")
    table = _formula_table_dev(rows, dim)
    g = workloads.rng(2024 + combiner)
    lens = g.integers(1, 9, size=300)
    offsets = np.zeros(301, dtype=np.int64)
    np.cumsum(lens, out=offsets[1:])
    ids = g.integers(0, rows, size=int(offsets[-1]), dtype=np.int64)
    ids[::3] = g.integers((1 << 31) // (4 * dim), rows, size=ids[::3].size)  # past 2 GiB
    uniq, inv = np.unique(ids, return_inverse=True)
    ref = ora.embedding_bag(_formula_rows_host(uniq, dim), inv.astype(np.int64), offsets, combiner)
    got = to_host(dev.embedding_bag(table, to_dev(ids), to_dev(offsets), combiner))
    np.testing.assert_array_equal(got, ref)
    # the same bags as a segment reduction: sorted segment ids (one-kernel
    # path) and shuffled positions (the sort paths), 64-bit addressing too
    seg = np.repeat(np.arange(300, dtype=np.int64), lens)
    got = to_host(dev.segment_reduce(table, to_dev(ids), to_dev(seg), 300, combiner,
                                     sorted_ids=True))
    np.testing.assert_array_equal(got, ref)
    order = g.permutation(seg.size)  # each segment sums in its shuffled order
    ref_shuffled = ora.segment_reduce(_formula_rows_host(uniq, dim), inv[order].astype(np.int64),
                                      seg[order], 300, combiner)
    got = to_host(dev.segment_reduce(table, to_dev(ids[order]), to_dev(seg[order]), 300,
                                     combiner))
    np.testing.assert_array_equal(got, ref_shuffled)
    del table
    torch.cuda.empty_cache()


# ------------------------------------------------------------ randomized sweep
@pytest.mark.parametrize("seed", range(12))
def test_bag_random_shapes_bit_exact(seed):
    """Seeded random shapes: dims 1..300, bags empty to 1500 long, int32 or
    int64 ids, padded output rows; every bag bit-exact against the oracle."""
    g = workloads.rng(7000 + seed)
    dim = int(g.choice([1, 2, 3, 5, 8, 12, 16, 24, 31, 48, 64, 96, 128, 200, 300]))
    rows = int(g.integers(1, 40000))
    nbags = int(g.integers(1, 700))
    lens = g.integers(0, 12, size=nbags)
    longs = g.random(nbags) < 0.05
    lens[longs] = g.integers(30, 1500, size=int(longs.sum()))
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    idx_dtype = np.int32 if seed % 2 else np.int64
    ids = g.integers(0, rows, size=int(offsets[-1])).astype(idx_dtype)
    combiner = seed % 3 % 2
    ldo = dim + int(g.integers(0, 5))
    note(f"bag random seed={seed}: dim={dim} rows={rows} bags={nbags} nnz={int(offsets[-1])} "
         f"ids={np.dtype(idx_dtype).name} combiner={combiner} ldo={ldo}")
    table = g.standard_normal((rows, dim)).astype(np.float32)
    ref = ora.embedding_bag(table, ids.astype(np.int64), offsets, combiner)
    out = to_dev(np.full((nbags, ldo), 3.0, dtype=np.float32))
    dev.embedding_bag(to_dev(table), to_dev(ids), to_dev(offsets), combiner, out=out[:, :dim])
    got = to_host(out)
    np.testing.assert_array_equal(got[:, :dim], ref)
    np.testing.assert_array_equal(got[:, dim:], 3.0)


@pytest.mark.parametrize("dim", [16, 32, 64])
def test_random_row_probe_reads_what_it_counts(dim):
    """The measurement kernel behind bench.py's gather_probe cases: every lane
    sums rows_per_group 16-byte chunks of a table of ones, so each lane's
    output is exactly 4 * rows_per_group (and the grid covers `out`)."""
    import bench
    note(f"random-row probe, dim {dim}")
    table = torch.ones((5000, dim), dtype=torch.float32, device=device())
    out = torch.full((3 * 256,), -1.0, dtype=torch.float32, device=device())
    bench.probe_random_rows(table, 3, 24, out)
    np.testing.assert_array_equal(to_host(out), np.full(3 * 256, 96.0, np.float32))
    with pytest.raises(ValueError, match="multiple of 8"):
        bench.probe_random_rows(table, 3, 12, out)


def test_tf_ops_from_concurrent_threads():
    """KPFusedSparseSegmentReduceNonzero (two phases), KPFusedGather and
    KPFusedSparseSegmentReduce called from 4 threads at once, each on its own
    inputs: the library stream, pinned read-back buffer and kept phase-1
    results are per thread, so every thread gets its own oracle result."""
    import threading
    note("TF ops from 4 threads")
    cases = []
    for t in range(4):
        g = workloads.rng(900 + t)
        rows, dim, n = 500 + 100 * t, 8 + 4 * t, 3000 + 700 * t
        data = g.standard_normal((rows, dim)).astype(np.float32)
        data[g.random((rows, dim)) < 0.2] = 0.0
        idx = g.integers(0, rows, size=n).astype(np.int64)
        seg = g.integers(0, 200 + 50 * t, size=n).astype(np.int64)
        sl = np.stack([np.zeros(n, np.int64), seg], axis=1)
        cases.append((data, idx, seg, sl))
    errors = []

    def work(c):
        data, idx, seg, sl = c
        try:
            want = ora.segment_reduce_nonzero(data, idx, seg, 1)
            want_u, want_i, want_r = ora.fused_gather(data, sl, 1)
            batch = int(seg.max()) + 1
            want_sr = ora.segment_reduce(data, idx, seg, batch, 0)
            for _ in range(3):
                shape, oi, ov = tf_ops.kp_fused_sparse_segment_reduce_nonzero(
                    data, idx, sl, np.array([0, 1], np.int32), 1)
                np.testing.assert_array_equal(shape, want[0])
                np.testing.assert_array_equal(oi, want[1])
                np.testing.assert_array_equal(ov, want[2])
                u, gi, gr = tf_ops.kp_fused_gather(data, sl, np.array([0, 1], np.int32))
                np.testing.assert_array_equal(u, want_u)
                np.testing.assert_array_equal(gi, want_i)
                np.testing.assert_array_equal(gr, want_r)
                out, so = tf_ops.kp_fused_sparse_segment_reduce(
                    data, idx, sl, np.array([0, 1], np.int32), np.array([0], np.int32), 0)
                np.testing.assert_array_equal(out, want_sr)
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(c,)) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


@pytest.mark.parametrize("m,n", [(7, 5), (1, 3), (64, 1), (100_000, 3), (300, 4097), (0, 2)])
@pytest.mark.parametrize("where", ["host", "device"])
def test_reduce_mean_custom_call(m, n, where):
    """__reduce_mean through the registered target (reduce_rewriter.cc:31-46):
    the mean of |x| over each run of m consecutive values, against the
    oracle's sequential sum at fp32 tolerance (cblas_sasum fixes no order);
    m = 0 gives 0/0."""
    note(f"__reduce_mean m={m} n={n} {where}")
    g = workloads.rng(m + n)
    x = g.standard_normal((m, n)).astype(np.float32)
    want = ora.reduce_mean(x)
    if where == "host":
        out = np.full(n, -1.0, np.float32)
        xla.reduce_mean(x, out)
    else:
        out_d = torch.full((n,), -1.0, device=device())
        xla.reduce_mean(to_dev(x), out_d)
        out = to_host(out_d)
    if m == 0:
        assert np.isnan(out).all()
    else:
        np.testing.assert_allclose(out, want, rtol=1e-5 + 2e-7 * np.sqrt(m))
