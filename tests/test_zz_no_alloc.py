"""The allocation-free segment reduction (annc_hip_segment_reduce_noalloc)
against annc_hip_segment_reduce, through the C ABI: bit-identical outputs on
two calls in a row, the second smaller, for sorted and unsorted segment ids,
both combiners; the caller's status word; the size limit."""
import ctypes

import numpy as np
import pytest
import torch

from annc_amd import _lib, workloads
from oracle import ora
from tests.gpu_util import device, note, to_dev, to_host

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _inputs(seed, n, rows, dim, batch, sorted_ids):
    g = workloads.rng(seed)
    data = g.standard_normal((rows, dim)).astype(np.float32)
    indices = g.integers(0, rows, size=n).astype(np.int64)
    seg = g.integers(0, batch, size=n).astype(np.int64)
    if sorted_ids:
        seg.sort()
    return data, indices, seg


def _run(fn_name, data, indices, seg, batch, combiner, sorted_ids, status=None):
    lib = _lib.lib()
    d, i, s = to_dev(data), to_dev(indices), to_dev(seg)
    out = torch.full((batch, data.shape[1]), 7.0, dtype=torch.float32, device=device())
    args = [_stream(), _lib.ptr(d), data.shape[0], data.shape[1], _lib.ptr(i), 1, _lib.ptr(s), 1,
            indices.size, combiner, batch, _lib.ptr(out), int(sorted_ids)]
    if fn_name.endswith("noalloc"):
        args.append(_lib.ptr(status) if status is not None else None)
    _lib.check(getattr(lib, fn_name)(*args))
    return to_host(out)


@pytest.mark.parametrize("sorted_ids", [True, False])
@pytest.mark.parametrize("combiner", [0, 1])
def test_noalloc_equals_segment_reduce_twice(sorted_ids, combiner):
    """Two calls in a row (the second with fewer positions, rows and
    segments, so stale scratch from the first would show) equal the
    allocating entry bit for bit, and the oracle."""
    for call, (n, rows, dim, batch) in enumerate([(30000, 5000, 64, 3000), (7000, 900, 16, 700)]):
        note(f"segment_reduce_noalloc sorted={sorted_ids} combiner={combiner} call={call} n={n}")
        data, indices, seg = _inputs(10 * call + 2 * sorted_ids + combiner, n, rows, dim, batch,
                                     sorted_ids)
        want = _run("annc_hip_segment_reduce", data, indices, seg, batch, combiner, sorted_ids)
        got = _run("annc_hip_segment_reduce_noalloc", data, indices, seg, batch, combiner,
                   sorted_ids)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(got, ora.segment_reduce(data, indices, seg, batch, combiner))


def test_noalloc_status_word_and_skipped_segments():
    """A row id outside the data sets bit 0 of the caller's status word and
    adds nothing; segment ids outside [0, batch) are skipped."""
    note("segment_reduce_noalloc status word")
    data, indices, seg = _inputs(5, 2000, 300, 8, 100, False)
    indices[17] = 300
    seg[3] = 100
    seg[4] = -2
    status = torch.zeros(1, dtype=torch.int32, device=device())
    got = _run("annc_hip_segment_reduce_noalloc", data, indices, seg, 100, 0, False, status)
    assert int(to_host(status)[0]) & 1 == 1
    keep = (seg >= 0) & (seg < 100) & (indices < 300)
    want = ora.segment_reduce(data, indices[keep], seg[keep], 100, 0)
    np.testing.assert_array_equal(got, want)


def test_noalloc_rejects_inputs_beyond_its_scratch():
    """Unsorted ids over 16384 segments at 2 M positions need more than the
    16 MiB scratch: refused before any GPU work, with the sizes named."""
    note("segment_reduce_noalloc size limit")
    lib = _lib.lib()
    n = 2_000_000
    d = torch.zeros((10, 4), dtype=torch.float32, device=device())
    # valid buffers of the stated sizes, though the call must not use them
    idx = torch.zeros(n, dtype=torch.int64, device=device())
    seg = torch.zeros(n, dtype=torch.int64, device=device())
    out = torch.zeros((20000, 4), dtype=torch.float32, device=device())
    rc = lib.annc_hip_segment_reduce_noalloc(_stream(), _lib.ptr(d), 10, 4, _lib.ptr(idx), 1,
                                             _lib.ptr(seg), 1, n, 0, 20000, _lib.ptr(out), 0, None)
    assert rc == 3
    assert "allocation-free" in _lib.last_error()
