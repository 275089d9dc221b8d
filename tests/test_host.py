"""Host-side logic of the library: exports, ANNC_FLAGS, pre-pack, validation.

CPU only: nothing here launches a kernel.
"""
import json
import os
import re

import numpy as np
import pytest

from annc_amd import _lib, flags, tf_ops, xla
from annc_amd._lib import AnncError
from annc_amd import device as dev
from oracle import ora

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    text = open(os.path.join(ROOT, "include", "annc_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(\w+)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("extern", "if")))


def test_library_exports_every_header_symbol():
    lib = _lib.lib()
    names = _header_functions()
    assert "__matmul_add_relu" in names and "annc_hip_gemm" in names
    for n in names:
        assert hasattr(lib, n), f"missing export {n}"
    # and the Python binding declares a prototype for each of them
    assert sorted(_lib.exported_names()) == names


def test_custom_call_registry():
    # REGISTER_ALL_GEMM_KERNELS's order (kdnn_rewriter.h:148-155)
    assert xla.registered_targets() == ["__matmul", "__batch_matmul", "__matmul_add",
                                        "__matmul_add_relu", "__reduce_mean", "__pooling",
                                        "__layout_matmul"]
    lib = _lib.lib()
    for t in xla.TARGETS:
        assert lib.annc_custom_call_target(t.encode())
    assert not lib.annc_custom_call_target(b"__softmax")


# ------------------------------------------------------------------ flags
FLAG_CASES = [
    "",
    "--matmul",
    "--layout-matmul --matmul-add-relu",
    "--gemm-opt",
    "--graph-opt",
    "--gemm-opt=false",
    "--matmul=1 --pooling=true --sps-emd-2=0",
    "--matmul=yes",
    "--matmul= --pooling",
    "--annc-pass=false",
    "   --matmul    --batch-matmul   ",
    "--unknown-flag --matmul",
    "--matmul bogus --pooling",
    "-matmul --pooling",
    "--matmul\t--pooling",
    "--matmul=true=1",
    "--",
    "--gemm-opt --matmul=false",
]
ALL_FLAGS = list(flags.FLAG_NAMES) + ["unknown-flag", "gemm-opt", "graph-opt", ""]

EXPECTED = {
    "": {"annc-pass"},
    "--matmul": {"matmul", "annc-pass"},
    "--gemm-opt": {"matmul", "layout-matmul", "disable-tf-matmul-fusion", "annc-pass"},
    "--graph-opt": {"sps-emd-2", "annc-pass"},
    "--gemm-opt=false": {"matmul", "layout-matmul", "disable-tf-matmul-fusion", "annc-pass"},
    "--matmul=yes": {"annc-pass"},
    "--annc-pass=false": set(),
    "--unknown-flag --matmul": {"unknown-flag", "matmul", "annc-pass"},
    "--matmul bogus --pooling": {"matmul", "annc-pass"},
    "--gemm-opt --matmul=false": {"layout-matmul", "disable-tf-matmul-fusion", "annc-pass"},
}


@pytest.mark.parametrize("s", FLAG_CASES)
def test_flags_grammar(s):
    flags.reset(s)
    got = {n for n in ALL_FLAGS if flags.is_enabled(n)}
    if s in EXPECTED:
        assert got == EXPECTED[s]
    ref = [ora.ref_flag_enabled(s, n) for n in ALL_FLAGS]
    if ref[0] is not None:  # oracle/_ref built from the reference's annc_flags.cc
        assert got == {n for n, r in zip(ALL_FLAGS, ref) if r}
    flags.reset(None)


def test_flags_env_default_set():
    flags.reset(None)
    assert flags.dump() == {n: n == "annc-pass" for n in flags.FLAG_NAMES}


# ------------------------------------------------------------------ pre-pack
def _offset_model(k, n, K, N):
    """Independent statement of the packed position (per region)."""
    kf, nf = K // 32 * 32, N // 32 * 32
    if n >= nf:
        return nf * K + k * (N - nf) + (n - nf)
    if k >= kf:
        return nf * kf + (k - kf) * nf + n
    block = (n // 32) * (kf // 32) + k // 32
    lane = 32 * ((k % 32) // 16) + n % 32
    step = k % 16
    return block * 1024 + (step // 4) * 256 + lane * 4 + step % 4


@pytest.mark.parametrize("k,n", [(1, 1), (32, 32), (64, 96), (845, 1024), (33, 31), (100, 70),
                                 (1024, 512), (31, 64), (12, 12)])
def test_pack_is_a_bijection_with_the_documented_order(k, n):
    w = np.arange(k * n, dtype=np.float32).reshape(k, n)
    p = dev.pack_weight_host(w)
    assert p.size == k * n
    assert np.array_equal(np.sort(p), w.reshape(-1))  # a permutation
    np.testing.assert_array_equal(dev.unpack_weight_host(p, k, n), w)
    g = np.random.Generator(np.random.PCG64(k * 1000 + n))
    for kk, nn in zip(g.integers(0, k, 64), g.integers(0, n, 64)):
        assert p[_offset_model(int(kk), int(nn), k, n)] == w[kk, nn]


def test_pack_small_n_is_row_major():
    w = np.random.default_rng(0).standard_normal((40, 20)).astype(np.float32)
    np.testing.assert_array_equal(dev.pack_weight_host(w), w.reshape(-1))


def test_fragment_block_is_mfma_b_operand():
    # lanes 0-31 of the first float4 hold k = 0..3 of columns 0..31
    w = np.arange(64 * 64, dtype=np.float32).reshape(64, 64)
    p = dev.pack_weight_host(w)
    blk = p[:1024].reshape(4, 64, 4)  # [q][lane][e]
    for lane in range(64):
        for q in range(4):
            for e in range(4):
                assert blk[q, lane, e] == w[16 * (lane // 32) + 4 * q + e, lane % 32]


def test_rhs_format_tag():
    assert _lib.lib().annc_layout_matmul_rhs_format().decode() == "mfma_f32_32x32x2_k16"


# ------------------------------------------------------------------ TF-op validation
_GOLD = json.load(open(os.path.join(ROOT, "tests", "golden", "segment_reduce_reference_gtest.json")))


@pytest.mark.parametrize("case", _GOLD["error_cases"], ids=lambda c: c["name"])
def test_segment_reduce_error_messages(case):
    data = np.arange(np.prod(case["data_shape"]), dtype=np.float32).reshape(case["data_shape"])
    idx = np.zeros(case["indices_shape"], dtype=np.int32)
    sl = np.ones(case["slice_shape"], dtype=np.int64)
    with pytest.raises(tf_ops.InvalidArgumentError) as ei:
        tf_ops.kp_fused_sparse_segment_reduce(data, idx, sl, np.array(case["begin"], np.int32),
                                              np.array(case["begin_1"], np.int32),
                                              case["combiner"])
    assert case["message"] in str(ei.value)


def test_segment_reduce_bad_combiner():
    with pytest.raises(tf_ops.InvalidArgumentError, match="combiner must be 0 or 1"):
        tf_ops.kp_fused_sparse_segment_reduce(np.zeros((2, 2), np.float32), np.zeros(1, np.int32),
                                              np.zeros((1, 2), np.int64), np.array([0, 0], np.int32),
                                              np.array([0], np.int32), combiner=2)


# The KPFusedSparseSegmentReduceNonzero checks, in the reference's order and
# text (embedding_fused_sparse_segment_reduce_nonzero.cc:33-57); all fail
# before any device work.
NONZERO_ERRORS = [
    ("combiner", dict(combiner=2), "combiner must be 0 or 1"),
    ("3-D data", dict(data=np.zeros((2, 2, 2), np.float32)),
     "Input data must be a 1-D vector or 2-D matrix"),
    ("1-D slice", dict(slice_input=np.zeros(3, np.int64)), "slice input must be 2-D"),
    ("begin of 3", dict(begin=np.array([0, 0, 0], np.int32)), "begin must have 2 elements"),
    ("column", dict(begin=np.array([0, 2], np.int32)), "Column index out of range"),
    ("sizes", dict(indices=np.zeros(2, np.int32)),
     "indices and slice_input.dim_size(0) should have same size"),
]


@pytest.mark.parametrize("what,override,message", NONZERO_ERRORS, ids=[e[0] for e in NONZERO_ERRORS])
def test_segment_reduce_nonzero_error_messages(what, override, message):
    args = dict(data=np.zeros((4, 2), np.float32), indices=np.zeros(3, np.int32),
                slice_input=np.zeros((3, 2), np.int64), begin=np.array([0, 1], np.int32),
                combiner=0)
    args.update(override)
    with pytest.raises(tf_ops.InvalidArgumentError) as ei:
        tf_ops.kp_fused_sparse_segment_reduce_nonzero(**args)
    assert message in str(ei.value)


def test_hash_ops_reject_zero_buckets():
    with pytest.raises(tf_ops.InvalidArgumentError):
        tf_ops.kp_fused_embedding_with_hash_bucket([b"a"], np.zeros((4, 2), np.float32), 0)
    with pytest.raises(tf_ops.InvalidArgumentError):
        tf_ops.kp_fused_sparse_embedding([b"a"], 0)


@pytest.mark.parametrize("n", [(1 << 29) + 1, 1 << 30, (1 << 31) - 2])
def test_unique_gather_rejects_key_counts_past_the_table_limit(n):
    """Slot numbers of the unique table are int32 and its capacity is the
    power of two at or above 2n, so n is capped at 2^29; the check runs before
    any launch (no device pointers are touched)."""
    import ctypes
    lib = _lib.lib()
    dummy = ctypes.c_void_p(16)
    rc = lib.annc_hip_unique_gather(None, None, 0, 0, dummy, 1, n, dummy, dummy, dummy, None)
    assert rc == _lib.INVALID_ARGUMENT
    assert b"at most 2^29" in lib.annc_hip_last_error()


@pytest.mark.parametrize("m,n,k,why", [(64, 96, 192, b"n must be"), (64, 256, 100, b"multiple of n"),
                                       (64, 256, 4096, b"multiple of n"), (64, 128, 64, b"multiple of n"),
                                       (-1, 256, 512, b"bad row count")])
def test_dense_score_rejects_unsupported_shapes(m, n, k, why):
    """annc_hip_dense_score checks its shape before any launch or pointer
    access; the tower falls back to one GEMM per layer for such shapes."""
    import ctypes
    from annc_amd import device as dev
    lib = _lib.lib()
    dummy = ctypes.c_void_p(16)
    rc = lib.annc_hip_dense_score(None, m, n, k, dummy, k, dummy, None, 1, dummy, None, 2, None, 0,
                                  dummy, 1)
    assert rc == _lib.INVALID_ARGUMENT
    assert why in lib.annc_hip_last_error()
    assert dev.dense_score_fits(k, n) == (m < 0)
    assert dev.dense_score_fits(512, 256) and dev.dense_score_fits(2048, 64)


def test_dense_score_zero_rows_is_a_no_op():
    """m = 0 returns OK before any pointer is looked at or any launch."""
    lib = _lib.lib()
    assert lib.annc_hip_dense_score(None, 0, 256, 512, None, 512, None, None, 1, None, None, 2,
                                    None, 0, None, 1) == _lib.OK


# (batch, m, n, k, lda, ldb, b_packed, b_aligned, epilogue, null_c, message): each
# rejected by annc_hip_gemm before any launch or pointer access
GEMM_BAD_ARGS = [
    (1, -1, 64, 64, 64, 64, 0, True, 0, False, b"negative GEMM dimension"),
    (-1, 4, 64, 64, 64, 64, 0, True, 0, False, b"negative GEMM dimension"),
    (1, 1 << 31, 64, 64, 64, 64, 0, True, 0, False, b"too large"),
    (1, 64, 64, 64, 64, 32, 0, True, 0, False, b"ldb < n"),
    (1, 64, 64, 64, 32, 64, 0, True, 0, False, b"leading dimension"),
    (1, 64, 64, 64, 64, 64, 0, True, 8, False, b"unknown epilogue"),
    (1, 64, 64, 64, 64, 64, 0, True, 0, True, b"null output"),
    (1, 4096, 64, 64, 64, 64, 1, False, 0, False, b"packed B must be 16-byte aligned"),
    (1, 64, 64, 64, 64, 64, 0, None, 0, False, b"null operand"),
]


@pytest.mark.parametrize("batch,m,n,k,lda,ldb,packed,aligned,epi,null_c,message", GEMM_BAD_ARGS)
def test_gemm_rejects_bad_arguments(batch, m, n, k, lda, ldb, packed, aligned, epi, null_c,
                                    message):
    """annc_hip_gemm validates its arguments before any launch (these run
    without a GPU); an empty product returns OK at once."""
    import ctypes
    lib = _lib.lib()
    a = ctypes.c_void_p(16)
    b = None if aligned is None else ctypes.c_void_p(16 if aligned else 20)
    c = None if null_c else ctypes.c_void_p(16)
    rc = lib.annc_hip_gemm(None, batch, m, n, k, a, lda, 0, b, ldb, 0, packed, None, 0, 0, None,
                           epi, c, n, 0)
    assert rc == _lib.INVALID_ARGUMENT
    assert message in lib.annc_hip_last_error()


@pytest.mark.parametrize("batch,m,n", [(0, 64, 64), (1, 0, 64), (1, 64, 0)])
def test_gemm_empty_product_is_a_no_op(batch, m, n):
    lib = _lib.lib()
    assert lib.annc_hip_gemm(None, batch, m, n, 64, None, 64, 0, None, 64, 0, 0, None, 0, 0,
                             None, 0, None, 64, 0) == _lib.OK


def test_shape_info_encoding():
    # hlo_util.h:14-21 -- dims then minor_to_major; row-major [512,256] -> {512,256,1,0}
    assert xla.shape_info((512, 256)).tolist() == [512, 256, 1, 0]
    assert xla.shape_info((2, 3, 4)).tolist() == [2, 3, 4, 2, 1, 0]


@pytest.mark.parametrize("case", [c for c in json.load(open(os.path.join(
    os.path.dirname(__file__), "golden", "fused_gather_reference_gtest.json")))["error_cases"]
    if not c.get("needs_gpu")], ids=lambda c: c["name"])
def test_fused_gather_error_messages(case):
    """The shape checks of KPFusedGather run on the host, before any GPU work."""
    from annc_amd import tf_ops
    data = np.ones(case["data_shape"], np.float32)
    keys = np.asarray(case["slice_input"], np.int64).reshape(case["slice_shape"])
    with pytest.raises(AnncError) as e:
        tf_ops.kp_fused_gather(data, keys, np.asarray(case["begin"], np.int32))
    assert case["message"] in e.value.message
    assert e.value.code == 13  # errors::Internal


@pytest.mark.parametrize("case", json.load(open(os.path.join(
    os.path.dirname(__file__), "golden", "batch_matmul_add_sigmoid_reference_gtest.json")))["error_cases"],
    ids=lambda c: c["name"])
def test_batch_matmul_add_sigmoid_error_messages(case):
    """Shape checks run on the host before any GPU work."""
    mk = lambda s: np.zeros(s, np.float32)  # noqa: E731
    with pytest.raises(_lib.InvalidArgumentError) as e:
        tf_ops.kp_fused_batch_matmul_add_sigmoid(mk(case["lhs_shape"]), mk(case["rhs_shape"]),
                                                 mk(case["bias_shape"]))
    assert case["message"] in e.value.message
