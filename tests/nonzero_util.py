"""The KPFusedSparseSegmentReduceNonzero output form built from a dense
segment reduction, for checking the reduction against that op's reference
goldens.

Follows annc/tensorflow/kernels/embedding_fused_sparse_segment_reduce_nonzero.cc:
segments are listed in order of first appearance in the segment column, each
segment's dims in increasing order, and only values != 0.0f are emitted
(1-D data: indices [nnz, 1] = segment; 2-D: [nnz, 2] = (segment, dim))."""
import numpy as np


def case_inputs(c):
    data = np.asarray(c["data"], np.float32).reshape(c["data_shape"])
    indices = np.asarray(c["indices"], np.int32)
    slice_input = np.asarray(c["slice_input"], np.int64).reshape(c["slice_shape"])
    seg = slice_input[:, c["begin"][1]].copy()
    return data, indices, slice_input, seg


def nonzero_coo(dense, seg, one_d):
    """(output_shape, output_indices, output_nonzero) from dense [batch, D]."""
    order = []
    for s in seg.tolist():
        if s not in order:
            order.append(s)
    idx, val = [], []
    for s in order:
        for d in range(dense.shape[1]):
            v = dense[s, d]
            if v != 0.0:
                idx.append([s] if one_d else [s, d])
                val.append(v)
    shape = [dense.shape[0]] if one_d else [dense.shape[0], dense.shape[1]]
    width = 1 if one_d else 2
    return (np.asarray(shape, np.int32), np.asarray(idx, np.int32).reshape(-1, width),
            np.asarray(val, np.float32))


def check_case(c, dense):
    """dense: the reduction of the case's rows, [max_seg + 1, D] (D = 1 for 1-D data)."""
    one_d = len(c["data_shape"]) == 1
    _, _, _, seg = case_inputs(c)
    shape, idx, val = nonzero_coo(dense, seg, one_d)
    assert shape.tolist() == c["expected_shape"]
    assert list(idx.shape) == c["expected_indices_shape"]
    assert idx.reshape(-1).tolist() == c["expected_indices"]
    np.testing.assert_array_equal(val, np.asarray(c["expected_values"], np.float32))
