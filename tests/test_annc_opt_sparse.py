"""annc-opt's dnn_sparse, dnn_hash_bucket and linear_sparse passes
(rec_embedding.py:6-211, 794-891) on hand-built TF feature-column subgraphs
that satisfy the reference matchers' check chains (node types, operand and
user order).  TensorFlow is absent, so agreement with graphs TensorFlow
exports is not pinned by these tests."""
import numpy as np
import pytest

from annc_amd import annc_opt
from tests.test_annc_opt import FORMS, _as_form, _shapes_attr

N = annc_opt.Node


def _front(p, inp, nb, c):
    """ExpandDims ... SparseFillEmptyRows of a DNN hash-bucket column
    (rec_embedding.py:9-53): 20 nodes, plus the Shape's fourth user (Cast)."""
    x = lambda s: f"{p}/{s}"
    return [
        N(x("ExpandDims"), "ExpandDims", [inp, c[0]]),
        N(x("NotEqual"), "NotEqual", [x("ExpandDims"), c[1]]),
        N(x("Where"), "Where", [x("NotEqual")]),
        N(x("GatherNd"), "GatherNd", [x("ExpandDims"), x("Where")]),
        N(x("Shape"), "Shape", [x("ExpandDims")], {"_output_shapes": [[2]]}),
        N(x("hash"), "StringToHashBucketFast", [x("GatherNd")],
          {"num_buckets": nb, "_output_shapes": [[-1]]}),
        N(x("Identity"), "Identity", [x("hash")]),
        N(x("GreaterEqual"), "GreaterEqual", [x("Identity"), c[2]]),
        N(x("Where_1"), "Where", [x("GreaterEqual")]),
        N(x("Reshape"), "Reshape", [x("Where_1"), c[3]]),
        N(x("Slice"), "Slice", [x("Shape"), c[4], c[5]]),
        N(x("GatherV2_3"), "GatherV2", [x("Shape"), c[6], c[7]]),
        N(x("Prod"), "Prod", [x("Slice"), c[7]]),
        N(x("Pack"), "Pack", [x("Prod"), x("GatherV2_3")]),
        N(x("SparseReshape"), "SparseReshape", [x("Where"), x("Shape"), x("Pack")],
          {"_output_shapes": [[-1, 2], [2]]}),
        N(x("Cast"), "Cast", [x("Shape")]),
        N(x("GatherV2_1"), "GatherV2", [x("SparseReshape"), x("Reshape"), c[7]]),
        N(x("Identity_2"), "Identity", [x("SparseReshape")]),
        N(x("GatherV2"), "GatherV2", [x("Identity"), x("Reshape"), c[7]]),
        N(x("SparseFillEmptyRows"), "SparseFillEmptyRows",
          [x("Identity_2"), x("GatherV2"), x("GatherV2_1"), c[8]],
          {"_output_shapes": [[-1, 2], [-1], [-1], [-1]]}),
    ]


def _dnn_hash_bucket_tail(p, weight, c):
    """SparseFillEmptyRows' users through the column's reshaped mean
    (rec_embedding.py:137-172): 23 nodes."""
    x = lambda s: f"{p}/{s}"
    return [
        N(x("strided_slice"), "StridedSlice", [x("SparseFillEmptyRows"), c[9], c[10], c[11]]),
        N(x("Unique"), "Unique", [x("SparseFillEmptyRows:1")]),
        N(x("Reshape_1"), "Reshape", [x("SparseFillEmptyRows:2"), c[12]]),
        N(x("embedding_lookup"), "GatherV2", [weight, x("Unique"), c[7]]),
        N(x("embedding_lookup/Identity"), "Identity", [x("embedding_lookup")]),
        N(x("Cast_1"), "Cast", [x("strided_slice")]),
        N(x("segment"), "SparseSegmentMean",
          [x("embedding_lookup/Identity"), x("Unique:1"), x("Cast_1")]),
        N(x("Shape_1"), "Shape", [x("segment")]),
        N(x("zeros_like"), "ZerosLike", [x("segment")]),
        N(x("strided_slice_1"), "StridedSlice", [x("Shape_1"), c[9], c[10], c[11]]),
        N(x("stack"), "Pack", [c[13], x("strided_slice_1")]),
        N(x("Tile"), "Tile", [x("Reshape_1"), x("stack")]),
        N(x("Select"), "Select", [x("Tile"), x("zeros_like"), x("segment")]),
        N(x("Shape_2"), "Shape", [x("Select")]),
        N(x("Slice_1"), "Slice", [x("Shape_2"), c[4], c[5]]),
        N(x("Slice_2"), "Slice", [x("Cast"), c[4], c[5]]),
        N(x("concat"), "ConcatV2", [x("Slice_2"), x("Slice_1"), c[14]]),
        N(x("Reshape_2"), "Reshape", [x("Select"), x("concat")]),
        N(x("Shape_3"), "Shape", [x("Reshape_2")]),
        N(x("strided_slice_2"), "StridedSlice", [x("Shape_3"), c[9], c[10], c[11]]),
        N(x("stack_1"), "Pack", [x("strided_slice_2"), c[15]]),
        N(x("Reshape_3"), "Reshape", [x("Reshape_2"), x("stack_1")],
          {"_output_shapes": [[-1, 16]]}),
    ]


def _linear(p, inp, nb, c):
    """ExpandDims ... SparseFillEmptyRows of a linear hash-bucket column
    (rec_embedding.py:797-855): 26 nodes, plus the SparseReshape's fifth user
    (a Cast of its dense shape)."""
    x = lambda s: f"{p}/{s}"
    return [
        N(x("ExpandDims"), "ExpandDims", [inp, c[0]]),
        N(x("NotEqual"), "NotEqual", [x("ExpandDims"), c[1]]),
        N(x("Where"), "Where", [x("NotEqual")]),
        N(x("GatherNd"), "GatherNd", [x("ExpandDims"), x("Where")]),
        N(x("Shape"), "Shape", [x("ExpandDims")]),
        N(x("hash"), "StringToHashBucketFast", [x("GatherNd")], {"num_buckets": nb}),
        N(x("Identity"), "Identity", [x("hash")]),
        N(x("Identity_1"), "Identity", [x("Identity")]),
        N(x("GreaterEqual"), "GreaterEqual", [x("Identity_1"), c[2]]),
        N(x("Where_1"), "Where", [x("GreaterEqual")]),
        N(x("Reshape"), "Reshape", [x("Where_1"), c[3]]),
        N(x("Cast"), "Cast", [x("Shape")]),
        N(x("strided_slice"), "StridedSlice", [x("Cast"), c[9], c[10], c[11]]),
        N(x("stack"), "Pack", [x("strided_slice"), c[12]]),
        N(x("Cast_1"), "Cast", [x("stack")]),
        N(x("SparseReshape"), "SparseReshape", [x("Where"), x("Shape"), x("Cast_1")],
          {"_output_shapes": [[-1, 2], [2]]}),
        N(x("Slice"), "Slice", [x("SparseReshape:1"), c[4], c[5]]),
        N(x("GatherV2_3"), "GatherV2", [x("SparseReshape:1"), c[6], c[7]]),
        N(x("Prod"), "Prod", [x("Slice"), c[7]]),
        N(x("Pack"), "Pack", [x("Prod"), x("GatherV2_3")]),
        N(x("SparseReshape_1"), "SparseReshape",
          [x("SparseReshape"), x("SparseReshape:1"), x("Pack")]),
        N(x("dense_shape"), "Cast", [x("SparseReshape:1")]),
        N(x("GatherV2_1"), "GatherV2", [x("SparseReshape_1"), x("Reshape"), c[7]]),
        N(x("Identity_2"), "Identity", [x("SparseReshape_1")]),
        N(x("GatherV2"), "GatherV2", [x("Identity_1"), x("Reshape"), c[7]]),
        N(x("SparseFillEmptyRows"), "SparseFillEmptyRows",
          [x("Identity_2"), x("GatherV2_1"), x("GatherV2"), c[8]],
          {"_output_shapes": [[-1, 2], [-1], [-1], [-1]]}),
    ]


def _model(tmp_path, kind, form, tweak=None):
    """Two columns of `kind` over placeholders in0/in1 with consumers of
    their outputs; returns (source dir, removed node names per column)."""
    nodes, variables, removed = [], {}, {}
    g = np.random.default_rng(5)
    for i in range(2):
        p, inp = f"col{i}", f"in{i}"
        c = [f"{p}/c{j}" for j in range(16)]
        nodes.append(N(inp, "Placeholder", [], {"dtype": "DT_STRING"}))
        nodes += [N(n, "Const") for n in c]
        if kind == "linear_sparse":
            col = _linear(p, inp, 100 + i, c)
            external = {f"{p}/dense_shape"}
        else:
            col = _front(p, inp, 100 + i, c)
            external = {f"{p}/Cast"} if kind == "dnn_sparse" else set()
        if kind == "dnn_hash_bucket":
            nodes.append(N(f"emb{i}", "VariableV2"))
            variables[f"emb{i}"] = g.standard_normal((100 + i, 16)).astype(np.float32)
            col += _dnn_hash_bucket_tail(p, f"emb{i}", c)
            nodes += col
            nodes.append(N(f"{p}/use", "Identity", [f"{p}/Reshape_3"]))
        else:
            nodes += col
            for k in range(3):
                nodes.append(N(f"{p}/use{k}", "Identity",
                               [f"{p}/SparseFillEmptyRows" + (f":{k}" if k else "")]))
            tail = f"{p}/Cast" if kind == "dnn_sparse" else f"{p}/dense_shape"
            nodes.append(N(f"{p}/use3", "Identity", [tail]))
        removed[p] = [n.name for n in col if n.name not in external] + [c[0]]
    if tweak:
        tweak(nodes)
    src = tmp_path / "in"
    annc_opt.save_model(_as_form(nodes, variables, form), str(src))
    return src, removed


def _shapes(form, *s):
    return [list(x) for x in s] if form == "json" else _shapes_attr(*s)


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("kind", ["dnn_sparse", "linear_sparse"])
def test_sparse_passes_emit_kp_fused_sparse_embedding(tmp_path, kind, form):
    src, removed = _model(tmp_path, kind, form)
    out = tmp_path / "out"
    assert annc_opt.main(["-I", str(src), "-O", str(out), kind]) == 0
    m = annc_opt.load_model(str(out))
    by = {n.name: n for n in m.nodes}
    names = [n.name for n in m.nodes]
    for i in range(2):
        p = f"col{i}"
        f = by[f"{p}/SparseFillEmptyRows/rec_embed_kp_sparse"]
        assert f.op == "KPFusedSparseEmbedding" and f.inputs == [f"in{i}"]
        assert f.attrs == {"num_buckets": 100 + i,
                           "_output_shapes": _shapes(form, [-1, 2], [-1], [-1], [2])}
        # rec_embedding.py:20 + 26 nodes removed (the ExpandDims' Const too)
        assert len(removed[p]) == (20 if kind == "dnn_sparse" else 26)
        assert not set(removed[p]) & set(names)
        # SparseFillEmptyRows' three outputs and the dense shape move over
        # (the dense shape's reader, a Cast outside the match, stays)
        cast = f"{p}/Cast" if kind == "dnn_sparse" else f"{p}/dense_shape"
        assert [by[f"{p}/use{k}"].inputs[0] for k in range(4)] == \
            [f.name, f.name + ":1", f.name + ":2", cast]
        if kind == "linear_sparse":
            assert by[f"{p}/dense_shape"].inputs == [f.name + ":3"]
        else:
            assert by[f"{p}/Cast"].inputs == [f.name + ":3"]
        # the fused node takes the ExpandDims' place: after its input, before its users
        pos = {n: j for j, n in enumerate(names)}
        assert pos[f"in{i}"] < pos[f.name] < pos[f"{p}/use0"]


@pytest.mark.parametrize("form", FORMS)
def test_dnn_hash_bucket_emits_kp_fused_dnn_embedding(tmp_path, form):
    src, removed = _model(tmp_path, "dnn_hash_bucket", form)
    out = tmp_path / "out"
    annc_opt.optimize(str(src), str(out), ["dnn_hash_bucket"])
    m = annc_opt.load_model(str(out))
    by = {n.name: n for n in m.nodes}
    for i in range(2):
        p = f"col{i}"
        f = by[f"{p}/SparseFillEmptyRows/rec_embed_kp_dnn_bucket"]
        assert f.op == "KPFusedDnnEmbeddingWithHashBucket"
        assert f.inputs == [f"in{i}", f"emb{i}"]
        assert f.attrs == {"num_buckets": 100 + i, "_output_shapes": _shapes(form, [-1, 16])}
        assert len(removed[p]) == 43  # rec_embedding.py:200-209
        assert not set(removed[p]) & set(by)
        assert by[f"{p}/use"].inputs == [f.name]
        assert f"emb{i}" in by  # the weight stays


@pytest.mark.parametrize("case", ["hash_read_outside", "extra_sfer_user", "wrong_op",
                                  "ctrl_dep_inside"])
def test_sparse_pass_near_misses_are_left_alone(tmp_path, case):
    """A removed node read outside the match, a changed op type or user
    count, or a control dependency on a removed node: that column stays,
    the other is fused."""
    def tweak(nodes):
        if case == "hash_read_outside":
            nodes.append(N("spy", "Identity", ["col0/hash"]))
        elif case == "extra_sfer_user":  # dnn_hash_bucket needs exactly 3 users
            nodes.append(N("spy", "Identity", ["col0/SparseFillEmptyRows:3"]))
        elif case == "wrong_op":
            for n in nodes:
                if n.name == "col0/segment":
                    n.op = "SparseSegmentSum"
        else:
            nodes.append(N("spy", "NoOp", ["^col0/Unique"]))

    src, removed = _model(tmp_path, "dnn_hash_bucket", "json", tweak)
    out = tmp_path / "out"
    annc_opt.optimize(str(src), str(out), ["dnn_hash_bucket"])
    names = {n.name for n in annc_opt.load_model(str(out)).nodes}
    assert set(removed["col0"]) <= names
    assert "col1/SparseFillEmptyRows/rec_embed_kp_dnn_bucket" in names


def test_sparse_passes_do_not_cross_match(tmp_path):
    """dnn_sparse leaves linear columns alone and linear_sparse DNN ones
    (the Identity chain and the Shape's users differ)."""
    for kind, other in (("linear_sparse", "dnn_sparse"), ("dnn_sparse", "linear_sparse")):
        src, removed = _model(tmp_path / kind, kind, "json")
        out = tmp_path / kind / "out"
        annc_opt.optimize(str(src), str(out), [other])
        names = {n.name for n in annc_opt.load_model(str(out)).nodes}
        assert set(removed["col0"]) <= names and set(removed["col1"]) <= names
