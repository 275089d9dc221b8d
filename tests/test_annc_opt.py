"""annc-opt layout_matmul (python/annc/main.py, optimize/constant_folding.py,
optimize/data_pack.py): CPU tests of the pass, the CLI and the kn4 reader."""
import os

import numpy as np
import pytest

from annc_amd import annc_opt
from annc_amd import device as dev
from annc_amd import savedmodel as sm

GOLD = os.path.join(os.path.dirname(__file__), "golden", "kn4_pack_vectors.npz")


def test_kn4_permutation_matches_reference_packing():
    """Pinned by tests/golden/kn4_pack_vectors.npz, written by the reference's
    own FormageChange (tests/golden/make_kn4_vectors.py)."""
    gold = np.load(GOLD)
    assert len(gold.files) >= 7
    for key in gold.files:
        k, n = (int(x) for x in key.split("_")[1].split("x"))
        np.testing.assert_array_equal(annc_opt.kn4_permutation(k, n), gold[key], err_msg=key)


@pytest.mark.parametrize("dim", [1, 11, 12, 128, 129, 352, 353, 365, 705, 1000, 1024])
@pytest.mark.parametrize("tile", [128, 352])
def test_kn4_tiles_cover_the_axis(dim, tile):
    b = annc_opt._tile_bounds(dim, tile, 12)
    assert b[0][0] == 0 and b[-1][1] == dim
    assert all(b[i][1] == b[i + 1][0] for i in range(len(b) - 1))
    assert all(e > s for s, e in b)


@pytest.mark.parametrize("k,n", [(12, 12), (37, 141), (400, 300)])
def test_kn4_round_trip(k, n):
    w = np.random.default_rng(k).standard_normal((k, n)).astype(np.float32)
    np.testing.assert_array_equal(annc_opt.unpack_kn4(annc_opt.pack_kn4(w), k, n), w)


def _shapes_attr(*shapes):
    """AttrValue {list {shape ...}} (an `_output_shapes` attr) as raw bytes."""
    lst = sm.Msg([(7, sm.LEN, sm.shape_proto(s)) for s in shapes])
    return sm.RawAttr(sm.Msg([(1, sm.LEN, lst)]).serialize())


def _as_form(nodes, variables, form):
    """The model in this build's plain form, or as a SavedModel (graph attrs
    as TensorFlow types them: dtype attrs as DataType, shape lists raw)."""
    if form == "json":
        return annc_opt.Model(nodes, variables)
    for n in nodes:
        for k, v in list(n.attrs.items()):
            if k == "_output_shapes":
                n.attrs[k] = _shapes_attr(*v)
            elif k == "dtype":
                n.attrs[k] = sm.DType(v)
    return annc_opt.Model(nodes, variables, sm.new_saved_model([]))


FORMS = ["json", "saved"]


def _model(tmp_path, form="json"):
    g = np.random.default_rng(7)
    f32 = lambda *s: g.standard_normal(s).astype(np.float32)  # noqa: E731
    orig = {"w1": f32(64, 48), "w2": f32(8, 64), "w3l": f32(4, 20), "w3": f32(20, 30),
            "w4": f32(40, 36), "w5": f32(32, 32), "w6": f32(3, 16, 16), "w7": f32(24, 16)}
    variables = dict(orig)
    variables["w4"] = annc_opt.pack_kn4(orig["w4"])            # packed by the reference
    variables["w5"] = annc_opt.pack_rhs(orig["w5"])            # already in this format
    nodes = [annc_opt.Node("x", "Placeholder")]
    for v in orig:
        nodes.append(annc_opt.Node(v, "VarHandleOp"))
        nodes.append(annc_opt.Node(v + "/read", "ReadVariableOp", [v]))
    nodes += [
        annc_opt.Node("m1", "MatMul", ["x", "w1/read"]),
        annc_opt.Node("m2", "MatMul", ["x", "w2/read"]),                 # k < 12: kept
        annc_opt.Node("m3", "MatMul", ["w3l/read", "w3/read"]),          # small lhs var: kept
        annc_opt.Node("m4", "MatMul", ["x", "w4/read"], {"rhs_format": "kn4"}),
        annc_opt.Node("m5", "MatMul", ["x", "w5"], {"rhs_format": annc_opt.mfma_rhs_format()}),
        annc_opt.Node("m6", "BatchMatMulV2", ["x", "w6/read"]),          # rank 3: kept
        annc_opt.Node("m7", "MatMul", ["x", "w7:0"], {"transpose_b": True}),
    ]
    src = tmp_path / "in"
    annc_opt.save_model(_as_form(nodes, variables, form), str(src))
    (src / "assets").mkdir()
    (src / "assets" / "vocab.txt").write_text("a\nb\n")
    return src, orig, variables


@pytest.mark.parametrize("form", FORMS)
def test_layout_matmul_cli(tmp_path, form):
    src, orig, before = _model(tmp_path, form)
    if form == "saved":  # made stale by the rewrite: not copied
        (src / "saved_model.pbtxt").write_text("stale")
        (src / "fingerprint.pb").write_bytes(b"stale")
    out = tmp_path / "out"
    assert annc_opt.main(["-I", str(src), "-O", str(out), "layout_matmul"]) == 0
    m = annc_opt.load_model(str(out))
    fmt = annc_opt.mfma_rhs_format()
    attrs = {n.name: n.attrs for n in m.nodes}
    assert attrs["m1"]["rhs_format"] == fmt
    np.testing.assert_array_equal(m.variables["w1"], annc_opt.pack_rhs(orig["w1"]))
    assert m.variables["w1"].shape == (64, 48)  # same shape, permuted
    np.testing.assert_array_equal(dev.unpack_weight_host(m.variables["w1"], 64, 48), orig["w1"])
    # reference-packed kn4 weight converted
    assert attrs["m4"]["rhs_format"] == fmt
    np.testing.assert_array_equal(m.variables["w4"], annc_opt.pack_rhs(orig["w4"]))
    # untouched: small k, small variable lhs, already packed, rank-3, transposed
    for name, node in (("w2", "m2"), ("w3", "m3"), ("w3l", "m3"), ("w6", "m6"), ("w7", "m7")):
        np.testing.assert_array_equal(m.variables[name], before[name])
        assert "rhs_format" not in attrs[node] or node == "m5"
    np.testing.assert_array_equal(m.variables["w5"], before["w5"])
    assert (out / "assets" / "vocab.txt").read_text() == "a\nb\n"
    if form == "saved":
        assert sorted(os.listdir(out)) == ["assets", "saved_model.pb", "variables"]
        assert sorted(os.listdir(out / "variables")) == ["variables.data-00000-of-00001",
                                                         "variables.index"]
        # the attrs TensorFlow reads: rhs_format a string, transpose_b a bool
        g = sm.read_saved_model(str(out))
        raw = {n.name: n for n in g.nodes}
        assert raw["m1"].attrs["rhs_format"] == fmt and raw["m7"].attrs["transpose_b"] is True


def test_unknown_and_unsupported_passes_are_rejected(tmp_path):
    src, _, _ = _model(tmp_path)
    with pytest.raises(TypeError, match="not found"):
        annc_opt.optimize(str(src), str(tmp_path / "o1"), ["layout_matmul", "fold_all"])
    for p in ("embed", "softmax"):
        with pytest.raises(TypeError, match="does not implement"):
            annc_opt.optimize(str(src), str(tmp_path / "o2"), [p])


# ---------------------------------------------------------------------------
# embed_hash_bucket: the TF feature-column subgraph of
# embedding_column(categorical_column_with_hash_bucket(...), combiner=...)
# as TF 1.x lowers it (ops, operand order and graph order), built by hand.
# ---------------------------------------------------------------------------
def _column(p, inp, weight, combiner, num_buckets):
    """Nodes of one column in graph order; returns (nodes, result name,
    names of the nodes the fused op replaces)."""
    N = annc_opt.Node
    consts = [N(f"{p}/c{i}", "Const") for i in range(12)]
    c = [x.name for x in consts]
    if combiner == "sum":
        body = [
            N(f"{p}/ExpandDims", "ExpandDims", [inp, c[0]]),
            N(f"{p}/NotEqual", "NotEqual", [f"{p}/ExpandDims", c[1]]),
            N(f"{p}/Where", "Where", [f"{p}/NotEqual"]),
            N(f"{p}/GatherNd", "GatherNd", [f"{p}/ExpandDims", f"{p}/Where"]),
            N(f"{p}/hash", "StringToHashBucketFast", [f"{p}/GatherNd"],
              {"num_buckets": num_buckets}),
            N(f"{p}/Shape", "Shape", [f"{p}/ExpandDims"]),
            N(f"{p}/Cast", "Cast", [f"{p}/Shape"]),
            N(f"{p}/strided_slice", "StridedSlice", [f"{p}/Cast", c[2], c[3], c[4]]),
            N(f"{p}/stack", "Pack", [f"{p}/strided_slice", c[5]]),
            N(f"{p}/Cast_1", "Cast", [f"{p}/stack"]),
            N(f"{p}/SparseReshape", "SparseReshape", [f"{p}/Where", f"{p}/Shape", f"{p}/Cast_1"]),
            N(f"{p}/Slice", "Slice", [f"{p}/SparseReshape:1", c[6], c[7]]),
            N(f"{p}/Prod", "Prod", [f"{p}/Slice", c[8]]),
            N(f"{p}/GatherV2", "GatherV2", [f"{p}/SparseReshape:1", c[9], c[8]]),
            N(f"{p}/Cast_2", "Pack", [f"{p}/Prod", f"{p}/GatherV2"]),
            N(f"{p}/SparseReshape_1", "SparseReshape",
              [f"{p}/SparseReshape", f"{p}/SparseReshape:1", f"{p}/Cast_2"]),
            N(f"{p}/Identity", "Identity", [f"{p}/SparseReshape_1:1"]),
            N(f"{p}/Identity_1", "Identity", [f"{p}/hash"]),
            N(f"{p}/Identity_2", "Identity", [f"{p}/Identity_1"]),
            N(f"{p}/GreaterEqual", "GreaterEqual", [f"{p}/Identity_2", c[10]]),
            N(f"{p}/Where_1", "Where", [f"{p}/GreaterEqual"]),
            N(f"{p}/Reshape", "Reshape", [f"{p}/Where_1", c[11]]),
            N(f"{p}/GatherV2_1", "GatherV2", [f"{p}/SparseReshape_1", f"{p}/Reshape", c[8]]),
            N(f"{p}/GatherV2_2", "GatherV2", [f"{p}/Identity_2", f"{p}/Reshape", c[8]]),
            N(f"{p}/SparseFillEmptyRows", "SparseFillEmptyRows",
              [f"{p}/GatherV2_1", f"{p}/GatherV2_2", f"{p}/Identity", c[10]]),
            N(f"{p}/strided_slice_1", "StridedSlice", [f"{p}/SparseFillEmptyRows", c[2], c[3], c[4]]),
            N(f"{p}/Unique", "Unique", [f"{p}/SparseFillEmptyRows:1"]),
            N(f"{p}/Reshape_1", "Reshape", [f"{p}/SparseFillEmptyRows:2", c[11]]),
            N(f"{p}/embedding_lookup", "ResourceGather", [weight, f"{p}/Unique"]),
            N(f"{p}/embedding_lookup/Identity", "Identity", [f"{p}/embedding_lookup"]),
            N(f"{p}/embedding_lookup/Identity_1", "Identity", [f"{p}/embedding_lookup/Identity"]),
            N(f"{p}/Cast_3", "Cast", [f"{p}/strided_slice_1"]),
            N(f"{p}/segment", "SparseSegmentSum",
              [f"{p}/embedding_lookup/Identity_1", f"{p}/Unique:1", f"{p}/Cast_3"]),
        ]
    else:
        body = [
            N(f"{p}/ExpandDims", "ExpandDims", [inp, c[0]]),
            N(f"{p}/Shape", "Shape", [f"{p}/ExpandDims"]),
            N(f"{p}/NotEqual", "NotEqual", [f"{p}/ExpandDims", c[1]]),
            N(f"{p}/Where", "Where", [f"{p}/NotEqual"]),
            N(f"{p}/GatherNd", "GatherNd", [f"{p}/ExpandDims", f"{p}/Where"]),
            N(f"{p}/hash", "StringToHashBucketFast", [f"{p}/GatherNd"],
              {"num_buckets": num_buckets}),
            N(f"{p}/Slice", "Slice", [f"{p}/Shape", c[6], c[7]]),
            N(f"{p}/Prod", "Prod", [f"{p}/Slice", c[8]]),
            N(f"{p}/GatherV2", "GatherV2", [f"{p}/Shape", c[9], c[8]]),
            N(f"{p}/stack", "Pack", [f"{p}/Prod", f"{p}/GatherV2"]),
            N(f"{p}/SparseReshape", "SparseReshape", [f"{p}/Where", f"{p}/Shape", f"{p}/stack"]),
            N(f"{p}/Identity", "Identity", [f"{p}/SparseReshape:1"]),
            N(f"{p}/Identity_1", "Identity", [f"{p}/hash"]),
            N(f"{p}/GreaterEqual", "GreaterEqual", [f"{p}/Identity_1", c[10]]),
            N(f"{p}/Where_1", "Where", [f"{p}/GreaterEqual"]),
            N(f"{p}/Reshape", "Reshape", [f"{p}/Where_1", c[11]]),
            N(f"{p}/GatherV2_1", "GatherV2", [f"{p}/SparseReshape", f"{p}/Reshape", c[8]]),
            N(f"{p}/GatherV2_2", "GatherV2", [f"{p}/Identity_1", f"{p}/Reshape", c[8]]),
            N(f"{p}/SparseFillEmptyRows", "SparseFillEmptyRows",
              [f"{p}/GatherV2_1", f"{p}/GatherV2_2", f"{p}/Identity", c[10]]),
            N(f"{p}/strided_slice_1", "StridedSlice", [f"{p}/SparseFillEmptyRows", c[2], c[3], c[4]]),
            N(f"{p}/Unique", "Unique", [f"{p}/SparseFillEmptyRows:1"]),
            N(f"{p}/Reshape_1", "Reshape", [f"{p}/SparseFillEmptyRows:2", c[11]]),
            N(f"{p}/embedding_lookup", "GatherV2", [weight, f"{p}/Unique", c[8]]),
            N(f"{p}/embedding_lookup/Identity", "Identity", [f"{p}/embedding_lookup"]),
            N(f"{p}/Cast_3", "Cast", [f"{p}/strided_slice_1"]),
            N(f"{p}/segment", "SparseSegmentMean",
              [f"{p}/embedding_lookup/Identity", f"{p}/Unique:1", f"{p}/Cast_3"]),
        ]
    tail = [
        N(f"{p}/Shape_1", "Shape", [f"{p}/segment"]),
        N(f"{p}/strided_slice_2", "StridedSlice", [f"{p}/Shape_1", c[2], c[3], c[4]]),
        N(f"{p}/stack_1", "Pack", [c[5], f"{p}/strided_slice_2"]),
        N(f"{p}/Tile", "Tile", [f"{p}/Reshape_1", f"{p}/stack_1"]),
        N(f"{p}/zeros_like", "ZerosLike", [f"{p}/segment"]),
        N(f"{p}/Select", "Select", [f"{p}/Tile", f"{p}/zeros_like", f"{p}/segment"]),
        N(f"{p}/Shape_2", "Shape", [f"{p}/Select"]),
        N(f"{p}/Slice_1", "Slice", [f"{p}/Shape_2", c[6], c[7]]),
        N(f"{p}/Cast_4", "Cast", [f"{p}/SparseReshape:1" if combiner == "sum" else f"{p}/Shape"]),
        N(f"{p}/Slice_2", "Slice", [f"{p}/Cast_4", c[6], c[7]]),
        N(f"{p}/concat", "ConcatV2", [f"{p}/Slice_2", f"{p}/Slice_1", c[8]]),
        N(f"{p}/Reshape_2", "Reshape", [f"{p}/Select", f"{p}/concat"],
          {"_output_shapes": [[-1, 16]]}),
    ]
    if combiner == "mean":
        tail += [
            N(f"{p}/Shape_3", "Shape", [f"{p}/Reshape_2"]),
            N(f"{p}/strided_slice_3", "StridedSlice", [f"{p}/Shape_3", c[2], c[3], c[4]]),
            N(f"{p}/stack_2", "Pack", [f"{p}/strided_slice_3", c[5]]),
            N(f"{p}/Reshape_3", "Reshape", [f"{p}/Reshape_2", f"{p}/stack_2"],
              {"_output_shapes": [[-1, 16]]}),
        ]
    nodes = consts + body + tail
    fused = [n.name for n in body + tail]
    return nodes, tail[-1].name, fused


def _embedding_model(tmp_path, columns=(("sum", 1000), ("mean", 77)), extra=None, form="json"):
    N = annc_opt.Node
    nodes, results, fused = [], [], {}
    g = np.random.default_rng(3)
    variables = {}
    for i, (comb, nb) in enumerate(columns):
        nodes.append(N(f"in{i}", "Placeholder", [], {"dtype": "DT_STRING"}))
        nodes.append(N(f"emb{i}", "VarHandleOp" if comb == "sum" else "VariableV2"))
        variables[f"emb{i}"] = g.standard_normal((nb, 16)).astype(np.float32)
        weight = f"emb{i}"
        if comb == "mean":
            nodes.append(N(f"emb{i}/read", "Identity", [f"emb{i}"]))
            weight = f"emb{i}/read"
        col, res, f = _column(f"col{i}", f"in{i}", weight, comb, nb)
        nodes += col
        results.append(res)
        fused[f"col{i}"] = f
    nodes.append(N("concat", "ConcatV2", results + ["axis"]))
    nodes.append(N("axis", "Const"))
    nodes.append(N("w_dense", "VarHandleOp"))
    variables["w_dense"] = g.standard_normal((16 * len(columns), 32)).astype(np.float32)
    nodes.append(N("w_dense/read", "ReadVariableOp", ["w_dense"]))
    nodes.append(N("dense", "MatMul", ["concat", "w_dense/read"]))
    nodes.append(N("after", "NoOp", [], {}))
    nodes[-1].inputs = ["^" + results[0]]
    if extra:
        extra(nodes)
    src = tmp_path / "emb_in"
    annc_opt.save_model(_as_form(nodes, variables, form), str(src))
    return src, results, fused


@pytest.mark.parametrize("form", FORMS)
def test_embed_hash_bucket_fuses_sum_and_mean_columns(tmp_path, form):
    src, results, fused = _embedding_model(tmp_path, form=form)
    before = annc_opt.load_model(str(src))
    out = tmp_path / "emb_out"
    # layout_matmul given first still runs last, on the fused graph
    assert annc_opt.main(["-I", str(src), "-O", str(out), "layout_matmul",
                          "embed_hash_bucket"]) == 0
    m = annc_opt.load_model(str(out))
    names = [n.name for n in m.nodes]
    by = {n.name: n for n in m.nodes}
    f0 = by["col0/SparseFillEmptyRows/rec_embed_kp_bucket"]
    f1 = by["col1/SparseFillEmptyRows/rec_embed_kp_bucket"]
    assert f0.op == f1.op == "KPFusedEmbeddingWithHashBucket"
    assert f0.inputs == ["in0", "emb0"] and f1.inputs == ["in1", "emb1/read"]
    shapes = [[-1, 16]] if form == "json" else _shapes_attr([-1, 16])
    assert f0.attrs == {"num_buckets": 1000, "combiner": 0, "T_weight": "DT_RESOURCE",
                        "_output_shapes": shapes}
    assert f1.attrs == {"num_buckets": 77, "combiner": 1, "T_weight": "DT_FLOAT",
                        "_output_shapes": shapes}
    if form == "saved":  # T_weight is a DataType attr (DT_RESOURCE 20, DT_FLOAT 1)
        assert isinstance(f0.attrs["T_weight"], sm.DType)
        assert sm.Msg.parse(sm.encode_attr(f0.attrs["T_weight"])).fields == [(6, sm.VARINT, 20)]
        assert sm.Msg.parse(sm.encode_attr(f1.attrs["T_weight"])).fields == [(6, sm.VARINT, 1)]
    assert len(fused["col0"]) == 45 and len(fused["col1"]) == 42
    for col in fused.values():
        assert not set(col) & set(names)
    assert by["concat"].inputs[:2] == [f0.name, f1.name]
    assert by["after"].inputs == ["^" + f0.name]
    # graph order still puts every node after its inputs
    pos = {n: i for i, n in enumerate(names)}
    for n in m.nodes:
        for i in n.inputs:
            src_name = i.lstrip("^").split(":")[0]
            if src_name in pos:
                assert pos[src_name] < pos[n.name] or n.name == "concat", (n.name, i)
    # everything outside the columns is unchanged
    kept = [n.name for n in before.nodes if n.name not in set(sum(fused.values(), []))]
    assert [x for x in names if not x.endswith("rec_embed_kp_bucket")] == kept
    assert by["dense"].attrs["rhs_format"] == annc_opt.mfma_rhs_format()


def test_lookup_embedding_hash_emits_its_own_op(tmp_path):
    src, _, _ = _embedding_model(tmp_path, columns=(("mean", 50),))
    out = tmp_path / "o"
    annc_opt.optimize(str(src), str(out), ["lookup_embedding_hash"])
    m = annc_opt.load_model(str(out))
    ops = {n.name: n.op for n in m.nodes}
    assert ops["col0/SparseFillEmptyRows/rec_embed_kp_hash"] == "KPLookupEmbeddingByHash"


@pytest.mark.parametrize("case", ["sfer_extra_user", "hash_read_outside", "wrong_segment_op",
                                  "ctrl_dep_inside"])
def test_embed_hash_bucket_near_misses_are_left_alone(tmp_path, case):
    N = annc_opt.Node

    def extra(nodes):
        if case == "sfer_extra_user":      # SparseFillEmptyRows must have exactly 3 users
            nodes.append(N("spy", "Identity", ["col0/SparseFillEmptyRows:3"]))
        elif case == "hash_read_outside":  # a removed node read elsewhere
            nodes.append(N("spy", "Identity", ["col0/hash"]))
        elif case == "wrong_segment_op":
            for n in nodes:
                if n.name == "col0/segment":
                    n.op = "SparseSegmentSqrtN"
        else:
            nodes.append(N("spy", "NoOp", ["^col0/Unique"]))

    src, _, fused = _embedding_model(tmp_path, columns=(("sum", 1000), ("mean", 77)),
                                     extra=extra)
    out = tmp_path / "o"
    annc_opt.optimize(str(src), str(out), ["embed_hash_bucket"])
    names = {n.name for n in annc_opt.load_model(str(out)).nodes}
    assert set(fused["col0"]) <= names                                # untouched
    assert "col1/SparseFillEmptyRows/rec_embed_kp_bucket" in names   # the other column fused
