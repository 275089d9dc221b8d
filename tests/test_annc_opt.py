"""annc-opt layout_matmul (python/annc/main.py, optimize/constant_folding.py,
optimize/data_pack.py): CPU tests of the pass, the CLI and the kn4 reader."""
import os

import numpy as np
import pytest

from annc_amd import annc_opt
from annc_amd import device as dev

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


def _model(tmp_path):
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
    annc_opt.save_model(annc_opt.Model(nodes, variables), str(src))
    (src / "assets").mkdir()
    (src / "assets" / "vocab.txt").write_text("a\nb\n")
    return src, orig, variables


def test_layout_matmul_cli(tmp_path):
    src, orig, before = _model(tmp_path)
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


def test_unknown_and_tensorflow_passes_are_rejected(tmp_path):
    src, _, _ = _model(tmp_path)
    with pytest.raises(TypeError, match="not found"):
        annc_opt.optimize(str(src), str(tmp_path / "o1"), ["layout_matmul", "fold_all"])
    with pytest.raises(TypeError, match="TensorFlow"):
        annc_opt.optimize(str(src), str(tmp_path / "o2"), ["embed_hash_bucket"])
