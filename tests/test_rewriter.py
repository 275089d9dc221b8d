"""Host tests of the KDnnRewriter restatement (annc_hlo_rewrite_instruction).

Expectations come from the reference's registration rules
(gemm_rewriter.cc:65-134, graph_opt.cc:8-129, kdnn_rewriter.cc:8-69) and
from the operand lists its custom-call kernels read (gemm_rewriter.cc:
161-281: __matmul {A, B}, __matmul_add {E, A, B}, __matmul_add_relu
{Z, E, A, B}, each followed by one shape info per operand)."""
import pytest

from annc_amd import _lib, hlo


@pytest.fixture
def flags():
    lib = _lib.lib()

    def set_flags(s: str):
        lib.annc_flags_reset(s.encode())

    yield set_flags
    lib.annc_flags_reset(b"")


def test_defaults_rewrite_nothing(flags):
    flags("")
    f, dot, _ = hlo.dense_layer(64, 32, 16)
    assert hlo.rewrite(f, dot) is None


def test_matmul_add_relu_operand_order_and_commutativity(flags):
    flags("--matmul-add-relu")
    for swap in (False, True):
        f = hlo.Fragment()
        x = f.add("parameter", (64, 32))
        w = f.add("parameter", (32, 16))
        dot = f.add("dot", (64, 16), operands=(x, w))
        b = f.add("parameter", (16,))
        bb = f.add("broadcast", (64, 16), operands=(b,))
        add = f.add("add", (64, 16), operands=(bb, dot) if swap else (dot, bb))
        z = f.add("constant", ())
        zb = f.add("broadcast", (64, 16), operands=(z,))
        mx = f.add("maximum", (64, 16), operands=(zb, add) if swap else (add, zb))
        r = hlo.rewrite(f, dot)
        assert r.target == "__matmul_add_relu" and r.custom_call and r.benefit == 3
        assert r.fused == [mx, add, dot]
        assert r.operands == [zb, bb, x, w]  # {Z, E, A, B}
        assert r.shape_infos == r.operands


def test_matmul_add_and_matmul_operands(flags):
    flags("--matmul-add")
    f, dot, out = hlo.dense_layer(64, 32, 16, activation=None)
    r = hlo.rewrite(f, dot)
    assert r.target == "__matmul_add" and r.benefit == 2 and r.operands == [4, 0, 1]  # {E, A, B}
    flags("--matmul")
    r = hlo.rewrite(f, dot)
    assert r.target == "__matmul" and r.operands == [0, 1] and r.fused == [dot]


def test_priority_by_benefit(flags):
    flags("--matmul --layout-matmul --matmul-add --matmul-add-relu")
    f, dot, _ = hlo.dense_layer(4096, 1024, 512)
    assert hlo.rewrite(f, dot).target == "__matmul_add_relu"
    f2, dot2, _ = hlo.dense_layer(4096, 1024, 512, activation=None)
    assert hlo.rewrite(f2, dot2).target == "__matmul_add"
    f3, dot3, _ = hlo.dense_layer(4096, 1024, 512, activation=None, bias=False)
    assert hlo.rewrite(f3, dot3).target == "__layout_matmul"  # registration order on ties


def test_gemm_opt_leaves_the_add_patterns_off(flags):
    """--gemm-opt enables matmul and layout-matmul, not matmul-add(-relu)
    (annc_flags.cc:88-104): a parameter rhs goes to __layout_matmul, a
    constant rhs to __matmul."""
    flags("--gemm-opt")
    f, dot, _ = hlo.dense_layer(4096, 1024, 512)
    assert hlo.rewrite(f, dot).target == "__layout_matmul"
    f2, dot2, _ = hlo.dense_layer(4096, 1024, 512, weight_parameter=False)
    assert hlo.rewrite(f2, dot2).target == "__matmul"


def test_layout_matmul_rules(flags):
    flags("--layout-matmul")
    # every dimension of both operands must be >= 12
    for m, k, n, ok in ((12, 12, 12, True), (4096, 256, 1, False), (11, 64, 64, False),
                        (64, 11, 64, False), (64, 64, 11, False)):
        f, dot, _ = hlo.dense_layer(m, k, n)
        r = hlo.rewrite(f, dot)
        assert (r is not None and r.target == "__layout_matmul") == ok, (m, k, n)
    # rhs must be an HLO parameter; dtype and layout are not checked
    f, dot, _ = hlo.dense_layer(64, 64, 64, weight_parameter=False)
    assert hlo.rewrite(f, dot) is None
    f = hlo.Fragment()
    x = f.add("parameter", (64, 64), dtype="other", minor_to_major=(0, 1))
    w = f.add("parameter", (64, 64), dtype="other")
    dot = f.add("dot", (64, 64), dtype="other", operands=(x, w))
    r = hlo.rewrite(f, dot)
    assert r.target == "__layout_matmul" and r.operands == [x, w]


def test_matmul_dim_range_dtype_layout(flags):
    flags("--matmul")
    for m, n, ok in ((12, 12, True), (11, 64, False), (64, 11, False), (4096, 1, False)):
        f, dot, _ = hlo.dense_layer(m, 64, n, weight_parameter=False)
        assert (hlo.rewrite(f, dot) is not None) == ok, (m, n)
    f = hlo.Fragment()
    x = f.add("parameter", (64, 64), minor_to_major=(0, 1))  # column-major lhs
    w = f.add("constant", (64, 64))
    dot = f.add("dot", (64, 64), operands=(x, w))
    assert hlo.rewrite(f, dot) is None
    f = hlo.Fragment()
    x = f.add("parameter", (64, 64), dtype="s32")
    w = f.add("constant", (64, 64))
    dot = f.add("dot", (64, 64), operands=(x, w))
    assert hlo.rewrite(f, dot) is None


def test_batch_matmul_dim_range(flags):
    flags("--batch-matmul")
    for shape, ok in (((1, 8, 8), True), ((4, 7, 8), False), ((4, 8, 7), False)):
        b, m, n = shape
        f = hlo.Fragment()
        a = f.add("parameter", (b, m, 16))
        w = f.add("parameter", (b, 16, n))
        dot = f.add("dot", shape, operands=(a, w))
        r = hlo.rewrite(f, dot)
        assert (r is not None and r.target == "__batch_matmul" and r.operands == [a, w]) == ok
    f, dot, _ = hlo.dense_layer(64, 64, 64)  # rank-2 dot is not a batch matmul
    assert hlo.rewrite(f, dot) is None


def test_users_order_matters(flags):
    """users()[0] must be the add (kdnn_rewriter.cc:33-40)."""
    flags("--matmul-add")
    f = hlo.Fragment()
    x = f.add("parameter", (64, 32))
    w = f.add("parameter", (32, 16))
    dot = f.add("dot", (64, 16), operands=(x, w))
    f.add("other", (64, 16), operands=(dot,))  # first user is not the add
    e = f.add("parameter", (64, 16))
    f.add("add", (64, 16), operands=(dot, e))
    assert hlo.rewrite(f, dot) is None


def test_control_dependencies_block_rewrites(flags):
    flags("--matmul-add-relu --matmul")
    f, dot, _ = hlo.dense_layer(64, 32, 16, weight_parameter=False)
    f.instrs[dot].control_deps = True
    assert hlo.rewrite(f, dot) is None


def _sparse_embedding2_fragment(f):
    ids = f.add("parameter", (32, 8), dtype="s64")
    c0 = f.add("constant", (), dtype="s64")
    c0b = f.add("broadcast", (32, 8), dtype="s64", operands=(c0,))
    cmp0 = f.add("compare", (32, 8), dtype="pred", operands=(ids, c0b))
    idsc = f.add("convert", (32, 8), dtype="s64", operands=(ids,))
    c1 = f.add("constant", (), dtype="s64")
    c1b = f.add("broadcast", (32, 8), dtype="s64", operands=(c1,))
    cmp1 = f.add("compare", (32, 8), dtype="pred", operands=(idsc, c1b))
    both = f.add("and", (32, 8), dtype="pred", operands=(cmp0, cmp1))
    fill = f.add("broadcast", (32, 8), dtype="s64", operands=(c0,))
    sel = f.add("select", (32, 8), dtype="s64", operands=(both, idsc, fill))
    table = f.add("parameter", (1000, 16))
    gat = f.add("gather", (32, 8, 16), operands=(table, sel))
    mask = f.add("convert", (32, 8), operands=(both,))
    maskb = f.add("broadcast", (32, 8, 16), operands=(mask,))
    mul = f.add("multiply", (32, 8, 16), operands=(maskb, gat))
    return mul, dict(ids=ids, table=table, sel=sel, gather=gat)


def test_sparse_embedding2_fusion(flags):
    flags("--sps-emd-2")
    f = hlo.Fragment()
    mul, n = _sparse_embedding2_fragment(f)
    r = hlo.rewrite(f, mul)
    assert r.target == "sparse_embedding2" and not r.custom_call and r.benefit == 3
    assert len(r.fused) == 12 and r.fused[0] == mul and n["gather"] in r.fused
    assert n["table"] in r.operands and n["ids"] in r.operands
    flags("")
    assert hlo.rewrite(f, mul) is None


def test_sparse_embedding2_missing_broadcast_is_safe(flags):
    """compare_0's operand 1 is read without an opcode check
    (graph_opt.cc:26-28); a compare with one operand must not match."""
    flags("--sps-emd-2")
    f = hlo.Fragment()
    mul, _ = _sparse_embedding2_fragment(f)
    cmp0 = f.instrs[3]
    f.instrs[3] = hlo.Instr(cmp0.opcode, cmp0.shape, cmp0.dtype, cmp0.operands[:1])
    assert hlo.rewrite(f, mul) is None


def test_pooling_tree(flags):
    flags("--pooling")
    f = hlo.Fragment()
    ids = f.add("parameter", (32, 8), dtype="s64")
    z64 = f.add("broadcast", (32, 8), dtype="s64", operands=(f.add("constant", (), dtype="s64"),))
    cmp = f.add("compare", (32, 8), dtype="pred", operands=(ids, z64))
    cnt = f.add("reduce", (32,), dtype="s32", operands=(f.add("convert", (32, 8), dtype="s32",
                                                                operands=(cmp,)),))
    cmp2 = f.add("compare", (32,), dtype="pred", operands=(cnt,))
    g = f.add("parameter", (32, 8, 16))
    sl = f.add("slice", (32, 8, 16), operands=(g,))
    m = f.add("broadcast", (32, 8, 16), dtype="pred", operands=(cmp,))
    zf = f.add("broadcast", (32, 8, 16), operands=(f.add("constant", ()),))
    s1 = f.add("select", (32, 8, 16), operands=(m, sl, zf))
    red = f.add("reduce", (32, 16), operands=(s1,))
    rs = f.add("reshape", (32, 16), operands=(red,))
    cntf = f.add("broadcast", (32, 16), operands=(f.add("convert", (32,), operands=(cnt,)),))
    div = f.add("divide", (32, 16), operands=(rs, cntf))
    b0 = f.add("broadcast", (32, 16), dtype="pred", operands=(cmp2,))
    zo = f.add("broadcast", (32, 16), operands=(f.add("constant", ()),))
    sel = f.add("select", (32, 16), operands=(b0, zo, div))
    r = hlo.rewrite(f, sel)
    assert r.target == "__pooling" and r.custom_call and len(r.fused) == 13
    assert r.operands[2:] == ["slice_starts", "slice_limits"] and len(r.shape_infos) == 2
    broken = hlo.Fragment(list(f.instrs))
    broken.instrs[div] = hlo.Instr("add", (32, 16), "f32", (rs, cntf))
    assert hlo.rewrite(broken, sel) is None


def test_malformed_fragment_rejected(flags):
    f = hlo.Fragment()
    f.add("parameter", (4, 4))
    f.instrs.append(hlo.Instr("dot", (4, 4), "f32", (0, 7)))
    with pytest.raises(_lib.InvalidArgumentError):
        hlo.rewrite(f, 1)


def test_config2_tower_lowering(flags):
    """configs[1] under --layout-matmul: layers 1-2 become __layout_matmul,
    the 256 -> 1 scoring layer stays an XLA dot (gemm_rewriter.cc:27-36)."""
    from annc_amd import workloads
    from annc_amd.rec_graph import MLPTower
    w = workloads.config2(seed=0, batch=64)
    tower = MLPTower(w.weights, w.biases, device="cpu", packed=False)
    flags("--layout-matmul")
    assert tower.lowering(4096) == ["__layout_matmul", "__layout_matmul", None]
    flags("--matmul-add-relu --matmul")
    assert tower.lowering(4096) == ["__matmul_add_relu", "__matmul_add_relu", None]
