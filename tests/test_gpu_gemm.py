"""GPU parity: fp32 MFMA GEMM custom calls against OpenBLAS 0.3.29.

Tolerance per element: |got - ref| <= 1e-4*|ref| + 1e-4*(|A||B| + |E|)."""
import numpy as np
import pytest
import torch

from annc_amd import EPI_NONE, EPI_RELU, EPI_SIGMOID, _lib, workloads, xla
from annc_amd import device as dev
from annc_amd.rec_graph import CapturedGraph, MLPTower, WideDeepConfig, WideDeepGraph
from oracle import ora
from tests.gpu_util import assert_gemm_close, device, gemm_bound, note, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_config1_matmul_add_relu_custom_call_host_and_device():
    note("config1 __matmul_add_relu")
    w = workloads.config1(seed=0)
    ref = ora.matmul_add_relu(w.e, w.a, w.b)
    bound = gemm_bound(w.a, w.b, w.e)
    out = np.empty_like(ref)
    xla.matmul_add_relu(w.z, w.e, w.a, w.b, out)  # host pointers: staged
    assert_gemm_close(out, ref, bound)
    assert (out >= 0).all()
    d = [to_dev(x) for x in (w.z, w.e, w.a, w.b)]
    dout = torch.empty(ref.shape, dtype=torch.float32, device=device())
    xla.matmul_add_relu(*d, dout)  # device pointers: in place
    assert_gemm_close(to_host(dout), ref, bound)


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_config1_seeds(seed):
    note(f"config1 seed {seed}")
    w = workloads.config1(seed=seed)
    out = np.empty((512, 256), np.float32)
    xla.matmul_add_relu(w.z, w.e, w.a, w.b, out)
    assert_gemm_close(out, ora.matmul_add_relu(w.e, w.a, w.b), gemm_bound(w.a, w.b, w.e))


SHAPES = [(512, 256, 256), (1, 1, 1), (33, 65, 17), (64, 128, 32), (100, 300, 845),
          (4096, 512, 1024), (257, 129, 63), (5, 700, 3), (128, 128, 1), (96, 40, 1000),
          (4096, 1, 256), (7, 3, 50)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_matmul_and_matmul_add(m, n, k):
    note(f"__matmul/__matmul_add {m}x{n}x{k}")
    g = workloads.rng(m + n + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    b = g.standard_normal((k, n)).astype(np.float32)
    e = g.standard_normal((m, n)).astype(np.float32)
    out = np.empty((m, n), np.float32)
    xla.matmul(a, b, out)
    assert_gemm_close(out, ora.matmul(a, b), gemm_bound(a, b))
    xla.matmul_add(e, a, b, out)
    assert_gemm_close(out, ora.matmul_add(e, a, b), gemm_bound(a, b, e))


@pytest.mark.parametrize("m,n,k", [(512, 256, 256), (4096, 512, 1024), (100, 300, 845),
                                   (64, 96, 31), (40, 33, 12), (300, 20, 64)])
def test_layout_matmul_packed(m, n, k):
    note(f"__layout_matmul {m}x{n}x{k}")
    g = workloads.rng(m * 7 + n)
    a = g.standard_normal((m, k)).astype(np.float32)
    w = g.standard_normal((k, n)).astype(np.float32)
    packed = dev.pack_weight_host(w)
    ref = ora.matmul(a, w)
    out = np.empty((m, n), np.float32)
    xla.layout_matmul(a, packed, k, n, out)
    assert_gemm_close(out, ref, gemm_bound(a, w))
    # device packer produces the same bytes
    pw = dev.pack_weight(to_dev(w))
    np.testing.assert_array_equal(to_host(pw.data), packed)
    got = dev.gemm(to_dev(a), pw)
    assert_gemm_close(to_host(got), ref, gemm_bound(a, w))


# Packed B with N % 32 == 0 runs the LDS-DMA pipelined kernel: each of its
# tile configurations (256x128, 128x128, 128x64 in 4 or 3 stages, 64x64,
# chosen from the tile area the busiest CU computes, and K; 64x32 is covered
# by test_packed_mid_batches), partial M and N tiles, a K tail with and
# without full k-blocks, padded lda, addend and sigmoid; A rows that are not 16-byte
# aligned (lda % 4 != 0) take the 4-byte DMA variant.
PIPE_CASES = [
    (4096, 1024, 845, 845, "128x128 tiles, unaligned A rows (4-byte DMA)"),
    (4096, 512, 1023, 1023, "128x64 tiles, unaligned A rows"),
    (4096, 256, 510, 510, "64x64 split-K tiles, unaligned A rows"),
    (1000, 96, 845, 845, "partial tiles and K tail, unaligned A rows"),
    (130, 64, 96, 97, "3 k-blocks, lda % 4 == 1"),
    (4096, 1024, 864, 864, "128x128 tiles"),
    (4096, 512, 1024, 1024, "128x64 tiles"),
    (4096, 256, 512, 516, "64x64 tiles, padded lda"),
    (1000, 96, 845, 848, "partial M tile, partial N tile, K tail after 26 k-blocks"),
    (65, 32, 31, 32, "K < 32: tail only"),
    (33, 160, 64, 64, "2 k-blocks"),
    (130, 64, 96, 100, "3 k-blocks (one full pipeline round), lda not a multiple of 32"),
    (7, 64, 300, 300, "tiny M"),
    # few k-blocks in each tile class: the prologue and the mid-stage waits
    # of the 4- and 3-stage pipelines
    (4096, 1024, 40, 40, "128x64 tiles, two per CU (3 stages), 1 k-block + tail"),
    (4096, 1024, 97, 97, "128x64 3-stage tiles, unaligned A, 3 k-blocks + tail"),
    (4096, 1024, 128, 128, "128x64 3-stage tiles, 4 k-blocks"),
    (4096, 1024, 544, 544, "128x128 tiles (K > 512), 17 k-blocks"),
    (4096, 512, 160, 160, "128x64 tiles, 5 k-blocks"),
    (4096, 512, 64, 67, "128x64 tiles, 2 k-blocks, unaligned A"),
    (4096, 256, 224, 224, "64x64 split-K tiles, 7 k-blocks"),
    (8192, 1024, 845, 845, "256x128 tiles, unaligned A rows (4-byte DMA), K tail"),
    (8192, 1024, 1024, 1028, "256x128 tiles, padded lda"),
    (8192, 1024, 544, 544, "256x128 tiles, 17 k-blocks"),
]


@pytest.mark.parametrize("m,n,k,lda,what", PIPE_CASES)
def test_layout_matmul_pipeline_edges(m, n, k, lda, what):
    note(f"packed pipeline {m}x{n}x{k} lda={lda}: {what}")
    g = workloads.rng(m + 3 * n + 7 * k)
    buf = g.standard_normal((m, lda)).astype(np.float32)
    a = np.ascontiguousarray(buf[:, :k])
    w = (g.standard_normal((k, n)) * 0.05).astype(np.float32)
    bias = g.standard_normal(n).astype(np.float32)
    e = g.standard_normal((m, n)).astype(np.float32)
    pw = dev.pack_weight(to_dev(w))
    da = to_dev(buf)[:, :k]
    ref = ora.dense_layer(a, w, bias, 1)
    got = to_host(dev.gemm(da, pw, bias=to_dev(bias), epilogue=EPI_RELU))
    assert_gemm_close(got, ref, gemm_bound(a, w, np.broadcast_to(bias, (m, n))))
    # addend instead of bias, sigmoid epilogue
    got = to_host(dev.gemm(da, pw, addend=to_dev(e), epilogue=EPI_SIGMOID))
    lin = ora.matmul_add(e, a, w)
    np.testing.assert_allclose(got, 1.0 / (1.0 + np.exp(-lin.astype(np.float64))), rtol=1e-4,
                               atol=1e-5)
    # the same numbers through the XLA custom call with host buffers
    out = np.empty((m, n), np.float32)
    xla.layout_matmul(a, dev.pack_weight_host(w), k, n, out)
    assert_gemm_close(out, ora.matmul(a, w), gemm_bound(a, w))


@pytest.mark.parametrize("batch,m,n,k", [(3, 40, 50, 60), (8, 64, 64, 64), (2, 8, 8, 8),
                                         (5, 100, 13, 200)])
def test_batch_matmul(batch, m, n, k):
    note(f"__batch_matmul {batch}x{m}x{n}x{k}")
    g = workloads.rng(batch * m)
    a = g.standard_normal((batch, m, k)).astype(np.float32)
    b = g.standard_normal((batch, k, n)).astype(np.float32)
    out = np.empty((batch, m, n), np.float32)
    xla.batch_matmul(a, b, out)
    ref = ora.batch_matmul(a, b)
    for i in range(batch):
        assert_gemm_close(out[i], ref[i], gemm_bound(a[i], b[i]))


# N <= 4 runs the 16-lanes-per-row kernel: float4 loads of A and of the dense
# [K, N] B block when both are aligned (four chunks at a time while k + 195 < K,
# then single chunks), scalar loads otherwise; rows past M are clamped.
SKINNY_CASES = [
    (1, 4096, 1, 256, "tower scoring layer"),
    (1, 257, 4, 1000, "K with unrolled, single and tail chunks"),
    (1, 5, 4, 196, "K at the unrolled-loop boundary"),
    (1, 1000, 3, 130, "lda % 4 != 0: scalar path"),
    (1, 33, 2, 7, "tiny K"),
    (1, 64, 1, 1, "K = 1"),
    (3, 100, 2, 300, "batched A and B"),
]


@pytest.mark.parametrize("batch,m,n,k,what", SKINNY_CASES)
@pytest.mark.parametrize("layout", ["dense", "ldb>n", "a offset"])
def test_skinny_n(batch, m, n, k, what, layout):
    note(f"skinny-N gemm {batch}x{m}x{n}x{k} {layout}: {what}")
    g = workloads.rng(batch * m + 11 * n + k)
    a = g.standard_normal((batch, m, k)).astype(np.float32)
    b = (g.standard_normal((batch, k, n)) * 0.1).astype(np.float32)
    e = g.standard_normal((batch, m, n)).astype(np.float32)
    bias = g.standard_normal(n).astype(np.float32)
    if layout == "ldb>n":  # B as the first n columns of a wider matrix
        wide = to_dev(np.concatenate([b, np.ones((batch, k, 3), np.float32)], axis=2))
        db = wide[:, :, :n]
    else:
        db = to_dev(b)
    if layout == "a offset":  # A rows start 4 bytes past an aligned address
        flat = torch.zeros(batch * m * k + 1, dtype=torch.float32, device=device())
        flat[1:] = to_dev(a).reshape(-1)
        da = flat[1:].view(batch, m, k)
    else:
        da = to_dev(a)
    if batch == 1:
        da, db = da[0], db[0]
    got = to_host(dev.gemm(da, db, bias=to_dev(bias), epilogue=EPI_RELU)).reshape(batch, m, n)
    for z in range(batch):
        ref = ora.dense_layer(a[z], b[z], bias, 1)
        assert_gemm_close(got[z], ref, gemm_bound(a[z], b[z], np.broadcast_to(bias, (m, n))))
    de = to_dev(e) if batch > 1 else to_dev(e[0])
    got = to_host(dev.gemm(da, db, addend=de, epilogue=EPI_SIGMOID)).reshape(batch, m, n)
    for z in range(batch):
        lin = ora.matmul_add(e[z], a[z], b[z]).astype(np.float64)
        np.testing.assert_allclose(got[z], 1.0 / (1.0 + np.exp(-lin)), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("epi", [EPI_NONE, EPI_RELU, EPI_SIGMOID])
@pytest.mark.parametrize("packed", [False, True])
def test_bias_epilogues_and_padded_lda(epi, packed):
    note(f"epilogue {epi} packed={packed}")
    g = workloads.rng(epi * 2 + packed)
    m, k, n, ld = 300, 845, 200, 848
    buf = g.standard_normal((m, ld)).astype(np.float32)
    a = buf[:, :k]
    w = g.standard_normal((k, n)).astype(np.float32) * np.float32(0.05)
    bias = g.standard_normal(n).astype(np.float32)
    act = {EPI_NONE: 0, EPI_RELU: 1, EPI_SIGMOID: 2}[epi]
    ref = ora.dense_layer(np.ascontiguousarray(a), w, bias, act)
    wt = dev.pack_weight(to_dev(w)) if packed else to_dev(w)
    got = to_host(dev.gemm(to_dev(buf)[:, :k], wt, bias=to_dev(bias), epilogue=epi))
    bound = gemm_bound(a, w, np.broadcast_to(bias, (m, n)))
    if epi == EPI_SIGMOID:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        assert_gemm_close(got, ref, bound)


def test_relu_propagates_nan_and_clamps():
    note("relu semantics")
    a = np.zeros((32, 32), np.float32)
    a[0, 0] = np.nan
    b = np.eye(32, dtype=np.float32)
    e = np.zeros((32, 32), np.float32)
    e[1, 1] = -0.0
    e[2, 2] = -3.0
    out = np.empty((32, 32), np.float32)
    xla.matmul_add_relu(np.zeros_like(e), e, a, b, out)
    assert np.isnan(out[0, 0])  # std::max(NaN, 0.f) returns NaN
    assert out[2, 2] == 0.0


def _check_tower_layers(tower, x_host, hidden, y, weights, biases, lda=None):
    """Each layer against the oracle fed with the GPU's previous layer: the
    ReLU layers at the GEMM bound, the sigmoid head at rtol 1e-4."""
    h = x_host
    outs = list(hidden) + [y]
    for i in range(len(weights)):
        out = outs[i]
        act = 2 if i == len(weights) - 1 else 1
        ref = ora.dense_layer(h, weights[i], biases[i], act)
        note(f"  layer {i + 1}: [{h.shape[0]}x{h.shape[1]}] . [{weights[i].shape[0]}x"
             f"{weights[i].shape[1]}] act {act}")
        if act == 2:
            np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-6)
        else:
            assert_gemm_close(out, ref, gemm_bound(h, weights[i],
                                                   np.broadcast_to(biases[i], ref.shape)))
        h = out


def test_config2_mlp_tower():
    """The configs[1] tower as the benchmark runs it (layer 1 as a GEMM, layers
    2 and 3 as one dense_score kernel) and with every layer a GEMM launch:
    each layer against the oracle, the fused tail's hidden layer stored or
    not giving the same bits."""
    note("config2 MLP tower")
    w = workloads.config2(seed=0)
    x = to_dev(w.x)
    ref = ora.mlp_tower(w.x, w.weights, w.biases)
    ys = {}
    for fuse in (True, False):
        tower = MLPTower(w.weights, w.biases, device=device(), packed=True, fuse_score=fuse,
                         keep_hidden=True)
        assert tower.fused_tail == fuse
        ys[fuse] = to_host(tower(x)).copy()
        bufs = [to_host(b) for b in tower.buffers(x.shape[0])]
        _check_tower_layers(tower, w.x, bufs[:-1], bufs[-1], w.weights, w.biases)
        np.testing.assert_allclose(ys[fuse], ref, rtol=1e-3, atol=1e-5)
    bench_tower = MLPTower(w.weights, w.biases, device=device(), packed=True)
    assert bench_tower.fused_tail and not bench_tower.keep_hidden
    np.testing.assert_array_equal(to_host(bench_tower(x)), ys[True])


@pytest.mark.parametrize("batch", [64, 1024, 2048, 2049])
def test_tower_fuses_its_tail_above_2048_rows(batch):
    """configs[1]'s tower runs its 512 -> 256 -> 1 tail as two GEMM launches
    up to 2048 rows (where the small-batch GEMM kernels beat the fused
    kernel) and as one dense_score launch above: the hidden layer reaches its
    buffer only on the first path (keep_hidden off).  Both against the
    oracle."""
    note(f"config2 tower tail path at batch {batch}")
    w = workloads.config2(seed=3, batch=batch)
    tower = MLPTower(w.weights, w.biases, device=device(), packed=True)
    assert tower.fused_tail
    bufs = tower.buffers(batch)
    bufs[-2].fill_(float("nan"))
    y = to_host(tower(to_dev(w.x)))
    np.testing.assert_allclose(y, ora.mlp_tower(w.x, w.weights, w.biases), rtol=1e-3, atol=1e-5)
    hidden = to_host(bufs[-2])
    if batch >= 2049:
        assert np.isnan(hidden).all()
    else:
        assert np.isfinite(hidden).all()


@pytest.mark.parametrize("widths,offset", [((512, 256, 1), 1), ((512, 256, 1), 4), ((512, 96, 1), 0)])
def test_tower_tail_fallbacks(widths, offset):
    """Towers whose tail the fused kernel does not take run it as two GEMM
    launches: an input whose rows are not 16-byte aligned (column offset 1)
    and a hidden width outside 64/128/256; an aligned offset (4) keeps the
    fused kernel.  Each against the oracle."""
    note(f"tower {widths}, input column offset {offset}")
    g = workloads.rng(sum(widths) + offset)
    m = 300
    ws = [workloads.glorot_uniform(g, a, b) for a, b in zip(widths[:-1], widths[1:])]
    bs = [(g.standard_normal(b) * 0.01).astype(np.float32) for b in widths[1:]]
    xbuf = g.standard_normal((m, widths[0] + 8)).astype(np.float32)
    x = xbuf[:, offset:offset + widths[0]]
    tower = MLPTower(ws, bs, device=device(), packed=True, fuse_min_rows=1)
    assert tower.fused_tail == (widths[1] in (64, 128, 256))
    y = to_host(tower(to_dev(xbuf)[:, offset:offset + widths[0]]))
    np.testing.assert_allclose(y, ora.mlp_tower(np.ascontiguousarray(x), ws, bs), rtol=1e-4,
                               atol=1e-6)


@pytest.mark.parametrize("fuse", [True, False])
def test_config2_tower_graph_replays(fuse):
    """The benchmark's graph form of the tower: a captured forward replayed
    three times, with eager forwards of other inputs and synchronisations
    between the replays, gives the eager result bit for bit every time."""
    note(f"config2 tower as a HIP graph, fused tail {fuse}")
    w = workloads.config2(seed=0)
    tower = MLPTower(w.weights, w.biases, device=device(), packed=True, fuse_score=fuse)
    x = to_dev(w.x)
    eager = to_host(tower(x)).copy()
    graph = CapturedGraph(tower, x)
    other = to_dev(workloads.config2(seed=1).x)
    for r in range(3):
        y = to_host(graph.replay()).copy()
        np.testing.assert_array_equal(y, eager, err_msg=f"replay {r}")
        y_other = to_host(tower(other)).copy()  # eager work on the same buffers
        assert not np.array_equal(y_other, eager)
        torch.cuda.synchronize()


@pytest.mark.parametrize("batch_rows", [1, 64])
def test_small_batch_tower_graph_replays(batch_rows):
    """A small-batch tower with a long-K first layer (4096 -> 1024, K split
    across workgroups and reduced in a second launch) and the unfused tail,
    captured into a HIP graph: three replays, each after new inputs were
    copied into the captured input buffer and after eager forwards of other
    inputs on the same buffers, each equal to an eager forward of the same
    input and within the oracle's tolerance."""
    note(f"small-batch tower graph, {batch_rows} rows")
    widths = (4096, 1024, 256, 1)
    g = workloads.rng(batch_rows + 11)
    ws = [workloads.glorot_uniform(g, a, b) for a, b in zip(widths[:-1], widths[1:])]
    bs = [(g.standard_normal(b) * 0.01).astype(np.float32) for b in widths[1:]]
    tower = MLPTower(ws, bs, device=device(), packed=True)
    xs = [g.standard_normal((batch_rows, widths[0])).astype(np.float32) for _ in range(4)]
    x = to_dev(xs[0])
    graph = CapturedGraph(tower, x)
    for r in range(1, 4):
        x.copy_(to_dev(xs[r]))
        y = to_host(graph.replay()).copy()
        torch.cuda.synchronize()
        eager = to_host(tower(to_dev(xs[r]))).copy()
        np.testing.assert_array_equal(y, eager, err_msg=f"replay {r}")
        np.testing.assert_allclose(y, ora.mlp_tower(xs[r], ws, bs), rtol=1e-3, atol=1e-5)
        to_host(tower(to_dev(xs[(r + 1) % 4])))  # eager work on the same buffers
        torch.cuda.synchronize()


@pytest.mark.parametrize("m,n,k,ldb_pad", [(1, 1024, 4096, 0), (4096, 512, 256, 1)])
def test_gemm_captured_without_warm_up(m, n, k, ldb_pad):
    """GEMMs that use the per-stream workspace (a K-split small product, a
    row-major B with unaligned rows) captured on a fresh stream with no call
    before: no allocation happens under capture (the library takes a path
    without workspace), and the replays give the oracle's result."""
    note(f"GEMM captured without warm-up {m}x{n}x{k} ldb+{ldb_pad}")
    g = workloads.rng(m + n + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    wide = (g.standard_normal((k, n + ldb_pad)) / np.sqrt(k)).astype(np.float32)
    w = np.ascontiguousarray(wide[:, :n])
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    da, dbias = to_dev(a), to_dev(bias)
    b = to_dev(wide)[:, :n] if ldb_pad else dev.pack_weight(to_dev(w))
    out = torch.empty((m, n), dtype=torch.float32, device=device())
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        dev.gemm(da, b, bias=dbias, epilogue=EPI_RELU, out=out)
    ref = ora.dense_layer(a, w, bias, 1)
    for _ in range(2):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert_gemm_close(to_host(out), ref, gemm_bound(a, w, np.broadcast_to(bias, ref.shape)))


def test_graph_replays_after_the_workspace_grows():
    """A GEMM that packs unaligned B rows into the workspace, captured after a
    warm-up on the capture stream; eager calls of the same thread on that
    stream then need a larger workspace (it grows; the outgrown one, which
    the graph holds, is kept): later replays equal the first bit for bit and
    stay within the GEMM bound."""
    note("graph replay after the workspace grows")
    g = workloads.rng(77)
    m, n, k = 600, 1024, 512
    a = g.standard_normal((m, k)).astype(np.float32)
    wide = (g.standard_normal((k, n + 1)) / np.sqrt(k)).astype(np.float32)
    w = np.ascontiguousarray(wide[:, :n])
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    da, db, dbias = to_dev(a), to_dev(wide)[:, :n], to_dev(bias)
    out = torch.empty((m, n), dtype=torch.float32, device=device())
    graph = CapturedGraph(lambda: dev.gemm(da, db, bias=dbias, epilogue=EPI_RELU, out=out))
    first = to_host(graph.replay()).copy()
    ref = ora.dense_layer(a, w, bias, 1)
    assert_gemm_close(first, ref, gemm_bound(a, w, np.broadcast_to(bias, ref.shape)))
    big_k = 4096
    a2 = g.standard_normal((m, big_k)).astype(np.float32)
    wide2 = (g.standard_normal((big_k, 2 * n + 1)) / np.sqrt(big_k)).astype(np.float32)
    with torch.cuda.stream(graph.stream):
        big = dev.gemm(to_dev(a2), to_dev(wide2)[:, :2 * n])
    torch.cuda.synchronize()
    assert_gemm_close(to_host(big), ora.matmul(a2, np.ascontiguousarray(wide2[:, :2 * n])),
                      gemm_bound(a2, wide2[:, :2 * n]))
    for _ in range(3):
        out.zero_()
        np.testing.assert_array_equal(to_host(graph.replay()), first)


def test_workspace_calls_from_two_threads_on_one_stream():
    """Two threads enqueue workspace-using calls (per-call packing of
    unaligned B rows, K split, the any-order segment reduction) on one stream
    at once, each in its own order, so their launches interleave and each
    thread's workspace grows meanwhile: every result equals the same call's
    single-threaded result bit for bit."""
    import threading
    note("workspace calls from two threads on one stream")
    g = workloads.rng(78)
    stream = torch.cuda.Stream()
    calls = []
    for m, n, k, pad in [(600, 2048, 1024, 1), (1, 1024, 4096, 0), (300, 1000, 2100, 3),
                         (64, 512, 4096, 0), (600, 2048, 2048, 1)]:
        a = to_dev(g.standard_normal((m, k)).astype(np.float32))
        b = to_dev((g.standard_normal((k, n + pad)) / np.sqrt(k)).astype(np.float32))[:, :n]
        calls.append(lambda a=a, b=b: dev.gemm(a, b, epilogue=EPI_RELU))
    table = to_dev(g.standard_normal((100_000, 64)).astype(np.float32))
    idx = to_dev(g.integers(0, 100_000, size=80_000).astype(np.int64))
    seg = to_dev(g.permutation(np.repeat(np.arange(4096), 20)[:80_000]).astype(np.int64))
    calls.append(lambda: dev.segment_reduce(table, idx, seg, 4096, 1))
    with torch.cuda.stream(stream):
        expected = [to_host(c()).copy() for c in calls]
    got = {0: [], 1: []}
    errors = []

    def run(t):
        try:
            order = list(range(len(calls)))
            if t:
                order.reverse()
            with torch.cuda.stream(stream):
                for _ in range(4):
                    for i in order:
                        got[t].append((i, calls[i]()))
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(t,)) for t in (0, 1)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    torch.cuda.synchronize()
    for t in (0, 1):
        assert len(got[t]) == 4 * len(calls)
        for i, y in got[t]:
            np.testing.assert_array_equal(to_host(y), expected[i], err_msg=f"thread {t} call {i}")


def test_config5_wide_deep_graph():
    note("config5 wide&deep")
    w = workloads.config5(seed=0)
    h = w.hashed
    cfg = WideDeepConfig()
    graph = WideDeepGraph(cfg, [to_dev(t) for t in h.tables], w.weights, w.biases, device=device())
    assert graph.tower.fused_tail  # 512 -> 256 -> 1 as one dense_score kernel
    graph.tower.keep_hidden = True  # the 256-wide layer stored too, for the per-layer check
    y = to_host(graph(to_dev(h.ids), to_dev(h.offsets), to_dev(w.dense))).copy()
    emb = ora.hashed_embedding_bags(h.tables, h.num_buckets, h.ids, h.offsets, h.batch, 1, threads=8)
    x = np.concatenate([emb, w.dense], axis=1)
    concat = to_host(graph.concat_buffer(h.batch))[:, :x.shape[1]]
    np.testing.assert_array_equal(concat, x)  # embeddings bit-exact, dense copied
    # the four GEMM layers at full size, each against the oracle fed with the
    # GPU's previous layer: 4096x845 (concat rows, padded to 864 with zero columns and zero weight rows) -> 1024 -> 512
    # -> 256 at the GEMM bound, then the 256 -> 1 sigmoid head
    bufs = [to_host(b) for b in graph.tower.buffers(h.batch)]
    _check_tower_layers(graph.tower, x, bufs[:-1], bufs[-1], w.weights, w.biases)
    np.testing.assert_allclose(y, ora.mlp_tower(x, w.weights, w.biases), rtol=1e-3, atol=1e-5)
    # dense features written straight into the concat buffer: same result, no copy
    graph.concat_buffer(h.batch).zero_()
    view = graph.dense_view(h.batch)
    view.copy_(to_dev(w.dense))
    y2 = to_host(graph(to_dev(h.ids), to_dev(h.offsets), view))
    np.testing.assert_array_equal(to_host(graph.concat_buffer(h.batch))[:, :x.shape[1]], x)
    np.testing.assert_array_equal(y2, y)
    # as served: the fused tail without the hidden store, same bits
    graph.tower.keep_hidden = False
    y3 = to_host(graph(to_dev(h.ids), to_dev(h.offsets), view))
    np.testing.assert_array_equal(y3, y)


DENSE_SCORE_CASES = [
    # m, k, n, hidden epilogue, score epilogue, biases
    (4096, 512, 256, 1, 2, True),    # configs[1] / configs[4] tail
    (1000, 256, 256, 1, 2, True),    # one round, partial last workgroup
    (4099, 2048, 256, 1, 2, True),   # largest K, 8 rounds
    (17, 512, 128, 2, 0, False),     # 8 waves, no biases, sigmoid hidden
    (300, 1024, 64, 0, 1, True),     # 4 waves, 16 rounds
    (1, 64, 64, 1, 2, True),         # one row
    (4096, 768, 256, 1, 2, True),    # 3 rounds: rotation by 0, 1, 2
    (128, 2048, 64, 1, 2, True),     # 4 waves, 32 rounds, largest K
    (200, 1024, 128, 1, 2, False),   # 8 waves, 8 rounds
    (64, 1536, 128, 1, 0, True),     # 8 waves, 12 rounds (K buffer of 2048)
]


@pytest.mark.parametrize("m,k,n,epi,sepi,with_bias", DENSE_SCORE_CASES)
def test_dense_score(m, k, n, epi, sepi, with_bias):
    """annc_hip_dense_score: the hidden layer against the oracle's sgemm
    (GEMM bound), the score against the oracle's dense layer fed with the
    GPU's hidden layer (rtol 1e-4); the score is the same bits with and
    without the hidden store and with a strided output column."""
    note(f"dense_score {m}x{k} . [{k}x{n}] epi {epi} -> [{n}x1] epi {sepi} bias {with_bias}")
    g = workloads.rng(m + 7 * k + n)
    a = np.maximum(g.standard_normal((m, k)), 0).astype(np.float32)
    w = (g.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    ws = (g.standard_normal((n, 1)) / np.sqrt(n)).astype(np.float32)
    b = (g.standard_normal(n) * 0.1).astype(np.float32) if with_bias else None
    bs = np.array([0.25], dtype=np.float32) if with_bias else None
    pw = dev.pack_weight(to_dev(w))
    hid_buf = torch.full((m, n + 8), float("nan"), device=device())  # ldh = n + 8
    hid = hid_buf[:, :n]
    out = torch.full((m, 1), float("nan"), device=device())
    dev.dense_score(to_dev(a), pw, to_dev(ws), bias=None if b is None else to_dev(b),
                    epilogue=epi, score_bias=None if bs is None else to_dev(bs),
                    score_epilogue=sepi, hidden=hid, out=out)
    h = to_host(hid).copy()
    assert np.isnan(to_host(hid_buf)[:, n:]).all()  # the row padding is not written
    href = ora.dense_layer(a, w, b, epi)
    bias_e = None if b is None else np.broadcast_to(b, href.shape)
    assert_gemm_close(h, href, gemm_bound(a, w, bias_e))
    y = to_host(out).copy()
    np.testing.assert_allclose(y, ora.dense_layer(h, ws, bs, sepi), rtol=1e-4, atol=1e-6)
    wide = torch.full((m, 3), float("nan"), device=device())
    dev.dense_score(to_dev(a), pw, to_dev(ws), bias=None if b is None else to_dev(b),
                    epilogue=epi, score_bias=None if bs is None else to_dev(bs),
                    score_epilogue=sepi, out=wide[:, 1:2])
    cols = to_host(wide)
    np.testing.assert_array_equal(cols[:, 1:2], y)
    assert np.isnan(cols[:, 0]).all() and np.isnan(cols[:, 2]).all()


def test_dense_score_consecutive_calls_of_different_sizes():
    """Two calls in a row on one stream, the second smaller: nothing carries
    over between launches (the kernel keeps no state outside its LDS)."""
    note("dense_score 4096 then 40 rows")
    g = workloads.rng(11)
    w = (g.standard_normal((512, 256)) / 23.0).astype(np.float32)
    ws = (g.standard_normal((256, 1)) / 16.0).astype(np.float32)
    pw = dev.pack_weight(to_dev(w))
    for m in (4096, 40):
        a = np.maximum(g.standard_normal((m, 512)), 0).astype(np.float32)
        y = to_host(dev.dense_score(to_dev(a), pw, to_dev(ws)))
        h = np.maximum(ora.dense_layer(a, w, None, 0), 0)
        np.testing.assert_allclose(y, ora.dense_layer(h, ws, None, 2), rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("pipe", ["mi16", "mi16w8"])
@pytest.mark.parametrize("m,n,k", [(4096, 512, 1024), (4096, 256, 512), (100, 96, 64),
                                   (257, 160, 256), (4100, 64, 32)])
def test_packed_gemm_16x16_blocks(pipe, m, n, k, monkeypatch):
    """The 16x16-block forms of the packed pipeline (ANNC_GEMM_PIPE): k fed
    as 4*(lane/16) + step from the 32x32 stage layouts, 16x16 accumulator
    map in the epilogue; within the GEMM bound of OpenBLAS, edge tiles
    included."""
    note(f"packed GEMM, ANNC_GEMM_PIPE={pipe}, {m}x{n}x{k}")
    g = workloads.rng(m + 3 * n + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    b = (g.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    pw = dev.pack_weight(to_dev(b))
    monkeypatch.setenv("ANNC_GEMM_PIPE", pipe)
    out = to_host(dev.gemm(to_dev(a), pw, bias=to_dev(bias), epilogue=EPI_RELU))
    ref = ora.dense_layer(a, b, bias, 1)
    assert_gemm_close(out, ref, gemm_bound(a, b, np.broadcast_to(bias, ref.shape)))


# ---------------------------------------------------------------- KPFusedBatchMatMulAddSigmoid
import json  # noqa: E402
import os  # noqa: E402

from annc_amd import tf_ops  # noqa: E402
from tests.test_oracle import BMS_GOLD, bms_inputs  # noqa: E402


@pytest.mark.parametrize("case", BMS_GOLD["cases"], ids=lambda c: c["name"])
@pytest.mark.parametrize("where", ["host", "device"])
def test_batch_matmul_add_sigmoid_reference_cases(case, where):
    note(f"KPFusedBatchMatMulAddSigmoid {case['name']} ({where})")
    lhs, rhs, bias = bms_inputs(case)
    ref = ora.batch_matmul_add_sigmoid(lhs, rhs, bias)
    args = (lhs, rhs, bias) if where == "host" else tuple(to_dev(x) for x in (lhs, rhs, bias))
    got = tf_ops.kp_fused_batch_matmul_add_sigmoid(*args)
    got = got if where == "host" else to_host(got)
    np.testing.assert_allclose(got, ref, rtol=0, atol=BMS_GOLD["tolerance"])


@pytest.mark.parametrize("bias_shape", [(64,), (1, 64), (300, 64), (7, 1, 64), (7, 300, 64),
                                        (7, 300, 1), (1,), ()])
@pytest.mark.parametrize("rhs_batched", [False, True])
def test_batch_matmul_add_sigmoid_broadcasts(bias_shape, rhs_batched):
    note(f"KPFusedBatchMatMulAddSigmoid bias {bias_shape} rhs_batched={rhs_batched}")
    g = workloads.rng(len(bias_shape) * 2 + rhs_batched)
    b, m, k, n = 7, 300, 96, 64
    lhs = (g.standard_normal((b, m, k)) * 0.1).astype(np.float32)
    rhs = (g.standard_normal((b, k, n) if rhs_batched else (k, n)) * 0.1).astype(np.float32)
    bias = g.standard_normal(bias_shape).astype(np.float32)
    ref = ora.batch_matmul_add_sigmoid(lhs, rhs, bias)
    got = tf_ops.kp_fused_batch_matmul_add_sigmoid(lhs, rhs, bias)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5)


# (each shape has n % 32 == 0 and at least 128 64x64 tiles, the condition for
# the pipelined kernel.  Rows of B that are 16-byte aligned (n + ldb_pad a
# multiple of 4) are read in place; the others need m >= 512 and are packed
# per call, the packer grouping 1, 2 or 4 n-panels per workgroup by grid size:
# (1, 8192, 64, 33, 7) takes 1 and (70, 512, 224, 64, 3) 2 with a remainder
# group.  The tile rule gives 64x64, 128x64 in 4 and 3 stages, and a grid of
# 1.25 CU rounds among these shapes.)
@pytest.mark.parametrize("batch,m,n,k,ldb_pad", [(1, 2048, 320, 845, 80), (1, 4096, 512, 1024, 0),
                                                 (3, 1024, 256, 200, 0), (1, 8192, 64, 33, 7),
                                                 (2, 4000, 96, 64, 32), (32, 512, 256, 256, 0),
                                                 (64, 512, 160, 101, 4), (70, 512, 224, 64, 3),
                                                 (64, 256, 128, 256, 0), (4, 2048, 320, 845, 0),
                                                 (2, 4096, 1024, 1024, 0), (1, 8192, 1024, 845, 3),
                                                 (3, 40, 64, 96, 0), (4, 33, 96, 845, 5),
                                                 (1, 500, 2048, 1024, 1), (2, 256, 2048, 512, 3)])
def test_row_major_b_packed_per_call(batch, m, n, k, ldb_pad):
    """Large row-major-B GEMMs run the pipelined kernel, on B read in place or
    packed into the stream workspace: within tolerance of OpenBLAS, and
    bit-identical to the same GEMM on weights packed ahead of time (so the
    in-place reads and the per-call packing both equal the layout_matmul
    packer, K tails and strided B included, and the pipelined kernel ran).
    Batches of at most 256 32x32 blocks run the small kernel on both forms
    (batched packed B included), bit-identical likewise."""
    note(f"row-major B packed per call b={batch} {m}x{n}x{k} ldb+{ldb_pad}")
    g = workloads.rng(m + n + k + batch)
    a = g.standard_normal((batch, m, k)).astype(np.float32)
    wide = (g.standard_normal((batch, k, n + ldb_pad)) * 0.05).astype(np.float32)
    b = wide[:, :, :n]
    e = g.standard_normal((batch, m, n)).astype(np.float32)
    da, de = to_dev(a), to_dev(e)
    db = to_dev(wide)[:, :, :n]
    if batch == 1:
        got = to_host(dev.gemm(da[0], db[0], addend=de[0], epilogue=EPI_RELU))[None]
    else:
        got = to_host(dev.gemm(da, db, addend=de, epilogue=EPI_RELU))
    packed = [dev.pack_weight(to_dev(b[z])).data for z in range(batch)]
    if batch == 1:
        pre = to_host(dev.gemm(da[0], dev.PackedWeight(packed[0], k, n), addend=de[0],
                               epilogue=EPI_RELU))[None]
    else:  # one batched call over the concatenated packed weights: same tile class
        pre_d = torch.empty((batch, m, n), dtype=torch.float32, device=device())
        _lib.check(_lib.lib().annc_hip_gemm(
            _lib.stream_ptr(), batch, m, n, k, _lib.ptr(da), k, m * k, _lib.ptr(torch.cat(packed)),
            n, k * n, 1, _lib.ptr(de), n, m * n, None, EPI_RELU, _lib.ptr(pre_d), n, m * n))
        pre = to_host(pre_d)
    for z in range(batch):
        ref = ora.matmul_add_relu(e[z], a[z], np.ascontiguousarray(b[z]))
        assert_gemm_close(got[z], ref, gemm_bound(a[z], b[z], e[z]))
    np.testing.assert_array_equal(got, pre)


@pytest.mark.parametrize("batch,m,n,k", [(1, 1, 512, 1024), (1, 16, 512, 1024), (1, 256, 256, 512),
                                         (1, 100, 96, 64), (1, 33, 256, 845), (1, 7, 32, 20),
                                         (3, 40, 64, 96), (1, 512, 512, 1024), (1, 256, 1000, 1024),
                                         (1, 100, 300, 845), (1, 17, 40, 33), (2, 40, 70, 96),
                                         (1, 4096, 16, 1024), (1, 3000, 24, 100),
                                         (1, 16384, 16, 1024), (1, 65536, 8, 40)])
def test_packed_small_batches(batch, m, n, k):
    """Packed GEMMs with at most one round of 32x32 blocks (small batches)
    run the small kernel: within the GEMM bound of OpenBLAS, and bit-identical
    to the same GEMM on row-major B, which takes the same kernel (K tails,
    K < 32, a partial last panel read from the format's N-tail region, and
    N < 32, where the format is row-major, included)."""
    note(f"packed small batch b={batch} {m}x{n}x{k}")
    g = workloads.rng(7 * m + n + k + batch)
    a = g.standard_normal((batch, m, k)).astype(np.float32)
    b = (g.standard_normal((batch, k, n)) / np.sqrt(k)).astype(np.float32)
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    da, dbias = to_dev(a), to_dev(bias)
    for z in range(batch):
        pw = dev.pack_weight(to_dev(b[z]))
        got = to_host(dev.gemm(da[z], pw, bias=dbias, epilogue=EPI_RELU))
        ref = ora.dense_layer(a[z], b[z], bias, 1)
        assert_gemm_close(got, ref, gemm_bound(a[z], b[z], np.broadcast_to(bias, ref.shape)))
        rm = to_host(dev.gemm(da[z], to_dev(b[z]), bias=dbias, epilogue=EPI_RELU))
        np.testing.assert_array_equal(got, rm)


@pytest.mark.parametrize("m,n,k,col0", [(768, 512, 1024, 0), (1024, 512, 1024, 0),
                                        (3072, 512, 1024, 0), (1536, 1024, 864, 0),
                                        (1200, 256, 100, 0), (1536, 256, 512, 1),
                                        (4000, 288, 845, 3)])
def test_packed_mid_batches(m, n, k, col0):
    """Batches between one round of 32x32 blocks and two rounds of 64x64
    tiles run 64x32 tiles of the pipelined kernel (16- and 4-byte A DMAs, K
    tails): within the GEMM bound of OpenBLAS, and bit-identical to the same
    GEMM on row-major B."""
    note(f"packed mid batch {m}x{n}x{k} col0={col0}")
    g = workloads.rng(5 * m + n + k + col0)
    buf = g.standard_normal((m, k + 4)).astype(np.float32)
    a = np.ascontiguousarray(buf[:, col0:col0 + k])
    b = (g.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    da, dbias = to_dev(buf)[:, col0:col0 + k], to_dev(bias)
    got = to_host(dev.gemm(da, dev.pack_weight(to_dev(b)), bias=dbias, epilogue=EPI_RELU))
    ref = ora.dense_layer(a, b, bias, 1)
    assert_gemm_close(got, ref, gemm_bound(a, b, np.broadcast_to(bias, ref.shape)))
    rm = to_host(dev.gemm(da, to_dev(b), bias=dbias, epilogue=EPI_RELU))
    np.testing.assert_array_equal(got, rm)


# N % 32 != 0 with more than one round of 32x32 blocks in the full panels:
# the pipelined kernel with a partial last panel (packed B, and row-major B
# with 16-byte aligned rows read in place; other row-major B is packed per
# call, tail columns included, and runs as packed B), or, where the extra
# column of tiles costs a CU round, the full panels and then the tail
# columns through the small kernel (N % 32 > 4) or the GEMV kernel.
N_TAIL_CASES = [
    (1, 4096, 1000, 1024, "8 tail columns"),
    (1, 4096, 515, 845, "3 tail columns; row-major rows unaligned (packed per call), K tail"),
    (1, 2048, 300, 845, "12 tail columns, K tail"),
    (3, 1024, 100, 64, "batched, 4 tail columns"),
    (1, 8200, 33, 256, "one full panel, 1 tail column (row-major: packed per call)"),
    (2, 777, 620, 100, "batched, partial M tile, 12 tail columns, K tail"),
    (1, 4096, 1001, 40, "unaligned rows (packed per call), 1 k-block + K tail"),
    (1, 8192, 1000, 864, "256x128 tiles with a partial panel"),
    (1, 1200, 340, 512, "64x32 tiles with a partial panel"),
    (1, 4096, 1000, 20, "K < 32 (K tail only), partial panel"),
    (1, 4096, 521, 1024, "unaligned rows, two launches (a fifth round of tiles)"),
    (2, 2048, 1001, 97, "batched, unaligned rows: K*N odd, batch strides of the per-call pack aligned"),
]


@pytest.mark.parametrize("batch,m,n,k,what", N_TAIL_CASES)
def test_n_tail_split(batch, m, n, k, what):
    """Within the GEMM bound of OpenBLAS with bias and ReLU, and with an
    addend and sigmoid; packed B and row-major B (read in place, or packed
    per call) bit-identical."""
    note(f"N-tail split b={batch} {m}x{n}x{k}: {what}")
    g = workloads.rng(3 * m + n + k + batch)
    a = g.standard_normal((batch, m, k)).astype(np.float32)
    w = (g.standard_normal((batch, k, n)) / np.sqrt(k)).astype(np.float32)
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    e = g.standard_normal((batch, m, n)).astype(np.float32)
    da, dbias, de = to_dev(a), to_dev(bias), to_dev(e)
    for z in range(batch):
        pw = dev.pack_weight(to_dev(w[z]))
        got = to_host(dev.gemm(da[z], pw, bias=dbias, epilogue=EPI_RELU))
        ref = ora.dense_layer(a[z], w[z], bias, 1)
        assert_gemm_close(got, ref, gemm_bound(a[z], w[z], np.broadcast_to(bias, ref.shape)))
        sg = to_host(dev.gemm(da[z], pw, addend=de[z], epilogue=EPI_SIGMOID))
        lin = ora.matmul_add(e[z], a[z], w[z])
        np.testing.assert_allclose(sg, 1.0 / (1.0 + np.exp(-lin.astype(np.float64))), rtol=1e-4,
                                   atol=1e-5)
        if batch == 1:
            rm = to_host(dev.gemm(da[z], to_dev(w[z]), bias=dbias, epilogue=EPI_RELU))
            np.testing.assert_array_equal(got, rm)
    if batch > 1:  # one batched row-major call: the same per-batch results
        got_b = to_host(dev.gemm(da, to_dev(w), bias=dbias, epilogue=EPI_RELU))
        for z in range(batch):
            ref = ora.dense_layer(a[z], w[z], bias, 1)
            assert_gemm_close(got_b[z], ref, gemm_bound(a[z], w[z], np.broadcast_to(bias, ref.shape)))


# 4 < N < 32 with more than one round of 32x32 blocks: 64x32 pipelined tiles
# with one partial panel and no full ones (B by 4-byte DMAs from any ldb);
# also the tail columns of a two-launch GEMM at such M
SKINNY_PIPE_CASES = [
    (1, 16384, 16, 1024, 0, 0, "one round of 64x32 tiles"),
    (1, 9216, 20, 845, 0, 0, "K tail, partial round"),
    (1, 65536, 8, 256, 0, 0, "1024 tiles: several rounds of three a CU"),
    (1, 20000, 31, 100, 0, 0, "partial M tile, K tail"),
    (1, 12000, 7, 300, 0, 0, "ldb = 7 (rows not 16-byte aligned)"),
    (1, 10000, 12, 96, 3, 1, "ldb padded, A from a column offset (4-byte A DMAs)"),
    (3, 4000, 12, 64, 0, 0, "batched: 375 blocks over the batch"),
    (1, 9000, 5, 40, 0, 0, "N = 5, one k-block and a K tail"),
    (1, 16384, 1009, 64, 1, 0, "row-major, unaligned rows: pipelined full panels, tail of 17 columns pipelined"),
]


@pytest.mark.parametrize("batch,m,n,k,ldb_pad,col0,what", SKINNY_PIPE_CASES)
def test_skinny_n_pipelined(batch, m, n, k, ldb_pad, col0, what):
    """Within the GEMM bound of OpenBLAS with bias and ReLU, and with an
    addend and sigmoid; packed B (the format is row-major below 32 columns)
    bit-identical to row-major B."""
    note(f"skinny N pipelined b={batch} {m}x{n}x{k} ldb+{ldb_pad} col0={col0}: {what}")
    g = workloads.rng(5 * m + n + k + batch)
    abuf = g.standard_normal((batch, m, k + col0 + 3)).astype(np.float32)
    a = np.ascontiguousarray(abuf[:, :, col0:col0 + k])
    wide = (g.standard_normal((batch, k, n + ldb_pad)) / np.sqrt(k)).astype(np.float32)
    w = np.ascontiguousarray(wide[:, :, :n])
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    e = g.standard_normal((batch, m, n)).astype(np.float32)
    da = to_dev(abuf)[:, :, col0:col0 + k]
    dw = to_dev(wide)[:, :, :n]
    dbias, de = to_dev(bias), to_dev(e)
    if batch == 1:
        got = to_host(dev.gemm(da[0], dw[0], bias=dbias, epilogue=EPI_RELU))[None]
        sg = to_host(dev.gemm(da[0], dw[0], addend=de[0], epilogue=EPI_SIGMOID))[None]
        if n < 32:
            pk = to_host(dev.gemm(da[0], dev.pack_weight(dw[0]), bias=dbias, epilogue=EPI_RELU))
            np.testing.assert_array_equal(pk, got[0])
    else:
        got = to_host(dev.gemm(da, dw, bias=dbias, epilogue=EPI_RELU))
        sg = to_host(dev.gemm(da, dw, addend=de, epilogue=EPI_SIGMOID))
    for z in range(batch):
        ref = ora.dense_layer(a[z], w[z], bias, 1)
        assert_gemm_close(got[z], ref, gemm_bound(a[z], w[z], np.broadcast_to(bias, ref.shape)))
        lin = ora.matmul_add(e[z], a[z], w[z])
        np.testing.assert_allclose(sg[z], 1.0 / (1.0 + np.exp(-lin.astype(np.float64))),
                                   rtol=1e-4, atol=1e-5)


# Few 32x32 blocks with a long K: K split over up to 8 workgroups, partial sums
# added in split order by a second launch (K tails in the last split)
SPLITK_CASES = [
    (1, 1, 1024, 4096, "8 splits"),
    (1, 64, 512, 4096, "8 splits, 2 row blocks"),
    (1, 16, 512, 1024, "4 splits (few blocks)"),
    (1, 100, 1000, 2100, "partial panel, K tail"),
    (3, 20, 96, 3000, "batched, K tail"),
    (1, 128, 1024, 4096, "2 splits"),
]


@pytest.mark.parametrize("batch,m,n,k,what", SPLITK_CASES)
def test_split_k_small_gemm(batch, m, n, k, what):
    """Within the GEMM bound of OpenBLAS with an addend, bias and ReLU, on
    packed and row-major B (bit-identical: the same kernels), batched through
    one call."""
    note(f"split-K small GEMM b={batch} {m}x{n}x{k}: {what}")
    g = workloads.rng(m + 3 * n + k + batch)
    a = g.standard_normal((batch, m, k)).astype(np.float32)
    w = (g.standard_normal((batch, k, n)) / np.sqrt(k)).astype(np.float32)
    e = g.standard_normal((batch, m, n)).astype(np.float32)
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    da, de, dbias = to_dev(a), to_dev(e), to_dev(bias)
    for z in range(batch):
        got = to_host(dev.gemm(da[z], dev.pack_weight(to_dev(w[z])), addend=de[z], bias=dbias,
                               epilogue=EPI_RELU))
        ref = np.maximum(ora.matmul_add(e[z] + bias, a[z], w[z]), 0)
        assert_gemm_close(got, ref, gemm_bound(a[z], w[z], np.abs(e[z]) + np.abs(bias)))
        if n % 4 == 0:
            rm = to_host(dev.gemm(da[z], to_dev(w[z]), addend=de[z], bias=dbias, epilogue=EPI_RELU))
            np.testing.assert_array_equal(got, rm)
    got_b = to_host(dev.gemm(da, to_dev(w), addend=de, bias=dbias, epilogue=EPI_RELU))
    for z in range(batch):
        ref = np.maximum(ora.matmul_add(e[z] + bias, a[z], w[z]), 0)
        assert_gemm_close(got_b[z], ref, gemm_bound(a[z], w[z], np.abs(e[z]) + np.abs(bias)))


@pytest.mark.parametrize("m,n", [(4096, 1024), (4096, 1000), (64, 40), (8192, 16)])
def test_k_zero_is_the_epilogue_alone(m, n):
    """K = 0 through the C ABI with null A and B: every output is the
    epilogue of addend + bias alone, on each path (pipelined, partial panel,
    small kernel)."""
    note(f"K = 0 {m}x{n}")
    g = workloads.rng(m + n)
    e = g.standard_normal((m, n)).astype(np.float32)
    bias = g.standard_normal(n).astype(np.float32)
    de, dbias = to_dev(e), to_dev(bias)
    out = torch.empty((m, n), dtype=torch.float32, device=device())
    _lib.check(_lib.lib().annc_hip_gemm(_lib.stream_ptr(), 1, m, n, 0, None, 0, 0, None, n, 0, 0,
                                        _lib.ptr(de), n, 0, _lib.ptr(dbias), EPI_RELU,
                                        _lib.ptr(out), n, 0))
    np.testing.assert_array_equal(to_host(out), np.maximum(e + bias, np.float32(0)))


@pytest.mark.parametrize("m,n,k,col0", [(2048, 512, 256, 1), (8192, 64, 333, 3)])
def test_pipeline_misaligned_a_base(m, n, k, col0):
    """A starting mid-row of a wider buffer (base not 16-byte aligned, lda a
    multiple of 4): the 4-byte DMA variant, bit-identical between packed and
    per-call-packed row-major B."""
    note(f"misaligned A base {m}x{n}x{k} col0={col0}")
    g = workloads.rng(m + n + k + col0)
    buf = g.standard_normal((m, k + 8)).astype(np.float32)
    a = np.ascontiguousarray(buf[:, col0:col0 + k])
    w = (g.standard_normal((k, n)) * 0.05).astype(np.float32)
    da = to_dev(buf)[:, col0:col0 + k]
    ref = ora.matmul(a, w)
    got = to_host(dev.gemm(da, dev.pack_weight(to_dev(w))))
    assert_gemm_close(got, ref, gemm_bound(a, w))
    np.testing.assert_array_equal(to_host(dev.gemm(da, to_dev(w))), got)


def _log_uniform(g, lo, hi):
    return int(np.exp(g.uniform(np.log(lo), np.log(hi + 1))))


def _sweep_case(seed):
    """A seeded random GEMM call: shape, batch, B layout, operand strides and
    epilogue drawn so that every dispatch path turns up over the seeds (GEMV,
    small kernel with and without K split, 64x32, 128x64, 128x128 and
    256x128 tiles, partial panels, N < 32, K tails, per-call packing)."""
    g = workloads.rng(1000 + seed)
    batch = int(g.choice([1, 1, 1, 2, 3]))
    m = _log_uniform(g, 1, 9000) if g.random() < 0.5 else _log_uniform(g, 512, 9000)
    n = _log_uniform(g, 1, 1100) if g.random() < 0.5 else _log_uniform(g, 64, 1100)
    k = _log_uniform(g, 1, 4500)
    if g.random() < 0.3:
        n = max(32, n // 32 * 32)
    if g.random() < 0.3:
        k = max(32, k // 32 * 32)
    while batch * m * n * k > 1_500_000_000:
        m = max(1, m // 2)
    return dict(
        batch=batch, m=m, n=n, k=k,
        packed=batch == 1 and bool(g.random() < 0.5),
        ldb_pad=int(g.choice([0, 0, 1, 3, 4, 33])),
        col0=int(g.choice([0, 0, 1, 4])),
        ldc_pad=int(g.choice([0, 0, 5])),
        addend=bool(g.random() < 0.5),
        bias=bool(g.random() < 0.5),
        epi=int(g.choice([EPI_NONE, EPI_RELU, EPI_SIGMOID])),
    )


@pytest.mark.parametrize("seed", range(256))
def test_gemm_random_shapes(seed):
    """Seeded random calls through annc_hip_gemm: within the GEMM bound of
    OpenBLAS (sigmoid: within 1e-4 relative, 1e-5 absolute of the logistic of
    OpenBLAS's sum), padding columns of the output untouched."""
    c = _sweep_case(seed)
    batch, m, n, k = c["batch"], c["m"], c["n"], c["k"]
    note(f"random GEMM seed={seed} {c}")
    g = workloads.rng(seed)
    abuf = g.standard_normal((batch, m, k + c["col0"] + 3)).astype(np.float32)
    a = abuf[:, :, c["col0"]:c["col0"] + k]
    w = (g.standard_normal((batch, k, n + c["ldb_pad"])) / np.sqrt(max(k, 1))).astype(np.float32)
    wv = w[:, :, :n]
    e = g.standard_normal((batch, m, n)).astype(np.float32) if c["addend"] else None
    bias = (g.standard_normal(n) * 0.1).astype(np.float32) if c["bias"] else None
    da = to_dev(abuf)[:, :, c["col0"]:c["col0"] + k]
    dw = to_dev(w)[:, :, :n]
    obuf = torch.full((batch, m, n + c["ldc_pad"]), float("nan"), device=device())
    if batch == 1:
        b_arg = dev.pack_weight(dw[0]) if c["packed"] else dw[0]
        dev.gemm(da[0], b_arg, addend=None if e is None else to_dev(e[0]),
                 bias=None if bias is None else to_dev(bias), epilogue=c["epi"],
                 out=obuf[0, :, :n])
    else:
        dev.gemm(da, dw, addend=None if e is None else to_dev(e),
                 bias=None if bias is None else to_dev(bias), epilogue=c["epi"],
                 out=obuf[:, :, :n])
    got = to_host(obuf)
    assert np.isnan(got[:, :, n:]).all(), "padding columns of the output were written"
    for z in range(batch):
        add = np.zeros((m, n), np.float32) if e is None else e[z]
        if bias is not None:
            add = add + bias
        lin = ora.matmul_add(add, np.ascontiguousarray(a[z]), np.ascontiguousarray(wv[z]))
        gz = got[z, :, :n]
        if c["epi"] == EPI_SIGMOID:
            np.testing.assert_allclose(gz, 1.0 / (1.0 + np.exp(-lin.astype(np.float64))),
                                       rtol=1e-4, atol=1e-5)
        else:
            ref = np.maximum(lin, 0) if c["epi"] == EPI_RELU else lin
            assert_gemm_close(gz, ref, gemm_bound(a[z], wv[z], np.abs(add)))


def test_custom_calls_from_concurrent_threads():
    """The synchronous custom calls run on a stream of the calling thread:
    threads calling __matmul_add_relu at once (host buffers staged through
    each thread's scratch; threads 2 and 3 have at least 128 64x64 tiles and
    run the pipelined kernel) each get their own result; so do their device
    calls on their own streams, where threads 2 and 3 pack an unaligned
    row-major B into that stream's workspace."""
    import threading
    note("custom calls from 4 threads")
    g = workloads.rng(77)
    cases = []
    for t in range(4):
        m, k, n = 1024 + 512 * t, 96 + 8 * t, 256
        a = g.standard_normal((m, k)).astype(np.float32)
        b = (g.standard_normal((k, n)) * 0.05).astype(np.float32)
        e = g.standard_normal((m, n)).astype(np.float32)
        cases.append((a, b, e, np.zeros((m, n), np.float32), np.empty((m, n), np.float32)))
    errors = []

    def work(c):
        a, b, e, z, out = c
        try:
            ref = ora.matmul_add_relu(e, a, b)
            bound = gemm_bound(a, b, e)
            k, n = b.shape
            wide = np.zeros((k, n + 3), np.float32)  # rows not 16-byte aligned
            wide[:, :n] = b
            s = torch.cuda.Stream(device=device())
            with torch.cuda.stream(s):
                da, de, db = to_dev(a), to_dev(e), to_dev(wide)[:, :n]
                s.synchronize()
                for _ in range(5):
                    xla.matmul_add_relu(z, e, a, b, out)
                    assert_gemm_close(out, ref, bound)
                    got = dev.gemm(da, db, addend=de, epilogue=EPI_RELU)
                    s.synchronize()
                    assert_gemm_close(to_host(got), ref, bound)
        except Exception as ex:  # reported below
            errors.append(ex)

    threads = [threading.Thread(target=work, args=(c,)) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors[0]


def test_layout_matmul_on_weights_packed_in_a_saved_model(tmp_path):
    """annc-opt's layout_matmul on a SavedModel (graph and variables read and
    written without TensorFlow): the packed variable read back from the
    output's tensor bundle drives __layout_matmul to the row-major product."""
    from annc_amd import annc_opt
    from annc_amd import savedmodel as sm
    note("annc-opt layout_matmul on a SavedModel, then __layout_matmul 4096x512x1024")
    g = workloads.rng(41)
    w = g.standard_normal((1024, 512)).astype(np.float32)
    a = g.standard_normal((4096, 1024)).astype(np.float32)
    nodes = [sm.GraphNode("x", "Placeholder", [], {"dtype": sm.DType("DT_FLOAT")}),
             sm.GraphNode("dense/kernel", "VariableV2", [], {"dtype": sm.DType("DT_FLOAT")}),
             sm.GraphNode("dense/kernel/read", "Identity", ["dense/kernel"],
                          {"T": sm.DType("DT_FLOAT")}),
             sm.GraphNode("dense/MatMul", "MatMul", ["x", "dense/kernel/read"],
                          {"T": sm.DType("DT_FLOAT"), "transpose_a": False,
                           "transpose_b": False})]
    src, out_dir = tmp_path / "in", tmp_path / "out"
    sm.write_saved_model(str(src), sm.new_saved_model(nodes))
    sm.write_variables(str(src), {"dense/kernel": w})
    assert annc_opt.main(["-I", str(src), "-O", str(out_dir), "layout_matmul"]) == 0
    graph = sm.read_saved_model(str(out_dir))
    mm = sm.find_node(graph.nodes, "dense/MatMul")
    assert mm.attrs["rhs_format"] == annc_opt.mfma_rhs_format()
    packed = sm.read_variables(str(out_dir))["dense/kernel"]
    assert packed.shape == w.shape and not np.array_equal(packed, w)
    out = np.empty((4096, 512), np.float32)
    xla.layout_matmul(a, packed, 1024, 512, out)
    assert_gemm_close(out, ora.matmul(a, w), gemm_bound(a, w))
