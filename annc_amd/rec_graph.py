"""Recommendation-model graphs assembled from the fused operators.

These are the graphs the reference reaches through XLA clustering of a TF
Serving model (the patched cpu_compiler.cc running the KDnnRewriter passes,
install/tensorflow.patch:187-198, then the rewriters of
annc/service/cpu/gemm_rewriter.cc and graph_opt.cc): dense layers lowered to
__layout_matmul / __matmul_add_relu custom calls plus bias/activation loop
fusions, and hashed categorical fields lowered to the embed_hash_bucket op
family.  Here every layer is one gfx950 kernel with the bias and activation
fused into the GEMM epilogue, all buffers are allocated once per batch size,
and the tower runs back to back on one stream.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from . import _lib
from . import device as dev


class CapturedGraph:
    """A callable captured once into a HIP graph and replayed.

    Every launch of the wrapped callable goes to the capture stream (the
    library reads torch's current stream), so one replay re-issues the whole
    sequence with no host work per kernel.  Buffers must be allocated before
    capture (the graphs above keep theirs per batch size); nothing in the
    captured kernels allocates or memsets.
    """

    def __init__(self, fn, *args, warmup: int = 2):
        self.stream = torch.cuda.Stream()  # default priority
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                self.out = fn(*args)
        torch.cuda.current_stream().wait_stream(self.stream)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.out = fn(*args)
        torch.cuda.synchronize()

    def replay(self):
        self.graph.replay()
        return self.out

    __call__ = replay


@dataclass
class DenseLayer:
    weight: dev.PackedWeight | torch.Tensor  # packed [k, n] or row-major [k, n]
    bias: torch.Tensor                        # [n]
    activation: int                           # _lib.EPI_*


class MLPTower:
    """relu(x W1 + b1) ... -> sigmoid(h Wl + bl) with pre-packed weights.

    With `fuse_score` (the default) a tower whose last layer has one output
    runs its last two layers as one kernel (annc_hip_dense_score) when the
    shapes allow and the batch has at least `fuse_min_rows` rows: the scoring
    dot reads the hidden layer from registers, and that hidden layer reaches
    memory only with `keep_hidden`.  Every other layer, and the tail when it
    does not fit, is one GEMM launch.  The fused kernel gives each 16 rows a
    workgroup that streams the whole hidden-layer weight, so its time is
    flat up to 4096 rows; below 2049 rows the GEMM's small-batch kernels and
    the GEMV are faster (configs[1]'s 512 -> 256 -> 1 tail: 7.7-8.9 us
    against 10.6-10.9 up to 1024 rows, tower steps 31.8 against 32.6 us at
    2048; fused 11.1 against 14.9 us from 2304 rows)."""

    def __init__(self, weights: Sequence[np.ndarray], biases: Sequence[np.ndarray],
                 device: torch.device | str = "cuda", packed: bool = True,
                 final_activation: int = _lib.EPI_SIGMOID, fuse_score: bool = True,
                 keep_hidden: bool = False, fuse_min_rows: int = 2049):
        self.device = torch.device(device)
        self.keep_hidden = keep_hidden
        self.fuse_min_rows = fuse_min_rows
        self.layers: list[DenseLayer] = []
        for i, (w, b) in enumerate(zip(weights, biases)):
            wt = torch.as_tensor(np.ascontiguousarray(w, dtype=np.float32)).to(self.device)
            if packed:
                wt = dev.pack_weight(wt)
            act = final_activation if i == len(weights) - 1 else _lib.EPI_RELU
            bt = torch.as_tensor(np.ascontiguousarray(b, dtype=np.float32)).to(self.device)
            self.layers.append(DenseLayer(wt, bt, act))
        self._buffers: dict[int, list[torch.Tensor]] = {}
        self.fused_tail = False
        if fuse_score and packed and len(self.layers) >= 2:
            hid, last = self.layers[-2].weight, self.layers[-1].weight
            self.fused_tail = last.n == 1 and dev.dense_score_fits(hid.k, hid.n)

    @property
    def widths(self) -> list[int]:
        return [(l.weight.n if isinstance(l.weight, dev.PackedWeight) else l.weight.shape[1])
                for l in self.layers]

    def lowering(self, batch: int) -> list:
        """Custom-call target ANNC's rewriters pick for each layer's dot under
        the current ANNC_FLAGS (None: the dot stays an XLA dot), for the HLO
        XLA emits from the layer: dot -> add(broadcast(bias)) -> maximum for
        ReLU, weights as parameters (annc_hlo_rewrite_instruction).  With
        --layout-matmul the configs[1] tower lowers to __layout_matmul,
        __layout_matmul, None (256 -> 1 fails the >= 12 rule)."""
        from . import hlo
        out, k = [], None
        for l in self.layers:
            w = l.weight
            k, n = (w.k, w.n) if isinstance(w, dev.PackedWeight) else tuple(w.shape)
            act = "relu" if l.activation == _lib.EPI_RELU else (
                "sigmoid" if l.activation == _lib.EPI_SIGMOID else None)
            f, dot, _ = hlo.dense_layer(batch, k, n, activation=act)
            r = hlo.rewrite(f, dot)
            out.append(None if r is None else r.target)
        return out

    def flops(self, batch: int) -> int:
        total = 0
        for l in self.layers:
            w = l.weight
            k, n = (w.k, w.n) if isinstance(w, dev.PackedWeight) else tuple(w.shape)
            total += 2 * batch * k * n
        return total

    def buffers(self, batch: int) -> list[torch.Tensor]:
        bufs = self._buffers.get(batch)
        if bufs is None:
            bufs = [torch.empty((batch, n), dtype=torch.float32, device=self.device)
                    for n in self.widths]
            self._buffers[batch] = bufs
        return bufs

    def forward(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        """x: [batch, k0] (any row stride).  Returns the final [batch, 1] buffer."""
        bufs = self.buffers(x.shape[0])
        h = x
        fused = self.fused_tail and x.shape[0] >= self.fuse_min_rows
        plain = len(self.layers) - (2 if fused else 0)
        for layer, out in zip(self.layers[:plain], bufs):
            dev.gemm(h, layer.weight, bias=layer.bias, epilogue=layer.activation, out=out,
                     stream=stream)
            h = out
        if plain == len(self.layers):
            return h
        if h.data_ptr() % 16 or h.stride(0) % 4:  # the fused tail reads float4 rows
            for layer, out in zip(self.layers[plain:], bufs[plain:]):
                dev.gemm(h, layer.weight, bias=layer.bias, epilogue=layer.activation, out=out,
                         stream=stream)
                h = out
            return h
        hid, last = self.layers[-2], self.layers[-1]
        return dev.dense_score(h, hid.weight, last.weight.data, bias=hid.bias,
                               epilogue=hid.activation, score_bias=last.bias,
                               score_epilogue=last.activation,
                               hidden=bufs[-2] if self.keep_hidden else None, out=bufs[-1],
                               stream=stream)

    __call__ = forward


@dataclass
class WideDeepConfig:
    num_fields: int = 26
    dim: int = 32
    table_rows: int = 100_000
    num_buckets: int = 100_000
    num_dense: int = 13
    hidden: tuple = (1024, 512, 256)
    combiner: int = _lib.COMBINER_MEAN


class WideDeepGraph:
    """Hashed categorical fields + dense features -> concat -> MLP -> sigmoid.

    The concat buffer is [batch, F*dim + num_dense] with its row padded to a
    multiple of 32 floats; the embedding kernel writes its columns in place.
    The padding columns stay zero, and the first layer's weight is packed
    with as many zero rows, so the first GEMM reads whole rows and runs
    whole 32-deep k-blocks (no K tail; the zero terms change no sum).
    Column order: field 0 .. field F-1 embeddings, then the dense features.
    """

    def __init__(self, cfg: WideDeepConfig, tables: Sequence[torch.Tensor],
                 weights: Sequence[np.ndarray], biases: Sequence[np.ndarray],
                 device: torch.device | str = "cuda"):
        self.cfg = cfg
        self.device = torch.device(device)
        self.tables = [t.to(self.device).contiguous() for t in tables]
        self.concat_width = cfg.num_fields * cfg.dim + cfg.num_dense
        self.ld = (self.concat_width + 31) // 32 * 32
        w0 = np.asarray(weights[0], dtype=np.float32)
        if w0.shape[0] != self.concat_width:
            raise ValueError(f"first weight has {w0.shape[0]} rows, the concat {self.concat_width}")
        w0_padded = np.zeros((self.ld, w0.shape[1]), dtype=np.float32)
        w0_padded[:self.concat_width] = w0
        self._shapes = [tuple(np.shape(w)) for w in weights]
        self.tower = MLPTower([w0_padded] + list(weights[1:]), biases, device=self.device,
                              packed=True)
        self._concat: dict[int, torch.Tensor] = {}

    def concat_buffer(self, batch: int) -> torch.Tensor:
        buf = self._concat.get(batch)
        if buf is None:
            buf = torch.zeros((batch, self.ld), dtype=torch.float32, device=self.device)
            self._concat[batch] = buf
        return buf

    def flops(self, batch: int) -> int:
        """The model's GEMM flops (the first layer at its own K, not the padded one)."""
        return sum(2 * batch * k * n for k, n in self._shapes)

    def dense_view(self, batch: int) -> torch.Tensor:
        """The dense-feature columns of the concat buffer ([batch, num_dense],
        row stride ld).  A producer that writes the dense features here (the
        host-to-device copy of a serving loop) makes the concat free: forward()
        skips the copy when it is given this view."""
        emb_cols = self.cfg.num_fields * self.cfg.dim
        return self.concat_buffer(batch)[:, emb_cols:self.concat_width]

    def forward(self, ids: torch.Tensor, offsets: torch.Tensor, dense: torch.Tensor,
                stream=None) -> torch.Tensor:
        batch = dense.shape[0]
        cfg = self.cfg
        buf = self.concat_buffer(batch)
        emb_cols = cfg.num_fields * cfg.dim
        dev.hashed_embedding_bags(self.tables, [cfg.num_buckets] * cfg.num_fields, ids, offsets,
                                  batch, cfg.combiner, out=buf[:, :emb_cols], stream=stream)
        view = buf[:, emb_cols:self.concat_width]
        if not (dense.data_ptr() == view.data_ptr() and dense.stride() == view.stride()
                and dense.shape == view.shape):
            view.copy_(dense)
        return self.tower.forward(buf, stream=stream)

    __call__ = forward
