"""Helpers shared by the GPU parity tests."""
import sys

import numpy as np
import torch


def device():
    if not torch.cuda.is_available():
        raise RuntimeError("gpu-marked test run without a visible GPU")
    return torch.device("cuda:0")


def note(msg: str) -> None:
    """Name the case before a GPU step (flushed, so it survives a crash)."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(x, dev=None):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev or device())


def to_host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def gemm_bound(a, b, e=None, rel=1e-4):
    """Elementwise tolerance 1e-4*|ref| + 1e-4*(|A||B| + |E|)."""
    mag = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    if e is not None:
        mag = mag + np.abs(e)
    return rel * mag


def assert_gemm_close(got, ref, bound):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    tol = 1e-4 * np.abs(ref) + bound
    bad = np.abs(got - ref) > tol
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{bad.sum()} elements out of tolerance; first at {tuple(i)}: "
                             f"got {got[tuple(i)]!r} ref {ref[tuple(i)]!r} tol {tol[tuple(i)]!r}")
