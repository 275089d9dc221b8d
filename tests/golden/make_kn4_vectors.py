"""Writes tests/golden/kn4_pack_vectors.npz: the reference annc-opt's "kn4"
weight packing (python/annc/optimize/data_pack.py:24-149, as called from
constant_folding.py:77-88 with FormageChange(12) and the tiling
[(axis 0, 352), (axis 1, 128)]) applied to arange-valued [k, n] matrices, so
each packed array is the source index of every packed element.

Run in a tree that holds the reference at /root/reference; only data_pack.py
(numpy-only) is loaded.  The fixture is the data; this script is how it was
made.
"""
import importlib.util
import os
import sys

import numpy as np

REF = "/root/reference/python/annc/optimize/data_pack.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kn4_pack_vectors.npz")
# shapes chosen to exercise: single tiles, N tails of 4/2/1 inside a block,
# the re-split of the last two K tiles (k > 352) and of the last two N
# tiles (n > 128), and three K tiles
SHAPES = [(12, 12), (13, 27), (37, 141), (365, 13), (705, 12), (30, 263), (401, 40)]


def main():
    spec = importlib.util.spec_from_file_location("ref_data_pack", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    arrays = {}
    for k, n in SHAPES:
        src = np.arange(k * n, dtype=np.int64).reshape(k, n)
        packed = mod.FormageChange(12).run(
            src, src_format=mod.DataFormat.kn, dst_format=mod.DataFormat.kn4,
            tiling_info=[mod.MatrixTiling(0, 352), mod.MatrixTiling(1, 128)])
        perm = np.asarray(packed, dtype=np.int64).reshape(-1)
        assert sorted(perm.tolist()) == list(range(k * n)), "kn4 must be a permutation"
        arrays[f"perm_{k}x{n}"] = perm.astype(np.int32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {sorted(arrays)}")


if __name__ == "__main__":
    sys.exit(main())
