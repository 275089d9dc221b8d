"""ANNC_FLAGS access (annc/service/cpu/annc_flags.h:25-39).

The flag set is parsed once from the ANNC_FLAGS environment variable by the
native library, with the reference grammar; ``reset`` re-parses a string.
"""
from __future__ import annotations

import ctypes

from . import _lib

FLAG_NAMES = ("matmul", "layout-matmul", "batch-matmul", "matmul-add", "matmul-add-relu",
              "sps-emd-2", "pooling", "disable-tf-matmul-fusion", "annc-pass")


def is_enabled(name: str) -> bool:
    return bool(_lib.lib().annc_flag_enabled(name.encode()))


def reset(flags: str | None) -> None:
    _lib.lib().annc_flags_reset(None if flags is None else flags.encode())


def dump() -> dict[str, bool]:
    lib = _lib.lib()
    need = lib.annc_flags_dump(None, 0)
    buf = ctypes.create_string_buffer(int(need) + 1)
    lib.annc_flags_dump(buf, len(buf))
    out = {}
    for line in buf.value.decode().splitlines():
        k, _, v = line.rpartition("=")
        out[k] = v == "1"
    return out
