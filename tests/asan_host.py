"""The CPU test suite against the host-code AddressSanitizer and
UndefinedBehaviorSanitizer build of the library (the host C++ -- custom
calls, TF-op entries, flags, rewriter, packers, runtime -- instrumented;
device code is not).  UBSan reports print as "runtime error" lines.

    make -C annc_amd/csrc asan
    ASAN_OPTIONS=detect_leaks=0 \\
      LD_PRELOAD=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so) \\
      python tests/asan_host.py

The interpreter itself is not instrumented, hence the preloaded runtime and
no leak check.  Not collected by pytest (no test_ prefix).
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from annc_amd import _lib  # noqa: E402

_lib.LIB_PATH = os.path.join(ROOT, "annc_amd", "_build", "asan", "libannc_hip_asan.so")
if not os.path.exists(_lib.LIB_PATH):
    sys.exit(f"{_lib.LIB_PATH} is missing: run `make -C annc_amd/csrc asan` first")

import pytest  # noqa: E402

sys.exit(pytest.main(["-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                      os.path.join(ROOT, "tests")]))
