"""annc_amd -- MI355X (gfx950) implementation of ANNC's fused-operator path.

Layers:
  include/annc_hip.h     C-ABI (XLA custom calls, TF-op entries, device API)
  annc_amd/csrc          HIP kernels + C++ host side (libannc_hip.so)
  annc_amd._lib          ctypes binding; raises if the library is not built
  annc_amd.flags         ANNC_FLAGS
  annc_amd.xla           custom-call invocation with XLA's operand encoding
  annc_amd.tf_ops        TF custom-op mirror (same inputs, attrs, messages)
  annc_amd.device        asynchronous device-pointer API on torch tensors
  annc_amd.rec_graph     MLP tower and wide&deep graph built on the above
  annc_amd.annc_opt      `annc-opt ... layout_matmul` pre-pack counterpart
"""
from ._lib import (AnncError, InvalidArgumentError, LibraryNotBuilt, LIB_PATH, lib,  # noqa: F401
                   EPI_NONE, EPI_RELU, EPI_SIGMOID, COMBINER_SUM, COMBINER_MEAN)

__version__ = "0.1.0"
