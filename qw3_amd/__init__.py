"""qw3_amd -- MI355X (gfx950) MoE-FFN hot path of the qw3 engine.

The product is the C-ABI library qw3_amd/lib/libds3_hip.so (include/ds3_hip.h):
hand-written HIP kernels for routing, bucketing, quantised expert products and
the weighted combine.  This package is its Python host mirror:

    qw3_amd.ds3       buffers and wrappers of the ds3_hip entry points
    qw3_amd.workload  deterministic synthetic layers and inputs
    qw3_amd.build     compiles the native libraries in-tree
"""
from . import ds3  # noqa: F401

__all__ = ["ds3"]
