"""tiler-hip: the MI355X (gfx950) execution backend for Tiler's hot path.

The product is the C ABI in include/tiler_hip.h, implemented by
tiler_amd/_build/libtiler_hip.so over hand-written gfx950 kernels compiled
ahead of time.  This package is its Python host mirror: `runtime` (bound
context, device buffers, launches), `families` (the tiler-reference family
functions run on the device), `adapter` (the RuntimeAdapter route), and
`build` (the offline build).  Nothing here computes on the CPU.
"""
from . import _lib
from .runtime import (Context, DeviceBuffer, Failure, GatherIndexOutOfBounds, HipError, Refusal,
                      profile, row_grouping, validate_gather_index)

__all__ = ["Context", "DeviceBuffer", "Failure", "GatherIndexOutOfBounds", "HipError", "Refusal",
           "profile", "row_grouping", "validate_gather_index", "_lib"]
