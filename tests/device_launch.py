"""Runs a kernel from a test-only code object through the adapter's own stages
(tiler_hip_prepare_entries -> plan_dispatch -> dispatch), the route a routed
payload takes (tiler-runtime/src/adapter.rs:387-506).  Every storage slot is
caller-supplied, so nothing is allocated by the route."""
from __future__ import annotations

import ctypes

from tiler_amd import _lib as L

_prepared = {}


def prepare(ctx, code: bytes, symbol: str) -> int:
    key = (id(ctx), symbol, len(code))
    if key not in _prepared:
        buf = ctypes.create_string_buffer(code, len(code))
        entry = L.RoutedEntry(ctypes.cast(buf, ctypes.c_void_p), len(code), symbol.encode())
        first = ctypes.c_uint32()
        st = L.lib().tiler_hip_prepare_entries(ctx.handle, ctypes.byref(entry), 1, ctypes.byref(first))
        assert st == L.OK, (st, ctx.diagnostic)
        _prepared[key] = (first.value, buf)
    return _prepared[key][0]


def launch(ctx, code: bytes, symbol: str, grid: int, block: int, kernargs: bytes,
           bindings: list, slots: list) -> None:
    """bindings: (byte offset of a pointer field in kernargs, slot index);
    slots: DeviceBuffers (or raw device addresses), one per slot."""
    prepared = prepare(ctx, code, symbol)
    ka = ctypes.create_string_buffer(kernargs, len(kernargs))
    nb = len(bindings)
    bslots = (ctypes.c_uint32 * max(nb, 1))(*[s for _, s in bindings])
    boffs = (ctypes.c_uint32 * max(nb, 1))(*[o for o, _ in bindings])
    e = L.DispatchEntry(prepared, (ctypes.c_uint32 * 3)(grid, 1, 1), (ctypes.c_uint32 * 3)(block, 1, 1), 0,
                        ctypes.cast(ka, ctypes.c_void_p), len(kernargs), nb, bslots, boffs)
    sizes = [getattr(s, "nbytes", 1) for s in slots]
    slot_bytes = (ctypes.c_uint64 * len(slots))(*sizes)
    plan = L.DispatchPlan(len(slots), slot_bytes, 1, ctypes.pointer(e))
    st = L.lib().tiler_hip_plan_dispatch(ctx.handle, ctypes.byref(plan))
    assert st == L.OK, (st, ctx.diagnostic)
    ptrs = (ctypes.c_void_p * len(slots))(*[getattr(s, "ptr", s) for s in slots])
    st = L.lib().tiler_hip_dispatch(ctx.handle, ctypes.byref(plan), ptrs)
    assert st == L.OK, (st, ctx.diagnostic)
