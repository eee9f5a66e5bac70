"""GPU: the RuntimeAdapter route over the C ABI, and graph replay.

The route mirrors tiler-runtime/src/adapter.rs:545-678: validate the payload
from its bytes, observe the live device, prepare the entry, observe the
prepared entry, plan (acquiring nothing), allocate after the commit, dispatch
and read back -- here with the library's own gfx950 code object as the routed
payload and a softmax entry whose kernel arguments are packed by hand.
"""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest

import oracle
import tiler_amd
from helpers import bits
from tiler_amd import _lib as L

pytestmark = pytest.mark.gpu


def _payload():
    v = L.PayloadView()
    assert L.lib().tiler_hip_payload(ctypes.byref(v)) == L.OK
    return ctypes.string_at(v.code, v.code_bytes)


def test_live_device_observations(ctx):
    assert ctx.observe_live_device("wavefront-size") == 64
    assert ctx.observe_live_device("target-is-gfx950") == 1
    assert ctx.observe_live_device("compute-units") >= 1
    assert ctx.observe_live_device("lds-bytes-per-workgroup") >= 64 * 1024
    assert ctx.observe_live_device("no-such-key") is None  # Unrecognized, fail-closed
    assert ctx.observe_live_device("device-address-bits") == 64
    assert min(ctx.observe_live_device(f"max-grid-{a}") for a in "xyz") >= 1


def test_measured_subnormal_behaviour(ctx):
    # Measured by the probe kernel on the device: the code object is built
    # without denormal flushing, so both sides preserve (mode 1), which is what
    # the declared profile states (f32_subnormals_preserved) and what the
    # oracle's PRESERVE mode computes.
    assert ctx.observe_live_device("f32-input-subnormals") == 1
    assert ctx.observe_live_device("f32-result-subnormals") == 1
    assert tiler_amd.runtime.profile()["f32_subnormals_preserved"] == 1
    # Cached: a second query answers without another probe and agrees.
    assert ctx.observe_live_device("f32-input-subnormals") == 1


def test_route_prepare_plan_allocate_dispatch(ctx):
    code = _payload()
    buf = ctypes.create_string_buffer(code, len(code))
    symbol = b"tiler_softmax_f32_ch1"
    entry = L.RoutedEntry(ctypes.cast(buf, ctypes.c_void_p), len(code), symbol)
    first = ctypes.c_uint32()
    h = ctx.handle
    assert L.lib().tiler_hip_prepare_entries(h, ctypes.byref(entry), 1, ctypes.byref(first)) == L.OK
    v = ctypes.c_uint64()
    assert L.lib().tiler_hip_observe_prepared_entry(h, first.value, b"max-threads-per-workgroup",
                                                    ctypes.byref(v)) == L.OK
    assert v.value >= 256
    assert L.lib().tiler_hip_observe_prepared_entry(h, first.value, b"bogus",
                                                    ctypes.byref(v)) == L.REFUSE_UNRECOGNIZED_KEY

    rows, extent = 8, 200
    x = (np.random.default_rng(61).standard_normal((rows, extent)) * 3).astype(np.float32)
    dx = ctx.to_device(x)
    # kernargs: const float* x, float* y, uint64 rows, uint32 extent  (28 bytes)
    kernargs = ctypes.create_string_buffer(struct.pack("<QQQI", 0, 0, rows, extent), 28)
    slots = (ctypes.c_uint32 * 2)(0, 1)
    offsets = (ctypes.c_uint32 * 2)(0, 8)
    e = L.DispatchEntry(first.value, (ctypes.c_uint32 * 3)((rows + 3) // 4, 1, 1),
                        (ctypes.c_uint32 * 3)(256, 1, 1), 0, ctypes.cast(kernargs, ctypes.c_void_p), 28,
                        2, slots, offsets)
    slot_bytes = (ctypes.c_uint64 * 2)(x.nbytes, x.nbytes)
    plan = L.DispatchPlan(2, slot_bytes, 1, ctypes.pointer(e))
    assert L.lib().tiler_hip_plan_dispatch(h, ctypes.byref(plan)) == L.OK
    ptrs = (ctypes.c_void_p * 2)(dx.ptr, None)  # slot 0 caller-supplied, slot 1 allocated
    assert L.lib().tiler_hip_allocate_dispatch(h, ctypes.byref(plan), ptrs) == L.OK
    assert ptrs[1]
    assert L.lib().tiler_hip_dispatch(h, ctypes.byref(plan), ptrs) == L.OK
    out = np.empty(rows * extent, np.float32)
    assert L.lib().tiler_hip_download(h, out.ctypes.data_as(ctypes.c_void_p), ptrs[1], out.nbytes) == L.OK
    assert np.array_equal(bits(out), bits(oracle.softmax_grouped(x, rows, extent, 4, 1)))
    owned = (ctypes.c_void_p * 2)(1, None)
    assert L.lib().tiler_hip_release_dispatch(h, ctypes.byref(plan), ptrs, owned) == L.OK
    dx.free()


def test_plan_refuses_before_commit(ctx):
    code = _payload()
    buf = ctypes.create_string_buffer(code, len(code))
    entry = L.RoutedEntry(ctypes.cast(buf, ctypes.c_void_p), len(code), b"tiler_softmax_f32_ch1")
    first = ctypes.c_uint32()
    h = ctx.handle
    assert L.lib().tiler_hip_prepare_entries(h, ctypes.byref(entry), 1, ctypes.byref(first)) == L.OK
    kernargs = ctypes.create_string_buffer(28)
    slots = (ctypes.c_uint32 * 2)(0, 1)
    offsets = (ctypes.c_uint32 * 2)(0, 8)
    slot_bytes = (ctypes.c_uint64 * 2)(64, 64)

    def plan_with(prepared, block, offs=offsets, slot_count=2):
        e = L.DispatchEntry(prepared, (ctypes.c_uint32 * 3)(1, 1, 1), (ctypes.c_uint32 * 3)(block, 1, 1),
                            0, ctypes.cast(kernargs, ctypes.c_void_p), 28, 2, slots, offs)
        p = L.DispatchPlan(slot_count, slot_bytes, 1, ctypes.pointer(e))
        return L.lib().tiler_hip_plan_dispatch(h, ctypes.byref(p))

    assert plan_with(first.value, 256) == L.OK
    assert plan_with(first.value, 2048) == L.REFUSE_CAPACITY          # wider than the pipeline
    assert plan_with(first.value + 1000, 256) == L.REFUSE_NOT_PREPARED
    assert plan_with(first.value, 256, (ctypes.c_uint32 * 2)(0, 24)) == L.REFUSE_BINDING_MISMATCH
    assert plan_with(first.value, 256, slot_count=1) == L.REFUSE_BINDING_MISMATCH
    # a malformed payload refuses at prepare, before anything is committed
    bad = ctypes.create_string_buffer(b"\x7fELF" + b"\0" * 60, 64)
    e2 = L.RoutedEntry(ctypes.cast(bad, ctypes.c_void_p), 64, b"tiler_softmax_f32_ch1")
    assert L.lib().tiler_hip_prepare_entries(h, ctypes.byref(e2), 1, ctypes.byref(first)) < 0


def test_graph_replay_matches_eager_on_every_replay(ctx):
    rows, extent, eps = 64, 4096, 0x3727C5AC
    rng = np.random.default_rng(62)
    xb = oracle.bf16_narrow(rng.standard_normal((rows, extent)).astype(np.float32))
    wb = oracle.bf16_narrow(rng.normal(1.0, 0.1, extent).astype(np.float32))
    sx = (np.random.default_rng(63).uniform(-1, 1, 1 << 20)).astype(np.float32)
    dx, dw, dy = ctx.to_device(xb), ctx.to_device(wb), ctx.alloc(xb.nbytes)
    ds, dso = ctx.to_device(sx), ctx.alloc(4)
    try:
        ctx.rms_norm(L.BF16, dx, dw, rows, extent, eps, dy)
        ctx.sum_f32(ds, 1, sx.size, dso, topology=L.SUM_TREE)
        ctx.synchronize()
        eager_y = dy.download(np.uint16, (rows, extent))
        eager_s = dso.download(np.float32, (1,))
        ctx.capture_begin()
        ctx.rms_norm(L.BF16, dx, dw, rows, extent, eps, dy)
        ctx.sum_f32(ds, 1, sx.size, dso, topology=L.SUM_TREE)
        graph = ctx.capture_end()
        for _ in range(4):
            ctx.fill_u32(dy, 0, xb.nbytes // 4)
            ctx.fill_u32(dso, 0, 1)
            ctx.synchronize()
            ctx.graph_launch(graph)
            ctx.synchronize()
            assert np.array_equal(dy.download(np.uint16, (rows, extent)), eager_y)
            assert bits(dso.download(np.float32, (1,)))[0] == bits(eager_s)[0]
        ctx.graph_destroy(graph)
    finally:
        for b in (dx, dw, dy, ds, dso):
            b.free()


def test_graph_replay_of_split_softmax(ctx):
    # 4 rows of 7 segments: the split form's three launches, partials in the
    # context workspace, captured and replayed; every replay matches eager.
    rows, extent = 4, 50001
    x = (np.random.default_rng(64).standard_normal((rows, extent)) * 3).astype(np.float32)
    dx, dy = ctx.to_device(x), ctx.alloc(x.nbytes)
    try:
        ctx.softmax_f32(dx, rows, extent, dy)
        ctx.synchronize()
        eager = dy.download(np.float32, x.shape)
        assert np.array_equal(bits(eager).reshape(-1), bits(oracle.softmax_grouped(x, rows, extent, 4, 4, 8192)))
        ctx.capture_begin()
        ctx.softmax_f32(dx, rows, extent, dy)
        graph = ctx.capture_end()
        for _ in range(4):
            ctx.fill_u32(dy, 0, x.size)
            ctx.synchronize()
            ctx.graph_launch(graph)
            ctx.synchronize()
            assert np.array_equal(bits(dy.download(np.float32, x.shape)), bits(eager))
        ctx.graph_destroy(graph)
    finally:
        dx.free(); dy.free()


def test_split_softmax_needing_allocation_refuses_under_capture(ctx):
    # 6600 x 40960 needs 33000 segment partials, beyond the workspace: eager it
    # allocates them on the stream; under capture it refuses before any launch
    # (the buffers are full size all the same).
    rows, extent = 6600, 40960
    dx, dy = ctx.alloc(rows * extent * 4), ctx.alloc(rows * extent * 4)
    try:
        ctx.capture_begin()
        with pytest.raises(tiler_amd.Refusal):
            ctx.softmax_f32(dx, rows, extent, dy)
        ctx.fill_u32(dy, 0, 16)
        graph = ctx.capture_end()
        ctx.graph_destroy(graph)
    finally:
        dx.free(); dy.free()
