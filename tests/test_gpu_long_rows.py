"""GPU: RMSNorm and softmax rows longer than one wave holds (> 8192 elements).

RMSNorm: one 1024-thread workgroup per row, register-resident up to 1024 x 8
chunks per row and streamed beyond.  Softmax: the exponent sum folds by
8192-element segments, run by one 1024-thread workgroup per row with the row
in registers (up to 4 segments), or by one workgroup per segment: in one
row-synchronized launch when rows x segments <= 2 x CUs, else in three
launches (the partials in the context workspace up to 32768 segments,
allocated beyond).  The fold order is
the declared grouping tiler_hip_row_grouping reports, restated by the
oracle's grouped forms (tiler-reference/src/rms_norm.rs:405-489,
softmax.rs:200-315 with that reassociation).  Bit-exact against the oracle on
the same inputs, whichever form runs.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import tiler_amd
from helpers import bf16_widen, bits
from tiler_amd import _lib as L

pytestmark = pytest.mark.gpu

EPS = 0x3727C5AC


def _dev_rms(ctx, dtype, x, w, rows, extent, broadcast, offset_elems=0):
    elem = x.dtype.itemsize
    dx = ctx.alloc(x.nbytes + 16)
    dw = ctx.to_device(w)
    dy = ctx.alloc(x.nbytes + 16)
    try:
        vx, vy = dx.offset(offset_elems * elem), dy.offset(offset_elems * elem)
        vx.upload(x)
        ctx.rms_norm(dtype, vx, dw, rows, extent, EPS, vy, weight_broadcast=broadcast)
        ctx.synchronize()
        return vy.download(x.dtype, x.shape)
    finally:
        dx.free(); dw.free(); dy.free()


@pytest.mark.parametrize("rows,extent,broadcast,offset", [
    (3, 8200, True, 0),      # register-resident, 2 chunks per thread
    (2, 12345, True, 0),     # unaligned rows (element path)
    (2, 65536, True, 0),     # 8 chunks per thread
    (2, 65544, False, 0),    # streamed, full weight
    (2, 100001, True, 1),    # streamed, unaligned base
])
def test_rms_norm_bf16_long_rows(ctx, rows, extent, broadcast, offset):
    rng = np.random.default_rng(extent)
    xb = oracle.bf16_narrow(rng.standard_normal((rows, extent)).astype(np.float32))
    wshape = (extent,) if broadcast else (rows, extent)
    wb = oracle.bf16_narrow(rng.normal(1.0, 0.1, wshape).astype(np.float32))
    vec, waves, _ = tiler_amd.row_grouping(L.ROWS_RMS_NORM, L.BF16, extent)
    assert (vec, waves) == (8, 16)
    got = _dev_rms(ctx, L.BF16, xb, wb, rows, extent, broadcast, offset)
    y = oracle.rms_norm_grouped(bf16_widen(xb), bf16_widen(wb), rows, extent, EPS, broadcast, vec, waves)
    assert np.array_equal(got, oracle.bf16_narrow(y).reshape(rows, extent))


@pytest.mark.parametrize("rows,extent", [(3, 8193), (2, 32768), (2, 40003)])
def test_rms_norm_f32_long_rows(ctx, rows, extent):
    rng = np.random.default_rng(extent + 7)
    x = rng.standard_normal((rows, extent)).astype(np.float32)
    w = rng.normal(1.0, 0.1, (rows, extent)).astype(np.float32)
    vec, waves, _ = tiler_amd.row_grouping(L.ROWS_RMS_NORM, L.F32, extent)
    got = _dev_rms(ctx, L.F32, x, w, rows, extent, False)
    want = oracle.rms_norm_grouped(x, w, rows, extent, EPS, False, vec, waves).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want))


def _form(rows, extent, cus=256):
    nseg = -(-extent // 8192)
    if nseg <= 4:
        return "resident"
    if rows * nseg <= min(2 * cus, 1024):
        return "row-synchronized"
    return "split" if rows * nseg <= 32768 else "split, allocated partials"


# Every launch form, aligned and element-wise (extent % 4, base offset).
@pytest.mark.parametrize("rows,extent,offset", [
    (4, 8196, 0), (2, 20000, 0), (2, 32768, 0), (140, 20001, 0), (1, 8193, 0),   # resident
    (3, 50001, 0), (5, 131072, 1), (131, 50000, 0), (130, 90001, 1),              # split
])
def test_softmax_long_rows(ctx, rows, extent, offset):
    rng = np.random.default_rng(extent + 11)
    x = (rng.standard_normal((rows, extent)) * 3).astype(np.float32)
    x[0, ::7] = -np.inf                  # masked positions
    if rows > 2:
        x[2, extent // 2] = np.nan          # a NaN poisons its row
    if rows > 3:
        x[3, :min(extent, 8192)] = -np.inf  # a whole segment masked
    vec, waves, seg = tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.F32, extent)
    assert (vec, waves, seg) == (4, 4, 8192)
    print(f"softmax long rows={rows} extent={extent} offset={offset} form={_form(rows, extent, ctx.observe_live_device('compute-units'))}", flush=True)
    dx, dy = ctx.alloc(x.nbytes + 16), ctx.alloc(x.nbytes + 16)
    try:
        vx, vy = dx.offset(offset * 4), dy.offset(offset * 4)
        vx.upload(x)
        ctx.softmax_f32(vx, rows, extent, vy)
        ctx.synchronize()
        got = vy.download(np.float32, x.shape)
    finally:
        dx.free(); dy.free()
    want = oracle.softmax_grouped(x, rows, extent, vec, waves, seg).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want))


def test_softmax_split_with_allocated_partials(ctx):
    # 6600 rows of 5 segments: 33000 segment partials exceed the 32768 the
    # workspace holds, so the call allocates them on the stream.  Rows repeat
    # 8 distinct inputs; every row must equal the oracle's for its input
    # (rows are independent), checked on the 8 distinct rows and by equality.
    rows, extent, distinct = 6600, 40960, 8
    assert _form(rows, extent) == "split, allocated partials"
    base = (np.random.default_rng(77).standard_normal((distinct, extent)) * 3).astype(np.float32)
    base[1, 100:9000] = -np.inf
    x = np.tile(base, (rows // distinct, 1))
    print(f"softmax split allocated partials rows={rows} extent={extent}", flush=True)
    dx, dy = ctx.to_device(x), ctx.alloc(x.nbytes)
    try:
        ctx.softmax_f32(dx, rows, extent, dy)
        ctx.synchronize()
        got = dy.download(np.float32, x.shape)
    finally:
        dx.free(); dy.free()
    del x
    want = oracle.softmax_grouped(base, distinct, extent, 4, 4, 8192).reshape(distinct, extent)
    assert np.array_equal(bits(got[:distinct]), bits(want))
    assert np.array_equal(got.reshape(rows // distinct, distinct, extent).view(np.uint32),
                          np.broadcast_to(want.view(np.uint32), (rows // distinct, distinct, extent)))


def test_long_row_softmax_matches_f64_within_tolerance(ctx):
    rows, extent = 2, 300000
    x = (np.random.default_rng(5).standard_normal((rows, extent)) * 3).astype(np.float32)
    dx, dy = ctx.to_device(x), ctx.alloc(x.nbytes)
    try:
        ctx.softmax_f32(dx, rows, extent, dy)
        ctx.synchronize()
        got = dy.download(np.float32, x.shape)
    finally:
        dx.free(); dy.free()
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    ref = e / e.sum(axis=1, keepdims=True)
    assert float((np.abs(got - ref) / ref).max()) <= 1e-5


def test_row_synchronized_softmax_fallback_matches(ctx):
    # With the wait bound at 0 ticks no workgroup waits for its row: each one
    # computes the row maximum and sum from the row itself.  The result is the
    # same segmented fold, bit for bit, as the waiting form and the oracle.
    import os
    rows, extent = 3, 70001
    assert _form(rows, extent, ctx.observe_live_device("compute-units")) == "row-synchronized"
    x = (np.random.default_rng(91).standard_normal((rows, extent)) * 3).astype(np.float32)
    x[1, 9000:20000] = -np.inf
    want = oracle.softmax_grouped(x, rows, extent, 4, 4, 8192).reshape(rows, extent)
    os.environ["TILER_HIP_ROW_SYNC_WAIT_TICKS"] = "0"
    try:
        c0 = tiler_amd.Context(0)
    finally:
        del os.environ["TILER_HIP_ROW_SYNC_WAIT_TICKS"]
    try:
        for c in (c0, ctx):
            dx, dy = c.to_device(x), c.alloc(x.nbytes)
            try:
                for _ in range(3):  # every call raises the epoch past its own tag
                    c.fill_u32(dy, 0, x.size)
                    c.softmax_f32(dx, rows, extent, dy)
                    c.synchronize()
                    assert np.array_equal(bits(dy.download(np.float32, x.shape)), bits(want))
            finally:
                dx.free(); dy.free()
    finally:
        c0.close()


def test_row_synchronized_softmax_calls_of_changing_shapes(ctx):
    # Calls of different shapes share the context's epoch and word area: a
    # call's segment positions hold an earlier call's words (of other rows,
    # other values) under earlier tags, which must never be taken for its own.
    cus = ctx.observe_live_device("compute-units")
    shapes = [(32, 131072), (5, 50001), (31, 90000), (2, 70001), (32, 131072), (5, 50001)]
    rng = np.random.default_rng(17)
    for i, (rows, extent) in enumerate(shapes * 2):
        assert _form(rows, extent, cus) == "row-synchronized"
        x = (rng.standard_normal((rows, extent)) * (1 + i)).astype(np.float32)
        print(f"[row-sync call {i}] {rows}x{extent}", flush=True)
        dx, dy = ctx.to_device(x), ctx.alloc(x.nbytes)
        try:
            ctx.softmax_f32(dx, rows, extent, dy)
            ctx.synchronize()
            got = dy.download(np.float32, x.shape)
        finally:
            dx.free(); dy.free()
        want = oracle.softmax_grouped(x, rows, extent, 4, 4, 8192).reshape(rows, extent)
        assert np.array_equal(bits(got), bits(want)), (rows, extent)
