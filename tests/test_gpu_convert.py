"""GPU: the bf16 <-> binary32 conversion families (ADR 0091 decision 2).

Widening is checked on every one of the 65,536 bf16 patterns, narrowing on
every high half crossed with the low halves that sit at rounding boundaries
(0x0000, 0x0001, 0x7fff, 0x8000, 0x8001, 0xffff) plus a million random
patterns. Both are bit-exact against the oracle's restatement of the ADR's
rules, through the 16-byte vector kernel, the tail, unaligned storage and a
realized plan routed through the runtime seam.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tiler_amd import _lib as L
from tiler_amd import families
from tiler_amd.realize import realize, route

pytestmark = pytest.mark.gpu

ALL_BF16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)


def _narrow_corpus():
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    edge = (hi[:, None] | lows[None, :]).reshape(-1)
    rnd = np.random.default_rng(81).integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([edge, rnd]).view(np.float32)


def test_widen_every_pattern(ctx):
    got = families.widen_bf16_f32(ALL_BF16, ctx=ctx)
    assert np.array_equal(got.view(np.uint32), ALL_BF16.astype(np.uint32) << 16)
    assert np.array_equal(got.view(np.uint32), oracle.bf16_widen(ALL_BF16).view(np.uint32))


def test_narrow_boundaries_and_random(ctx):
    x = _narrow_corpus()
    got = families.narrow_f32_bf16(x, ctx=ctx)
    want = oracle.bf16_narrow(x)
    assert np.array_equal(got, want)
    assert (got[np.isnan(x)] == 0x7FC0).all()
    # overflow at the inclusive midpoint above the largest finite bf16 (0x7f7f)
    edge = np.array([0x7F7F7FFF, 0x7F7F8000, 0xFF7F8000, 0x00000001, 0x80000000], np.uint32).view(np.float32)
    assert list(families.narrow_f32_bf16(edge, ctx=ctx)) == [0x7F7F, 0x7F80, 0xFF80, 0x0000, 0x8000]


@pytest.mark.parametrize("n,offset", [(8, 0), (1000003, 0), (77, 4), (4096, 2)])
def test_tails_and_unaligned_storage(ctx, n, offset):
    x = _narrow_corpus()[:n + offset]
    dx = ctx.to_device(x)
    dy = ctx.alloc((n + offset) * 2 + 64)
    try:
        ctx.convert(L.CONVERT_NARROW_F32_BF16, dx.offset(4 * offset), n, dy.offset(2 * offset))
        ctx.synchronize()
        got = dy.download(np.uint16, (n + offset,))[offset:]
    finally:
        dx.free(); dy.free()
    assert np.array_equal(got, oracle.bf16_narrow(x[offset:]))
    b = ALL_BF16[:n + offset] if n + offset <= ALL_BF16.size else np.resize(ALL_BF16, n + offset)
    db = ctx.to_device(b)
    dw = ctx.alloc((n + offset) * 4)
    try:
        ctx.convert(L.CONVERT_WIDEN_BF16_F32, db.offset(2 * offset), n, dw.offset(4 * offset))
        ctx.synchronize()
        gotw = dw.download(np.uint32, (n + offset,))[offset:]
    finally:
        db.free(); dw.free()
    assert np.array_equal(gotw, b[offset:].astype(np.uint32) << 16)


def test_round_trips(ctx):
    finite = ALL_BF16[(ALL_BF16 & 0x7F80) != 0x7F80]
    assert np.array_equal(families.narrow_f32_bf16(families.widen_bf16_f32(finite, ctx=ctx), ctx=ctx), finite)
    nans = ALL_BF16[((ALL_BF16 & 0x7F80) == 0x7F80) & ((ALL_BF16 & 0x7F) != 0)]
    assert (families.narrow_f32_bf16(families.widen_bf16_f32(nans, ctx=ctx), ctx=ctx) == 0x7FC0).all()


@pytest.mark.parametrize("direction", [L.CONVERT_NARROW_F32_BF16, L.CONVERT_WIDEN_BF16_F32])
def test_routed_conversion(ctx, direction):
    if direction == L.CONVERT_NARROW_F32_BF16:
        src = _narrow_corpus()[:1 << 18]
        want, out_t = oracle.bf16_narrow(src), np.uint16
    else:
        src = np.resize(ALL_BF16, 1 << 18)
        want, out_t = (src.astype(np.uint32) << 16), np.uint32
    rz = realize(L.PROGRAM_CONVERT, (src.size,), variant=direction, ctx=ctx)
    ds, dd = ctx.to_device(src), ctx.alloc(src.size * np.dtype(out_t).itemsize)
    try:
        route(ctx, rz, [ds, dd])
        got = dd.download(out_t, (src.size,))
    finally:
        ds.free(); dd.free()
    assert np.array_equal(got, want)
