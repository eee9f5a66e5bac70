"""GPU: empty inputs and argument refusals on the device path.

Empty reductions commit the empty identity (+0.0, tiler-reference
src/evaluate.rs:498-589); empty maps, rows and contractions over zero
outputs launch nothing and leave the output untouched; an empty contracted
extent refuses (contraction.rs:420-428).  Every buffer here is allocated at
the size the call is given, so no case reaches memory it does not own.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import tiler_amd
from helpers import bits
from tiler_amd import _lib as L

pytestmark = pytest.mark.gpu

SENTINEL = 0xDEADBEEF


def _sentinel(ctx, words):
    buf = ctx.alloc(4 * words)
    ctx.fill_u32(buf, SENTINEL, words)
    return buf


def _words(buf, n):
    return buf.download(np.uint32, (n,))


@pytest.mark.parametrize("topology", [L.SUM_TREE, L.SUM_SERIAL])
def test_empty_sum_commits_positive_zero(ctx, topology):
    x = ctx.alloc(16)
    out = _sentinel(ctx, 1)
    try:
        ctx.sum_f32(x, 1, 0, out, topology=topology)
        ctx.synchronize()
        assert _words(out, 1)[0] == 0x00000000
        assert bits(oracle.strict_sum(np.zeros(0, np.float32), (0,), 0))[0] == 0x00000000
    finally:
        x.free(); out.free()


def test_empty_rows_leave_outputs_untouched(ctx):
    x, w = ctx.alloc(64), ctx.alloc(64)
    y = _sentinel(ctx, 16)
    try:
        ctx.rms_norm(L.BF16, x, w, 0, 16, 0x3727C5AC, y)
        ctx.rms_norm(L.F32, x, w, 4, 0, 0x3727C5AC, y)
        ctx.softmax_f32(x, 0, 16, y)
        ctx.softmax_f32(x, 4, 0, y)
        ctx.map(L.MAP_SILU, L.F32, x, 0, y)
        ctx.contract_bf16(x, w, 0, 8, 8, y)
        ctx.contract_strict_f32(x, w, 8, 0, 8, y)
        ctx.synchronize()
        assert (_words(y, 16) == SENTINEL).all()
    finally:
        x.free(); w.free(); y.free()


def test_empty_contracted_extent_refuses(ctx):
    a, b, c = ctx.alloc(64), ctx.alloc(64), _sentinel(ctx, 16)
    try:
        with pytest.raises(tiler_amd.Refusal):
            ctx.contract_bf16(a, b, 2, 2, 0, c)
        with pytest.raises(tiler_amd.Refusal):
            ctx.contract_strict_f32(a, b, 2, 2, 0, c)
        ctx.synchronize()
        assert (_words(c, 16) == SENTINEL).all()
    finally:
        a.free(); b.free(); c.free()


def test_rms_norm_dtype_and_map_op_refusals(ctx):
    x, y = ctx.alloc(64), ctx.alloc(64)
    try:
        with pytest.raises(tiler_amd.Refusal):
            ctx.rms_norm(7, x, x, 1, 8, 0x3727C5AC, y)
        with pytest.raises(tiler_amd.Refusal):
            ctx.map(99, L.F32, x, 8, y)
    finally:
        x.free(); y.free()


def test_single_element_rows(ctx):
    xs = np.array([[3.0], [-0.0], [np.inf]], np.float32)
    dx, dy = ctx.to_device(xs), ctx.alloc(xs.nbytes)
    try:
        ctx.softmax_f32(dx, 3, 1, dy)
        ctx.synchronize()
        got = dy.download(np.float32, xs.shape)
    finally:
        dx.free(); dy.free()
    assert np.array_equal(bits(got), bits(oracle.softmax_f32(xs, xs.shape, 1).reshape(xs.shape)))
