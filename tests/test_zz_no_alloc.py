"""GPU: tiler_hip_sum_f32_noalloc -- the sum with its partials in the
library's static device array -- gives the bits tiler_hip_sum_f32 gives, on
two calls in a row (the second smaller, so stale partials from the first
would show), for the tree and the multi-pass split (the latter beyond the
context workspace, where tiler_hip_sum_f32 allocates on the stream), and
refuses partials beyond the array's 8 MiB.  Called through the C ABI."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from helpers import bits
from tiler_amd import _lib as L

pytestmark = pytest.mark.gpu


def _sum(ctx, fn, dx, rows, extent, do, plan):
    st = getattr(L.lib(), fn)(ctx.handle, dx.ptr, rows, extent, do.ptr, ctypes.byref(plan), None)
    return st


@pytest.mark.parametrize("calls", [
    # (topology, rows, extent, partitions) per call: first large, then smaller
    [(L.SUM_TREE, 1, 1 << 24, 0), (L.SUM_TREE, 1, 1000003, 0)],
    [(L.SUM_MULTIPASS, 64, 1 << 16, 256), (L.SUM_MULTIPASS, 16, 1 << 12, 64)],
    [(L.SUM_MULTIPASS, 1024, 1 << 15, 512), (L.SUM_MULTIPASS, 100, 1 << 14, 128)],
])
def test_noalloc_sum_matches_the_allocating_entry_point(ctx, calls):
    rng = np.random.default_rng(31)
    for topology, rows, extent, parts in calls:
        print(f"[noalloc] topology={topology} rows={rows} extent={extent} partitions={parts}", flush=True)
        x = rng.uniform(-1, 1, rows * extent).astype(np.float32)
        plan = L.SumPlan(topology, 0, parts, 0, extent // parts if parts else 0, 0)
        dx, d1, d2 = ctx.to_device(x), ctx.alloc(4 * rows), ctx.alloc(4 * rows)
        try:
            assert _sum(ctx, "tiler_hip_sum_f32", dx, rows, extent, d1, plan) == L.OK
            assert _sum(ctx, "tiler_hip_sum_f32_noalloc", dx, rows, extent, d2, plan) == L.OK, ctx.diagnostic()
            ctx.synchronize()
            want = d1.download(np.float32, (rows,))
            got = d2.download(np.float32, (rows,))
        finally:
            for b in (dx, d1, d2):
                b.free()
        assert np.array_equal(bits(got), bits(want))


def test_noalloc_sum_refuses_partials_beyond_its_array(ctx):
    rows, extent, parts = 4096, 1 << 11, 1024      # 4096 * 1024 partials = 16 MiB
    plan = L.SumPlan(L.SUM_MULTIPASS, 0, parts, 0, extent // parts, 0)
    dx, do = ctx.alloc(4 * rows * extent), ctx.alloc(4 * rows)
    try:
        assert _sum(ctx, "tiler_hip_sum_f32_noalloc", dx, rows, extent, do, plan) == L.REFUSE_CAPACITY
        assert "8 MiB" in ctx.diagnostic()
    finally:
        dx.free(); do.free()
