"""GPU: realized regions routed through the RuntimeAdapter seam.

For each family the region is realized (`tiler_hip_realize`, with the bound
device deciding tile sizes and groupings), routed the way route_with_adapter
drives an adapter:
1. prepare the payload entries;
2. plan, acquiring nothing;
3. allocate scratch after the commit;
4. dispatch.

The result is compared bit for bit with the family entry point's on the same
inputs, and with the oracle where the family is bit-exact. Routing refusals
(storage too small, misaligned against the realization's assumption, missing)
arrive before anything is committed.
"""
from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

import oracle
from helpers import bf16_widen, bits
from tiler_amd import _lib as L
from tiler_amd.realize import realize, route
from tiler_amd.runtime import GatherIndexOutOfBounds, Refusal

pytestmark = pytest.mark.gpu

EPS = 0x3727C5AC


def _routed(ctx, rz, inputs, outputs):
    """Routes `rz` with device copies of `inputs` and fresh `outputs`
    ((dtype, shape) per output slot); returns the outputs on the host."""
    dev_in = [ctx.to_device(a) for a in inputs]
    dev_out = [ctx.alloc(max(1, int(np.prod(shape)) * np.dtype(dt).itemsize)) for dt, shape in outputs]
    storage, i_in, i_out = [], 0, 0
    for role, _ in rz.slots:
        if role == L.SLOT_INPUT:
            storage.append(dev_in[i_in]); i_in += 1
        elif role == L.SLOT_OUTPUT:
            storage.append(dev_out[i_out]); i_out += 1
        else:
            storage.append(None)
    try:
        route(ctx, rz, storage)
        return [b.download(dt, shape) for b, (dt, shape) in zip(dev_out, outputs)]
    finally:
        for b in dev_in + dev_out:
            b.free()


@pytest.mark.parametrize("rows,extent,symbol", [(1000, 37, "tiler_sum_f32_staged_r256_u"),
                                               (1000, 9, "tiler_sum_f32_serial"),
                                               (3, 5000, "tiler_sum_f32_staged_r1")])
def test_serial_sum_routed(ctx, rows, extent, symbol):
    x = np.random.default_rng(71).standard_normal((rows, extent)).astype(np.float32)
    rz = realize(L.PROGRAM_SERIAL_SUM, (rows, extent), topology=L.SUM_SERIAL, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    assert rz.symbols == [symbol]
    (got,) = _routed(ctx, rz, [x], [(np.float32, (rows,))])
    assert np.array_equal(bits(got), bits(oracle.strict_sum(x, (rows, extent), 1)))


@pytest.mark.parametrize("topology,rows,extent,grouping,flags", [
    (L.SUM_MULTIPASS, 7, 120, (4, 30), L.REGION_ALIGNED16),
    (L.SUM_MULTIPASS, 40, 4000, (200, 20), L.REGION_ALIGNED16),   # partials beyond the context workspace
    (L.SUM_COOPERATIVE, 5, 24, (4, 3, 2), L.REGION_ALIGNED16 | L.REGION_PARTICIPANT_MAJOR),
    (L.SUM_TREE, 1, (1 << 20) + 3, (), L.REGION_ALIGNED16),
    (L.SUM_TREE, 33, 5000, (), L.REGION_ALIGNED16),
])
def test_grouped_sums_routed(ctx, topology, rows, extent, grouping, flags):
    x = np.random.default_rng(rows + extent).uniform(-1, 1, (rows, extent)).astype(np.float32)
    rz = realize(L.PROGRAM_SERIAL_SUM, (rows, extent), topology=topology, grouping=grouping, flags=flags, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [x], [(np.float32, (rows,))])
    from tiler_amd import families
    if topology == L.SUM_MULTIPASS:
        want = families.strict_partitioned_sum(x, (rows, extent), 1, grouping[0], grouping[1], ctx=ctx)
    elif topology == L.SUM_COOPERATIVE:
        want = families.cooperative_grouped_sum(x, (rows, extent), 1, grouping[0], grouping[1], grouping[2],
                                                participant_major=True, ctx=ctx)
    else:
        want = families.tree_sum(x, (rows, extent), 1, ctx=ctx)
    assert np.array_equal(bits(got).reshape(-1), bits(want).reshape(-1))


@pytest.mark.parametrize("dtype,rows,extent", [(L.BF16, 64, 4096), (L.F32, 9, 1000), (L.BF16, 3, 20000)])
def test_rms_norm_routed(ctx, dtype, rows, extent):
    rng = np.random.default_rng(rows * extent)
    if dtype == L.BF16:
        x = oracle.bf16_narrow(rng.standard_normal((rows, extent)).astype(np.float32))
        w = oracle.bf16_narrow(rng.normal(1.0, 0.1, extent).astype(np.float32))
        out_t = np.uint16
    else:
        x = rng.standard_normal((rows, extent)).astype(np.float32)
        w = rng.normal(1.0, 0.1, extent).astype(np.float32)
        out_t = np.float32
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=dtype, scalars=(EPS,),
                 flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [x, w], [(out_t, (rows, extent))])
    dx, dw, dy = ctx.to_device(x), ctx.to_device(w), ctx.alloc(x.nbytes)
    try:
        ctx.rms_norm(dtype, dx, dw, rows, extent, EPS, dy, weight_broadcast=True)
        want = dy.download(out_t, (rows, extent))
    finally:
        dx.free(); dw.free(); dy.free()
    assert np.array_equal(got.view(np.uint16 if dtype == L.BF16 else np.uint32),
                          want.view(np.uint16 if dtype == L.BF16 else np.uint32))


@pytest.mark.parametrize("rows,extent", [(64, 2048), (5, 300), (2, 40000), (150, 20001)])
def test_softmax_routed(ctx, rows, extent):
    x = (np.random.default_rng(extent).standard_normal((rows, extent)) * 3).astype(np.float32)
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [x], [(np.float32, (rows, extent))])
    import tiler_amd
    vec, waves, seg = tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.F32, extent)
    assert np.array_equal(bits(got).reshape(-1), bits(oracle.softmax_grouped(x, rows, extent, vec, waves, seg)))


@pytest.mark.parametrize("op,n", [(L.MAP_ADD, 4096), (L.MAP_MULTIPLY, 1001), (L.MAP_SILU, 8192), (L.MAP_SILU, 77)])
def test_maps_routed(ctx, op, n):
    rng = np.random.default_rng(n + op)
    x = (rng.standard_normal(n) * 5).astype(np.float32)
    x2 = rng.standard_normal(n).astype(np.float32)
    rz = realize(L.PROGRAM_POINTWISE, (n,), variant=op, ctx=ctx)
    binary = op in (L.MAP_ADD, L.MAP_MULTIPLY)
    (got,) = _routed(ctx, rz, [x, x2] if binary else [x], [(np.float32, (n,))])
    if op == L.MAP_ADD:
        want = x + x2            # one binary32 rounding; no NaN among these operands
    elif op == L.MAP_MULTIPLY:
        want = x * x2
    else:
        want = oracle.silu_f32(x)
    assert np.array_equal(bits(got), bits(np.asarray(want, np.float32).reshape(-1)))


def test_broadcast_and_gather_routed(ctx):
    rng = np.random.default_rng(72)
    w = rng.integers(0, 1 << 16, 4096, dtype=np.uint16)
    rz = realize(L.PROGRAM_BROADCAST, (8, 4096), variant=2, rank=2, strides=(0, 1), grouping=(4096,), ctx=ctx)
    (got,) = _routed(ctx, rz, [w], [(np.uint16, (8, 4096))])
    assert np.array_equal(got, np.broadcast_to(w, (8, 4096)))

    table = rng.integers(0, 1 << 16, (500, 256), dtype=np.uint16)
    idx = rng.integers(0, 500, 300).astype(np.uint32)
    rz = realize(L.PROGRAM_GATHER, (1, 500, 256, 300), variant=2, ctx=ctx)
    assert rz.symbols == ["tiler_fill_u32", "tiler_gather_u128"]
    (got,) = _routed(ctx, rz, [table, idx], [(np.uint16, (300, 256))])
    assert np.array_equal(got, table[idx])


def test_gather_record_reports_post_commit(ctx):
    """An index the host did not validate is caught by the kernel's own bound
    check (its run is skipped, nothing is read out of range) and surfaces as
    the post-commit failure naming the lowest position."""
    table = np.arange(40 * 8, dtype=np.uint32).reshape(40, 8)
    idx = np.array([3, 39, 40, 7, 1000], np.uint32)
    rz = realize(L.PROGRAM_GATHER, (1, 40, 8, 5), variant=4, ctx=ctx)
    with pytest.raises(GatherIndexOutOfBounds) as e:
        _routed(ctx, rz, [table, idx], [(np.uint32, (5, 8))])
    assert e.value.position == 2 and not e.value.fallback_permitted


@pytest.mark.parametrize("m,n,k,silu", [(512, 512, 256, True), (16, 1024, 512, False), (300, 130, 72, True)])
def test_bf16_contraction_routed(ctx, m, n, k, silu):
    rng = np.random.default_rng(m + n + k)
    a = oracle.bf16_narrow((rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32))
    b = oracle.bf16_narrow((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))
    ep = L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16, variant=ep, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [a, b], [(np.uint16, (m, n))])
    from tiler_amd import families
    assert np.array_equal(got, families.contract_bf16(a, b, ep, ctx=ctx))


def test_strict_contraction_routed(ctx):
    rng = np.random.default_rng(73)
    a = rng.standard_normal((40, 9)).astype(np.float32)
    b = rng.standard_normal((70, 9)).astype(np.float32)
    rz = realize(L.PROGRAM_CONTRACTION, (40, 70, 9), permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [a, b], [(np.float32, (40, 70))])
    assert np.array_equal(bits(got).reshape(-1), bits(oracle.contract_strict_f32(a, b, 40, 70, 9)).reshape(-1))


def test_route_refuses_before_commit(ctx):
    rz = realize(L.PROGRAM_SOFTMAX, (4, 256), permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    x = ctx.alloc(4 * 256 * 4)
    small = ctx.alloc(64)
    try:
        with pytest.raises(Refusal):
            route(ctx, rz, [x, small])                  # output slot too small
        with pytest.raises(Refusal):
            route(ctx, rz, [x.offset(4), x])            # not 16-byte aligned as assumed
        with pytest.raises(Refusal):
            route(ctx, rz, [x, None])                   # an output needs caller storage
        with pytest.raises(Refusal):
            route(ctx, rz, [x])                         # one binding per slot
    finally:
        x.free(); small.free()


LIVE = L.REGION_ALIGNED16 | L.REGION_LIVE_EXTENT


def _route_live(ctx, rz, bufs, a, b, k, out_dtype, m, n):
    """Routes one live-k realization with A [m, k] and B [n, k] packed at the
    start of bound-sized slots; returns C [m, n]."""
    bufs[0].upload(np.ascontiguousarray(a))
    bufs[1].upload(np.ascontiguousarray(b))
    print(f"[live k] {rz.symbols} m={m} n={n} k={k}", flush=True)
    route(ctx, rz, bufs, extents=(k,))
    return bufs[2].download(out_dtype, (m, n))


@pytest.mark.parametrize("dtype,variant,permissions", [
    (L.F32, L.EPILOGUE_NONE, 0),                                   # the strict f32 fold
    (L.BF16, L.EPILOGUE_SILU, 0),                                  # strict bf16 fold, then SiLU
    (L.BF16, L.EPILOGUE_SILU, L.PERMITS_REASSOCIATION),            # the general MFMA form
    (L.BF16, L.EPILOGUE_NONE, L.PERMITS_REASSOCIATION),
])
def test_live_contracted_extent_routes_every_value(ctx, dtype, variant, permissions):
    """One realization (LiveContraction: k read at dispatch) routed at several
    k up to the bound it was sized for, each result against the oracle at
    that k: the strict folds bit for bit, the MFMA form within 1e-2 relative
    Frobenius of the f64 contraction of the widened operands."""
    m, n, bound = 300, 264, 200
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, bound), dtype=dtype, variant=variant, permissions=permissions,
                 flags=LIVE, ctx=ctx)
    assert rz.live_extents == [(0, 1, 1, bound)]
    bufs = [ctx.alloc(nbytes) for _, nbytes in rz.slots]
    try:
        for k in (1, 7, 64, 131, bound):
            rng = np.random.default_rng(k)
            a = rng.standard_normal((m, k)).astype(np.float32)
            b = rng.standard_normal((n, k)).astype(np.float32)
            if dtype == L.F32:
                got = _route_live(ctx, rz, bufs, a, b, k, np.float32, m, n)
                assert np.array_equal(bits(got).reshape(-1), bits(oracle.contract_strict_f32(a, b, m, n, k)).reshape(-1)), k
                continue
            a16, b16 = oracle.bf16_narrow(a), oracle.bf16_narrow(b)
            got = _route_live(ctx, rz, bufs, a16, b16, k, np.uint16, m, n)
            if not permissions:
                want = oracle.contract_general(a16, "mk", b16, "nk", "mn", silu=variant == L.EPILOGUE_SILU)
                assert np.array_equal(got, want), k
                continue
            wide = bf16_widen(a16).astype(np.float64) @ bf16_widen(b16).astype(np.float64).T
            if variant == L.EPILOGUE_SILU:
                wide = oracle.silu_f32(wide.astype(np.float32).reshape(-1)).reshape(m, n).astype(np.float64)
            g = bf16_widen(got).astype(np.float64)
            assert np.linalg.norm(g - wide) / np.linalg.norm(wide) <= 1e-2, k
    finally:
        for x in bufs:
            x.free()


def test_live_extent_outside_its_range_is_refused_before_commit(ctx):
    m, n, bound = 40, 70, 64
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, bound), flags=LIVE, ctx=ctx)
    bufs = [ctx.alloc(nbytes) for _, nbytes in rz.slots]
    try:
        for k in (0, bound + 1, 1 << 32):
            with pytest.raises(Refusal) as e:
                route(ctx, rz, bufs, extents=(k,))
            assert e.value.status == L.REFUSE_CAPACITY, k
        with pytest.raises(Refusal) as e:
            route(ctx, rz, bufs)                        # the live extent's value is not supplied
        assert e.value.status == L.REFUSE_BINDING_MISMATCH
        with pytest.raises(Refusal):
            route(ctx, realize(L.PROGRAM_CONTRACTION, (m, n, bound), ctx=ctx), bufs, extents=(3,))
    finally:
        for x in bufs:
            x.free()


@pytest.mark.parametrize("dtype", [L.F32, L.BF16])
def test_live_contracted_extent_decode_shape(ctx, dtype):
    """A decode-shaped LiveContraction (m = 8 rows, n = 1000, k bound 5000):
    the f32 region runs the staged strict fold along B's rows
    (tiler_contract_strict_f32_s*_u, whose rows per workgroup and stages were
    sized from the bound), the bf16 region the register-blocked strict tiles.
    Routed at k far below the bound, at k not a multiple of 4 and at the
    bound, each bit for bit with the strict fold at that k."""
    m, n, bound = 8, 1000, 5000
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, bound), dtype=dtype, flags=LIVE, ctx=ctx)
    if dtype == L.F32:
        assert re.fullmatch(r"tiler_contract_strict_f32_s\d+_u", rz.symbols[0]), rz.symbols
    else:
        assert rz.symbols[0].startswith("tiler_contract_strict_bf16"), rz.symbols
    bufs = [ctx.alloc(nbytes) for _, nbytes in rz.slots]
    try:
        for k in (1, 7, 130, 4999, bound):
            rng = np.random.default_rng(k + 1)
            a = rng.standard_normal((m, k)).astype(np.float32)
            b = rng.standard_normal((n, k)).astype(np.float32)
            if dtype == L.F32:
                got = _route_live(ctx, rz, bufs, a, b, k, np.float32, m, n)
                want = oracle.contract_strict_f32(a, b, m, n, k)
                assert np.array_equal(bits(got).reshape(-1), bits(want).reshape(-1)), k
            else:
                a16, b16 = oracle.bf16_narrow(a).reshape(m, k), oracle.bf16_narrow(b).reshape(n, k)
                got = _route_live(ctx, rz, bufs, a16, b16, k, np.uint16, m, n)
                assert np.array_equal(got, oracle.contract_general(a16, "mk", b16, "nk", "mn")), k
    finally:
        for x in bufs:
            x.free()


def test_dispatch_rechecks_live_extents_and_requires_ranges(ctx):
    """A plan whose live extent lies outside its range, or that carries
    values without ranges, is refused at plan_dispatch and fails at dispatch
    before any entry is launched (the output slot keeps its contents)."""
    from tiler_amd.realize import _prepared
    m, n, bound = 40, 70, 64
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, bound), flags=LIVE, ctx=ctx)
    e = rz.raw.entries[0]
    count = e.binding_count
    slots = (ctypes.c_uint32 * count)(*e.binding_slots[:count])
    offs = (ctypes.c_uint32 * count)(*e.binding_offsets[:count])
    ids = (ctypes.c_uint32 * e.extent_count)(*e.extent_ids[:e.extent_count])
    xoffs = (ctypes.c_uint32 * e.extent_count)(*e.extent_offsets[:e.extent_count])
    ka = ctypes.create_string_buffer(bytes(e.kernargs[:e.kernarg_bytes]), e.kernarg_bytes)
    de = L.DispatchEntry(_prepared(ctx, rz.symbols[0]), (ctypes.c_uint32 * 3)(*e.grid), (ctypes.c_uint32 * 3)(*e.block),
                         0, ctypes.cast(ka, ctypes.c_void_p), e.kernarg_bytes, count, slots, offs,
                         e.extent_count, ids, xoffs)
    sb = (ctypes.c_uint64 * len(rz.slots))(*[b for _, b in rz.slots])
    bufs = [ctx.alloc(b) for _, b in rz.slots]
    ptrs = (ctypes.c_void_p * len(bufs))(*[x.ptr for x in bufs])
    ranges = (L.LiveExtent * 1)(*rz.raw.live_extents[:1])
    try:
        ctx.fill_u32(bufs[2], 0x7FC00001, m * n)
        ctx.synchronize()
        too_big = (ctypes.c_uint64 * 1)(bound + 1)
        plan = L.DispatchPlan(len(rz.slots), sb, 1, ctypes.pointer(de), None, 1, too_big, ranges)
        assert L.lib().tiler_hip_plan_dispatch(ctx.handle, ctypes.byref(plan)) == L.REFUSE_CAPACITY
        assert L.lib().tiler_hip_dispatch(ctx.handle, ctypes.byref(plan), ptrs) == L.FAIL_LAUNCH
        ok = (ctypes.c_uint64 * 1)(bound)
        bare = L.DispatchPlan(len(rz.slots), sb, 1, ctypes.pointer(de), None, 1, ok, None)
        assert L.lib().tiler_hip_plan_dispatch(ctx.handle, ctypes.byref(bare)) == L.REFUSE_INVALID_ARGUMENT
        assert L.lib().tiler_hip_dispatch(ctx.handle, ctypes.byref(bare), ptrs) == L.FAIL_LAUNCH
        assert (bufs[2].download(np.uint32, (m * n,)) == 0x7FC00001).all()  # nothing ran
    finally:
        for x in bufs:
            x.free()


def test_workspace_calls_refuse_a_foreign_stream(ctx):
    """The tree sum's partials, the split softmax's partials and the gather
    record live in the context workspace, ordered by the context's stream
    only: given another stream (here a second context's) those calls refuse
    before anything is enqueued; calls that bind no workspace (RMSNorm) run
    on any stream; the context's own stream, given explicitly, is accepted."""
    import tiler_amd
    other = tiler_amd.Context(0)
    x = np.ones((1, 1 << 20), np.float32)
    dx, dout = ctx.to_device(x), ctx.alloc(4)
    dy = ctx.alloc(x.nbytes)
    idx = ctx.to_device(np.zeros(4, np.uint32))
    try:
        foreign = other.stream
        with pytest.raises(Refusal) as e:
            ctx.sum_f32(dx, 1, 1 << 20, dout, topology=L.SUM_TREE, stream=foreign)
        assert e.value.status == L.REFUSE_UNSUPPORTED
        with pytest.raises(Refusal) as e:
            ctx.softmax_f32(dx, 1, 1 << 20, dy, stream=foreign)
        assert e.value.status == L.REFUSE_UNSUPPORTED
        with pytest.raises(Refusal) as e:
            ctx.gather(dx, 1, 1 << 20, 1, 4, idx, 4, dy, stream=foreign)
        assert e.value.status == L.REFUSE_UNSUPPORTED
        ctx.sum_f32(dx, 1, 1 << 20, dout, topology=L.SUM_TREE, stream=ctx.stream)
        ctx.synchronize()
        assert dout.download(np.float32, (1,))[0] == np.float32(1 << 20)
        w = ctx.to_device(np.ones(1 << 10, np.float32))
        try:
            ctx.rms_norm(L.F32, dx, w, 1 << 10, 1 << 10, 0x3727C5AC, dy, stream=foreign)
            other.synchronize()
        finally:
            w.free()
    finally:
        for b in (dx, dout, dy, idx):
            b.free()
        other.close()
