"""GPU: seeded random shapes for every family against the oracle.

Each case draws its shape (and, where the family has them, the axis, offsets
and groupings) from a fixed seed, so a failure names a reproducible case.
Sizes stay small enough for the oracle to finish in well under a second each.
Comparison is bit-exact wherever the oracle restates the kernel's order (or
its declared grouping), and to the contraction's 1e-2 relative Frobenius bound
for the bf16 MFMA path.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import tiler_amd
from helpers import bf16_widen, bits
from tiler_amd import _lib as L
from tiler_amd import families

pytestmark = pytest.mark.gpu

EPS = 0x3727C5AC
CASES = 12


def _rng(case, salt):
    return np.random.default_rng(1000 * salt + case)


@pytest.mark.parametrize("case", range(CASES))
def test_sums(ctx, case):
    r = _rng(case, 1)
    rank = int(r.integers(1, 4))
    shape = tuple(int(v) for v in r.integers(1, 40, rank))
    axis = int(r.integers(0, rank))
    x = (r.standard_normal(shape) * 10).astype(np.float32)
    assert np.array_equal(bits(families.strict_sum(x, shape, axis, ctx=ctx)).reshape(-1),
                          bits(oracle.strict_sum(x, shape, axis)).reshape(-1)), (shape, axis)
    extent = shape[axis]
    parts = [p for p in range(1, extent + 1) if extent % p == 0]
    p = parts[int(r.integers(0, len(parts)))]
    got = families.strict_partitioned_sum(x, shape, axis, p, extent // p, ctx=ctx)
    moved = np.moveaxis(x, axis, -1)
    want = oracle.strict_partitioned_sum(moved, moved.size // extent, extent, p, extent // p)
    assert np.array_equal(bits(got).reshape(-1), bits(want).reshape(-1))


def _staged_shape(r, max_elements):
    """(rows, extent) spread over every staged form: rows from 1 to 20000,
    extents from 16 to 20000, at most `max_elements` in all."""
    rows = int(np.exp(r.uniform(0, np.log(20000))))
    extent = int(np.exp(r.uniform(np.log(16), np.log(20000))))
    while rows * extent > max_elements:
        rows = max(1, rows // 2)
        extent = max(16, extent * 3 // 4)
    return rows, extent


@pytest.mark.parametrize("case", range(CASES))
def test_staged_folds(ctx, case):
    """Random rows and extents, an aligned or unaligned base: the strict
    serial fold (staged for rows of >= 16), the multi-pass split at the
    reference's partition, the workgroup tree over rows, each bit for bit."""
    from tiler_amd.calibrate import split_partitions
    r = _rng(case, 9)
    rows, extent = _staged_shape(r, 2_000_000)
    offset = int(r.choice([0, 4]))
    x = (r.standard_normal((rows, extent)) * np.exp2(r.integers(-30, 30, (rows, extent)))).astype(np.float32)
    if rows > 1:
        x[0] = -0.0
    dx, do = ctx.alloc(x.nbytes + offset), ctx.alloc(rows * 4)
    try:
        src = dx.offset(offset)
        src.upload(x)
        print(f"[staged folds] case {case}: rows={rows} extent={extent} offset={offset}", flush=True)
        ctx.sum_f32(src, rows, extent, do, topology=L.SUM_SERIAL)
        assert np.array_equal(bits(do.download(np.float32, (rows,))), bits(oracle.strict_sum(x, (rows, extent), 1)))
        p = split_partitions(extent)
        if extent % p == 0:
            ctx.sum_f32(src, rows, extent, do, topology=L.SUM_MULTIPASS, partitions=p, per_partition=extent // p)
            want = oracle.strict_partitioned_sum(x, rows, extent, p, extent // p)
            assert np.array_equal(bits(do.download(np.float32, (rows,))), bits(want))
        if rows > 1:
            ctx.sum_f32(src, rows, extent, do, topology=L.SUM_TREE)
            want = oracle.row_grouped_sum(x, rows, extent, 4, 4)
            assert np.array_equal(bits(do.download(np.float32, (rows,))), bits(want))
    finally:
        dx.free()
        do.free()


@pytest.mark.parametrize("case", range(CASES))
def test_strict_rows(ctx, case):
    """Random shapes through the strict (no reassociation) RMSNorm and
    softmax realizations, staged for rows of >= 64: bit for bit."""
    from tiler_amd.realize import realize, route
    r = _rng(case, 10)
    rows, extent = _staged_shape(r, 300_000)
    x = (r.standard_normal((rows, extent)) * 3).astype(np.float32)
    w = r.normal(1.0, 0.1, extent).astype(np.float32)
    print(f"[strict rows] case {case}: rows={rows} extent={extent}", flush=True)
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), scalars=(EPS,),
                 flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, ctx=ctx)
    bufs = [ctx.to_device(x), ctx.to_device(w), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[2].download(np.float32, x.shape)
    finally:
        for b in bufs:
            b.free()
    want = oracle.rms_norm_f32(x, np.broadcast_to(w, x.shape).copy(), x.shape, 1, EPS).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want)), rz.symbols
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), flags=L.REGION_ALIGNED16, ctx=ctx)
    bufs = [ctx.to_device(x), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[1].download(np.float32, x.shape)
    finally:
        for b in bufs:
            b.free()
    want = oracle.softmax_f32(x, x.shape, 1).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want)), rz.symbols


@pytest.mark.parametrize("case", range(8))
def test_resident_strict_rows(ctx, case):
    """Random shapes through the register-resident strict forms
    (tiler_{rms_norm_f32,rms_norm_bf16,softmax_f32}_strict_rr8_p*): 2048 to
    2600 rows (ragged last workgroups included), extents drawn over their
    whole range, bit for bit -- every RMSNorm row, and for the softmax 64
    sampled rows plus the last workgroup's."""
    from tiler_amd.realize import realize, route
    r = _rng(case, 11)
    rows = int(r.integers(2048, 2601))
    # f32 RMSNorm, extent a multiple of 4 in [64, 2048]
    extent = 4 * int(r.integers(16, 513))
    x = (r.standard_normal((rows, extent)) * 3).astype(np.float32)
    x[int(r.integers(rows)), int(r.integers(extent))] = np.nan
    w = r.normal(1.0, 0.1, extent).astype(np.float32)
    print(f"[resident rows] case {case}: rms f32 rows={rows} extent={extent}", flush=True)
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), scalars=(EPS,),
                 flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, ctx=ctx)
    assert "_strict_rr8_p" in rz.symbols[-1], rz.symbols
    bufs = [ctx.to_device(x), ctx.to_device(w), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[2].download(np.float32, x.shape)
    finally:
        for b in bufs:
            b.free()
    want = oracle.rms_norm_f32(x, np.broadcast_to(w, x.shape).copy(), x.shape, 1, EPS).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want)), rz.symbols
    # bf16 RMSNorm, extent a multiple of 8 in [128, 4096], a weight row per row
    extent = 8 * int(r.integers(16, 513))
    xb = oracle.bf16_narrow(r.standard_normal((rows, extent)).astype(np.float32)).reshape(rows, extent)
    wb = oracle.bf16_narrow(r.normal(1.0, 0.1, (rows, extent)).astype(np.float32)).reshape(rows, extent)
    print(f"[resident rows] case {case}: rms bf16 rows={rows} extent={extent}", flush=True)
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=L.BF16, scalars=(EPS,), flags=L.REGION_ALIGNED16,
                 ctx=ctx)
    assert "_strict_rr8_p" in rz.symbols[-1], rz.symbols
    bufs = [ctx.to_device(xb), ctx.to_device(wb), ctx.alloc(xb.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[2].download(np.uint16, xb.shape)
    finally:
        for b in bufs:
            b.free()
    wantf = oracle.rms_norm_f32(bf16_widen(xb), bf16_widen(wb), xb.shape, 1, EPS)
    assert np.array_equal(got.reshape(-1), oracle.bf16_narrow(wantf).reshape(-1)), rz.symbols
    # softmax, extent a multiple of 4 in [128, 4096]
    extent = 4 * int(r.integers(32, 1025))
    x = (r.standard_normal((rows, extent)) * 3).astype(np.float32)
    sample = np.unique(np.concatenate([r.choice(rows, 64, replace=False), np.arange(rows - rows % 8 - 8, rows)]))
    x[sample[3], int(r.integers(extent))] = np.nan
    x[sample[5]] = -np.inf
    print(f"[resident rows] case {case}: softmax rows={rows} extent={extent}", flush=True)
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), flags=L.REGION_ALIGNED16, ctx=ctx)
    assert "_strict_rr8_p" in rz.symbols[-1], rz.symbols
    bufs = [ctx.to_device(x), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[1].download(np.float32, x.shape)[sample]
    finally:
        for b in bufs:
            b.free()
    xs = np.ascontiguousarray(x[sample])
    want = oracle.softmax_f32(xs, xs.shape, 1).reshape(xs.shape)
    assert np.array_equal(bits(got), bits(want)), rz.symbols


def _tiny_rows(r, rows, extent, scale_log2):
    """Rows of magnitude 2^scale_log2 (their squares or exponents reach the
    subnormal range), every fifth row of ordinary values, a few subnormal
    entries planted."""
    x = (r.standard_normal((rows, extent)) * 2.0 ** scale_log2).astype(np.float32)
    x[::5] = r.standard_normal((len(range(0, rows, 5)), extent)).astype(np.float32)
    n = min(rows * extent, 64)
    sub = (r.integers(1, 1 << 23, n).astype(np.uint32) | (r.integers(0, 2, n).astype(np.uint32) << 31))
    x.reshape(-1)[r.choice(rows * extent, n, replace=False)] = sub.view(np.float32)
    return x


@pytest.mark.parametrize("case", range(10))
def test_strict_rows_under_modes(ctx, case):
    """Random shapes through the strict RMSNorm and softmax under a random
    flushing contract: the register-resident _m forms (2048 to 2600 rows) and
    the staged _m forms (1 to 1200 rows, aligned or not), bit for bit with the
    oracle under the same modes."""
    from tiler_amd.realize import realize, route
    r = _rng(case, 12)
    modes = [(2, 1), (1, 2), (2, 2), (3, 3), (2, 3), (3, 1)]
    im, rm = modes[int(r.integers(len(modes)))]
    resident = case % 2 == 0
    rows = int(r.integers(2048, 2601)) if resident else int(r.integers(1, 1201))
    dtype = L.BF16 if r.integers(2) else L.F32
    per16 = 8 if dtype == L.BF16 else 4
    if resident:
        extent = per16 * int(r.integers(16, 513))
    else:
        extent = int(r.integers(64, min(9000, 4_000_000 // rows) + 1))
    x = _tiny_rows(r, rows, extent, -70)
    w = r.normal(1.0, 0.1, extent).astype(np.float32)
    w[:3] = np.array([1, 0x80000001, 0x7FFFFF], np.uint32).view(np.float32)
    if dtype == L.BF16:
        x = bf16_widen(oracle.bf16_narrow(x)).reshape(x.shape)
        w = bf16_widen(oracle.bf16_narrow(w)).reshape(w.shape)
    print(f"[strict modes] case {case}: rms {'bf16' if dtype == L.BF16 else 'f32'} rows={rows} extent={extent} "
          f"modes=({im},{rm})", flush=True)
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=dtype, scalars=(EPS,), input_subnormals=im,
                 result_subnormals=rm, flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, ctx=ctx)
    assert rz.symbols[-1].endswith("_m") and ("_rr8_" in rz.symbols[-1]) == resident, rz.symbols
    host = [x, w] if dtype == L.F32 else [oracle.bf16_narrow(x).reshape(x.shape), oracle.bf16_narrow(w)]
    out = np.float32 if dtype == L.F32 else np.uint16
    bufs = [ctx.to_device(np.ascontiguousarray(h)) for h in host] + [ctx.alloc(rows * extent * np.dtype(out).itemsize)]
    try:
        route(ctx, rz, bufs)
        got = bufs[2].download(out, x.shape)
    finally:
        for b in bufs:
            b.free()
    want = oracle.rms_norm_f32(x, np.broadcast_to(w, x.shape).copy(), x.shape, 1, EPS, input_mode=im - 1,
                               result_mode=rm - 1).reshape(rows, extent)
    if dtype == L.BF16:
        assert np.array_equal(got, oracle.bf16_narrow(want).reshape(rows, extent)), rz.symbols
    else:
        assert np.array_equal(bits(got), bits(want)), rz.symbols
    # softmax: rows spread ~100 below their maximum, the same row counts
    extent = 4 * int(r.integers(32, 513)) if resident else int(r.integers(64, min(9000, 4_000_000 // rows) + 1))
    x = r.uniform(-100.0, 0.0, (rows, extent)).astype(np.float32)
    x[1::7] = _tiny_rows(r, len(range(1, rows, 7)), extent, -126)
    x[int(r.integers(rows)), int(r.integers(extent))] = np.nan
    print(f"[strict modes] case {case}: softmax rows={rows} extent={extent} modes=({im},{rm})", flush=True)
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), input_subnormals=im, result_subnormals=rm,
                 flags=L.REGION_ALIGNED16, ctx=ctx)
    assert rz.symbols[-1].endswith("_m") and ("_rr8_" in rz.symbols[-1]) == resident, rz.symbols
    bufs = [ctx.to_device(x), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[1].download(np.float32, x.shape)
    finally:
        for b in bufs:
            b.free()
    want = oracle.softmax_f32(x, x.shape, 1, input_mode=im - 1, result_mode=rm - 1).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want)), rz.symbols


@pytest.mark.parametrize("case", range(CASES))
def test_tree_sum(ctx, case):
    r = _rng(case, 2)
    n = int(r.integers(1, 200000))
    x = r.uniform(-1, 1, n).astype(np.float32)
    got = families.tree_sum(x, (n,), 0, ctx=ctx)
    assert bits(got)[0] == bits([oracle.grid_tree_sum(x, ctx.sum_tree_workgroups(n))])[0]


@pytest.mark.parametrize("case", range(CASES))
def test_rms_norm_bf16(ctx, case):
    r = _rng(case, 3)
    rows = int(r.integers(1, 9))
    extent = int(r.choice([int(r.integers(1, 9000)), int(r.integers(8193, 70000))]))
    xb = oracle.bf16_narrow(r.standard_normal((rows, extent)).astype(np.float32))
    wb = oracle.bf16_narrow(r.normal(1.0, 0.1, extent).astype(np.float32))
    got = families.rms_norm_bf16(xb, wb, EPS, ctx=ctx)
    vec, waves, _ = tiler_amd.row_grouping(L.ROWS_RMS_NORM, L.BF16, extent)
    y = oracle.rms_norm_grouped(bf16_widen(xb), bf16_widen(wb), rows, extent, EPS, True, vec, waves)
    assert np.array_equal(got, oracle.bf16_narrow(y).reshape(rows, extent)), (rows, extent)


@pytest.mark.parametrize("case", range(CASES))
def test_softmax(ctx, case):
    r = _rng(case, 4)
    rows = int(r.integers(1, 9))
    # short rows, rows of 2-4 segments (one workgroup per row) and longer
    # rows (one workgroup per segment, synchronized in one launch)
    extent = int(r.choice([int(r.integers(1, 9000)), int(r.integers(8193, 32769)),
                           int(r.integers(32769, 140000))]))
    x = (r.standard_normal((rows, extent)) * 4).astype(np.float32)
    if extent > 3:
        x[0, r.integers(0, extent, extent // 3)] = -np.inf
    got = families.softmax_f32((rows, extent), 1, x, ctx=ctx).reshape(rows, extent)
    vec, waves, seg = tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.F32, extent)
    want = oracle.softmax_grouped(x, rows, extent, vec, waves, seg).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want)), (rows, extent)


@pytest.mark.parametrize("case", range(CASES))
def test_gather(ctx, case):
    r = _rng(case, 5)
    rank = int(r.integers(1, 4))
    shape = tuple(int(v) for v in r.integers(1, 30, rank))
    axis = int(r.integers(0, rank))
    dtype = [np.uint8, np.uint16, np.uint32, np.uint64][int(r.integers(0, 4))]
    src = r.integers(0, np.iinfo(dtype).max, shape, dtype=dtype)
    idx = r.integers(0, shape[axis], tuple(int(v) for v in r.integers(0, 6, int(r.integers(0, 3)))))
    got = families.gather(src, axis, idx.astype(np.uint32), ctx=ctx)
    assert np.array_equal(got, np.take(src, idx, axis=axis))


@pytest.mark.parametrize("case", range(CASES))
def test_contractions(ctx, case):
    r = _rng(case, 6)
    m, n, k = (int(v) for v in r.integers(1, 300, 3))
    if case % 3 == 0:  # shapes on the staged path's 8-element grid
        n, k = 8 * max(1, n // 8), 8 * max(1, k // 8)
    a = r.standard_normal((m, k)).astype(np.float32) / np.float32(np.sqrt(k))
    b = r.standard_normal((n, k)).astype(np.float32) / np.float32(np.sqrt(k))
    ref = oracle.contract_strict_f32(a, b, m, n, k)
    got = families.contract_strict_f32(a, b, ctx=ctx)
    assert np.array_equal(bits(got).reshape(-1), bits(ref).reshape(-1))
    ab, bb = oracle.bf16_narrow(a), oracle.bf16_narrow(b)
    silu = bool(case % 2)
    gb = families.contract_bf16(ab, bb, L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE, ctx=ctx)
    rb = oracle.contract_strict_f32(bf16_widen(ab), bf16_widen(bb), m, n, k).reshape(m, n)
    if silu:
        rb = oracle.silu_f32(rb).reshape(m, n)
    g = bf16_widen(gb).astype(np.float64)
    den = np.linalg.norm(rb.astype(np.float64))
    if den > 0:
        assert np.linalg.norm(g - rb) / den <= 1e-2, (m, n, k, silu)


@pytest.mark.parametrize("case", range(CASES))
def test_maps(ctx, case):
    r = _rng(case, 7)
    n = int(r.integers(1, 20000))
    x = (r.standard_normal(n) * 6).astype(np.float32)
    assert np.array_equal(bits(families.silu_f32(x, ctx=ctx)), bits(oracle.silu_f32(x)))


def _route_vs_direct(ctx, rz, inputs, out_spec, direct):
    """Routes a realization with device copies of `inputs`; returns (routed, direct) outputs."""
    from tiler_amd.realize import route
    dev_in = [ctx.to_device(a) for a in inputs]
    out_t, out_n = out_spec
    dev_out = ctx.alloc(max(1, out_n * np.dtype(out_t).itemsize))
    storage, k = [], 0
    for role, _ in rz.slots:
        if role == L.SLOT_INPUT:
            storage.append(dev_in[k]); k += 1
        elif role == L.SLOT_OUTPUT:
            storage.append(dev_out)
        else:
            storage.append(None)
    try:
        route(ctx, rz, storage)
        routed = dev_out.download(out_t, (out_n,))
    finally:
        for b in dev_in + [dev_out]:
            b.free()
    return routed, np.asarray(direct()).reshape(-1)


@pytest.mark.parametrize("case", range(CASES))
def test_realized_plans_match_direct_calls(ctx, case):
    """The recognizer's plan, routed through the runtime seam, reproduces the
    family entry point bit for bit on random shapes of every family."""
    from tiler_amd.realize import realize
    r = _rng(case, 8)
    fam = case % 6
    if fam == 0:
        rows, extent = int(r.integers(1, 9)), int(r.integers(1, 20000))
        x = oracle.bf16_narrow(r.standard_normal((rows, extent)).astype(np.float32))
        w = oracle.bf16_narrow(r.normal(1.0, 0.1, extent).astype(np.float32))
        rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=L.BF16, scalars=(EPS,),
                     flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
        got, want = _route_vs_direct(ctx, rz, [x, w], (np.uint16, rows * extent),
                                     lambda: families.rms_norm_bf16(x, w, EPS, ctx=ctx))
    elif fam == 1:
        # up to 12 segments: the realized plan runs the three-launch split where
        # the direct call synchronizes rows in one launch; the bits must agree
        rows, extent = int(r.integers(1, 9)), int(r.integers(1, 98304))
        x = (r.standard_normal((rows, extent)) * 3).astype(np.float32)
        rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
        got, want = _route_vs_direct(ctx, rz, [x], (np.float32, rows * extent),
                                     lambda: families.softmax_f32((rows, extent), 1, x, ctx=ctx))
    elif fam == 2:
        rows, extent = int(r.integers(1, 40)), int(r.integers(1, 5000))
        x = r.uniform(-1, 1, (rows, extent)).astype(np.float32)
        rz = realize(L.PROGRAM_SERIAL_SUM, (rows, extent), topology=L.SUM_TREE, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
        got, want = _route_vs_direct(ctx, rz, [x], (np.float32, rows),
                                     lambda: families.tree_sum(x, (rows, extent), 1, ctx=ctx))
    elif fam == 3:
        m, n, k = (int(v) for v in r.integers(1, 400, 3))
        n, k = 8 * max(1, n // 8), 8 * max(1, k // 8)
        a = oracle.bf16_narrow((r.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32))
        b = oracle.bf16_narrow((r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))
        rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16, variant=L.EPILOGUE_SILU, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
        got, want = _route_vs_direct(ctx, rz, [a, b], (np.uint16, m * n),
                                     lambda: families.contract_bf16(a, b, L.EPILOGUE_SILU, ctx=ctx))
    elif fam == 4:
        n = 8 * int(r.integers(1, 50000))
        x = (r.standard_normal(n) * 6).astype(np.float32)
        rz = realize(L.PROGRAM_POINTWISE, (n,), variant=L.MAP_SILU, ctx=ctx)
        got, want = _route_vs_direct(ctx, rz, [x], (np.float32, n), lambda: families.silu_f32(x, ctx=ctx))
    else:
        n = int(r.integers(1, 100000))
        x = (r.standard_normal(n) * 1e3).astype(np.float32)
        rz = realize(L.PROGRAM_CONVERT, (n,), variant=L.CONVERT_NARROW_F32_BF16, ctx=ctx)
        got, want = _route_vs_direct(ctx, rz, [x], (np.uint16, n), lambda: families.narrow_f32_bf16(x, ctx=ctx))
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (case, rz.symbols)
