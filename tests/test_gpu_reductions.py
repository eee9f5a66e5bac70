"""GPU parity: the sum family under every topology, RMS normalization and
softmax, against the oracle on the same seeded inputs.

Bit-exact where the kernel's order is a reference order (serial, multipass,
cooperative) or its declared grouping (tree, row families); at the full
configuration sizes additionally within the stated tolerance of an f64
accumulation: 1e-5 relative (sum, softmax), 2 bf16 ulp (bf16 RMSNorm).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import bits, bf16_ulp_distance, bf16_widen, expected_bits, f32, golden, hexbits, values_of
from tiler_amd import _lib as L
from tiler_amd import families

pytestmark = pytest.mark.gpu
G = golden()
EPS = hexbits(G["rms_norm"]["eps_bits"])


def _sum_dev(ctx, x, rows, extent, **plan):
    dx = ctx.to_device(np.ascontiguousarray(x, np.float32))
    do = ctx.alloc(max(rows, 1) * 4)
    try:
        ctx.sum_f32(dx, rows, extent, do, **plan)
        ctx.synchronize()
        return do.download(np.float32, (rows,))
    finally:
        dx.free()
        do.free()


# -- sum: reference topologies ----------------------------------------------------

def test_serial_sum_golden_sets_and_random(ctx):
    s = G["serial_sum"]
    for key, want in [("parallel_operands", "parallel_sum"),
                      ("grouping_sensitive_operands", "grouping_sensitive_serial"),
                      ("separating_exact_operands", "separating_exact_sum")]:
        x = f32(s[key])
        got = _sum_dev(ctx, x, 1, x.size, topology=L.SUM_SERIAL)
        assert bits(got)[0] == hexbits(s[want])
    rows = f32([b for r in s["row_patterns"] for b in r])
    got = _sum_dev(ctx, rows, 4, 3, topology=L.SUM_SERIAL)
    assert list(bits(got)) == list(bits(oracle.strict_sum(rows, (4, 3), 1)))
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((37, 1001)) * 100).astype(np.float32)
    got = _sum_dev(ctx, x, 37, 1001, topology=L.SUM_SERIAL)
    assert np.array_equal(bits(got), bits(oracle.strict_sum(x, (37, 1001), 1)))


def _order_sensitive(rng, rows, extent):
    """Values over 80 binades, so that any other order of the fold gives
    other bits; row 0 all -0.0 (the fold's -0.0 total), row 1 with a NaN,
    row 2 with +inf and -inf (NaN), row 3 with one +inf."""
    x = (rng.standard_normal((rows, extent)) * np.exp2(rng.integers(-40, 40, (rows, extent)))).astype(np.float32)
    if rows >= 4:
        x[0] = -0.0
        x[1, extent // 2] = np.nan
        x[2, 0], x[2, -1] = np.inf, -np.inf
        x[3, extent - 1] = np.inf
    return x


@pytest.mark.parametrize("rows,extent,offset", [
    (3, 10000, 0),     # one row per workgroup, 16-byte loads, a ragged last stage
    (5, 9999, 0),      # rows off the 16-byte grid: 4-byte loads
    (4, 3000, 4),      # an unaligned base
    (700, 1500, 0),    # four rows per workgroup (one per wave), a ragged last workgroup
    (701, 1500, 0),    # four rows per workgroup, the last holding one row
    (2000, 300, 0),    # sixteen rows per workgroup
    (3000, 259, 0),    # sixteen rows, 4-byte loads
    (5000, 129, 0),    # sixty-four rows per workgroup, 4-byte loads
    (20000, 64, 0),    # sixty-four rows per workgroup, one stage
    (17000, 65, 0),    # sixty-four rows, a second stage of one element
    (1, 70000, 0),     # one long row
    (2, 100, 0),       # one row per workgroup, one pass that opens and ends the row
    (3, 8192, 0),      # whole stages and whole 256-element passes
    (600, 256, 0),     # four rows per workgroup, one whole pass
    (5000, 20, 0),     # rows of 16..63: 256 rows per workgroup, stages of 16
    (300, 63, 0),      # the same, 4-byte loads, a ragged last stage
    (257, 16, 4),      # one stage, an unaligned base, a second workgroup of one row
])
def test_serial_sum_staged_rows_are_the_strict_fold(ctx, rows, extent, offset):
    """Rows of 64 or more elements are folded from LDS stages
    (tiler_sum_f32_staged_r*); the fold is still evaluate.rs:555-585's, bit
    for bit."""
    x = _order_sensitive(np.random.default_rng(rows * 7 + extent), rows, extent)
    dx = ctx.alloc(x.nbytes + offset)
    do = ctx.alloc(rows * 4)
    try:
        src = dx.offset(offset)
        src.upload(x)
        ctx.sum_f32(src, rows, extent, do, topology=L.SUM_SERIAL)
        got = do.download(np.float32, (rows,))
    finally:
        dx.free()
        do.free()
    want = oracle.strict_sum(x, (rows, extent), 1)
    assert np.array_equal(bits(got), bits(want))
    if rows >= 4:
        assert bits(got)[0] == 0x80000000 and bits(got)[1] == bits(got)[2] == 0x7FC00000
        assert got[3] == np.inf


def test_multipass_sum_matches_strict_partitioned_sum(ctx):
    s = G["serial_sum"]
    sep = f32(s["separating_operands"])
    assert bits(_sum_dev(ctx, sep, 1, 12, topology=L.SUM_MULTIPASS, partitions=6,
                         per_partition=2))[0] == hexbits(s["separating_tree_6x2"])
    assert bits(_sum_dev(ctx, sep, 1, 12, topology=L.SUM_MULTIPASS, partitions=4,
                         per_partition=3))[0] == hexbits(s["separating_split_4x3"])
    rng = np.random.default_rng(22)
    x = (rng.standard_normal((9, 4096)) * 10).astype(np.float32)
    got = _sum_dev(ctx, x, 9, 4096, topology=L.SUM_MULTIPASS, partitions=64, per_partition=64)
    assert np.array_equal(bits(got), bits(oracle.strict_partitioned_sum(x, 9, 4096, 64, 64)))
    # partitions of 16..63: the staged fold with 256 rows per workgroup
    z = (rng.standard_normal((33, 1024)) * 10).astype(np.float32)
    got = _sum_dev(ctx, z, 33, 1024, topology=L.SUM_MULTIPASS, partitions=32, per_partition=32)
    assert np.array_equal(bits(got), bits(oracle.strict_partitioned_sum(z, 33, 1024, 32, 32)))
    y = (rng.standard_normal((70, 1024)) * 10).astype(np.float32)
    got = _sum_dev(ctx, y, 70, 1024, topology=L.SUM_MULTIPASS, partitions=64, per_partition=16)
    assert np.array_equal(bits(got), bits(oracle.strict_partitioned_sum(y, 70, 1024, 64, 16)))
    # 2100 x 512 partials (4.3 MB) exceed the context's 256 KiB partials
    # workspace: the stream-ordered allocation path
    w = (rng.standard_normal((2100, 1024)) * 10).astype(np.float32)
    got = _sum_dev(ctx, w, 2100, 1024, topology=L.SUM_MULTIPASS, partitions=512, per_partition=2)
    assert np.array_equal(bits(got), bits(oracle.strict_partitioned_sum(w, 2100, 1024, 512, 2)))


@pytest.mark.parametrize("major", [False, True])
def test_cooperative_sum_matches_cooperative_grouped_sum(ctx, major):
    rng = np.random.default_rng(23)
    P, c, R = 64, 3, 5
    x = (rng.standard_normal((6, P * c * R)) * 1e3).astype(np.float32)
    got = _sum_dev(ctx, x, 6, P * c * R, topology=L.SUM_COOPERATIVE, participants=P,
                   per_partition=c, rounds=R, participant_major=major)
    want = oracle.cooperative_grouped_sum(x, 6, P * c * R, P, c, R,
                                          oracle.PARTICIPANT_MAJOR if major else oracle.ROUND_MAJOR)
    assert np.array_equal(bits(got), bits(want))


# -- sum: the reassociating tree -------------------------------------------------------

@pytest.mark.parametrize("n", [1, 3, 1000, 1024, 4097, 300001])
def test_tree_sum_is_its_declared_grouping(ctx, n):
    rng = np.random.default_rng(n)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    got = _sum_dev(ctx, x, 1, n, topology=L.SUM_TREE)
    want = oracle.grid_tree_sum(x, ctx.sum_tree_workgroups(n))
    assert bits(got)[0] == bits([want])[0]


def test_tree_sum_exact_sets_and_special_values(ctx):
    ex = f32(G["serial_sum"]["separating_exact_operands"])
    assert bits(_sum_dev(ctx, ex, 1, 12, topology=L.SUM_TREE))[0] == 0x457FF000
    negz = np.full(5000, -0.0, np.float32)
    assert bits(_sum_dev(ctx, negz, 1, 5000, topology=L.SUM_TREE))[0] == 0x80000000
    nan = np.ones(3000, np.float32)
    nan[1234] = f32(["0x7fc01234"])[0]
    assert bits(_sum_dev(ctx, nan, 1, 3000, topology=L.SUM_TREE))[0] == 0x7FC00000


@pytest.mark.parametrize("rows,extent,offset", [(1000, 256, 0), (37, 255, 0), (4096, 64, 0), (5, 1, 0),
                                                (9, 200, 4)])
def test_tree_sum_short_rows_one_wave_each(ctx, rows, extent, offset):
    """Rows of at most 256 run one wave per row (tiler_sum_f32_rows_w): the
    same declared grouping as the 256-thread form, bit for bit."""
    x = np.random.default_rng(rows + extent).uniform(-1, 1, (rows, extent)).astype(np.float32)
    x[0, 0] = np.float32(2.0 ** 30)  # large enough that the grouping shows in the bits
    dx = ctx.alloc(x.nbytes + offset)
    do = ctx.alloc(rows * 4)
    try:
        dx.offset(offset).upload(x)
        ctx.sum_f32(dx.offset(offset), rows, extent, do, topology=L.SUM_TREE)
        got = do.download(np.float32, (rows,))
    finally:
        dx.free()
        do.free()
    assert np.array_equal(bits(got), bits(oracle.row_grouped_sum(x, rows, extent, 4, 4)))


def test_tree_sum_rows_declared_grouping(ctx):
    rng = np.random.default_rng(24)
    x = rng.uniform(-1, 1, (33, 5000)).astype(np.float32)
    got = _sum_dev(ctx, x, 33, 5000, topology=L.SUM_TREE)
    assert np.array_equal(bits(got), bits(oracle.row_grouped_sum(x, 33, 5000, 4, 4)))


def test_tree_sum_full_size_config(ctx):
    """C1: f32[2^24] ~ U[-1, 1] -> scalar, within 1e-5 of the f64 sum, and
    repeated launches (sharing the context's partials workspace) stay
    bit-identical."""
    n = 1 << 24
    x = np.random.default_rng(0).uniform(-1, 1, n).astype(np.float32)
    dx = ctx.to_device(x)
    do = ctx.alloc(4 * 4)
    try:
        for i in range(4):
            ctx.sum_f32(dx, 1, n, do.offset(4 * i), topology=L.SUM_TREE)
        ctx.synchronize()
        got = do.download(np.float32, (4,))
    finally:
        dx.free()
        do.free()
    ref = float(np.sum(x.astype(np.float64)))
    assert abs(float(got[0]) - ref) <= 1e-5 * abs(ref)
    assert len(set(bits(got).tolist())) == 1
    assert bits(got)[0] == bits([oracle.grid_tree_sum(x, ctx.sum_tree_workgroups(n))])[0]


# -- RMS normalization -------------------------------------------------------------------

@pytest.mark.parametrize("case", G["rms_norm"]["cases"], ids=lambda c: c["name"])
def test_rms_norm_golden_on_device(ctx, case):
    x = values_of(case, "x")
    w = values_of(case, "w")
    y = families.rms_norm_f32(case["shape"], case["axis"], EPS, x, w, ctx=ctx)
    assert list(bits(y)) == list(expected_bits(case))


def test_rms_norm_holed_rows_and_axis(ctx):
    hr = G["rms_norm"]["holed_rows"]
    for key in ("extent_1024", "extent_128"):
        n = int(key.split("_")[1])
        x = np.full(n, hr[key]["fill"], np.float32)
        x[hr[key]["hole"]] = 0.0
        y = families.rms_norm_f32((1, n), 1, EPS, x, np.ones(n, np.float32), ctx=ctx)
        assert bits(y)[0] == hexbits(hr[key]["first_bits"])
    v = np.arange(1, 7, dtype=np.float32)
    for axis in (0, 1):
        y = families.rms_norm_f32((2, 3), axis, EPS, v, np.ones(6, np.float32), ctx=ctx)
        assert np.array_equal(bits(y), bits(oracle.rms_norm_f32(v, np.ones(6, np.float32), (2, 3), axis, EPS)))


@pytest.mark.parametrize("rows,extent", [(64, 4096), (7, 1000), (5, 96), (3, 8192), (9, 4104)])
def test_rms_norm_bf16_declared_grouping(ctx, rows, extent):
    rng = np.random.default_rng(rows * 10000 + extent)
    xf = rng.standard_normal((rows, extent)).astype(np.float32)
    wf = rng.normal(1.0, 0.1, extent).astype(np.float32)
    xb, wb = oracle.bf16_narrow(xf), oracle.bf16_narrow(wf)
    got = families.rms_norm_bf16(xb, wb, EPS, ctx=ctx)
    y = oracle.rms_norm_grouped(bf16_widen(xb), bf16_widen(wb), rows, extent, EPS, True, 8, 1)
    want = oracle.bf16_narrow(y).reshape(rows, extent)
    assert np.array_equal(got, want)


def test_rms_norm_f32_declared_grouping_and_unaligned(ctx):
    rng = np.random.default_rng(31)
    for rows, extent in [(16, 2048), (5, 1001)]:
        x = rng.standard_normal((rows, extent)).astype(np.float32)
        w = rng.normal(1.0, 0.1, (rows, extent)).astype(np.float32)
        dx, dw, dy = ctx.to_device(x), ctx.to_device(w), ctx.alloc(x.nbytes)
        try:
            ctx.rms_norm(L.F32, dx, dw, rows, extent, EPS, dy, weight_broadcast=False)
            ctx.synchronize()
            got = dy.download(np.float32, (rows * extent,))
        finally:
            dx.free(); dw.free(); dy.free()
        want = oracle.rms_norm_grouped(x, w, rows, extent, EPS, False, 4, 1)
        assert np.array_equal(bits(got), bits(want))


def test_rms_norm_refuses_bad_eps(ctx):
    import tiler_amd
    for bad in G["rms_norm"]["bad_eps_bits"]:
        with pytest.raises(tiler_amd.Refusal):
            families.rms_norm_f32((1, 2), 1, hexbits(bad), [1.0, 2.0], [1.0, 1.0], ctx=ctx)


def test_rms_norm_full_size_config(ctx):
    """C2: bf16 [8192 x 4096], w bf16 [4096] ~ N(1, 0.1): bit-exact with the
    declared grouping and within 2 bf16 ulp of the f64 result."""
    rows, extent = 8192, 4096
    rng = np.random.default_rng(2)
    xb = oracle.bf16_narrow(rng.standard_normal((rows, extent)).astype(np.float32))
    wb = oracle.bf16_narrow(rng.normal(1.0, 0.1, extent).astype(np.float32))
    got = families.rms_norm_bf16(xb, wb, EPS, ctx=ctx)
    x64 = bf16_widen(xb).astype(np.float64)
    w64 = bf16_widen(wb).astype(np.float64)
    ms = np.mean(x64 * x64, axis=1, keepdims=True)
    ref = w64 * x64 / np.sqrt(ms + float(f32([EPS])[0]))
    dist = bf16_ulp_distance(got, ref)
    assert float(dist.max()) <= 2.0
    sample = slice(0, 256)
    y = oracle.rms_norm_grouped(bf16_widen(xb[sample]), bf16_widen(wb), 256, extent, EPS, True, 8, 1)
    assert np.array_equal(got[sample], oracle.bf16_narrow(y).reshape(256, extent))


# -- softmax ---------------------------------------------------------------------------------

@pytest.mark.parametrize("case", G["softmax"]["cases"], ids=lambda c: c["name"])
def test_softmax_golden_on_device(ctx, case):
    x = values_of(case, "x")
    y = families.softmax_f32(case["shape"], case.get("axis", 1), x, ctx=ctx)
    assert list(bits(y)) == list(expected_bits(case))


@pytest.mark.parametrize("rows,extent", [(64, 2048), (13, 1000), (4, 8192), (50, 3)])
def test_softmax_declared_grouping(ctx, rows, extent):
    rng = np.random.default_rng(rows + extent)
    x = (rng.standard_normal((rows, extent)) * 3).astype(np.float32)
    got = families.softmax_f32((rows, extent), 1, x, ctx=ctx)
    want = oracle.softmax_grouped(x, rows, extent, 4, 1)
    assert np.array_equal(bits(got), bits(want))


def test_softmax_axis_other_than_last(ctx):
    v = np.arange(1, 7, dtype=np.float32)
    y = families.softmax_f32((2, 3), 0, v, ctx=ctx)
    assert np.array_equal(bits(y), bits(oracle.softmax_f32(v, (2, 3), 0)))


def test_softmax_full_size_config(ctx):
    """C3: f32 [32 x 2048 x 2048] ~ N(0, 3) over the last axis: within 1e-5
    relative of the f64 softmax, bit-exact with the declared grouping on a
    sample of rows."""
    rows, extent = 32 * 2048, 2048
    x = (np.random.default_rng(3).standard_normal((rows, extent)) * 3).astype(np.float32)
    dx, dy = ctx.to_device(x), ctx.alloc(x.nbytes)
    try:
        ctx.softmax_f32(dx, rows, extent, dy)
        ctx.synchronize()
        got = dy.download(np.float32, (rows, extent))
    finally:
        dx.free(); dy.free()
    for lo in range(0, rows, 8192):
        x64 = x[lo:lo + 8192].astype(np.float64)
        e = np.exp(x64 - x64.max(axis=1, keepdims=True))
        ref = e / e.sum(axis=1, keepdims=True)
        rel = np.abs(got[lo:lo + 8192] - ref) / np.maximum(ref, 1e-300)
        assert float(rel.max()) <= 1e-5
    sample = x[:512]
    assert np.array_equal(bits(got[:512]), bits(oracle.softmax_grouped(sample, 512, extent, 4, 1)).reshape(512, extent))
