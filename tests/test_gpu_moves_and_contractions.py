"""GPU parity: pointwise maps, broadcast, gather and both contractions.

Gather and broadcast are byte moves and must be bit-exact; the strict f32
contraction must reproduce the reference's own device digests; the bf16 MFMA
contraction is held to the stated 1e-2 relative Frobenius error against
the strict f32 fold of the same (exactly widened) operands.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import tiler_amd
from helpers import (bits, bf16_widen, f32, golden, hexbits, sha256_le_f32, splitmix_operands)
from tiler_amd import _lib as L
from tiler_amd import families

pytestmark = pytest.mark.gpu
G = golden()


# -- maps -------------------------------------------------------------------------------

def test_silu_boundary_corpus_on_device(ctx):
    corpus = G["silu"]["corpus"]
    y = families.silu_f32(f32([a for a, _ in corpus]), ctx=ctx)
    assert [int(v) for v in bits(y)] == [hexbits(b) for _, b in corpus]


def test_silu_random_matches_oracle(ctx):
    x = (np.random.default_rng(41).standard_normal(100000) * 20).astype(np.float32)
    got = families.silu_f32(x, ctx=ctx)
    assert np.array_equal(bits(got), bits(oracle.silu_f32(x)))


def _map(ctx, op, dtype, x, x2=None, bcast=False, a=0.0, b=0.0):
    dx = ctx.to_device(x)
    d2 = ctx.to_device(x2) if x2 is not None else None
    dy = ctx.alloc(x.nbytes)
    try:
        ctx.map(op, dtype, dx, x.size, dy, x2=d2, x2_broadcast=bcast, a=a, b=b)
        ctx.synchronize()
        return dy.download(x.dtype, x.shape)
    finally:
        dx.free(); dy.free()
        if d2 is not None:
            d2.free()


def _canon(a):
    a = np.asarray(a, np.float32)
    return np.where(np.isnan(a), f32(["0x7fc00000"])[0], a).astype(np.float32)


def test_scale_bias_and_binary_maps(ctx):
    rng = np.random.default_rng(42)
    x = rng.standard_normal(7777).astype(np.float32)
    x[:4] = f32(["0x7fc01234", "0x7f800000", "0x00000001", "0x80000000"])
    y = _map(ctx, L.MAP_SCALE_BIAS, L.F32, x, a=2.0, b=1.0)
    want = _canon((x * np.float32(2.0)).astype(np.float32) + np.float32(1.0))
    assert np.array_equal(bits(y), bits(want))
    x2 = rng.standard_normal(7777).astype(np.float32)
    assert np.array_equal(bits(_map(ctx, L.MAP_ADD, L.F32, x, x2)), bits(_canon(x + x2)))
    s = np.asarray([3.0], np.float32)
    got = _map(ctx, L.MAP_MULTIPLY, L.F32, x, s, bcast=True)
    assert np.array_equal(bits(got), bits(_canon(x * s[0])))


def test_bf16_maps_round_once_per_operation(ctx):
    rng = np.random.default_rng(43)
    xb = oracle.bf16_narrow(rng.standard_normal(5000).astype(np.float32))
    yb = _map(ctx, L.MAP_SCALE_BIAS, L.BF16, xb, a=2.0, b=1.0)
    t = oracle.bf16_narrow(bf16_widen(xb) * np.float32(2.0))
    want = oracle.bf16_narrow(bf16_widen(t) + np.float32(1.0))
    assert np.array_equal(yb, want)
    x2 = oracle.bf16_narrow(rng.standard_normal(5000).astype(np.float32))
    got = _map(ctx, L.MAP_ADD, L.BF16, xb, x2)
    assert np.array_equal(got, oracle.bf16_narrow(bf16_widen(xb) + bf16_widen(x2)))


def _map_at(ctx, op, dtype, x, x2=None, bcast=False, a=0.0, b=0.0, offset=0):
    """Runs the map with every operand starting `offset` elements into its buffer."""
    eb = x.dtype.itemsize
    dx = ctx.alloc(x.nbytes + 16)
    dy = ctx.alloc(x.nbytes + 16)
    d2 = ctx.alloc(x2.nbytes + 16) if x2 is not None else None
    try:
        vx, vy = dx.offset(offset * eb), dy.offset(offset * eb)
        vx.upload(x)
        v2 = None
        if d2 is not None:
            v2 = d2.offset(0 if bcast else offset * eb)
            v2.upload(x2)
        ctx.map(op, dtype, vx, x.size, vy, x2=v2, x2_broadcast=bcast, a=a, b=b)
        ctx.synchronize()
        return vy.download(x.dtype, x.shape)
    finally:
        dx.free(); dy.free()
        if d2 is not None:
            d2.free()


@pytest.mark.parametrize("n", [1, 7, 8195])
@pytest.mark.parametrize("offset", [0, 1])
def test_maps_vector_tail_and_unaligned_paths(ctx, n, offset):
    """16-byte vector kernels with a scalar tail (aligned) and the scalar kernel
    alone (offset by one element): identical arithmetic either way."""
    rng = np.random.default_rng(n * 3 + offset)
    x = rng.standard_normal(n).astype(np.float32)
    x2 = rng.standard_normal(n).astype(np.float32)
    s = np.asarray([0.75], np.float32)
    got = _map_at(ctx, L.MAP_SCALE_BIAS, L.F32, x, a=2.0, b=-1.0, offset=offset)
    assert np.array_equal(bits(got), bits(_canon((x * np.float32(2.0)).astype(np.float32) + np.float32(-1.0))))
    assert np.array_equal(bits(_map_at(ctx, L.MAP_ADD, L.F32, x, x2, offset=offset)), bits(_canon(x + x2)))
    assert np.array_equal(bits(_map_at(ctx, L.MAP_MULTIPLY, L.F32, x, s, bcast=True, offset=offset)),
                          bits(_canon(x * s[0])))
    assert np.array_equal(bits(_map_at(ctx, L.MAP_SILU, L.F32, x * 8, offset=offset)),
                          bits(oracle.silu_f32(x * 8)))
    xb, x2b = oracle.bf16_narrow(x), oracle.bf16_narrow(x2)
    sb = oracle.bf16_narrow(s)
    t = oracle.bf16_narrow(bf16_widen(xb) * np.float32(2.0))
    assert np.array_equal(_map_at(ctx, L.MAP_SCALE_BIAS, L.BF16, xb, a=2.0, b=-1.0, offset=offset),
                          oracle.bf16_narrow(bf16_widen(t) + np.float32(-1.0)))
    assert np.array_equal(_map_at(ctx, L.MAP_MULTIPLY, L.BF16, xb, x2b, offset=offset),
                          oracle.bf16_narrow(bf16_widen(xb) * bf16_widen(x2b)))
    assert np.array_equal(_map_at(ctx, L.MAP_ADD, L.BF16, xb, sb, bcast=True, offset=offset),
                          oracle.bf16_narrow(bf16_widen(xb) + bf16_widen(sb)[0]))


def test_broadcast_moves_bytes(ctx):
    src = np.arange(6, dtype=np.float32).reshape(2, 3)
    src[0, 0] = f32(["0x7fc01234"])[0]
    ds = ctx.to_device(src)
    do = ctx.alloc(4 * 2 * 3 * 4)
    try:
        ctx.broadcast(ds, 6, [4, 2, 3], [0, 3, 1], 4, do)
        ctx.synchronize()
        got = do.download(np.uint32, (4, 2, 3))
    finally:
        ds.free(); do.free()
    assert np.array_equal(got, np.broadcast_to(bits(src), (4, 2, 3)))


def _broadcast(ctx, src, out_dims, strides):
    ds = ctx.to_device(src)
    n = int(np.prod(out_dims))
    do = ctx.alloc(max(n * src.itemsize, 4))
    try:
        ctx.broadcast(ds, src.size, list(out_dims), list(strides), src.itemsize, do)
        ctx.synchronize()
        return do.download(src.dtype, tuple(out_dims))
    finally:
        ds.free(); do.free()


@pytest.mark.parametrize("dtype,src_shape,out_dims,strides", [
    (np.uint32, (4, 300), (3, 4, 300), (0, 300, 1)),    # rows copied as 16-byte vectors
    (np.uint16, (5,), (5, 512), (1, 0)),                # inner axis broadcast: filled rows
    (np.uint32, (300, 2), (2, 300), (1, 2)),            # transposed: strided rows
    (np.uint16, (257,), (3, 257), (0, 1)),              # rows not a whole number of vectors
    (np.uint32, (2, 3), (4, 2, 3), (0, 3, 1)),          # short rows: per-element kernel
])
def test_broadcast_row_and_element_modes(ctx, dtype, src_shape, out_dims, strides):
    src = np.random.default_rng(len(out_dims) * 1000 + out_dims[-1]).integers(0, np.iinfo(dtype).max, src_shape,
                                                                             dtype=dtype)
    got = _broadcast(ctx, src, out_dims, strides)
    want = np.lib.stride_tricks.as_strided(src, shape=out_dims,
                                           strides=[s * src.itemsize for s in strides])
    assert np.array_equal(got, want)


def test_broadcast_refuses_reads_outside_the_source(ctx):
    src = np.arange(5, dtype=np.uint32)
    ds, do = ctx.to_device(src), ctx.alloc(64)
    try:
        with pytest.raises(tiler_amd.Refusal):
            ctx.broadcast(ds, 5, [2, 3], [3, 1], 4, do)   # largest offset 1*3 + 2*1 = 5
        ctx.broadcast(ds, 6 - 1, [2, 2], [3, 1], 4, do)     # largest offset 4: admitted
        ctx.synchronize()
    finally:
        ds.free(); do.free()


# -- gather -------------------------------------------------------------------------------

@pytest.mark.parametrize("case", G["gather"]["cases"], ids=lambda c: c["name"])
def test_gather_golden_on_device(ctx, case):
    shape = tuple(case["source_shape"])
    src = np.arange(int(np.prod(shape)), dtype=np.uint32).reshape(shape)
    idx = np.asarray(case["index"], np.uint32).reshape(case["index_shape"])
    got = families.gather(src, case["axis"], idx, ctx=ctx)
    assert list(got.shape) == case["result_shape"]
    assert got.reshape(-1).tolist() == case["result"]


def test_gather_refuses_before_commit_naming_position(ctx):
    src = np.arange(15, dtype=np.uint32).reshape(5, 3)
    for ref in G["gather"]["refusals"]:
        with pytest.raises(tiler_amd.GatherIndexOutOfBounds) as err:
            families.gather(src, 0, np.asarray(ref["index"], np.uint32), ctx=ctx)
        assert err.value.position == ref["position"] and err.value.value == ref["value"]
        assert err.value.fallback_permitted


def test_gather_device_bound_check_reports_lowest_position(ctx):
    """An index that reaches the device unvalidated is not clamped or wrapped:
    its run is not written and the committed dispatch fails naming it."""
    src = np.arange(15, dtype=np.uint32)
    idx = np.asarray([1, 7, 2, 5, 0], np.uint32)
    ds, di = ctx.to_device(src), ctx.to_device(idx)
    do = ctx.alloc(5 * 3 * 4)
    try:
        ctx.fill_u32(do, 0xDEADBEEF, 15)
        ctx.gather(ds, 1, 5, 3, 4, di, 5, do)
        with pytest.raises(tiler_amd.GatherIndexOutOfBounds) as err:
            ctx.gather_status()
        assert err.value.position == 1 and not err.value.fallback_permitted
        got = do.download(np.uint32, (5, 3))
        assert got[0].tolist() == [3, 4, 5] and got[2].tolist() == [6, 7, 8]
        assert got[1].tolist() == [0xDEADBEEF] * 3 and got[3].tolist() == [0xDEADBEEF] * 3
        ctx.gather_status()  # the record re-armed
        sidx = np.asarray([0, -3], np.int32).view(np.uint32)
        di2 = ctx.to_device(sidx)
        ctx.gather(ds, 1, 5, 3, 4, di2, 2, do, index_signed=True)
        with pytest.raises(tiler_amd.GatherIndexOutOfBounds) as err:
            ctx.gather_status()
        assert err.value.position == 1
        di2.free()
    finally:
        ds.free(); di.free(); do.free()


def test_gather_preserves_every_payload(ctx):
    p = G["gather"]["payloads"]
    src = np.asarray([hexbits(b) for b in p["source_bits"]], np.uint32)
    got = families.gather(src, 0, np.asarray(p["index"], np.uint32), ctx=ctx)
    assert [int(v) for v in got] == [hexbits(b) for b in p["result_bits"]]


@pytest.mark.parametrize("dtype,inner", [(np.uint16, 4096), (np.uint16, 7), (np.uint8, 33), (np.uint32, 12)])
def test_gather_ragged_runs_match_oracle(ctx, dtype, inner):
    rng = np.random.default_rng(inner)
    src = rng.integers(0, np.iinfo(dtype).max, (3, 50, inner), dtype=dtype)
    idx = rng.integers(0, 50, 77).astype(np.int32)
    got = families.gather(src, 1, idx, index_signed=True, ctx=ctx)
    want, err = oracle.gather(src.reshape(-1), 3, 50, inner, idx.view(np.uint32), index_signed=True)
    assert err is None and np.array_equal(got.reshape(-1), want)


def test_gather_full_size_config(ctx):
    """C4: bf16 table [128256 x 4096] ~ N(0, 0.02), int32 indices [16384]
    ~ U[0, 128256): bit-exact."""
    vocab, hidden, count = 128256, 4096, 16384
    rng = np.random.default_rng(4)
    table = oracle.bf16_narrow((rng.standard_normal((vocab, hidden), dtype=np.float32) * np.float32(0.02)))
    idx = rng.integers(0, vocab, count).astype(np.int32)
    got = families.gather(table, 0, idx, index_signed=True, ctx=ctx)
    assert np.array_equal(got, table[idx])


# -- contractions -------------------------------------------------------------------------

@pytest.mark.parametrize("cell", G["contraction"]["cells"], ids=lambda c: c["id"])
def test_strict_contraction_reproduces_reference_digests_on_device(ctx, cell):
    seed = hexbits(G["contraction"]["workload_seed"])
    mask = hexbits(G["contraction"]["right_seed_mask"])
    a = splitmix_operands(seed, cell["m"] * cell["k"]).reshape(cell["m"], cell["k"])
    b = splitmix_operands(seed ^ mask, cell["n"] * cell["k"]).reshape(cell["n"], cell["k"])
    c = families.contract_strict_f32(a, b, ctx=ctx)
    assert sha256_le_f32(c) == cell["sha256"]


def test_strict_contraction_tails_and_signed_zero(ctx):
    rng = np.random.default_rng(51)
    a = rng.standard_normal((19, 37)).astype(np.float32)
    b = rng.standard_normal((23, 37)).astype(np.float32)
    got = families.contract_strict_f32(a, b, ctx=ctx)
    assert np.array_equal(bits(got), bits(oracle.contract_strict_f32(a, b, 19, 23, 37)))
    z = families.contract_strict_f32(np.asarray([[-0.0]], np.float32), np.asarray([[1.0]], np.float32), ctx=ctx)
    assert bits(z)[0, 0] == 0x80000000


@pytest.mark.parametrize("m,n,k,offset", [
    (1, 200, 1000, 0),   # one output column per workgroup, 16-byte loads
    (3, 300, 999, 0),    # four columns per workgroup, 4-byte loads, a ragged last stage
    (16, 200, 300, 0),   # sixteen columns per workgroup
    (5, 4000, 130, 0),   # sixty-four columns per workgroup, 4-byte loads
    (2, 3000, 64, 0),    # sixty-four columns, exactly one stage
    (1, 70, 4099, 0),    # one column per workgroup over two stages
    (4, 100, 512, 4),    # unaligned operands: 4-byte loads
    (40, 70, 100, 0),    # m > 16: 16 x 16 blocked tiles, ragged edges and k tile
    (33, 65, 77, 4),     # the same, unaligned
    (512, 1000, 96, 0),  # 32 x 32 tiles (2 x 2 per thread), a ragged n edge
    (2048, 2040, 70, 0), # 64 x 64 tiles (4 x 4 per thread), a ragged n edge and k tile
])
def test_strict_contraction_staged_and_blocked_are_the_first_product_fold(ctx, m, n, k, offset):
    """k >= 64 runs the staged fold of products for m <= 16
    (tiler_contract_strict_f32_s*) and register-blocked tiles above
    (tiler_contract_strict_f32_b16/_b32/_b64): still contraction.rs:558-630's fold,
    bit for bit, with values over 60 binades so any other order shows; row 0
    of A all -0.0 against positive B (a -0.0 total), a NaN in row 1, an inf
    against a zero in row 2."""
    rng = np.random.default_rng(m * 1000 + n + k)
    a = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-30, 30, (m, k)))).astype(np.float32)
    b = (rng.standard_normal((n, k)) * np.exp2(rng.integers(-30, 30, (n, k)))).astype(np.float32)
    if m >= 3:
        a[0] = -0.0
        b[0] = np.abs(b[0])
        a[1, k // 3] = np.nan
        a[2, 5], b[:, 5] = np.inf, 0.0
    da, db = ctx.alloc(a.nbytes + offset), ctx.alloc(b.nbytes + offset)
    dc = ctx.alloc(m * n * 4)
    try:
        da.offset(offset).upload(a)
        db.offset(offset).upload(b)
        print(f"[strict few rows] m={m} n={n} k={k} offset={offset}", flush=True)
        ctx.contract_strict_f32(da.offset(offset), db.offset(offset), m, n, k, dc)
        got = dc.download(np.float32, (m, n))
    finally:
        for x in (da, db, dc):
            x.free()
    want = oracle.contract_strict_f32(a, b, m, n, k).reshape(m, n)
    assert np.array_equal(bits(got), bits(want))
    if m >= 3:
        assert bits(got)[0, 0] == 0x80000000
        assert (bits(got)[1] == 0x7FC00000).all() and (bits(got)[2] == 0x7FC00000).all()


def _frob(got_bits, ref32):
    g = bf16_widen(got_bits).astype(np.float64)
    r = np.asarray(ref32, np.float64)
    return float(np.linalg.norm(g - r) / np.linalg.norm(r))


@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (256, 384, 512), (200, 136, 72), (77, 45, 13), (1, 300, 1000),
                                   (256, 256, 64), (512, 768, 1024), (1024, 2048, 256)])
@pytest.mark.parametrize("silu", [False, True])
def test_bf16_contraction_within_frobenius_bound(ctx, m, n, k, silu):
    rng = np.random.default_rng(m * n + k)
    ab = oracle.bf16_narrow((rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32))
    bb = oracle.bf16_narrow((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))
    got = families.contract_bf16(ab, bb, L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE, ctx=ctx)
    ref = oracle.contract_strict_f32(bf16_widen(ab), bf16_widen(bb), m, n, k)
    if silu:
        ref = oracle.silu_f32(ref).reshape(m, n)
    assert _frob(got, ref) <= 1e-2


@pytest.mark.parametrize("m,n,k", [(4000, 4104, 136), (4096, 4096, 72), (1000, 2048, 520), (64, 4096, 256),
                                   (3, 8, 8), (16, 4104, 4096), (33, 1000, 520), (1, 4096, 8)])
def test_bf16_contraction_ragged_edges(ctx, m, n, k):
    """Staged (m > 64) and skinny (m <= 64) paths on ragged shapes: rows past m
    and n load as zeros, k past a multiple of 64 is masked in both operands,
    and only in-range outputs are stored (the C buffer is poisoned with NaN
    bf16 first, so a stray store or a missed one shows)."""
    rng = np.random.default_rng(m + n + k)
    ab = oracle.bf16_narrow((rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32))
    bb = oracle.bf16_narrow((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))
    da, db = ctx.to_device(ab), ctx.to_device(bb)
    dc = ctx.alloc(m * n * 2 + 64)
    try:
        ctx.fill_u32(dc, 0x7FC17FC1, (m * n * 2 + 64) // 4)
        ctx.contract_bf16(da, db, m, n, k, dc, L.EPILOGUE_SILU)
        ctx.synchronize()
        raw = dc.download(np.uint16, (m * n + 32,))
    finally:
        da.free(); db.free(); dc.free()
    got, guard = raw[:m * n].reshape(m, n), raw[m * n:]
    assert (guard == 0x7FC1).all()
    ref = oracle.silu_f32(oracle.contract_strict_f32(bf16_widen(ab), bf16_widen(bb), m, n, k)).reshape(m, n)
    assert _frob(got, ref) <= 1e-2
    assert not np.isnan(bf16_widen(got)).any()


@pytest.mark.parametrize("m,n,k", [(16, 64, 64), (300, 264, 136), (70, 30, 20)])
@pytest.mark.parametrize("silu", [False, True])
def test_bf16_contraction_exceptional_values(ctx, m, n, k, silu):
    """Non-finite operands on every dispatch path (skinny m <= 64, staged, and
    the general form for n, k off the 8-element grid).  A NaN with a negative
    sign and a payload, +inf meeting a zero (inf * 0), and -inf are planted in
    A and B.  Every NaN output must be the canonical bf16 0x7fc0 (ADR 0091
    narrowing), infinities keep their sign, and the finite outputs stay
    within the Frobenius bound."""
    rng = np.random.default_rng(m * 7 + n + k)
    a = (rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32)
    b = np.abs(rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32) + np.float32(0.01)
    ab, bb = oracle.bf16_narrow(a), oracle.bf16_narrow(b)
    ab[0, 5] = 0xFFC1   # negative NaN with a payload: row 0 is NaN
    ab[1, 5] = 0x7F80   # +inf against positive B: +inf, except column 0 ...
    bb[0, 5] = 0x0000   # ... where it meets +0: inf * 0 = NaN
    ab[2, 7] = 0xFF80   # -inf: -inf (SiLU: NaN)
    bb[3, 9] = 0x7FA3   # a NaN payload in B: column 3 is NaN
    got = families.contract_bf16(ab, bb, L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE, ctx=ctx)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = oracle.contract_strict_f32(bf16_widen(ab), bf16_widen(bb), m, n, k).reshape(m, n)
        if silu:
            ref = oracle.silu_f32(ref).reshape(m, n)
    want = oracle.bf16_narrow(ref).reshape(m, n)
    special = ~np.isfinite(ref)
    assert special[0].all() and special[:, 3].all() and np.isnan(ref[1, 0])
    assert np.array_equal(got[special], want[special])
    assert (got[np.isnan(ref)] == 0x7FC0).all()
    fin = np.isfinite(ref)
    g = bf16_widen(got)[fin].astype(np.float64)
    r = ref[fin].astype(np.float64)
    assert np.linalg.norm(g - r) / np.linalg.norm(r) <= 1e-2


def test_bf16_contraction_full_size_config(ctx):
    """C5: bf16 A, B [4096 x 4096] ~ N(0, 1/sqrt(4096)), f32 accumulation,
    fused SiLU, bf16 C: the whole 4096 x 4096 output against the strict f32
    reference (the oracle's multithreaded fold, then silu_f32): relative
    Frobenius error <= 1e-2 over the output and over every row, and the
    non-finite pattern identical."""
    m = n = k = 4096
    rng = np.random.default_rng(5)
    ab = oracle.bf16_narrow((rng.standard_normal((m, k), dtype=np.float32) / np.float32(64.0)))
    bb = oracle.bf16_narrow((rng.standard_normal((n, k), dtype=np.float32) / np.float32(64.0)))
    got = families.contract_bf16(ab, bb, L.EPILOGUE_SILU, ctx=ctx)
    print("[C5] device done; strict f32 oracle over the whole output", flush=True)
    ref = oracle.contract_strict_f32(bf16_widen(ab), bf16_widen(bb), m, n, k)
    ref = oracle.silu_f32(ref).reshape(m, n)
    assert np.isfinite(ref).all() and np.isfinite(bf16_widen(got)).all()
    assert _frob(got, ref) <= 1e-2
    g = bf16_widen(got).astype(np.float64)
    r = ref.astype(np.float64)
    per_row = np.linalg.norm(g - r, axis=1) / np.linalg.norm(r, axis=1)
    assert per_row.max() <= 1e-2, f"row {int(per_row.argmax())}: {per_row.max():.3e}"
