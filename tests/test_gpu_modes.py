"""GPU parity for the flushing contracts (the declared subnormal modes,
tiler-reference/src/conformance.rs:498-521; FLUSH_SUBNORMALS_TO_ZERO_F32,
FLUSH_AND_REASSOCIATE_F32 and the bf16 flush, tiler-compiler/src/session.rs:
1795-1870) on every family that realizes them:

* the sums and folds -- serial, multi-pass split, cooperative workgroup,
  with the scale-bias and squared prologues -- bit for bit with the oracle's
  strict_sum / strict_partitioned_sum / cooperative_grouped_sum / fold_f32
  under the same modes, and the reference's own split-and-modes rows
  (tests.rs:2125-2260) on the device;
* RMSNorm (f32 and bf16 storage) and softmax, with the modes at every site;
* the f32 maps (scale-bias, SiLU, add, multiply) and the bf16 maps and
  expressions (operand and rounded-result encodings), including bf16.rs's
  seven counterexamples (bf16/tests.rs:722-835) on the device;
* the contractions (td,od->to in f32 and bf16 with SiLU, and an attention
  structure) on the strict fold with the modes at every site
  (contraction.rs:600-625).

Inputs are built so that operands, products and partial sums land in the
subnormal range.  Mode numbers: the region's (1 preserve, 2 flush to the
zero of the value's sign, 3 flush to +0); the oracle's are one less.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import bits, golden
from tiler_amd import _lib as L
from tiler_amd.realize import realize, route

pytestmark = pytest.mark.gpu

RE = L.PERMITS_REASSOCIATION
P, FS, FP = L.SUBNORMALS_PRESERVE, L.SUBNORMALS_FLUSH_SIGN, L.SUBNORMALS_FLUSH_POSITIVE
MODES = [(FS, P), (P, FS), (FS, FS), (FP, FP), (FS, FP)]
G = golden()["subnormal_modes"]
READINGS = [(P, P), (FS, P), (P, FS), (FS, FS)]


def om(m):
    """The oracle's number for a region mode."""
    return m - 1


def tiny_f32(rng, n, scale_log2=-126):
    """binary32 values around the least normal: subnormals of both signs,
    normals a few steps above 2^-126 that cancel into the subnormal range,
    and a few ordinary values."""
    kind = rng.integers(0, 4, n)
    sub = (rng.integers(1, 1 << 23, n).astype(np.uint32) | (rng.integers(0, 2, n).astype(np.uint32) << 31))
    near = ((rng.integers(1, 4, n).astype(np.uint32) << 23) + rng.integers(0, 64, n).astype(np.uint32)) | \
        (rng.integers(0, 2, n).astype(np.uint32) << 31)
    out = np.where(kind == 0, sub, near).view(np.float32).copy()
    out[kind == 3] = (rng.standard_normal(int((kind == 3).sum())) * np.float32(2.0 ** (scale_log2 + 4))).astype(np.float32)
    return out


def _route(ctx, rz, host_inputs, out_shape, out_dtype):
    bufs = [ctx.to_device(np.ascontiguousarray(h)) for h in host_inputs]
    nout = int(np.prod(out_shape)) * np.dtype(out_dtype).itemsize
    bufs.append(ctx.alloc(max(nout, 4)))
    extra = [None] * (len(rz.slots) - len(bufs))
    try:
        route(ctx, rz, bufs + extra)
        return bufs[len(host_inputs)].download(out_dtype, out_shape)
    finally:
        for b in bufs:
            b.free()


def _sum(ctx, x, im, rm, **kw):
    rows, extent = x.shape
    flags = kw.pop("flags", L.REGION_ALIGNED16)
    rz = realize(L.PROGRAM_SERIAL_SUM, (rows, extent), input_subnormals=im, result_subnormals=rm, flags=flags,
                 ctx=ctx, **kw)
    print(f"[modes sum] {rz.symbols} {rows}x{extent} modes=({im},{rm})", flush=True)
    return _route(ctx, rz, [x], (rows,), np.float32)


@pytest.mark.parametrize("reading", range(4))
def test_reference_split_rows_on_the_device(ctx, reading):
    """tests.rs:2125-2260: the two rows under the four readings, the 2x2
    and 4x1 splits and the serial fold, straight from the reference's bits."""
    im, rm = READINGS[reading]
    for row in G["f32_split"]["rows"]:
        x = np.array([int(v, 16) for v in row["contributors"]], np.uint32).view(np.float32).reshape(1, 4)
        want = row["readings"][reading]
        t22 = _sum(ctx, x, im, rm, topology=L.SUM_MULTIPASS, grouping=(2, 2), permissions=RE)
        t41 = _sum(ctx, x, im, rm, topology=L.SUM_MULTIPASS, grouping=(4, 1), permissions=RE)
        assert int(bits(t22)[0]) == int(want["total_2x2"], 16), (row["name"], reading)
        assert int(bits(t41)[0]) == int(want["total_4x1"], 16), (row["name"], reading)
        # the serial fold of four is the 4x1 split's second pass over the same operands
        assert int(bits(_sum(ctx, x, im, rm))[0]) == int(want["total_4x1"], 16), (row["name"], reading)


@pytest.mark.parametrize("rows,extent,flags", [(33, 7, L.REGION_ALIGNED16), (300, 40, L.REGION_ALIGNED16),
                                               (300, 41, 0), (2000, 300, L.REGION_ALIGNED16),
                                               (5, 20000, L.REGION_ALIGNED16), (1, 1, L.REGION_ALIGNED16),
                                               (10, 100, L.REGION_ALIGNED16), (1, 70, L.REGION_ALIGNED16),
                                               (700, 1000, L.REGION_ALIGNED16), (3, 512, L.REGION_ALIGNED16),
                                               (700, 1001, 0), (701, 1000, L.REGION_ALIGNED16)])
@pytest.mark.parametrize("modes", MODES)
def test_serial_sum_under_modes(ctx, rows, extent, flags, modes):
    rng = np.random.default_rng(rows * 7 + extent)
    x = tiny_f32(rng, rows * extent).reshape(rows, extent)
    got = _sum(ctx, x, *modes, flags=flags)
    want = oracle.strict_sum(x, x.shape, 1, input_mode=om(modes[0]), result_mode=om(modes[1]))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("rows,extent,partitions", [(40, 100, 10), (7, 4096, 64), (3, 6, 6), (64, 512, 2)])
@pytest.mark.parametrize("modes", MODES)
def test_split_and_workgroup_sums_under_modes(ctx, rows, extent, partitions, modes):
    rng = np.random.default_rng(rows + extent)
    x = tiny_f32(rng, rows * extent).reshape(rows, extent)
    im, rm = modes
    c = extent // partitions
    got = _sum(ctx, x, im, rm, topology=L.SUM_MULTIPASS, grouping=(partitions, c), permissions=RE)
    want = oracle.strict_partitioned_sum(x, rows, extent, partitions, c, input_mode=om(im), result_mode=om(rm))
    assert np.array_equal(bits(got), bits(want))
    for rounds, major in ((1, False), (2, True)):
        if partitions % rounds:
            continue
        pp = partitions // rounds
        flags = L.REGION_ALIGNED16 | (L.REGION_PARTICIPANT_MAJOR if major else 0)
        got = _sum(ctx, x, im, rm, topology=L.SUM_COOPERATIVE, grouping=(pp, c, rounds), permissions=RE, flags=flags)
        want = oracle.cooperative_grouped_sum(x, rows, extent, pp, c, rounds,
                                              layout=oracle.PARTICIPANT_MAJOR if major else oracle.ROUND_MAJOR,
                                              input_mode=om(im), result_mode=om(rm))
        assert np.array_equal(bits(got), bits(want)), (rounds, major)


def _scale_bias(x, s_bits, b_bits, im, rm):
    """The materialized prologue fl(fl(x * s) + b) under the modes, by the
    oracle's expression evaluator (each node a binary site)."""
    nodes = [(0, 0, 0), (1, s_bits, 0), (3, 0, 1), (1, b_bits, 0), (2, 2, 3)]
    return oracle.expression_f32(nodes, [x.reshape(-1)], input_mode=om(im), result_mode=om(rm)).reshape(x.shape)


@pytest.mark.parametrize("modes", MODES)
def test_scale_bias_fold_under_modes_every_topology(ctx, modes):
    """FusedMultiplyAddSerialSum over the trailing axis (the reference's
    reduction program, x * scale + bias into a sum): serial against
    oracle.fold_f32; the split and the workgroup against the oracle's
    grouping of the materialized prologue, as the reference's split divides
    the materialized reduction."""
    im, rm = modes
    rows, extent = 48, 1024
    rng = np.random.default_rng(11)
    x = tiny_f32(rng, rows * extent).reshape(rows, extent)
    s_bits, b_bits = 0x3F000000, 0x00000003  # 0.5, a subnormal bias
    base = dict(rank=2, variant=L.FOLD_FMA, scalars=(s_bits, b_bits), input_subnormals=im, result_subnormals=rm,
                flags=L.REGION_ALIGNED16, ctx=ctx)
    rz = realize(L.PROGRAM_FOLD, (rows, extent), grouping=(2,), **base)
    got = _route(ctx, rz, [x], (rows,), np.float32)
    want = oracle.fold_f32(x, x.shape, (1,), op=2, scale_bits=s_bits, bias_bits=b_bits, input_mode=om(im),
                           result_mode=om(rm))
    assert np.array_equal(bits(got), bits(want)), rz.symbols
    t = _scale_bias(x, s_bits, b_bits, im, rm)
    rz = realize(L.PROGRAM_FOLD, (rows, extent), grouping=(2, 32, 32), topology=L.SUM_MULTIPASS, permissions=RE,
                 **base)
    got = _route(ctx, rz, [x], (rows,), np.float32)
    want = oracle.strict_partitioned_sum(t, rows, extent, 32, 32, input_mode=om(im), result_mode=om(rm))
    assert np.array_equal(bits(got), bits(want)), rz.symbols
    rz = realize(L.PROGRAM_FOLD, (rows, extent), grouping=(2, 256, 2), topology=L.SUM_COOPERATIVE, permissions=RE,
                 **base)
    got = _route(ctx, rz, [x], (rows,), np.float32)
    want = oracle.cooperative_grouped_sum(t, rows, extent, 256, 2, 2, input_mode=om(im), result_mode=om(rm))
    assert np.array_equal(bits(got), bits(want)), rz.symbols


@pytest.mark.parametrize("variant", [L.FOLD_SUM, L.FOLD_SQUARED, L.FOLD_FMA])
def test_folds_over_leading_axes_under_modes(ctx, variant):
    shape, axes, mask = (6, 7, 8), (0, 2), 0b101
    rng = np.random.default_rng(variant + 5)
    x = tiny_f32(rng, int(np.prod(shape)), scale_log2=-70 if variant == L.FOLD_SQUARED else -126).reshape(shape)
    s_bits, b_bits = 0x3E800000, 0x80000002
    for im, rm in MODES:
        rz = realize(L.PROGRAM_FOLD, shape, rank=3, grouping=(mask,), variant=variant, scalars=(s_bits, b_bits),
                     input_subnormals=im, result_subnormals=rm, flags=L.REGION_ALIGNED16, ctx=ctx)
        assert rz.symbols == ["tiler_fold_f32_m"]
        got = _route(ctx, rz, [x], (7,), np.float32)
        want = oracle.fold_f32(x, shape, axes, op=variant, scale_bits=s_bits, bias_bits=b_bits,
                               input_mode=om(im), result_mode=om(rm))
        assert np.array_equal(bits(got), bits(want)), (im, rm)


@pytest.mark.parametrize("dtype", [L.F32, L.BF16])
@pytest.mark.parametrize("modes", MODES)
def test_rms_norm_under_modes(ctx, dtype, modes):
    """Rows of ~2^-70 (their squares are subnormal), one of normal values, a
    weight with subnormal entries: every site of rms_norm.rs:134-195, 453-489
    under the modes."""
    im, rm = modes
    rows, extent = 12, 300
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((rows, extent)) * 2.0 ** -70).astype(np.float32)
    x[0] = rng.standard_normal(extent).astype(np.float32)
    x[1, :10] = tiny_f32(rng, 10)
    w = rng.normal(1.0, 0.1, extent).astype(np.float32)
    w[:5] = tiny_f32(rng, 5)
    if dtype == L.BF16:
        x = oracle.bf16_widen(oracle.bf16_narrow(x)).reshape(x.shape)
        w = oracle.bf16_widen(oracle.bf16_narrow(w)).reshape(w.shape)
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=dtype, scalars=(0x3727C5AC,), input_subnormals=im,
                 result_subnormals=rm, flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, permissions=RE, ctx=ctx)
    host = [x, w] if dtype == L.F32 else [oracle.bf16_narrow(x).reshape(x.shape), oracle.bf16_narrow(w)]
    got = _route(ctx, rz, host, (rows, extent), np.float32 if dtype == L.F32 else np.uint16)
    want = oracle.rms_norm_f32(x, np.broadcast_to(w, x.shape).copy(), x.shape, 1, 0x3727C5AC, input_mode=om(im),
                               result_mode=om(rm)).reshape(rows, extent)
    if dtype == L.BF16:
        want = oracle.bf16_narrow(want).reshape(rows, extent)
        assert np.array_equal(got, want)
    else:
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("modes", MODES)
def test_softmax_under_modes(ctx, modes):
    """Rows spread over ~100 below their maximum, so exponents and products
    fall into the subnormal range (softmax.rs:237-315 under the modes)."""
    im, rm = modes
    rows, extent = 20, 700
    rng = np.random.default_rng(4)
    x = rng.uniform(-100.0, 0.0, (rows, extent)).astype(np.float32)
    x[0, :8] = tiny_f32(rng, 8)
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), input_subnormals=im, result_subnormals=rm, permissions=RE,
                 flags=L.REGION_ALIGNED16, ctx=ctx)
    got = _route(ctx, rz, [x], (rows, extent), np.float32)
    want = oracle.softmax_f32(x, x.shape, 1, input_mode=om(im), result_mode=om(rm)).reshape(rows, extent)
    assert np.array_equal(bits(got), bits(want))


RESIDENT_RMS = [
    # (rows, extent, dtype, kernel suffix): rows held in registers, 8 per
    # workgroup (tiler_rms_norm_*_strict_rr8_p*_m)
    (2048, 1000, L.BF16, "_strict_rr8_p8_m"),   # a partial fourth chunk
    (2050, 1100, L.F32, "_strict_rr8_p16_m"),   # a ragged last workgroup, a partial chunk
    (2100, 4096, L.BF16, "_strict_rr8_p16_m"),  # the longest resident row
    (2048, 64, L.F32, "_strict_rr8_p8_m"),      # one partial chunk
]
STAGED_RMS = [
    # (rows, extent, dtype, kernel suffix): R rows per staged workgroup
    # (tiler_rms_norm_*_strict_r{1,4,16,64}[_u]_m)
    (3, 9000, L.BF16, "_strict_r1_m"),       # three stages, the last partial
    (1025, 2000, L.F32, "_strict_r4_m"),     # a ragged last workgroup
    (4100, 4104, L.BF16, "_strict_r16_m"),   # longer than the resident rows
    (16400, 102, L.F32, "_strict_r64_u_m"),  # unaligned rows, a lane per row
    (300, 40, L.F32, "_strict"),             # rows under 64: one wave per row
    (33, 63, L.BF16, "_strict"),
]


@pytest.mark.parametrize("rows,extent,dtype,kernel", RESIDENT_RMS + STAGED_RMS)
@pytest.mark.parametrize("modes", MODES)
def test_strict_rms_norm_forms_under_modes(ctx, rows, extent, dtype, kernel, modes):
    """The register-resident and staged strict RMSNorm under the modes: rows
    of ~2^-70 (subnormal squares), rows of normal values, rows opening with
    subnormal entries, a weight with subnormal entries, bit for bit with the
    oracle."""
    im, rm = modes
    rng = np.random.default_rng(rows + extent)
    x = (rng.standard_normal((rows, extent)) * 2.0 ** -70).astype(np.float32)
    x[::7] = rng.standard_normal((len(range(0, rows, 7)), extent)).astype(np.float32)
    x[1::5, :10] = tiny_f32(rng, 10 * len(range(1, rows, 5))).reshape(-1, 10)
    w = rng.normal(1.0, 0.1, extent).astype(np.float32)
    w[:5] = tiny_f32(rng, 5)
    if dtype == L.BF16:
        x = oracle.bf16_widen(oracle.bf16_narrow(x)).reshape(x.shape)
        w = oracle.bf16_widen(oracle.bf16_narrow(w)).reshape(w.shape)
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=dtype, scalars=(0x3727C5AC,), input_subnormals=im,
                 result_subnormals=rm, flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, permissions=RE, ctx=ctx)
    print(f"[modes rms] {rz.symbols} {rows}x{extent} modes=({im},{rm})", flush=True)
    assert len(rz.symbols) == 1 and rz.symbols[0].endswith(kernel), rz.symbols
    host = [x, w] if dtype == L.F32 else [oracle.bf16_narrow(x).reshape(x.shape), oracle.bf16_narrow(w)]
    got = _route(ctx, rz, host, (rows, extent), np.float32 if dtype == L.F32 else np.uint16)
    want = oracle.rms_norm_f32(x, np.broadcast_to(w, x.shape).copy(), x.shape, 1, 0x3727C5AC, input_mode=om(im),
                               result_mode=om(rm)).reshape(rows, extent)
    if dtype == L.BF16:
        assert np.array_equal(got, oracle.bf16_narrow(want).reshape(rows, extent))
    else:
        assert np.array_equal(bits(got), bits(want))


RESIDENT_SOFTMAX = [
    # (rows, extent, kernel suffix): tiler_softmax_f32_strict_rr8_p*_m
    (4096, 200, "_strict_rr8_p8_m"),    # two chunks, the second partial
    (2050, 1100, "_strict_rr8_p16_m"),  # a ragged last workgroup, a partial ninth chunk
    (2048, 2048, "_strict_rr8_p16_m"),  # two whole ring rounds
    (2050, 3000, "_strict_rr8_p32_m"),  # a ragged last workgroup, a partial third ring round
]
STAGED_SOFTMAX = [
    # (rows, extent, kernel suffix): tiler_softmax_f32_strict_r{1,4,16}[_u]_m
    (6, 9000, "_strict_r1_m"),      # three stages, the last partial
    (300, 1001, "_strict_r1_u_m"),  # unaligned rows
    (1025, 2048, "_strict_r4_m"),   # a ragged last workgroup
    (4100, 4100, "_strict_r16_m"),  # longer than the resident rows
    (300, 40, "_strict"),           # rows under 64: one wave per row
    (33, 63, "_strict"),
]


@pytest.mark.parametrize("rows,extent,kernel", RESIDENT_SOFTMAX + STAGED_SOFTMAX)
@pytest.mark.parametrize("modes", MODES)
def test_strict_softmax_forms_under_modes(ctx, rows, extent, kernel, modes):
    """The register-resident and staged strict softmax under the modes: rows
    spread over ~100 below their maximum (subnormal exponents and products),
    rows of subnormal inputs, and a NaN row, bit for bit with the oracle."""
    im, rm = modes
    rng = np.random.default_rng(rows * 3 + extent)
    x = rng.uniform(-100.0, 0.0, (rows, extent)).astype(np.float32)
    x[1::9] = tiny_f32(rng, extent * len(range(1, rows, 9))).reshape(-1, extent)
    x[5, extent // 2] = np.nan
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), input_subnormals=im, result_subnormals=rm, permissions=RE,
                 flags=L.REGION_ALIGNED16, ctx=ctx)
    print(f"[modes softmax] {rz.symbols} {rows}x{extent} modes=({im},{rm})", flush=True)
    assert len(rz.symbols) == 1 and rz.symbols[0].endswith(kernel), rz.symbols
    got = _route(ctx, rz, [x], (rows, extent), np.float32)
    # rows are independent: past 2.5M elements (the oracle's certified exp
    # takes ~1.7 s per million) compare the planted rows, the first and last
    # workgroups and 64 drawn rows
    if rows * extent > 2_500_000:
        keep = np.unique(np.concatenate([np.arange(16), np.arange(rows - 16, rows), rng.choice(rows, 64, replace=False)]))
        x, got = np.ascontiguousarray(x[keep]), got[keep]
    want = oracle.softmax_f32(x, x.shape, 1, input_mode=om(im), result_mode=om(rm)).reshape(x.shape)
    assert np.array_equal(bits(got), bits(want))


def _map(ctx, op, dtype, x, x2=None, a=0.0, b=0.0, modes=(P, P)):
    n = x.size
    import struct
    sa = struct.unpack("<I", struct.pack("<f", a))[0]
    sb = struct.unpack("<I", struct.pack("<f", b))[0]
    rz = realize(L.PROGRAM_POINTWISE, (n,), dtype=dtype, variant=op, scalars=(sa, sb), input_subnormals=modes[0],
                 result_subnormals=modes[1], flags=L.REGION_ALIGNED16, ctx=ctx)
    assert rz.symbols[0].endswith("_m"), rz.symbols
    return _route(ctx, rz, [x] + ([x2] if x2 is not None else []), (n,), x.dtype)


@pytest.mark.parametrize("modes", MODES)
def test_f32_maps_under_modes(ctx, modes):
    im, rm = modes
    rng = np.random.default_rng(5)
    x = tiny_f32(rng, 5000)
    x2 = tiny_f32(rng, 5000) * np.float32(2.0 ** 3)
    x[:4] = np.array([0x7FC01234, 0x7F800000, 0xFF800000, 0x80000000], np.uint32).view(np.float32)
    sb_nodes = [(0, 0, 0), (1, 0x3F000000, 0), (3, 0, 1), (1, 0x00000005, 0), (2, 2, 3)]
    want = oracle.expression_f32(sb_nodes, [x], input_mode=om(im), result_mode=om(rm))
    got = _map(ctx, L.MAP_SCALE_BIAS, L.F32, x, a=0.5, b=float(np.uint32(5).view(np.float32)), modes=modes)
    assert np.array_equal(bits(got), bits(want))
    for op, node in ((L.MAP_ADD, 2), (L.MAP_MULTIPLY, 3)):
        want = oracle.expression_f32([(0, 0, 0), (0, 1, 0), (node, 0, 1)], [x, x2], input_mode=om(im),
                                     result_mode=om(rm))
        assert np.array_equal(bits(_map(ctx, op, L.F32, x, x2, modes=modes)), bits(want)), op
    want = oracle.silu_f32(x, input_mode=om(im), result_mode=om(rm))
    assert np.array_equal(bits(_map(ctx, L.MAP_SILU, L.F32, x, modes=modes)), bits(want))


@pytest.mark.parametrize("reading", range(4))
def test_bf16_counterexamples_on_the_device(ctx, reading):
    """bf16/tests.rs:722-835: the seven cases under each reading, through the
    bf16 maps and the bf16 expression kernels."""
    im, rm = READINGS[reading]
    cases = G["bf16_counterexamples"]["cases"]
    left = np.array([int(c["left"], 16) for c in cases], np.uint16)
    right = np.array([int(c["right"], 16) for c in cases], np.uint16)
    want = np.array([int(c["readings"][reading], 16) for c in cases], np.uint16)
    if (im, rm) == (P, P):
        return  # the preserving reading is the vector kernels' (test_gpu_programs)
    for i, c in enumerate(cases):
        op = L.MAP_ADD if c["op"] == "add" else L.MAP_MULTIPLY
        got = _map(ctx, op, L.BF16, left[i:i + 1].copy(), right[i:i + 1].copy(), modes=(im, rm))
        assert int(got[0]) == int(want[i]), (c, reading)
        node = 2 if c["op"] == "add" else 3
        rz = realize(L.PROGRAM_EXPRESSION, (1,), dtype=L.BF16, nodes=[(0, 0, 0), (0, 1, 0), (node, 0, 1)],
                     input_subnormals=im, result_subnormals=rm, flags=L.REGION_ALIGNED16, ctx=ctx)
        got = _route(ctx, rz, [left[i:i + 1], right[i:i + 1]], (1,), np.uint16)
        assert int(got[0]) == int(want[i]), (c, reading, rz.symbols)


@pytest.mark.parametrize("modes", MODES)
def test_bf16_expressions_and_maps_under_modes(ctx, modes):
    im, rm = modes
    rng = np.random.default_rng(6)
    n = 6000
    x = oracle.bf16_narrow(tiny_f32(rng, n) * np.float32(2.0 ** rng.integers(0, 8)))
    x2 = oracle.bf16_narrow(rng.uniform(-2, 2, n).astype(np.float32))
    nodes = [(0, 0, 0), (0, 1, 0), (3, 0, 1), (1, 0x3F00, 0), (3, 2, 3), (2, 4, 0)]
    want = oracle.expression_bf16(nodes, [x, x2], input_mode=om(im), result_mode=om(rm))
    rz = realize(L.PROGRAM_EXPRESSION, (n,), dtype=L.BF16, nodes=nodes, input_subnormals=im, result_subnormals=rm,
                 flags=L.REGION_ALIGNED16, ctx=ctx)
    got = _route(ctx, rz, [x, x2], (n,), np.uint16)
    assert np.array_equal(got, want), rz.symbols
    sb = [(0, 0, 0), (1, 0x3F00, 0), (3, 0, 1), (1, 0x0003, 0), (2, 2, 3)]
    want = oracle.expression_bf16(sb, [x], input_mode=om(im), result_mode=om(rm))
    got = _map(ctx, L.MAP_SCALE_BIAS, L.BF16, x, a=0.5, b=float(oracle.bf16_widen(np.array([3], np.uint16))[0]),
               modes=modes)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("modes", MODES)
def test_contractions_under_modes(ctx, modes):
    """contraction.rs:600-625 under the modes: td,od->to in f32 and bf16
    (+SiLU) and an attention-shaped structure, against oracle.contract_general
    with the same modes; operands ~2^-65 so products and partial sums fall
    into the subnormal range."""
    im, rm = modes
    rng = np.random.default_rng(8)
    m, n, k = 37, 45, 29
    a = (rng.standard_normal((m, k)) * 2.0 ** -65).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 2.0 ** -65).astype(np.float32)
    a[0, :5] = tiny_f32(rng, 5)
    b[1, :5] = tiny_f32(rng, 5)
    b[2] = rng.standard_normal(k).astype(np.float32) * 2.0 ** 60
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), input_subnormals=im, result_subnormals=rm, permissions=RE,
                 flags=L.REGION_ALIGNED16, ctx=ctx)
    assert rz.symbols == ["tiler_contract_general_f32_m"], rz.symbols
    got = _route(ctx, rz, [a, b], (m, n), np.float32)
    want = oracle.contract_general(a, "mk", b, "nk", "mn", input_mode=om(im), result_mode=om(rm))
    assert np.array_equal(bits(got), bits(want))
    a16 = oracle.bf16_narrow(a * np.float32(2.0 ** 60)).reshape(m, k)
    b16 = oracle.bf16_narrow(b * np.float32(2.0 ** -60)).reshape(n, k)
    for ep in (L.EPILOGUE_NONE, L.EPILOGUE_SILU):
        rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16, variant=ep, input_subnormals=im,
                     result_subnormals=rm, permissions=RE, flags=L.REGION_ALIGNED16, ctx=ctx)
        got = _route(ctx, rz, [a16, b16], (m, n), np.uint16)
        want = oracle.contract_general(a16, "mk", b16, "nk", "mn", silu=ep == L.EPILOGUE_SILU,
                                       input_mode=om(im), result_mode=om(rm))
        assert np.array_equal(got, want), (ep, rz.symbols)
    # attention scores bhqd,bkd->bhqk (the key shared across heads)
    q = (rng.standard_normal((2, 3, 5, 16)) * 2.0 ** -66).astype(np.float32)
    kk = (rng.standard_normal((2, 7, 16)) * 2.0 ** -66).astype(np.float32)
    st = L.contraction_structure("bhqd", q.shape, "bkd", kk.shape, "bhqk")
    rz = realize(L.PROGRAM_CONTRACTION, (), structure=st, input_subnormals=im, result_subnormals=rm,
                 flags=L.REGION_ALIGNED16, ctx=ctx)
    got = _route(ctx, rz, [q, kk], (2, 3, 5, 7), np.float32)
    want = oracle.contract_general(q, "bhqd", kk, "bkd", "bhqk", input_mode=om(im), result_mode=om(rm))
    assert np.array_equal(bits(got), bits(want)), rz.symbols
