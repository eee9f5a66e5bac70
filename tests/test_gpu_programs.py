"""GPU parity for the realizations added behind the numerical contract:

* pointwise expression DAGs (ScalarProgram::PointwiseF32 / PointwiseBf16,
  tiler-ir/src/schedule/pointwise.rs:74-140, pointwise_bf16.rs:114-168):
  the tiler-metal golden expressions, seeded random DAGs up to the 4096-node
  limit, special values, the subnormal modes, every kernel form -- bit-exact
  with the oracle (f32: IEEE nodes + certified exp/rsqrt; bf16: each node
  rounded once from its exact binary128 value);
* serial folds over any axis set (StrictSerialSum multi-axis,
  SquaredSerialSum, FusedMultiplyAddSerialSum, StrictSerialMaximum,
  SquaredSerialSumThenEpilogue) -- bit-exact with oracle.fold_f32;
* the strict realizations a region without permits_reassociation gets:
  RMSNorm and softmax with the reference's serial fold (bit-exact with
  oracle.rms_norm_f32 / softmax_f32, the reference's own forms) and the
  strict bf16 contraction;
* the mirrored reindex golden, the target environment, and plan_dispatch's
  grid check.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from helpers import bits, bf16_widen
from tiler_amd import _lib as L
from tiler_amd import runtime
from tiler_amd.realize import realize, route

pytestmark = pytest.mark.gpu

RE = L.PERMITS_REASSOCIATION


def _random_dag(rng, inputs, extra, ops, max_nodes=4096):
    """A DAG over `inputs` leaves with `extra` random interior nodes, every
    node reachable from the root (dangling values are added into it)."""
    nodes = [(L.NODE_INPUT, k, 0) for k in range(inputs)]
    consts = [0x3F800000, 0x40000000, 0xBF000000, 0x3E800000, 0x00000001, 0x7F800000, 0x80000000, 0x3F7FFFFF]
    for _ in range(extra):
        op = ops[rng.integers(len(ops))]
        i = len(nodes)
        if op == L.NODE_CONSTANT:
            c = consts[rng.integers(len(consts))]
            nodes.append((op, c, 0))
        elif op in (L.NODE_EXP, L.NODE_RSQRT):
            nodes.append((op, int(rng.integers(i)), 0))
        else:
            nodes.append((op, int(rng.integers(i)), int(rng.integers(i))))
    used = set()
    for op, a, b in nodes:
        if op >= L.NODE_ADD:
            used.add(a)
            if op <= L.NODE_DIVIDE:
                used.add(b)
    dangling = [i for i in range(len(nodes)) if i not in used]
    acc = dangling[0]
    for d in dangling[1:]:
        nodes.append((L.NODE_ADD, acc, d))
        acc = len(nodes) - 1
    assert len(nodes) <= max_nodes
    return nodes


def _f32_inputs(rng, count, n):
    out = []
    for k in range(count):
        x = (rng.standard_normal(n) * np.exp2(rng.integers(-4, 5))).astype(np.float32)
        x[rng.integers(n, size=max(1, n // 97))] = rng.choice(
            np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -3e-39, 88.0, -104.5], np.float32))
        out.append(x)
    return out


def _run_direct(ctx, dtype, nodes, xs, modes=(0, 0)):
    n = xs[0].size
    dev = [ctx.to_device(x) for x in xs]
    dy = ctx.alloc(max(1, n * xs[0].itemsize))
    try:
        ctx.expression(dtype, nodes, dev, n, dy, input_subnormals=modes[0], result_subnormals=modes[1])
        ctx.synchronize()
        return dy.download(xs[0].dtype, (n,))
    finally:
        for b in dev + [dy]:
            b.free()


def _run_routed(ctx, dtype, nodes, xs, modes=(0, 0), flags=L.REGION_ALIGNED16):
    n = xs[0].size
    rz = realize(L.PROGRAM_EXPRESSION, (n,), dtype=dtype, nodes=nodes, flags=flags,
                 input_subnormals=modes[0], result_subnormals=modes[1], ctx=ctx)
    dev = [ctx.to_device(x) for x in xs]
    dy = ctx.alloc(max(1, n * xs[0].itemsize))
    storage = dev + [dy] + [None] * (len(rz.slots) - len(dev) - 1)
    try:
        route(ctx, rz, storage)
        return dy.download(xs[0].dtype, (n,)), rz.symbols
    finally:
        for b in dev + [dy]:
            b.free()


_O_MODE = {0: oracle.PRESERVE, 1: oracle.PRESERVE, 2: oracle.FLUSH_SIGN_PRESERVING, 3: oracle.FLUSH_POSITIVE_ZERO}


def test_expression_goldens(ctx):
    # pointwise_scale_bias{,_bf16}.metal: y = x*2 + 1, one rounding per node
    x = np.array([1.0, -2.5, np.nan, 3e38, -0.0, 1e-45, 7.0, 0.1], np.float32)
    sb = [(0, 0, 0), (1, 0x40000000, 0), (3, 0, 1), (1, 0x3F800000, 0), (2, 2, 3)]
    want = oracle.expression_f32(sb, [x])
    assert np.array_equal(bits(_run_direct(ctx, L.F32, sb, [x])), bits(want))
    assert bits(want)[2] == 0x7FC00000 and np.isinf(want[3])
    xb = oracle.bf16_narrow(x)
    sbb = [(0, 0, 0), (1, 0x4000, 0), (3, 0, 1), (1, 0x3F80, 0), (2, 2, 3)]
    got = _run_direct(ctx, L.BF16, sbb, [xb])
    assert np.array_equal(got, oracle.expression_bf16(sbb, [xb]))
    assert got[2] == 0x7FC0
    # elementary_silu_activation.metal: x / (1 + exp(-x)) spelled as a DAG
    xs = (np.random.default_rng(3).standard_normal(4096) * 30).astype(np.float32)
    silu = [(0, 0, 0), (1, 0xBF800000, 0), (3, 0, 1), (5, 2, 0), (1, 0x3F800000, 0), (2, 4, 3), (4, 0, 5)]
    got = _run_direct(ctx, L.F32, silu, [xs])
    assert np.array_equal(bits(got), bits(oracle.silu_f32(xs)))


@pytest.mark.parametrize("seed", range(6))
def test_random_f32_dags(ctx, seed):
    rng = np.random.default_rng(100 + seed)
    inputs = int(rng.integers(1, 6))
    extra = int(rng.integers(3, 40))
    nodes = _random_dag(rng, inputs, extra, [L.NODE_CONSTANT, L.NODE_ADD, L.NODE_MULTIPLY, L.NODE_DIVIDE,
                                             L.NODE_EXP, L.NODE_RSQRT])
    n = (1 << 16) if seed % 2 == 0 else 50021
    xs = _f32_inputs(rng, inputs, n)
    print(f"[expr f32] seed={seed} nodes={len(nodes)} inputs={inputs} n={n}", flush=True)
    want = oracle.expression_f32(nodes, xs)
    got = _run_direct(ctx, L.F32, nodes, xs)
    assert np.array_equal(bits(got), bits(want)), np.flatnonzero(bits(got) != bits(want))[:5]
    got2, symbols = _run_routed(ctx, L.F32, nodes, xs)
    assert np.array_equal(bits(got2), bits(want)), symbols


@pytest.mark.parametrize("seed", range(4))
def test_random_bf16_dags(ctx, seed):
    rng = np.random.default_rng(200 + seed)
    inputs = int(rng.integers(1, 5))
    nodes = _random_dag(rng, inputs, int(rng.integers(3, 40)), [L.NODE_CONSTANT, L.NODE_ADD, L.NODE_MULTIPLY])
    # the f32 constants' upper halves are bf16 constants (0x3F80 = 1, 0x7F80 = inf, ...)
    nodes = [(op, a >> 16 if op == L.NODE_CONSTANT else a, b) for op, a, b in nodes]
    n = (1 << 16) if seed % 2 == 0 else 30011
    xs = [oracle.bf16_narrow(x) for x in _f32_inputs(rng, inputs, n)]
    print(f"[expr bf16] seed={seed} nodes={len(nodes)} inputs={inputs} n={n}", flush=True)
    want = oracle.expression_bf16(nodes, xs)
    assert np.array_equal(_run_direct(ctx, L.BF16, nodes, xs), want)
    got, symbols = _run_routed(ctx, L.BF16, nodes, xs)
    assert np.array_equal(got, want), symbols


def test_expressions_at_the_node_limit_and_sixteen_inputs(ctx):
    # 4096 nodes whose register program needs far more than 16 registers:
    # the value-store form, through both the direct call and the route
    rng = np.random.default_rng(7)
    nodes = [(L.NODE_INPUT, 0, 0), (L.NODE_INPUT, 1, 0)]
    while len(nodes) < 2048:
        i = len(nodes)
        nodes.append((int(rng.choice([L.NODE_ADD, L.NODE_MULTIPLY])), int(rng.integers(i)), int(rng.integers(i))))
    used = set(a for op, a, b in nodes if op >= 2) | set(b for op, a, b in nodes if 2 <= op <= 4)
    dangling = [i for i in range(len(nodes)) if i not in used]
    acc = dangling[0]
    for d in dangling[1:]:
        nodes.append((L.NODE_ADD, acc, d))
        acc = len(nodes) - 1
    while len(nodes) < 4096:
        nodes.append((L.NODE_MULTIPLY, len(nodes) - 1, 0))
    assert len(nodes) == 4096
    xs = [(rng.standard_normal(20001) * 0.5).astype(np.float32) for _ in range(2)]
    want = oracle.expression_f32(nodes, xs)
    got, symbols = _run_routed(ctx, L.F32, nodes, xs)
    print(f"[expr limit] {symbols}", flush=True)
    assert symbols == ["tiler_expr_f32_mem"]
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(_run_direct(ctx, L.F32, nodes, xs)), bits(want))
    # sixteen inputs summed in order
    sixteen = [(L.NODE_INPUT, k, 0) for k in range(16)]
    acc = 0
    for k in range(1, 16):
        sixteen.append((L.NODE_ADD, acc, k))
        acc = len(sixteen) - 1
    ys = _f32_inputs(rng, 16, 4096)
    assert np.array_equal(bits(_run_direct(ctx, L.F32, sixteen, ys)), bits(oracle.expression_f32(sixteen, ys)))


@pytest.mark.parametrize("modes", [(2, 2), (3, 3), (2, 1), (1, 3)])
def test_f32_expression_subnormal_modes(ctx, modes):
    rng = np.random.default_rng(11)
    n = 8192
    x0 = (rng.standard_normal(n) * 1e-38).astype(np.float32)   # many subnormal operands
    x1 = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    x0[:4] = [-1e-45, 1e-45, -0.0, 5e-39]
    # x0*0.5 + (x0 / rsqrt(x1*x1)) * x1: subnormal operands (x0) and
    # subnormal results (x0*0.5, x0*|x1|, ...) on most elements, every node kind
    nodes = [(0, 0, 0), (0, 1, 0), (3, 1, 1), (6, 2, 0), (4, 0, 3), (3, 4, 1), (1, 0x3F000000, 0), (3, 0, 6),
             (2, 7, 5)]
    want = oracle.expression_f32(nodes, [x0, x1], input_mode=_O_MODE[modes[0]], result_mode=_O_MODE[modes[1]])
    preserve = oracle.expression_f32(nodes, [x0, x1])
    assert not np.array_equal(bits(want), bits(preserve))  # the modes are observable here
    assert np.array_equal(bits(_run_direct(ctx, L.F32, nodes, [x0, x1], modes)), bits(want))
    got, symbols = _run_routed(ctx, L.F32, nodes, [x0, x1], modes)
    assert symbols == ["tiler_expr_f32_r16f_i2"] and np.array_equal(bits(got), bits(want))
    got, symbols = _run_routed(ctx, L.F32, nodes, [x0, x1], modes, flags=0)
    assert symbols == ["tiler_expr_f32_r16s_i2"] and np.array_equal(bits(got), bits(want))


def test_expression_forms_agree_on_unaligned_storage(ctx):
    rng = np.random.default_rng(12)
    nodes = [(0, 0, 0), (0, 1, 0), (3, 0, 1), (5, 2, 0)]
    xs = _f32_inputs(rng, 2, 4096)
    want = oracle.expression_f32(nodes, xs)
    got, symbols = _run_routed(ctx, L.F32, nodes, xs, flags=0)
    assert symbols == ["tiler_expr_f32_r16s_i2"] and np.array_equal(bits(got), bits(want))
    # a direct call on storage 4 bytes off a 16-byte boundary
    base = [ctx.alloc(4 * 4097) for _ in range(2)]
    dy = ctx.alloc(4 * 4097)
    try:
        views = [b.offset(4) for b in base]
        for v, x in zip(views, xs):
            v.upload(x)
        ctx.expression(L.F32, nodes, views, 4096, dy.offset(4))
        ctx.synchronize()
        out = dy.download(np.float32, (4097,))[1:]
        assert np.array_equal(bits(out), bits(want))
    finally:
        for b in base + [dy]:
            b.free()


# --- folds ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape,axes", [((2, 3, 4), (1, 2)), ((7, 5, 9), (0, 2)), ((64, 33), (0,)),
                                        ((3, 4, 5, 6), (1, 3)), ((1000, 257), (1,)), ((6,), (0,))])
@pytest.mark.parametrize("variant", [L.FOLD_SUM, L.FOLD_SQUARED, L.FOLD_FMA, L.FOLD_MAXIMUM])
def test_folds_over_any_axes(ctx, shape, axes, variant):
    rng = np.random.default_rng(hash((shape, axes, variant)) & 0xFFFF)
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    flat = x.reshape(-1)
    flat[rng.integers(flat.size, size=max(1, flat.size // 50))] = rng.choice(
        np.array([0.0, -0.0, 1e-40, np.inf, 3e38], np.float32))
    if variant == L.FOLD_MAXIMUM and flat.size > 10:
        flat[3] = np.nan
    sb = (0x40000000, 0x3F800000) if variant == L.FOLD_FMA else (0, 0)
    want = oracle.fold_f32(x, shape, axes, op=variant, scale_bits=sb[0], bias_bits=sb[1])
    dx, do = ctx.to_device(x), ctx.alloc(max(4, want.nbytes))
    try:
        ctx.fold_f32(variant, dx, shape, axes, do, scale_bits=sb[0], bias_bits=sb[1])
        ctx.synchronize()
        got = do.download(np.float32, want.shape)
    finally:
        dx.free(); do.free()
    assert np.array_equal(bits(got), bits(want))


def test_fold_goldens_and_epilogue(ctx):
    # reduction_multi_axis.metal [2,3,4] over axes (1,2); reduction_fused_multiply_add.metal [2,3] x*2+1
    x = np.arange(24, dtype=np.float32)
    rz = realize(L.PROGRAM_FOLD, (2, 3, 4), rank=3, grouping=(0b110,), ctx=ctx)
    dx, do = ctx.to_device(x), ctx.alloc(8)
    try:
        route(ctx, rz, [dx, do])
        assert do.download(np.float32, (2,)).tolist() == [66.0, 210.0]
        fma = realize(L.PROGRAM_FOLD, (2, 3), rank=2, grouping=(0b10,), variant=L.FOLD_FMA,
                      scalars=(0x40000000, 0x3F800000), ctx=ctx)
        route(ctx, fma, [dx, do])
        assert do.download(np.float32, (2,)).tolist() == [9.0, 27.0]
    finally:
        dx.free(); do.free()
    # SquaredSerialSumThenEpilogue: rsqrt(a / N + eps), the RMSNorm row scale
    rows, n, eps = 64, 4096, 0x3727C5AC
    y = np.random.default_rng(13).standard_normal((rows, n)).astype(np.float32)
    epi = [(0, 0, 0), (1, int(bits(np.array([float(n)], np.float32))[0]), 0), (4, 0, 1), (1, eps, 0),
           (2, 2, 3), (6, 4, 0)]
    rz = realize(L.PROGRAM_FOLD, (rows, n), rank=2, grouping=(0b10,), variant=L.FOLD_SQUARED, nodes=epi, ctx=ctx)
    sq = oracle.fold_f32(y, y.shape, (1,), op=1)
    want = oracle.expression_f32(epi, [sq])
    dx, do = ctx.to_device(y), ctx.alloc(4 * rows)
    try:
        route(ctx, rz, [dx, do, None])
        assert np.array_equal(bits(do.download(np.float32, (rows,))), bits(want))
    finally:
        dx.free(); do.free()


# --- strict rows and contraction ------------------------------------------------------

def _route_rows(ctx, program, x, w=None, dtype=L.F32, eps=0, broadcast=True):
    rows, extent = x.shape
    flags = L.REGION_ALIGNED16 | (L.REGION_OPERAND_BROADCAST if broadcast else 0)
    rz = realize(program, (rows, extent), dtype=dtype, scalars=(eps,), flags=flags, ctx=ctx)
    assert "_strict" in rz.symbols[-1], rz.symbols
    bufs = [ctx.to_device(x)] + ([ctx.to_device(w)] if w is not None else []) + [ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        return bufs[-1].download(x.dtype, x.shape)
    finally:
        for b in bufs:
            b.free()


def test_strict_rms_norm_is_the_reference_fold(ctx):
    # worked example (rms_norm/tests.rs:253-276): x=[3,4], w=[1,2], eps 0x358637bd
    y = _route_rows(ctx, L.PROGRAM_RMS_NORM, np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32),
                    eps=0x358637BD)
    assert bits(y).reshape(-1).tolist() == [0x3F593923, 0x4010D0C2]
    rng = np.random.default_rng(21)
    for rows, extent in ((37, 1000), (8, 4096), (3, 20000)):
        x = rng.standard_normal((rows, extent)).astype(np.float32)
        w = rng.normal(1.0, 0.1, extent).astype(np.float32)
        want = oracle.rms_norm_f32(x, np.broadcast_to(w, x.shape).copy(), x.shape, 1, 0x3727C5AC)
        got = _route_rows(ctx, L.PROGRAM_RMS_NORM, x, w, eps=0x3727C5AC)
        assert np.array_equal(bits(got).reshape(-1), bits(want).reshape(-1)), (rows, extent)
    # bf16 storage: the strict fold on exactly widened values, one narrowing
    xb = oracle.bf16_narrow(rng.standard_normal((64, 4096)).astype(np.float32)).reshape(64, 4096)
    wb = oracle.bf16_narrow(rng.normal(1.0, 0.1, 4096).astype(np.float32))
    wantf = oracle.rms_norm_f32(bf16_widen(xb), np.broadcast_to(bf16_widen(wb), xb.shape).copy(), xb.shape, 1,
                                0x3727C5AC)
    got = _route_rows(ctx, L.PROGRAM_RMS_NORM, xb, wb, dtype=L.BF16, eps=0x3727C5AC)
    assert np.array_equal(got.reshape(-1), oracle.bf16_narrow(wantf).reshape(-1))


@pytest.mark.parametrize("rows,extent,dtype,broadcast,form", [
    (4096, 4104, L.BF16, True, "_strict_r16"),  # 16-byte loads, staged (rows past 4096 bf16)
    (1500, 300, L.F32, True, "_strict_r4"),
    (1025, 2000, L.BF16, True, "_strict_r4"),  # the last workgroup holding one row
    (20000, 64, L.BF16, True, "_strict_r64"),   # one stage
    (700, 1001, L.F32, False, "_strict_r1_u"),  # 4-byte loads, a weight row per row, a ragged stage
    (300, 1030, L.BF16, True, "_strict_r1_u"),
    (32, 4096, L.BF16, True, "_strict_r1"),     # decode rows: one row per workgroup, one whole stage
    (3, 10000, L.F32, True, "_strict_r1"),      # long rows: three stages, the last ragged
    # rows held in registers, 8 per workgroup (tiler_rms_norm_*_strict_rr8_p*)
    (8192, 4096, L.BF16, True, "_strict_rr8_p16"),   # the C2 configuration
    (2050, 1100, L.F32, False, "_strict_rr8_p16"),   # a weight row per row, a ragged last workgroup, a partial chunk
    (2048, 1000, L.BF16, True, "_strict_rr8_p8"),    # a partial fourth chunk, one ring round
    (2100, 2048, L.BF16, False, "_strict_rr8_p8"),   # two whole ring rounds
    (3000, 64, L.F32, True, "_strict_rr8_p8"),       # one partial chunk
])
def test_strict_rms_norm_staged_rows(ctx, rows, extent, dtype, broadcast, form):
    """Rows of >= 64 run the staged strict fold (tiler_rms_norm_*_strict_r*)
    or, for aligned rows of at most 512 16-byte pieces and enough of them,
    the register-resident one (_rr8_p*): the reference's serial fold of the
    squares, then its division, eps and certified rsqrt, bit for bit against
    the oracle (bf16: on exactly widened values, one narrowing).  Row 0 is all
    zeros (0 / N + eps), row 1 holds a NaN and row 2 an infinity; a ragged
    last workgroup also gets a NaN row and a zero row."""
    rng = np.random.default_rng(rows + extent)
    x = rng.standard_normal((rows, extent)).astype(np.float32) * np.float32(3.0)
    x[0] = 0.0
    x[1, extent // 2] = np.nan
    x[2, 0] = np.inf
    if rows % 8:
        x[rows - 1, extent - 1] = np.nan
        x[rows - 2] = 0.0
    w = rng.normal(1.0, 0.1, extent if broadcast else (rows, extent)).astype(np.float32)
    if dtype == L.BF16:
        x, w = oracle.bf16_narrow(x).reshape(x.shape), oracle.bf16_narrow(w).reshape(w.shape)
        xf, wf = bf16_widen(x), bf16_widen(w)
    else:
        xf, wf = x, w
    flags = L.REGION_ALIGNED16 | (L.REGION_OPERAND_BROADCAST if broadcast else 0)
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=dtype, scalars=(0x3727C5AC,), flags=flags, ctx=ctx)
    assert rz.symbols[-1].endswith(form), rz.symbols
    print(f"[strict rms] {rz.symbols[-1]} rows={rows} extent={extent}", flush=True)
    bufs = [ctx.to_device(x), ctx.to_device(w), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[-1].download(x.dtype, x.shape)
    finally:
        for b in bufs:
            b.free()
    want = oracle.rms_norm_f32(xf, np.broadcast_to(wf, xf.shape).copy(), xf.shape, 1, 0x3727C5AC).reshape(rows, extent)
    if dtype == L.BF16:
        want = oracle.bf16_narrow(want).reshape(rows, extent)
    assert np.array_equal(bits(got) if dtype == L.F32 else got, bits(want) if dtype == L.F32 else want)


def test_strict_softmax_is_the_reference_fold(ctx):
    # worked example (softmax/tests.rs:362-455): [1, 2, 3, mask]
    x = np.array([[1.0, 2.0, 3.0, -np.inf]], np.float32)
    got = _route_rows(ctx, L.PROGRAM_SOFTMAX, x)
    assert bits(got).reshape(-1).tolist() == [0x3DB861F3, 0x3E7A9A1A, 0x3F2A4D3B, 0]
    rng = np.random.default_rng(22)
    for rows, extent in ((100, 2048), (5, 9000), (2, 70000)):
        x = (rng.standard_normal((rows, extent)) * 3).astype(np.float32)
        x[0, 5] = np.nan
        want = oracle.softmax_f32(x, x.shape, 1)
        got = _route_rows(ctx, L.PROGRAM_SOFTMAX, x)
        assert np.array_equal(bits(got).reshape(-1), bits(want).reshape(-1)), (rows, extent)


@pytest.mark.parametrize("rows,extent,form", [
    (16384, 64, "_strict_r16"),    # one partial stage (the oracle's certified exp keeps these small)
    (4500, 530, "_strict_r16_u"),  # 4-byte loads, three stages, a ragged last workgroup
    (1500, 301, "_strict_r4_u"),   # 4-byte loads, a ragged last stage
    (300, 72, "_strict_r1"),
    (1024, 2048, "_strict_r4"),    # 16-byte loads, whole stages, four rows per workgroup
    (1025, 2048, "_strict_r4"),    # the last workgroup holding one row
    (32, 2048, "_strict_r1"),      # decode rows: one row per workgroup, one partial stage
    (4, 9000, "_strict_r1"),       # long rows: three stages, the last ragged
    # rows held in registers, 8 per workgroup (tiler_softmax_f32_strict_rr8_p*)
    (4096, 200, "_strict_rr8_p8"),   # two chunks, the second partial
    (4096, 512, "_strict_rr8_p8"),
    (2050, 1100, "_strict_rr8_p16"),  # a ragged last workgroup, a partial ninth chunk, two ring rounds
    (2048, 1028, "_strict_rr8_p16"),  # one 4-column group in the ninth chunk
    (2100, 1024, "_strict_rr8_p8"),   # eight whole chunks, one ring round
    (3000, 128, "_strict_rr8_p8"),    # one chunk
    (2050, 4096, "_strict_rr8_p32"),  # four whole ring rounds, a ragged last workgroup
    (2048, 2052, "_strict_rr8_p32"),  # one 4-column group in the seventeenth chunk
    (2048, 3000, "_strict_rr8_p32"),  # a partial third ring round
    (4100, 4100, "_strict_r16"),      # past the resident rows: staged, 16-byte loads
])
def test_strict_softmax_staged_rows(ctx, rows, extent, form):
    """Rows of >= 64 run the staged strict softmax (tiler_softmax_f32_strict_r*)
    or, for 128..4096 aligned elements and enough rows, the register-resident
    one (_rr8_p*): the maximum, the exponent sum folded in order, the
    reciprocal multiply -- bit for bit against the oracle.  Row 0 all -inf,
    row 1 with a NaN, row 2 with a +inf, row 3 with -0.0 and +0.0 as its only
    large values; a ragged last workgroup also gets a NaN row and a -inf
    row."""
    rng = np.random.default_rng(rows * 3 + extent)
    x = (rng.standard_normal((rows, extent)) * 3).astype(np.float32)
    x[0] = -np.inf
    x[1, extent // 3] = np.nan
    x[2, extent - 1] = np.inf
    x[3] = -np.abs(x[3]) - 1
    x[3, 0], x[3, 1] = -0.0, 0.0
    if rows % 8:
        x[rows - 1, extent // 2] = np.nan
        x[rows - 2] = -np.inf
    flags = L.REGION_ALIGNED16
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), flags=flags, ctx=ctx)
    assert rz.symbols[-1].endswith(form), rz.symbols
    print(f"[strict softmax] {rz.symbols[-1]} rows={rows} extent={extent}", flush=True)
    bufs = [ctx.to_device(x), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[-1].download(np.float32, x.shape)
    finally:
        for b in bufs:
            b.free()
    # rows are independent: past 2.5M elements (the oracle's certified exp
    # takes ~1.7 s per million) compare the planted rows, every residue mod 8
    # of the first and last workgroups and 64 drawn rows
    if rows * extent > 2_500_000:
        keep = np.unique(np.concatenate([np.arange(16), np.arange(rows - 16, rows), rng.choice(rows, 64, replace=False)]))
        x, got = np.ascontiguousarray(x[keep]), got[keep]
    want = oracle.softmax_f32(x, x.shape, 1).reshape(x.shape)
    assert np.array_equal(bits(got), bits(want))


def _sampled_rows(rng, rows, per_group, groups_sampled):
    """Rows covering every residue mod `per_group` (the rows one workgroup
    holds): the first and last workgroup whole, plus `groups_sampled` - 2
    other workgroups, each contributing one row per residue."""
    groups = rows // per_group
    picked = set(range(per_group)) | set(range(rows - per_group, rows))
    others = rng.choice(np.arange(1, groups - 1), size=groups_sampled - 2, replace=False)
    for r in range(per_group):
        for g in others:
            picked.add(int(g) * per_group + r)
    return np.array(sorted(picked))


def test_strict_softmax_staged_whole_stages_sampled_rows(ctx):
    """The staged strict softmax with 16 rows per workgroup, 16-byte loads
    and whole stages (tiler_softmax_f32_strict_r16, rows past the resident
    form's 4096 elements): 4096 x 4352, 17 stages of 256 -- every row of the
    first and last workgroup and one row of every residue mod 16 from 14
    others, bit for bit with the oracle."""
    rows, extent = 4096, 4352
    rng = np.random.default_rng(2304)
    x = rng.standard_normal((rows, extent), dtype=np.float32) * np.float32(3)
    sample = _sampled_rows(rng, rows, 16, 16)
    x[sample[1], 100] = np.nan
    x[sample[20]] = -np.inf
    x[sample[-3], extent - 1] = np.inf
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), flags=L.REGION_ALIGNED16, ctx=ctx)
    assert rz.symbols == ["tiler_softmax_f32_strict_r16"], rz.symbols
    print(f"[strict softmax staged] {rz.symbols} rows={rows} extent={extent} sampled={len(sample)}", flush=True)
    bufs = [ctx.to_device(x), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[-1].download(np.float32, x.shape)[sample]
    finally:
        for b in bufs:
            b.free()
    xs = np.ascontiguousarray(x[sample])
    want = oracle.softmax_f32(xs, xs.shape, 1).reshape(xs.shape)
    assert np.array_equal(bits(got), bits(want))


def test_strict_softmax_c3_shape_sampled_rows(ctx):
    """The strict softmax at the C3 configuration (f32 [32 x 2048 x 2048],
    65536 rows of 2048; tiler_softmax_f32_strict_rr8_p16, 8 rows per
    workgroup held in registers) routed under the strict contract (no
    PERMITS_REASSOCIATION) -- 264 rows compared bit for bit with the oracle's
    softmax_f32 (softmax.rs:237-315): the first and last workgroup whole and
    one row of every residue mod 8 from 31 other workgroups.  Planted rows:
    all -inf, a NaN, a +inf, -0.0 and +0.0 as the only large values, and a
    row of one repeated value."""
    rows, extent = 65536, 2048
    rng = np.random.default_rng(65536)
    x = rng.standard_normal((rows, extent), dtype=np.float32) * np.float32(3)
    sample = _sampled_rows(rng, rows, 8, 33)
    planted = {int(sample[0]): "ninf", int(sample[17]): "nan", int(sample[40]): "pinf",
               int(sample[-1]): "zeros", int(sample[-6]): "flat", int(sample[100]): "nan"}
    for r, kind in planted.items():
        if kind == "ninf":
            x[r] = -np.inf
        elif kind == "nan":
            x[r, (r * 7) % extent] = np.nan
        elif kind == "pinf":
            x[r, extent - 1 - r % 16] = np.inf
        elif kind == "zeros":
            x[r] = -np.abs(x[r]) - 1
            x[r, 0], x[r, extent - 1] = -0.0, 0.0
        else:
            x[r] = np.float32(0.75)
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), flags=L.REGION_ALIGNED16, ctx=ctx)
    assert rz.symbols == ["tiler_softmax_f32_strict_rr8_p16"], rz.symbols
    print(f"[strict softmax C3] {rz.symbols} rows={rows} extent={extent} sampled={len(sample)}", flush=True)
    bufs = [ctx.to_device(x), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[-1].download(np.float32, x.shape)[sample]
    finally:
        for b in bufs:
            b.free()
    xs = np.ascontiguousarray(x[sample])
    del x
    want = oracle.softmax_f32(xs, xs.shape, 1).reshape(xs.shape)
    diff = np.argwhere(bits(got) != bits(want))
    assert diff.size == 0, f"{len(diff)} elements differ, first in row {sample[diff[0][0]]} at {diff[0][1]}"


def test_strict_bf16_silu_contraction_c5_shape_sampled_rows(ctx):
    """The strict bf16 contraction with the SiLU epilogue at the C5
    configuration (A, B bf16 [4096 x 4096] ~N(0, 1/64), C = bf16(silu(A.B^T)))
    routed under the strict contract: tiler_contract_strict_bf16_silu_b64,
    64 x 64 outputs per workgroup.  192 whole output rows -- the first and
    last row tile whole, and one row of every residue mod 64, each from
    another tile --
    bit for bit with bf16_narrow(silu_f32(contract_strict_f32(widened))),
    the reference's fold (contraction.rs:558-630) and SiLU (silu.rs:511-533)
    on exactly widened operands."""
    m = n = k = 4096
    rng = np.random.default_rng(4096)
    a = oracle.bf16_narrow(rng.standard_normal((m, k), dtype=np.float32) / np.float32(64)).reshape(m, k)
    b = oracle.bf16_narrow(rng.standard_normal((n, k), dtype=np.float32) / np.float32(64)).reshape(n, k)
    sample = np.array(sorted(set(range(64)) | set(range(m - 64, m)) |
                             {int(g) * 64 + r for r, g in enumerate(rng.integers(1, m // 64 - 1, 64))}))
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16, variant=L.EPILOGUE_SILU, ctx=ctx)
    assert rz.symbols == ["tiler_contract_strict_bf16_silu_b64"], rz.symbols
    print(f"[strict bf16 silu C5] {rz.symbols} {m}x{n}x{k} sampled rows={len(sample)}", flush=True)
    bufs = [ctx.to_device(a), ctx.to_device(b), ctx.alloc(m * n * 2)]
    try:
        route(ctx, rz, bufs)
        got = bufs[2].download(np.uint16, (m, n))[sample]
    finally:
        for x in bufs:
            x.free()
    ref = oracle.contract_strict_f32(bf16_widen(a[sample]), bf16_widen(b), len(sample), n, k)
    want = oracle.bf16_narrow(oracle.silu_f32(ref)).reshape(len(sample), n)
    diff = np.argwhere(got != want)
    assert diff.size == 0, f"{len(diff)} outputs differ, first at row {sample[diff[0][0]]} column {diff[0][1]}"


@pytest.mark.parametrize("m,n,k,form", [(70, 90, 300, "b16"), (512, 1000, 96, "b32"), (2048, 2040, 70, "b64"),
                                        (40, 70, 9, "")])
@pytest.mark.parametrize("silu", [False, True])
def test_strict_bf16_contraction(ctx, silu, m, n, k, form):
    """The strict bf16 contraction (no reassociation): register-blocked tiles
    of 16/32/64 for k >= 64, one output per thread below; the first-product
    fold on exactly widened operands, then (SiLU) the reference SiLU, one
    narrowing -- bit for bit."""
    rng = np.random.default_rng(23 + m)
    a = oracle.bf16_narrow(rng.standard_normal((m, k)).astype(np.float32)).reshape(m, k)
    b = oracle.bf16_narrow(rng.standard_normal((n, k)).astype(np.float32)).reshape(n, k)
    ref = oracle.contract_strict_f32(bf16_widen(a), bf16_widen(b), m, n, k)
    if silu:
        ref = oracle.silu_f32(ref).reshape(m, n)
    want = oracle.bf16_narrow(ref).reshape(m, n)
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16,
                 variant=L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE, ctx=ctx)
    assert rz.symbols[0].startswith("tiler_contract_strict_bf16") and rz.symbols[0].endswith(form)
    print(f"[strict bf16] {rz.symbols[0]} m={m} n={n} k={k}", flush=True)
    bufs = [ctx.to_device(a), ctx.to_device(b), ctx.alloc(m * n * 2)]
    try:
        route(ctx, rz, bufs)
        assert np.array_equal(bufs[2].download(np.uint16, (m, n)), want)
    finally:
        for x in bufs:
            x.free()


# --- reindex, target environment, dispatch checks ------------------------------------

def test_mirrored_reindex(ctx):
    # structural_mirrored_reindex.metal: out[i] = src[(i/2)*2 + 1 - i%2]
    src = np.array([10.0, 11.0, 12.0, 13.0], np.float32)
    ds, do = ctx.to_device(src), ctx.alloc(16)
    try:
        ctx.reindex(ds, 4, (2, 2), (2, -1), 1, 4, do)
        ctx.synchronize()
        assert do.download(np.float32, (4,)).tolist() == [11.0, 10.0, 13.0, 12.0]
    finally:
        ds.free(); do.free()
    # a reversed long row (row mode) and a transposed reversal, bf16
    rng = np.random.default_rng(24)
    x = rng.integers(0, 1 << 16, (33, 1000), dtype=np.uint32).astype(np.uint16)
    want = x[::-1, ::-1].T.copy()
    rz = realize(L.PROGRAM_REINDEX, want.shape, rank=2, variant=2, strides=(-1, -1000),
                 grouping=(x.size, x.size - 1), ctx=ctx)
    ds, do = ctx.to_device(x), ctx.alloc(x.nbytes)
    try:
        route(ctx, rz, [ds, do])
        assert np.array_equal(do.download(np.uint16, want.shape), want)
    finally:
        ds.free(); do.free()


def test_observed_target_environment_validates(ctx):
    d, reason = ctx.observe_target_environment()
    assert reason is None, reason
    assert runtime.validate_target_environment(d) is None
    assert b"amdgcn-amd-amdhsa--gfx950:sramecc" in d
    assert ctx.environment["gcn_arch_name"].split(":")[0] == "gfx950"


def test_plan_dispatch_refuses_a_grid_beyond_the_profile(ctx):
    rz = realize(L.PROGRAM_CONVERT, (1024,), variant=L.CONVERT_NARROW_F32_BF16, ctx=ctx)
    from tiler_amd.realize import _prepared
    e = rz.raw.entries[0]
    slots = (ctypes.c_uint32 * 2)(*e.binding_slots[:2])
    offs = (ctypes.c_uint32 * 2)(*e.binding_offsets[:2])
    ka = ctypes.create_string_buffer(bytes(e.kernargs[:e.kernarg_bytes]), e.kernarg_bytes)
    de = L.DispatchEntry(_prepared(ctx, rz.symbols[0]), (ctypes.c_uint32 * 3)(0x80000000, 1, 1),
                         (ctypes.c_uint32 * 3)(256, 1, 1), 0, ctypes.cast(ka, ctypes.c_void_p), e.kernarg_bytes,
                         2, slots, offs)
    sb = (ctypes.c_uint64 * 2)(4096, 2048)
    plan = L.DispatchPlan(2, sb, 1, ctypes.pointer(de), None)
    assert L.lib().tiler_hip_plan_dispatch(ctx.handle, ctypes.byref(plan)) == L.REFUSE_CAPACITY
