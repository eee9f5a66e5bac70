"""Host-level entry points mirroring tiler-reference's family functions, run on
the MI355X through the C ABI.

Each function takes and returns host numpy arrays with the reference's
argument meaning and refusal behaviour, moves the operands to HBM, launches the
gfx950 realization, and reads the result back.  The device kernels reduce the
last axis; a reduction over another axis is presented to them by moving that
axis last on the host (a pure relayout that changes no value).

Reference functions mirrored (paths under /root/reference/crates/):
  strict_sum                tiler-reference/src/evaluate.rs:498-589
  strict_partitioned_sum    tiler-reference/src/evaluate.rs:788-832
  cooperative_grouped_sum   tiler-reference/src/evaluate.rs:536-659
  rms_norm_f32              tiler-reference/src/rms_norm.rs:405-451
  softmax_f32               tiler-reference/src/softmax.rs:200-234
  silu_f32                  tiler-reference/src/silu.rs:486-533
  gather                    tiler-reference/src/structural.rs:513-606
  contract_strict_f32       tiler-reference/src/contraction.rs:297-333 (td,od->to)
"""
from __future__ import annotations

import numpy as np

from . import _lib as L
from .runtime import Context, GatherIndexOutOfBounds, Refusal, validate_gather_index

_default: Context | None = None


def default_context() -> Context:
    global _default
    if _default is None:
        _default = Context(0)
    return _default


def _ctx(ctx):
    return ctx if ctx is not None else default_context()


def _axis_last(values: np.ndarray, shape, axis: int):
    shape = tuple(int(s) for s in shape)
    if not 0 <= axis < len(shape):
        raise Refusal(L.REFUSE_INVALID_ARGUMENT, "axis outside the shape")
    arr = np.asarray(values).reshape(shape)
    moved = np.moveaxis(arr, axis, -1)
    return np.ascontiguousarray(moved), moved.shape


def _run_rows(ctx, x: np.ndarray, out_dtype, out_count, launch):
    ctx = _ctx(ctx)
    dx = ctx.to_device(x)
    dy = ctx.alloc(max(out_count * np.dtype(out_dtype).itemsize, 1))
    try:
        launch(ctx, dx, dy)
        ctx.synchronize()
        return dy.download(out_dtype, (out_count,))
    finally:
        dx.free()
        dy.free()


# --- sums --------------------------------------------------------------------

def _sum(values, shape, axis, topology, ctx=None, **plan):
    x, moved_shape = _axis_last(np.asarray(values, dtype=np.float32), shape, axis)
    extent = moved_shape[-1]
    rows = int(np.prod(moved_shape[:-1], dtype=np.int64)) if len(moved_shape) > 1 else 1
    out = _run_rows(ctx, x.reshape(-1), np.float32, rows,
                    lambda c, dx, dy: c.sum_f32(dx, rows, extent, dy, topology=topology, **plan))
    return out.reshape(moved_shape[:-1])


def strict_sum(values, shape, axis: int, ctx=None) -> np.ndarray:
    """Serial topology: bit-exact with the strict left fold."""
    return _sum(values, shape, axis, L.SUM_SERIAL, ctx)


def strict_partitioned_sum(values, shape, axis: int, partitions: int,
                           contributors_per_partition: int, ctx=None) -> np.ndarray:
    return _sum(values, shape, axis, L.SUM_MULTIPASS, ctx, partitions=partitions,
                per_partition=contributors_per_partition)


def cooperative_grouped_sum(values, shape, axis: int, participants: int,
                            contributors_per_partition: int, rounds: int,
                            participant_major: bool = False, ctx=None) -> np.ndarray:
    return _sum(values, shape, axis, L.SUM_COOPERATIVE, ctx, participants=participants,
                per_partition=contributors_per_partition, rounds=rounds,
                participant_major=participant_major)


def tree_sum(values, shape, axis: int, ctx=None) -> np.ndarray:
    """The reassociating two-level tree (declared grouping)."""
    return _sum(values, shape, axis, L.SUM_TREE, ctx)


# --- row families --------------------------------------------------------------

def rms_norm_f32(shape, axis: int, eps_bits: int, values, weights, ctx=None) -> np.ndarray:
    """weights has the input's shape, as the reference requires."""
    x, moved_shape = _axis_last(np.asarray(values, dtype=np.float32), shape, axis)
    w, _ = _axis_last(np.asarray(weights, dtype=np.float32), shape, axis)
    extent = moved_shape[-1]
    rows = x.size // extent if extent else 0
    ctx = _ctx(ctx)
    dw = ctx.to_device(w.reshape(-1))
    try:
        out = _run_rows(ctx, x.reshape(-1), np.float32, x.size,
                        lambda c, dx, dy: c.rms_norm(L.F32, dx, dw, rows, extent, eps_bits, dy,
                                                     weight_broadcast=False))
    finally:
        dw.free()
    return np.moveaxis(out.reshape(moved_shape), -1, axis).reshape(-1)


def rms_norm_bf16(values_bits: np.ndarray, weight_bits: np.ndarray, eps_bits: int,
                  ctx=None) -> np.ndarray:
    """bf16 [rows, extent] x bf16 [extent] -> bf16 [rows, extent] (bit patterns)."""
    x = np.ascontiguousarray(values_bits, dtype=np.uint16)
    rows, extent = x.shape
    ctx = _ctx(ctx)
    dw = ctx.to_device(np.ascontiguousarray(weight_bits, dtype=np.uint16))
    try:
        out = _run_rows(ctx, x.reshape(-1), np.uint16, x.size,
                        lambda c, dx, dy: c.rms_norm(L.BF16, dx, dw, rows, extent, eps_bits, dy,
                                                     weight_broadcast=True))
    finally:
        dw.free()
    return out.reshape(rows, extent)


def softmax_f32(shape, axis: int, values, ctx=None) -> np.ndarray:
    x, moved_shape = _axis_last(np.asarray(values, dtype=np.float32), shape, axis)
    extent = moved_shape[-1]
    rows = x.size // extent if extent else 0
    out = _run_rows(ctx, x.reshape(-1), np.float32, x.size,
                    lambda c, dx, dy: c.softmax_f32(dx, rows, extent, dy))
    return np.moveaxis(out.reshape(moved_shape), -1, axis).reshape(-1)


def silu_f32(values, ctx=None) -> np.ndarray:
    x = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    return _run_rows(ctx, x, np.float32, x.size,
                     lambda c, dx, dy: c.map(L.MAP_SILU, L.F32, dx, x.size, dy))


# --- bf16 <-> binary32 conversion (ADR 0091 decision 2) -------------------------

def narrow_f32_bf16(values, ctx=None) -> np.ndarray:
    """binary32 -> bf16 bit patterns: round to nearest even, overflow to a
    signed infinity at the inclusive midpoint, every NaN -> 0x7fc0."""
    x = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    return _run_rows(ctx, x, np.uint16, x.size,
                     lambda c, dx, dy: c.convert(L.CONVERT_NARROW_F32_BF16, dx, x.size, dy))


def widen_bf16_f32(bits, ctx=None) -> np.ndarray:
    """bf16 bit patterns -> binary32, exactly (a NaN keeps its payload)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    return _run_rows(ctx, b, np.float32, b.size,
                     lambda c, dx, dy: c.convert(L.CONVERT_WIDEN_BF16_F32, dx, b.size, dy))


# --- gather --------------------------------------------------------------------

def gather(source: np.ndarray, axis: int, index: np.ndarray, index_signed: bool = False,
           ctx=None) -> np.ndarray:
    """Result shape = source.shape[:axis] + index.shape + source.shape[axis+1:].
    An out-of-range index raises GatherIndexOutOfBounds before any device work."""
    src = np.ascontiguousarray(source)
    idx = np.ascontiguousarray(np.asarray(index).astype(np.int64).astype(np.uint32)
                               if np.asarray(index).dtype != np.uint32 else index)
    gathered = src.shape[axis]
    validate_gather_index(idx.reshape(-1), gathered, index_signed)
    outer = int(np.prod(src.shape[:axis], dtype=np.int64)) if axis else 1
    inner = int(np.prod(src.shape[axis + 1:], dtype=np.int64)) if axis + 1 < src.ndim else 1
    out_shape = src.shape[:axis] + np.asarray(index).shape + src.shape[axis + 1:]
    count = idx.size
    ctx = _ctx(ctx)
    ds = ctx.to_device(src.reshape(-1))
    di = ctx.to_device(idx.reshape(-1))
    n_out = outer * count * inner
    do = ctx.alloc(max(n_out * src.itemsize, 1))
    try:
        ctx.gather(ds, outer, gathered, inner, src.itemsize, di, count, do,
                   index_signed=index_signed)
        ctx.gather_status()
        out = do.download(src.dtype, (n_out,))
    finally:
        ds.free()
        di.free()
        do.free()
    return out.reshape(out_shape)


# --- contraction ------------------------------------------------------------------

def contract_strict_f32(a: np.ndarray, b: np.ndarray, ctx=None) -> np.ndarray:
    """td,od->to: A [m, k], B [n, k] -> C [m, n], the strict fold."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    n, k2 = b.shape
    if k != k2:
        raise Refusal(L.REFUSE_INVALID_ARGUMENT, "contracted extents disagree")
    ctx = _ctx(ctx)
    da, db = ctx.to_device(a), ctx.to_device(b)
    dc = ctx.alloc(max(m * n * 4, 1))
    try:
        ctx.contract_strict_f32(da, db, m, n, k, dc)
        ctx.synchronize()
        return dc.download(np.float32, (m, n))
    finally:
        da.free()
        db.free()
        dc.free()


def contract_bf16(a_bits: np.ndarray, b_bits: np.ndarray, epilogue: int = L.EPILOGUE_NONE,
                  ctx=None) -> np.ndarray:
    """bf16 A [m, k], B [n, k] (bit patterns) -> bf16 C [m, n] on MFMA."""
    a = np.ascontiguousarray(a_bits, dtype=np.uint16)
    b = np.ascontiguousarray(b_bits, dtype=np.uint16)
    m, k = a.shape
    n, k2 = b.shape
    if k != k2:
        raise Refusal(L.REFUSE_INVALID_ARGUMENT, "contracted extents disagree")
    ctx = _ctx(ctx)
    da, db = ctx.to_device(a), ctx.to_device(b)
    dc = ctx.alloc(max(m * n * 2, 1))
    try:
        ctx.contract_bf16(da, db, m, n, k, dc, epilogue)
        ctx.synchronize()
        return dc.download(np.uint16, (m, n))
    finally:
        da.free()
        db.free()
        dc.free()


def dequantize_u4(packed: np.ndarray, n: int, scale_bits: int, zero_point: int, ctx=None) -> np.ndarray:
    """Strict-affine U4 -> f32 on the device (quantization.rs:218-246):
    `packed` holds n U4 codes LSB-first in (n + 1) // 2 U8 carriers."""
    p = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    if p.size < (n + 1) // 2:
        raise Refusal(L.REFUSE_INVALID_ARGUMENT, "dequantize_u4", "fewer carriers than codes")
    ctx = _ctx(ctx)
    dc = ctx.to_device(p) if p.size else ctx.alloc(1)
    dy = ctx.alloc(max(4 * n, 1))
    try:
        ctx.dequantize_u4(dc, n, scale_bits, zero_point, dy)
        ctx.synchronize()
        return dy.download(np.float32, (n,))
    finally:
        dc.free()
        dy.free()


__all__ = [
    "strict_sum", "strict_partitioned_sum", "cooperative_grouped_sum", "tree_sum",
    "rms_norm_f32", "rms_norm_bf16", "softmax_f32", "silu_f32", "gather",
    "contract_strict_f32", "contract_bf16", "dequantize_u4", "default_context", "GatherIndexOutOfBounds",
]
