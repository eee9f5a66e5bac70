"""CPU: the algebra the strict row kernels' flushing-contract forms rest on,
checked with the oracle's own subnormal-mode function (conformance.rs:498-521
apply(), restated in oracle/tiler_oracle.c), not with the kernels' code.

The `_m` forms of the strict RMSNorm and softmax (rows_strict.hip) carry
every value as the operand flush O reads it and fold the flushed
contributors with plain adds.  That is the reference's fold
acc = R(O(acc) + O(c)) seeded at c_0 (R the result flush) because:

1. O after R is a single flush, by the result mode when it flushes, else
   by the input mode (`tiler::result_as_operand`);
2. a sum of two non-negative values that are not subnormal is never
   subnormal, so that flush leaves every partial sum of squares or
   exponents alone, and -0.0 (the start and the padding) adds exactly;
3. hence O(reference fold) equals the plain fold of F(c_i) from -0.0 --
   checked directly on random contributor sequences.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle

MODES = (oracle.PRESERVE, oracle.FLUSH_SIGN_PRESERVING, oracle.FLUSH_POSITIVE_ZERO)


def _apply(mode, v):
    return np.float32(oracle.lib().tiler_oracle_apply_subnormal_mode(mode, ctypes.c_float(float(v))))


def _bits(v):
    return int(np.float32(v).view(np.uint32))


def _single_flush(in_mode, out_mode):
    """The mode result_as_operand picks (rows_strict / common.h)."""
    return out_mode if out_mode != oracle.PRESERVE else in_mode


def _values():
    """Zeros, both subnormal edges, the least normals, ordinary values,
    infinities and NaN, of both signs, plus random bit patterns."""
    rng = np.random.default_rng(5)
    edge = np.array([0, 1, 2, 0x7FFFFF, 0x7FFFFE, 0x400000, 0x800000, 0x800001, 0xFFFFFF, 0x1000000,
                     0x3F800000, 0x7F7FFFFF, 0x7F800000, 0x7FC00000, 0x7FA00000], np.uint32)
    rand = rng.integers(0, 1 << 32, 3000, dtype=np.uint64).astype(np.uint32)
    sub = rng.integers(1, 1 << 23, 1000, dtype=np.uint64).astype(np.uint32)
    allv = np.concatenate([edge, edge | np.uint32(0x80000000), rand, sub, sub | np.uint32(0x80000000)])
    return allv.view(np.float32)


@pytest.mark.parametrize("in_mode", MODES)
@pytest.mark.parametrize("out_mode", MODES)
def test_result_then_operand_is_one_flush(in_mode, out_mode):
    f = _single_flush(in_mode, out_mode)
    for v in _values():
        got = _apply(in_mode, _apply(out_mode, v))
        want = _apply(f, v)
        assert _bits(got) == _bits(want) or (np.isnan(got) and np.isnan(want)), (in_mode, out_mode, hex(_bits(v)))


def test_sums_of_nonnegative_normals_are_never_subnormal():
    """Every a + b with a, b in {+0, normals near 2^-126, ordinary values,
    +inf} is a zero, at least 2^-126, infinite or NaN; -0.0 adds exactly."""
    rng = np.random.default_rng(6)
    least = np.arange(0x800000, 0x800000 + 4096, dtype=np.uint32)  # 2^-126 and its next 4095 values
    near = rng.integers(0x800000, 0x2000000, 4000, dtype=np.uint64).astype(np.uint32)
    wide = rng.integers(0x800000, 0x7F800000, 4000, dtype=np.uint64).astype(np.uint32)
    pool = np.concatenate([[0, 0x7F800000], least, near, wide]).astype(np.uint32).view(np.float32)
    a = pool[::7][:, None]
    b = pool[None, :]
    with np.errstate(over="ignore"):
        s = (a + b).astype(np.float32)
    mag = np.abs(s)
    assert not np.any((mag > 0) & (mag < np.float32(2.0 ** -126))), "a subnormal sum"
    for v in pool:
        assert _bits(np.float32(v) + np.float32(-0.0)) == _bits(v)
        assert _bits(np.float32(-0.0) + np.float32(v)) == _bits(v)


def _contributors(rng, n, kind):
    """Non-negative contributors as the kernels' folds see them: squares of
    values around 2^-70 (subnormal squares), or exponent-like values from
    2^hi down into the subnormal range, hi drawn per sequence so that some
    sequences lie wholly among the subnormals; a few zeros."""
    if kind == "squares":
        x = (rng.standard_normal(n) * 2.0 ** rng.integers(-80, -55, n)).astype(np.float32)
        return x, "square"
    e = np.exp2(rng.uniform(-150.0, rng.uniform(-149.0, 0.0), n)).astype(np.float32)
    e[rng.random(n) < 0.05] = 0.0
    return e, "value"


@pytest.mark.parametrize("in_mode", MODES)
@pytest.mark.parametrize("out_mode", MODES)
@pytest.mark.parametrize("kind", ["squares", "exponents"])
def test_operand_read_of_the_reference_fold_is_the_plain_fold(in_mode, out_mode, kind):
    """O(acc) of the reference's seeded fold acc = R(O(acc) + O(c)) over
    c = R(O(x) * O(x)) (squares) or c = R(e) (exponents) equals the plain
    float32 fold of F(c) = O(R(c)) from -0.0, bit for bit."""
    rng = np.random.default_rng(100 * in_mode + 10 * out_mode + (kind == "squares"))
    f = _single_flush(in_mode, out_mode)
    for trial in range(60):
        n = int(rng.integers(1, 40))
        raw, how = _contributors(rng, n, kind)
        if how == "square":
            c = [_apply(out_mode, np.float32(_apply(in_mode, v) * _apply(in_mode, v))) for v in raw]
        else:
            c = [_apply(out_mode, v) for v in raw]
        acc = c[0]
        for ci in c[1:]:
            acc = _apply(out_mode, np.float32(_apply(in_mode, acc) + _apply(in_mode, ci)))
        b = np.float32(-0.0)
        for ci in c:
            b = np.float32(b + _apply(f, ci))
        assert _bits(_apply(in_mode, acc)) == _bits(b), (in_mode, out_mode, kind, trial, n)
