"""GPU: the device's exp on the inputs nearest a binary32 rounding boundary.

tests/golden/device_exp_hard_cases.json lists every binary32 input whose
binary64 exp lies within 2^-48 of a rounding boundary (see
test_device_exp_audit.py).  The device's SiLU (x = -s, so exp(-x) = exp(s))
and softmax (rows [0, s] for s <= 0, so the second exponent is exp(s)) must
match the oracle, which uses the certified exp, bit for bit.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from helpers import bits
from tiler_amd import families

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                       "device_exp_hard_cases.json")


def _hard():
    with open(FIXTURE) as f:
        fx = json.load(f)
    s = np.array([int(v, 16) for v in fx["inputs"]], np.uint32).view(np.float32)
    e = np.array([int(v, 16) for v in fx["certified_exp"]], np.uint32)
    return s, e


def test_silu_on_every_hard_exp_input(ctx):
    s, _ = _hard()
    x = (-s).astype(np.float32)
    got = families.silu_f32(x, ctx=ctx)
    assert np.array_equal(bits(got), bits(oracle.silu_f32(x)))


def test_softmax_on_every_nonpositive_hard_exp_input(ctx):
    s, _ = _hard()
    keep = s <= 0
    rows = np.stack([np.zeros(keep.sum(), np.float32), s[keep]], axis=1)
    got = families.softmax_f32(rows.shape, 1, rows, ctx=ctx).reshape(rows.shape)
    assert np.array_equal(bits(got), bits(oracle.softmax_f32(rows, rows.shape, 1).reshape(rows.shape)))


def test_resident_strict_softmax_on_every_nonpositive_hard_exp_input(ctx):
    """The register-resident strict softmax (tiler_softmax_f32_strict_rr8_p8,
    which evaluates exp_f32_cr_nonpositive) on rows [0, s_1, ..., s_127]
    whose s cycle through every hard input s <= 0 (the row's maximum is 0,
    so each exponent is exp(s) itself), bit for bit with the oracle."""
    from tiler_amd import _lib as L
    from tiler_amd.realize import realize, route

    s, _ = _hard()
    s = s[s <= 0]
    rows, extent = 2048, 128
    x = np.zeros((rows, extent), np.float32)
    x[:, 1:] = np.resize(s, (rows, extent - 1))
    rz = realize(L.PROGRAM_SOFTMAX, (rows, extent), flags=L.REGION_ALIGNED16, ctx=ctx)
    assert rz.symbols == ["tiler_softmax_f32_strict_rr8_p8"], rz.symbols
    bufs = [ctx.to_device(x), ctx.alloc(x.nbytes)]
    try:
        route(ctx, rz, bufs)
        got = bufs[-1].download(np.float32, x.shape)
    finally:
        for b in bufs:
            b.free()
    assert np.array_equal(bits(got), bits(oracle.softmax_f32(x, x.shape, 1).reshape(x.shape)))
