"""GPU: the contraction epilogue's SiLU is the reference SiLU.

The fused epilogue narrows bf16(silu_f32(acc)) -- tiler-reference/src/silu.rs:511-533
applied to the f32 accumulator, then the ADR 0091 narrowing -- on every
dispatch path (the staged 256- and 128-tiles, the skinny m <= 64 form, the
guarded general form).  Two checks:

* exhaustive: tiler::silu_for_bf16 (a fast path guarded near bf16 rounding
  midpoints, falling back to silu_f32) narrows to the same bf16 as silu_f32
  for all 2^32 binary32 inputs, run on the device by a test-only audit kernel
  (tests/native/silu_epilogue_audit.hip) loaded through the adapter's own
  prepare/plan/dispatch stages;
* through each contraction kernel: accumulators built exactly from bf16
  operands (each value v = hi + lo + lo2, three bf16 terms whose every partial
  sum is exact, against B rows of ones) must come out as
  bf16(oracle.silu_f32(v)), bit for bit, including values whose SiLU lies
  within a few binary32 steps of a bf16 midpoint (the fallback path).
"""
from __future__ import annotations

import os
import re
import struct

import numpy as np
import pytest

import oracle
from device_launch import launch
from helpers import bits, bf16_widen
from tiler_amd import _lib as L
from tiler_amd.realize import realize, route

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
AUDIT = os.path.join(ROOT, "tests", "_build", "silu_epilogue_audit.hsaco")
GUARD = 8  # tiler::kSiluGuard


def test_silu_for_bf16_matches_reference_on_every_binary32(ctx):
    with open(AUDIT, "rb") as fh:
        code = fh.read()
    res = ctx.to_device(np.array([0, 2**64 - 1, 0, 0, 0], dtype=np.uint64))
    try:
        step = 1 << 28
        for first in range(0, 1 << 32, step):
            launch(ctx, code, "tiler_audit_silu_for_bf16", 4096, 256,
                   struct.pack("<QQQ", first, step, 0), [(16, 0)], [res])
        print(f"[silu audit] scanned 2^32 inputs", flush=True)
        mis, low, fall, dist, fast = (int(v) for v in res.download(np.uint64, (5,)))
    finally:
        res.free()
    print(f"[silu audit] mismatches={mis} fast-domain={fast} fallbacks={fall} "
          f"({fall / max(fast, 1):.2e}) max distance={dist} steps (guard {GUARD})", flush=True)
    assert mis == 0, f"first mismatching input 0x{low:08x}"
    assert fast > 2_000_000_000
    assert dist < GUARD  # the guard covers the fast path's whole error
    assert fall < fast // 1000


def _split3(v: np.ndarray):
    """v = hi + lo + lo2 with bf16 terms and every partial sum exact; returns
    the terms and a mask of the values that split exactly."""
    v = v.astype(np.float32)
    hi = oracle.bf16_narrow(v)
    r1 = (v.astype(np.float64) - bf16_widen(hi).astype(np.float64)).astype(np.float32)
    lo = oracle.bf16_narrow(r1)
    r2 = (r1.astype(np.float64) - bf16_widen(lo).astype(np.float64)).astype(np.float32)
    lo2 = oracle.bf16_narrow(r2)
    t = [bf16_widen(x).astype(np.float64) for x in (hi, lo, lo2)]
    ok = (t[0] + t[1] + t[2]) == v.astype(np.float64)
    for i in range(3):
        for j in range(i + 1, 3):
            s = t[i] + t[j]
            ok &= s.astype(np.float32).astype(np.float64) == s
    return hi, lo, lo2, ok & (v != 0)


def _values(rng, count):
    """Accumulator values across SiLU's regimes, a third of them chosen so
    silu_f32(v) lies within a few binary32 steps of a bf16 midpoint (drawn
    from a pool of at most 1024 such values: finding one takes ~4000 SiLU
    evaluations)."""
    out = []
    near = []
    want = min(count // 3, 1024)
    while sum(len(x) for x in near) < want:
        c = rng.uniform(-95, 25, 1 << 18).astype(np.float32)
        s = oracle.silu_f32(c)
        lo16 = bits(s) & 0xFFFF
        near.append(c[np.abs(lo16.astype(np.int64) - 0x8000) <= 2 * GUARD])
    pool = np.concatenate(near)[:want]
    out.append(pool if want == count // 3 else rng.choice(pool, count // 3))
    k = count - count // 3
    out.append(rng.uniform(-20, 20, k // 3).astype(np.float32))
    out.append(rng.uniform(-100, 30, k // 3).astype(np.float32))
    rest = k - 2 * (k // 3)
    out.append((rng.standard_normal(rest) * np.exp2(rng.integers(-60, 6, rest))).astype(np.float32))
    v = np.concatenate(out)
    rng.shuffle(v)
    return v


def _contract_on_path(ctx, a, b, epilogue, path):
    """C = A.B^T (bf16 bits) realized under PERMITS_REASSOCIATION; the
    realization must dispatch the kernel form `path` names (its symbol ends in
    _<path>, a skinny form's row count after it), so every case below runs the
    epilogue it is labelled with."""
    m, k = a.shape
    n = b.shape[0]
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16, variant=epilogue,
                 permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    assert len(rz.symbols) == 1 and re.search(rf"_{path}\d*$", rz.symbols[0]), (path, rz.symbols)
    print(f"[silu path] {path}: {rz.symbols[0]} m={m} n={n} k={k}", flush=True)
    bufs = [ctx.to_device(a), ctx.to_device(b), ctx.alloc(m * n * 2)]
    try:
        route(ctx, rz, bufs)
        return bufs[2].download(np.uint16, (m, n))
    finally:
        for x in bufs:
            x.free()


@pytest.mark.parametrize("m,n,pad,path", [
    (4096, 4096, 0, "t256_kf"),  # 256 tiles of 256 fill every CU; k a multiple of 64
    (4096, 4096, 8, "t256"),     # the same with a ragged last k tile
    (300, 264, 0, "t128_kf"),
    (300, 264, 8, "t128"),
    (48, 200, 0, "skinny"),
    (130, 100, 0, "g128"),       # n off the 8-element grid: the general form
])
def test_fused_silu_is_reference_silu_on_each_path(ctx, m, n, pad, path):
    rng = np.random.default_rng(m + 7 * n)
    groups = 64 if n >= 64 else n
    vals = _values(rng, m * groups)
    hi, lo, lo2, ok = _split3(vals)
    while not ok.all():  # replace the few values that do not split exactly
        bad = ~ok
        vals[bad] = rng.uniform(-20, 20, int(bad.sum())).astype(np.float32)
        hi, lo, lo2, ok = _split3(vals)
    vals = vals.reshape(m, groups)
    k = 3 * groups
    k_pad = (k + 7) // 8 * 8 + pad  # zero columns past k change no accumulator
    a = np.zeros((m, k_pad), np.uint16)
    a[:, 0:k:3], a[:, 1:k:3], a[:, 2:k:3] = (x.reshape(m, groups) for x in (hi, lo, lo2))
    b = np.zeros((n, k_pad), np.uint16)
    g = np.arange(n) % groups
    for t in range(3):
        b[np.arange(n), 3 * g + t] = 0x3F80  # bf16 1.0
    got = _contract_on_path(ctx, a, b, L.EPILOGUE_SILU, path)
    acc = vals[:, g]  # C[i, j] = v[i, j % groups] exactly
    want = oracle.bf16_narrow(oracle.silu_f32(vals))[:, g]  # each distinct accumulator once
    plain = _contract_on_path(ctx, a, b, L.EPILOGUE_NONE, path)
    assert np.array_equal(plain, oracle.bf16_narrow(acc).reshape(m, n)), "accumulators are not exact"
    diff = np.argwhere(got != want)
    assert diff.size == 0, (f"{path}: {len(diff)} outputs differ, first at {tuple(diff[0])}: "
                            f"acc {acc[tuple(diff[0])]!r} got 0x{got[tuple(diff[0])]:04x} "
                            f"want 0x{want[tuple(diff[0])]:04x}")
