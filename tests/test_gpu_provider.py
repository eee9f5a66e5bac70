"""GPU: every implementation the provider proposes computes what its strategy
declares.

For each region, tiler_hip_propose offers strategies; each proposal's region
is realized (tiler_hip_realize) and routed through the RuntimeAdapter seam on
the device, and its result is checked against the oracle of the grouping
that strategy declares:
* sum: the serial baseline bit-exact with strict_sum; the multi-pass split
  with strict_partitioned_sum at the proposal's partition; the workgroup tree
  with row_grouped_sum, the grid tree with grid_tree_sum over the proposal's
  workgroup count; the cooperative workgroup with cooperative_grouped_sum at
  the proposal's grouping;
* softmax over long rows: the serial baseline bit-exact with softmax_f32, the
  row-synchronized and split launches with the segmented softmax_grouped;
* bf16 contraction with the SiLU epilogue: the serial baseline bit-exact with
  contract_general(..., silu=True); every MFMA form within the relative
  Frobenius bound of 1e-2 of the strict f32 fold (then the reference SiLU).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import bf16_widen, bits
from tiler_amd import _lib as L
from tiler_amd.realize import propose, route

pytestmark = pytest.mark.gpu

RE = L.PERMITS_REASSOCIATION


def _routed(ctx, rz, inputs, outputs):
    dev_in = [ctx.to_device(a) for a in inputs]
    dev_out = [ctx.alloc(max(1, int(np.prod(shape)) * np.dtype(dt).itemsize)) for dt, shape in outputs]
    storage, i_in, i_out = [], 0, 0
    for role, _ in rz.slots:
        if role == L.SLOT_INPUT:
            storage.append(dev_in[i_in])
            i_in += 1
        elif role == L.SLOT_OUTPUT:
            storage.append(dev_out[i_out])
            i_out += 1
        else:
            storage.append(None)
    try:
        route(ctx, rz, storage)
        return [b.download(dt, shape) for b, (dt, shape) in zip(dev_out, outputs)]
    finally:
        for b in dev_in + dev_out:
            b.free()


@pytest.mark.parametrize("rows,extent", [(3, 1 << 16), (1, 1 << 20)])
def test_every_sum_proposal_computes_its_grouping(ctx, rows, extent):
    x = np.random.default_rng(rows + extent).uniform(-1, 1, (rows, extent)).astype(np.float32)
    offer = propose(L.PROGRAM_SERIAL_SUM, (rows, extent), permissions=RE, ctx=ctx)
    assert len(offer.proposals) == 4
    for p in offer.proposals:
        print(f"[provider sum {rows}x{extent}] {p.strategy} {p.symbols}", flush=True)
        (got,) = _routed(ctx, p.realize(ctx), [x], [(np.float32, (rows,))])
        g = p.region.grouping
        if p.strategy == "tiler.region.serial-baseline":
            want = oracle.strict_sum(x, (rows, extent), 1)
        elif p.strategy == "tiler.reduction.multi-pass-split":
            want = oracle.strict_partitioned_sum(x, rows, extent, g[0], g[1])
        elif p.strategy == "tiler.reduction.single-workgroup-tree":
            want = oracle.row_grouped_sum(x, rows, extent, 4, 4)
        elif p.strategy == "gfx950.reduction.grid-tree":
            want = np.array([oracle.grid_tree_sum(x, p.workgroups[0])], np.float32)
        else:
            assert p.strategy == "gfx950.reduction.cooperative-workgroup"
            want = oracle.cooperative_grouped_sum(x, rows, extent, g[0], g[1], g[2])
        assert np.array_equal(bits(got), bits(want)), p.strategy


def test_every_long_row_softmax_proposal(ctx):
    rows, extent = 3, 50000  # seven 8192-element segments
    x = (np.random.default_rng(5).standard_normal((rows, extent)) * 4).astype(np.float32)
    offer = propose(L.PROGRAM_SOFTMAX, (rows, extent), permissions=RE, ctx=ctx)
    assert offer.strategies() == ["tiler.region.serial-baseline", "gfx950.softmax.row-synchronized",
                                  "gfx950.softmax.split"]
    for p in offer.proposals:
        print(f"[provider softmax {rows}x{extent}] {p.strategy} {p.symbols}", flush=True)
        (got,) = _routed(ctx, p.realize(ctx), [x], [(np.float32, (rows, extent))])
        if p.strategy == "tiler.region.serial-baseline":
            want = oracle.softmax_f32(x, (rows, extent), 1).reshape(rows, extent)
        else:
            want = oracle.softmax_grouped(x, rows, extent, 4, 4, 8192).reshape(rows, extent)
        assert np.array_equal(bits(got), bits(want)), p.strategy


def test_every_contraction_proposal(ctx):
    m, n, k = 300, 264, 192
    rng = np.random.default_rng(11)
    a = oracle.bf16_narrow(rng.standard_normal((m, k)).astype(np.float32))
    b = oracle.bf16_narrow(rng.standard_normal((n, k)).astype(np.float32))
    offer = propose(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16, variant=L.EPILOGUE_SILU, permissions=RE,
                    ctx=ctx)
    assert offer.strategies() == ["tiler.region.serial-baseline", "gfx950.contraction.mfma-staged-256",
                                  "gfx950.contraction.mfma-staged-128", "gfx950.contraction.mfma-general-128"]
    wide = oracle.contract_general(bf16_widen(a), "mk", bf16_widen(b), "nk", "mn")
    want = oracle.silu_f32(wide.reshape(-1)).reshape(m, n).astype(np.float64)
    for p in offer.proposals:
        print(f"[provider contraction {m}x{n}x{k}] {p.strategy} {p.symbols}", flush=True)
        (got,) = _routed(ctx, p.realize(ctx), [a, b], [(np.uint16, (m, n))])
        if p.strategy == "tiler.region.serial-baseline":
            assert np.array_equal(got, oracle.contract_general(a, "mk", b, "nk", "mn", silu=True))
        else:
            g = bf16_widen(got).astype(np.float64)
            assert np.linalg.norm(g - want) / np.linalg.norm(want) <= 1e-2, p.strategy
