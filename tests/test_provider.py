"""CPU: the physical-implementation provider (tiler_hip_propose).

The counterpart of PhysicalImplementationProvider::propose
(tiler-compiler/src/frontier.rs:1507-1527): for one region, every strategy
the library has, proposed with the region that realizes it, its launches and
its structural cost (PhysicalCostEstimate::structural, frontier.rs:351-400),
or declined with the reference's cause (StrategyDeclineCause,
frontier.rs:1311-1384).  Checked here without a device:
* the permission decides first: under the strict contract every regrouping
  strategy is declined for numerics.reassociation (frontier.rs:3925-3934);
* the split's partition is the reference's (physical.rs:2780-2798): checked
  against a brute-force search of the divisors;
* every proposal realizes (tiler_hip_realize on its region) to exactly the
  launches it states, and its structural cost is the sum over those launches;
* the sum's measured fold steps are sum over stages of max(work, depth * P)
  (measured_cost.rs:60-110), recomputed here from the launches' own fold
  structure, and the offer's choice is their minimum;
* the offer's choice elsewhere is what tiler_hip_realize picks by itself.
"""
from __future__ import annotations

import math

import pytest

from tiler_amd import _lib as L
from tiler_amd.realize import propose, realize
from tiler_amd.runtime import Refusal

RE = L.PERMITS_REASSOCIATION
P_ROW = 17870  # the profile's saturated_parallel_fold_steps


def _check_proposals(offer):
    for p in offer.proposals:
        rz = p.realize()
        assert rz.symbols == p.symbols, p.strategy
        assert [d.grid[0] * d.grid[1] for d in rz.dispatches] == p.workgroups
        assert [d.block[0] for d in rz.dispatches] == p.workgroup_threads
        assert p.dispatch_count == len(rz.dispatches)
        assert p.launched_threads == sum(w * t for w, t in zip(p.workgroups, p.workgroup_threads))
        assert p.temporary_bytes == sum(b for role, b in rz.slots if role == L.SLOT_SCRATCH)


def _brute_partition(n):
    best = None
    for c in range(2, math.isqrt(n) + 1):
        if n % c == 0 and n // c >= 2:
            best = (n // c, c)
    return best


def test_strict_contract_declines_every_regrouping():
    o = propose(L.PROGRAM_SERIAL_SUM, (64, 1000))
    assert o.strategies() == ["tiler.region.serial-baseline"] and o.chosen == 0
    assert {d.strategy for d in o.declined} == {"tiler.reduction.multi-pass-split",
                                                "tiler.reduction.single-workgroup-tree",
                                                "gfx950.reduction.cooperative-workgroup"}
    for d in o.declined:
        assert d.cause == L.DECLINE_NUMERICAL_PERMISSION_REFUSED and d.subject == "numerics.reassociation"
    for program, extents, kw in ((L.PROGRAM_RMS_NORM, (8, 4096), {"scalars": (0x3727C5AC,)}),
                                 (L.PROGRAM_SOFTMAX, (8, 2048), {}),
                                 (L.PROGRAM_CONTRACTION, (512, 512, 512), {"dtype": L.BF16})):
        o = propose(program, extents, **kw)
        assert o.strategies() == ["tiler.region.serial-baseline"]
        assert all(d.cause == L.DECLINE_NUMERICAL_PERMISSION_REFUSED for d in o.declined) and o.declined
        assert o.proposals[0].symbols == realize(program, extents, **kw).symbols
        _check_proposals(o)


@pytest.mark.parametrize("rows,extent", [(1, 1 << 24), (1, 4096), (3, 1 << 16), (100, 768), (7, 1000)])
def test_sum_strategies(rows, extent):
    o = propose(L.PROGRAM_SERIAL_SUM, (rows, extent), permissions=RE)
    _check_proposals(o)
    tree = "gfx950.reduction.grid-tree" if rows == 1 else "tiler.reduction.single-workgroup-tree"
    want = ["tiler.region.serial-baseline", "tiler.reduction.multi-pass-split", tree]
    if extent % 256 == 0:
        want.append("gfx950.reduction.cooperative-workgroup")
    assert o.strategies() == want
    by = {p.strategy: p for p in o.proposals}
    # the reference's partition, and the region that realizes it
    split = by["tiler.reduction.multi-pass-split"]
    assert (split.region.grouping[0], split.region.grouping[1]) == _brute_partition(extent)
    assert split.region.topology == L.SUM_MULTIPASS
    # fold steps: sum over stages of max(work, depth * P), from each form's fold structure
    n = rows * extent

    def steps(stages):
        return sum(max(w, d * P_ROW) for w, d in stages)

    parts, per = _brute_partition(extent)
    assert by["tiler.region.serial-baseline"].measured_fold_steps == steps([(n, extent)])
    assert split.measured_fold_steps == steps([(n, per), (rows * parts, parts)])
    t = by[tree]
    if rows == 1:
        g = t.workgroups[0]
        assert t.measured_fold_steps == steps([(n + g * 1540, -(-n // (256 * g)) + 10),
                                               (g + 1540, -(-g // 256) + 10)])
    else:
        assert t.measured_fold_steps == steps([(rows * (extent + 1540), -(-extent // 256) + 10)])
    if extent % 256 == 0:
        c = by["gfx950.reduction.cooperative-workgroup"]
        assert tuple(c.region.grouping) == (256, extent // 256, 1)
        assert c.measured_fold_steps == steps([(n + rows * 256, extent // 256 + 256)])
    else:
        (d,) = [d for d in o.declined if d.strategy == "gfx950.reduction.cooperative-workgroup"]
        assert d.cause == L.DECLINE_NO_ADMISSIBLE_SHAPE and d.subject == "no-admissible-participant-count"
        assert d.extent == extent
    chosen = o.proposals[o.chosen]
    assert chosen.measured_fold_steps == min(p.measured_fold_steps for p in o.proposals)


def test_sum_split_declined_without_a_partition():
    for extent in (3, 1009, (1 << 61) - 1):  # below four contributors; primes
        o = propose(L.PROGRAM_SERIAL_SUM, (2, extent), permissions=RE)
        (d,) = [d for d in o.declined if d.strategy == "tiler.reduction.multi-pass-split"]
        if extent < 1 << 48:
            assert d.cause == L.DECLINE_NO_ADMISSIBLE_SHAPE and d.subject == "no-admissible-partition"
        else:  # beyond any device's memory: the partition search is not run
            assert d.cause == L.DECLINE_UNREPRESENTABLE and d.subject == "split-extent-unrepresentable"
        assert d.extent == extent
    # the largest extents saturate the fold-step counts instead of wrapping
    o = propose(L.PROGRAM_SERIAL_SUM, (1, (1 << 64) - 1), permissions=RE)
    assert all(p.measured_fold_steps > 0 for p in o.proposals)


def test_the_measured_row_prefers_the_tree_for_one_long_row_and_serial_for_many_short():
    o = propose(L.PROGRAM_SERIAL_SUM, (1, 1 << 24), permissions=RE)
    assert o.proposals[o.chosen].strategy == "gfx950.reduction.grid-tree"
    o = propose(L.PROGRAM_SERIAL_SUM, (1 << 20, 4), permissions=RE)
    assert o.proposals[o.chosen].strategy == "tiler.region.serial-baseline"


def test_contraction_forms():
    kw = dict(dtype=L.BF16, variant=L.EPILOGUE_SILU, permissions=RE)
    o = propose(L.PROGRAM_CONTRACTION, (4096, 4096, 4096), **kw)
    _check_proposals(o)
    assert o.strategies() == ["tiler.region.serial-baseline", "gfx950.contraction.mfma-staged-256",
                              "gfx950.contraction.mfma-staged-128", "gfx950.contraction.mfma-general-128"]
    assert o.proposals[0].symbols == ["tiler_contract_strict_bf16_silu_b64"]
    by = {p.strategy: p for p in o.proposals}
    assert by["gfx950.contraction.mfma-staged-256"].workgroups == [256]
    assert by["gfx950.contraction.mfma-staged-256"].workgroup_threads == [1024]
    assert by["gfx950.contraction.mfma-staged-128"].workgroups == [1024]
    (d,) = o.declined
    assert (d.strategy, d.cause, d.subject, d.extent) == ("gfx950.contraction.mfma-skinny",
                                                          L.DECLINE_NO_ADMISSIBLE_SHAPE, "skinny-rows", 4096)
    assert o.proposals[o.chosen].symbols == realize(L.PROGRAM_CONTRACTION, (4096, 4096, 4096), **kw).symbols
    # decode: the skinny form is proposed and chosen
    o = propose(L.PROGRAM_CONTRACTION, (16, 4096, 4096), **kw)
    _check_proposals(o)
    assert o.proposals[o.chosen].strategy == "gfx950.contraction.mfma-skinny"
    assert o.proposals[o.chosen].symbols == realize(L.PROGRAM_CONTRACTION, (16, 4096, 4096), **kw).symbols
    # n off the 8-element grid: only the general form among the MFMA forms
    o = propose(L.PROGRAM_CONTRACTION, (300, 100, 64), **kw)
    _check_proposals(o)
    assert o.strategies() == ["tiler.region.serial-baseline", "gfx950.contraction.mfma-general-128"]
    staged = [d for d in o.declined if d.strategy.startswith("gfx950.contraction.mfma-staged")]
    assert len(staged) == 2 and all(d.subject == "staged-rows" and d.extent == 100 for d in staged)
    # f32 has the strict fold only
    o = propose(L.PROGRAM_CONTRACTION, (64, 64, 64), dtype=L.F32, permissions=RE)
    assert o.strategies() == ["tiler.region.serial-baseline"] and not o.declined


def test_general_contraction_forms():
    S = L.contraction_structure
    score = S("bhqd", (2, 8, 256, 64), "bkd", (2, 256, 64), "bhqk")
    o = propose(L.PROGRAM_CONTRACTION, (), dtype=L.BF16, structure=score, permissions=RE)
    _check_proposals(o)
    assert o.strategies() == ["tiler.region.serial-baseline", "gfx950.contraction.mfma-batched"]
    assert o.proposals[0].symbols == ["tiler_contract_general_bf16"] and o.chosen == 1
    assert o.proposals[1].symbols == ["tiler_contract_bf16_t128_b"]
    odd = S("km", (64, 32), "nk", (16, 64), "mn")  # the left operand stored [k, m]
    o = propose(L.PROGRAM_CONTRACTION, (), dtype=L.BF16, structure=odd, permissions=RE)
    assert o.strategies() == ["tiler.region.serial-baseline"] and o.chosen == 0
    (d,) = o.declined
    assert d.subject == "batched-operand-layout" and d.cause == L.DECLINE_NO_ADMISSIBLE_SHAPE


def test_softmax_and_rms_norm_forms():
    o = propose(L.PROGRAM_SOFTMAX, (32, 131072), permissions=RE)
    _check_proposals(o)
    assert o.strategies() == ["tiler.region.serial-baseline", "gfx950.softmax.row-synchronized",
                              "gfx950.softmax.split"]
    assert o.proposals[o.chosen].symbols == realize(L.PROGRAM_SOFTMAX, (32, 131072), permissions=RE).symbols
    by = {p.strategy: p for p in o.proposals}
    assert by["gfx950.softmax.split"].dispatch_count == 3
    assert by["gfx950.softmax.split"].temporary_bytes == 2 * 32 * 16 * 4
    # too many segments for every workgroup to be resident: the split only
    o = propose(L.PROGRAM_SOFTMAX, (4096, 131072), permissions=RE)
    assert o.strategies() == ["tiler.region.serial-baseline", "gfx950.softmax.split"]
    (d,) = o.declined
    assert (d.subject, d.extent) == ("row-sync-residency", 4096 * 16)
    # rows of at most four segments: the grouped fold
    o = propose(L.PROGRAM_SOFTMAX, (64, 2048), permissions=RE)
    assert o.strategies() == ["tiler.region.serial-baseline", "gfx950.rows.grouped-fold"] and o.chosen == 1
    o = propose(L.PROGRAM_RMS_NORM, (8192, 4096), dtype=L.BF16, scalars=(0x3727C5AC,), permissions=RE)
    _check_proposals(o)
    assert o.strategies() == ["tiler.region.serial-baseline", "gfx950.rows.grouped-fold"]
    assert o.proposals[1].symbols == ["tiler_rms_norm_bf16_ch8_full"] and o.chosen == 1


def test_single_form_programs_and_refusals():
    o = propose(L.PROGRAM_CONVERT, (1 << 20,), variant=L.CONVERT_NARROW_F32_BF16)
    assert o.strategies() == ["tiler.region.serial-baseline"] and not o.declined
    _check_proposals(o)
    # a form a program does not have, or one the shape does not admit, refuses
    with pytest.raises(Refusal):
        realize(L.PROGRAM_CONVERT, (1 << 20,), form=L.FORM_CONTRACT_SKINNY)
    with pytest.raises(Refusal):
        realize(L.PROGRAM_CONTRACTION, (4096, 4096, 4096), dtype=L.BF16, permissions=RE,
                form=L.FORM_CONTRACT_SKINNY)
    with pytest.raises(Refusal):  # a form needs the reassociation it regroups by
        realize(L.PROGRAM_CONTRACTION, (64, 64, 64), dtype=L.BF16, form=L.FORM_CONTRACT_STAGED_128)
    with pytest.raises(Refusal):
        realize(L.PROGRAM_SOFTMAX, (8, 2048), permissions=RE, form=L.FORM_SOFTMAX_SPLIT)
    # a malformed request every strategy refuses the same way
    with pytest.raises(Refusal) as e:
        propose(L.PROGRAM_RMS_NORM, (8, 4096), scalars=(0,), permissions=RE)
    assert e.value.status == L.REFUSE_INVALID_ARGUMENT
    assert propose(L.PROGRAM_SERIAL_SUM, (4, 4)).provider == "tiler.hip.gfx950-physical-provider"
