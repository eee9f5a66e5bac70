"""The realization recognizer, device-free: which entry points realize a
region, with what launch geometry, storage slots and argument segment, and
which regions it refuses.

`tiler_hip_realize` plays the role tiler-metal's emit_entry_point plays for
a scheduled region (tiler-metal/src/emit.rs:647-840).  Its answer is the
program the family entry point itself runs for the same request, so these
tests pin the choices the families make at the C5/C2/C3/C4/C1 shapes and at
the edges: tail variants, long rows, small grids, unaligned storage.
"""
from __future__ import annotations

import ctypes
import functools
import struct

import pytest

from tiler_amd import _lib as L
from tiler_amd.realize import realize
from tiler_amd.runtime import Refusal

EPS = 0x3727C5AC
RE = L.PERMITS_REASSOCIATION  # the REASSOCIATE_F32 contract's permission


def _descriptor_kernarg_bytes(symbol: str) -> int:
    for i in range(1000):
        e = L.EntryInfo()
        if L.lib().tiler_hip_payload_entry(i, ctypes.byref(e)) != L.OK:
            break
        if e.symbol.decode() == symbol:
            return e.kernarg_bytes
    raise KeyError(symbol)


def _check_segments(rz):
    """Every argument segment fits its kernel's descriptor, and kernels with
    no hidden arguments (descriptor below 256 bytes) match it exactly;
    pointer fields are 8-byte aligned and name declared slots."""
    for i, d in enumerate(rz.dispatches):
        e = rz.raw.entries[i]
        desc = _descriptor_kernarg_bytes(d.symbol)
        assert e.kernarg_bytes <= desc, d.symbol
        if desc < 256:
            assert (e.kernarg_bytes + 7) // 8 * 8 == (desc + 7) // 8 * 8, d.symbol
        for slot, off in d.bindings:
            assert off % 8 == 0 and slot < len(rz.slots)


def test_rms_norm_headline_and_variants():
    rz = realize(L.PROGRAM_RMS_NORM, (8192, 4096), dtype=L.BF16, scalars=(EPS,),
                 flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, permissions=RE)
    assert rz.symbols == ["tiler_rms_norm_bf16_ch8_full"]
    assert rz.dispatches[0].grid == (2048, 1, 1) and rz.dispatches[0].block == (256, 1, 1)
    assert rz.slots == [(L.SLOT_INPUT, 8192 * 4096 * 2), (L.SLOT_INPUT, 4096 * 2),
                        (L.SLOT_OUTPUT, 8192 * 4096 * 2)]
    assert rz.alignment == 16
    _check_segments(rz)
    # kernel arguments: x, w, w_row_stride (0: broadcast), y, rows, extent, eps
    seg = bytes(rz.raw.entries[0].kernargs[:rz.raw.entries[0].kernarg_bytes])
    assert struct.unpack_from("<QQQQQII", seg) == (0, 0, 0, 0, 8192, 4096, EPS)
    unaligned = realize(L.PROGRAM_RMS_NORM, (8, 4096), dtype=L.BF16, scalars=(EPS,), flags=0, permissions=RE)
    assert unaligned.symbols == ["tiler_rms_norm_bf16_ch8_u"] and unaligned.alignment == 1
    long_row = realize(L.PROGRAM_RMS_NORM, (3, 20000), dtype=L.BF16, scalars=(EPS,), permissions=RE)
    assert long_row.symbols == ["tiler_rms_norm_bf16_long4_a"]
    assert long_row.dispatches[0].grid == (3, 1, 1) and long_row.dispatches[0].block == (1024, 1, 1)
    _check_segments(long_row)


def test_softmax_long_rows_choose_a_launch_form():
    realize_re = functools.partial(realize, permissions=RE)
    # Rows of more than 4 segments, at most 2 workgroups per CU (the profile's
    # 256): one workgroup per 8192-element segment in one row-synchronized
    # launch, its area zeroed by a fill first (a realized plan's scratch is
    # fresh).  More workgroups: three launches, the partials in two scratch
    # slots of rows * segments f32.  Up to 4 segments: one workgroup per row.
    rs = realize_re(L.PROGRAM_SOFTMAX, (32, 131072), flags=L.REGION_ALIGNED16)
    assert rs.symbols == ["tiler_fill_u32", "tiler_softmax_f32_rowsync_a"]
    sync = 256 + 16 * 512
    assert rs.slots == [(L.SLOT_INPUT, 32 * 131072 * 4), (L.SLOT_OUTPUT, 32 * 131072 * 4), (L.SLOT_SCRATCH, sync)]
    assert rs.dispatches[1].grid == (512, 1, 1) and rs.dispatches[1].block == (256, 1, 1)
    assert struct.unpack_from("<QI4xQ", bytes(rs.raw.entries[0].kernargs[:24])) == (0, 0, sync // 4)
    _check_segments(rs)
    sp = realize_re(L.PROGRAM_SOFTMAX, (64, 131072), flags=L.REGION_ALIGNED16)
    assert sp.symbols == ["tiler_softmax_f32_split_max_a", "tiler_softmax_f32_split_sum_a",
                          "tiler_softmax_f32_split_out_a"]
    assert [d.grid for d in sp.dispatches] == [(16 * 64, 1, 1)] * 3
    assert all(d.block == (256, 1, 1) for d in sp.dispatches)
    assert sp.slots == [(L.SLOT_INPUT, 64 * 131072 * 4), (L.SLOT_OUTPUT, 64 * 131072 * 4),
                        (L.SLOT_SCRATCH, 64 * 16 * 4), (L.SLOT_SCRATCH, 64 * 16 * 4)]
    assert [sorted(s for s, _ in d.bindings) for d in sp.dispatches] == [[0, 2], [0, 2, 3], [0, 1, 2, 3]]
    _check_segments(sp)
    assert realize_re(L.PROGRAM_SOFTMAX, (3, 50001)).symbols == ["tiler_fill_u32", "tiler_softmax_f32_rowsync_u"]
    assert realize_re(L.PROGRAM_SOFTMAX, (1000, 32769)).symbols[0] == "tiler_softmax_f32_split_max_u"
    res = realize_re(L.PROGRAM_SOFTMAX, (2, 32768), flags=L.REGION_ALIGNED16)
    assert res.symbols == ["tiler_softmax_f32_long_r_a"] and res.dispatches[0].grid == (2, 1, 1)
    assert res.dispatches[0].block == (1024, 1, 1) and len(res.slots) == 2
    _check_segments(res)
    assert realize_re(L.PROGRAM_SOFTMAX, (7, 8193)).symbols == ["tiler_softmax_f32_long_r_u"]
    big = realize_re(L.PROGRAM_SOFTMAX, (100000, 65536), flags=L.REGION_ALIGNED16)
    assert big.dispatches[0].grid == (800000, 1, 1) and big.slots[2] == (L.SLOT_SCRATCH, 3200000)


def test_softmax_and_sums():
    sm = realize(L.PROGRAM_SOFTMAX, (65536, 2048), permissions=RE)
    assert sm.symbols == ["tiler_softmax_f32_ch8_full"] and sm.dispatches[0].grid == (16384, 1, 1)
    _check_segments(sm)

    tree = realize(L.PROGRAM_SERIAL_SUM, (1, 1 << 24), topology=L.SUM_TREE, permissions=RE)
    assert tree.symbols == ["tiler_sum_f32_grid", "tiler_sum_f32_grid_final"]
    G = L.lib().tiler_hip_sum_tree_workgroups(None, 1 << 24)
    assert tree.dispatches[0].grid == (G, 1, 1) and tree.dispatches[1].grid == (1, 1, 1)
    assert tree.slots[2] == (L.SLOT_SCRATCH, G * 4)
    assert [s for s, _ in tree.dispatches[0].bindings] == [0, 2]      # x, partials
    assert [s for s, _ in tree.dispatches[1].bindings] == [2, 1]      # partials, out
    _check_segments(tree)
    assert realize(L.PROGRAM_SERIAL_SUM, (1, 1000), topology=L.SUM_TREE, flags=0, permissions=RE).symbols[0] == \
        "tiler_sum_f32_grid_unaligned"
    assert realize(L.PROGRAM_SERIAL_SUM, (64, 1000), topology=L.SUM_TREE, permissions=RE).symbols == ["tiler_sum_f32_rows"]

    mp = realize(L.PROGRAM_SERIAL_SUM, (3, 120), topology=L.SUM_MULTIPASS, grouping=(4, 30), permissions=RE)
    # partitions of 30: pass 1 is the staged fold over 3 x 4 rows of 30 (stages of 16)
    assert mp.symbols == ["tiler_sum_f32_staged_r256_u", "tiler_sum_f32_serial"]
    assert realize(L.PROGRAM_SERIAL_SUM, (3, 120), topology=L.SUM_MULTIPASS, grouping=(12, 10),
                   permissions=RE).symbols == ["tiler_sum_f32_partials", "tiler_sum_f32_serial"]
    assert realize(L.PROGRAM_SERIAL_SUM, (9, 256), topology=L.SUM_TREE, permissions=RE).symbols == \
        ["tiler_sum_f32_rows_w"]
    assert mp.slots[2] == (L.SLOT_SCRATCH, 3 * 4 * 4)
    _check_segments(mp)

    coop = realize(L.PROGRAM_SERIAL_SUM, (5, 4 * 3 * 2), topology=L.SUM_COOPERATIVE, grouping=(4, 3, 2),
                   flags=L.REGION_ALIGNED16 | L.REGION_PARTICIPANT_MAJOR, permissions=RE)
    assert coop.symbols == ["tiler_sum_f32_cooperative"]
    assert coop.dispatches[0].grid == (5, 1, 1) and coop.dispatches[0].block == (4, 1, 1)
    seg = bytes(coop.raw.entries[0].kernargs[:coop.raw.entries[0].kernarg_bytes])
    # x, extent, participants, chunk, rounds, participant_major, out (natural alignment)
    assert struct.unpack_from("<QQI4xQQI4xQ", seg) == (0, 24, 4, 3, 2, 1, 0)
    _check_segments(coop)


def test_contraction_paths():
    c5 = realize(L.PROGRAM_CONTRACTION, (4096, 4096, 4096), dtype=L.BF16, permissions=RE, variant=L.EPILOGUE_SILU)
    assert c5.symbols == ["tiler_contract_bf16_silu_t256_kf"]  # k a multiple of 64: no last-tile masking
    assert c5.dispatches[0].grid == (256, 1, 1) and c5.dispatches[0].block == (1024, 1, 1)
    _check_segments(c5)
    assert realize(L.PROGRAM_CONTRACTION, (16, 4096, 4096), dtype=L.BF16, permissions=RE).symbols == \
        ["tiler_contract_bf16_skinny1"]
    small = realize(L.PROGRAM_CONTRACTION, (1000, 2048, 512), dtype=L.BF16, permissions=RE)
    assert small.symbols == ["tiler_contract_bf16_t128_kf"] and small.dispatches[0].grid == (8 * 16, 1, 1)
    assert realize(L.PROGRAM_CONTRACTION, (1000, 2048, 520), dtype=L.BF16, permissions=RE).symbols == \
        ["tiler_contract_bf16_t128"]
    assert realize(L.PROGRAM_CONTRACTION, (300, 130, 64), dtype=L.BF16, permissions=RE).symbols == \
        ["tiler_contract_bf16_g128"]
    assert realize(L.PROGRAM_CONTRACTION, (300, 128, 60), dtype=L.BF16, permissions=RE).symbols == \
        ["tiler_contract_bf16_g128_k"]
    strict = realize(L.PROGRAM_CONTRACTION, (40, 70, 9))
    assert strict.symbols == ["tiler_contract_strict_f32"] and strict.dispatches[0].grid == (5, 3, 1)
    _check_segments(strict)
    # k >= 64: register-blocked tiles of 16, 32 or 64 by the work on the busiest CU; m <= 16: staged rows
    assert realize(L.PROGRAM_CONTRACTION, (128, 1024, 3072)).symbols == ["tiler_contract_strict_f32_b16"]
    blocked = realize(L.PROGRAM_CONTRACTION, (512, 3072, 1024))
    assert blocked.symbols == ["tiler_contract_strict_f32_b32"] and blocked.dispatches[0].grid == (96, 16, 1)
    big = realize(L.PROGRAM_CONTRACTION, (2048, 2040, 70))
    assert big.symbols == ["tiler_contract_strict_f32_b64"] and big.dispatches[0].grid == (32, 32, 1)
    few = realize(L.PROGRAM_CONTRACTION, (1, 1024, 1024))
    assert few.symbols == ["tiler_contract_strict_f32_s4"] and few.dispatches[0].grid == (256, 1, 1)
    # up to 32 outputs per CU the relay-folded R = 16, beyond them R = 64 (a lane per output)
    slice_ = realize(L.PROGRAM_CONTRACTION, (1, 8192, 1024))
    assert slice_.symbols == ["tiler_contract_strict_f32_s16"] and slice_.dispatches[0].grid == (512, 1, 1)
    vocab = realize(L.PROGRAM_CONTRACTION, (1, 151936, 1024))
    assert vocab.symbols == ["tiler_contract_strict_f32_s64"] and vocab.dispatches[0].grid == (2374, 1, 1)
    prefill = realize(L.PROGRAM_CONTRACTION, (10, 2048, 1024))
    assert prefill.symbols == ["tiler_contract_strict_f32_s64"] and prefill.dispatches[0].grid == (32, 10, 1)
    for rz in (blocked, big, few):
        _check_segments(rz)


LIVE = L.REGION_ALIGNED16 | L.REGION_LIVE_EXTENT


def test_live_contracted_extent():
    """LiveContraction (tiler-ir/src/schedule/model.rs:1429-1450): k is an
    input-axis extent read at dispatch (InputExtentParameter, kernel/model.rs:
    375-390).  The realization sizes its slots for the bound, declares live
    extent 0 as input 0's axis 1 in [1, bound], and leaves the k field of the
    argument segment for the dispatch to patch."""
    m, n, bound = 40, 70, 512
    f = realize(L.PROGRAM_CONTRACTION, (m, n, bound), flags=LIVE)
    assert f.symbols == ["tiler_contract_strict_f32_b16"]
    assert f.live_extents == [(0, 1, 1, bound)]
    assert [s for s, _ in f.slots] == [L.SLOT_INPUT, L.SLOT_INPUT, L.SLOT_OUTPUT]
    assert [b for _, b in f.slots] == [m * bound * 4, n * bound * 4, m * n * 4]
    # a, b, m, n, k, c: the k field follows the two pointers and m, n
    assert f.dispatches[0].extents == [(0, 24)]
    assert bytes(f.raw.entries[0].kernargs[16:28]) == struct.pack("<III", m, n, 0)
    _check_segments(f)
    assert realize(L.PROGRAM_CONTRACTION, (m, n, bound)).live_extents == []
    # bf16: the MFMA path takes the general form, whatever the bound's alignment
    for variant, symbol in ((L.EPILOGUE_NONE, "tiler_contract_bf16_g128_k"),
                            (L.EPILOGUE_SILU, "tiler_contract_bf16_silu_g128_k")):
        b = realize(L.PROGRAM_CONTRACTION, (4096, 4096, 4096), dtype=L.BF16, permissions=RE, variant=variant,
                    flags=LIVE)
        assert b.symbols == [symbol] and b.live_extents == [(0, 1, 1, 4096)]
        assert b.dispatches[0].extents == [(0, 24)]
        _check_segments(b)
    g = realize(L.PROGRAM_CONTRACTION, (300, 264, 192), dtype=L.BF16, permissions=RE, flags=LIVE,
                form=L.FORM_CONTRACT_GENERAL_128)
    assert g.symbols == ["tiler_contract_bf16_g128_k"]
    s = realize(L.PROGRAM_CONTRACTION, (300, 264, 192), dtype=L.BF16, variant=L.EPILOGUE_SILU, flags=LIVE)
    assert s.symbols == ["tiler_contract_strict_bf16_silu_b16"] and s.dispatches[0].extents == [(0, 24)]
    # zero work still declares the extent (the route supplies it and skips the dispatch)
    z = realize(L.PROGRAM_CONTRACTION, (0, 64, 64), dtype=L.BF16, flags=LIVE)
    assert z.raw.entry_count == 0 and z.live_extents == [(0, 1, 1, 64)]


@pytest.mark.parametrize("kwargs,status,rule", [
    (dict(program=L.PROGRAM_CONTRACTION, extents=(300, 264, 192), dtype=L.BF16, permissions=RE,
          form=L.FORM_CONTRACT_STAGED_256), L.REFUSE_UNSUPPORTED, "live-extent"),
    (dict(program=L.PROGRAM_CONTRACTION, extents=(16, 264, 192), dtype=L.BF16, permissions=RE,
          form=L.FORM_CONTRACT_SKINNY), L.REFUSE_UNSUPPORTED, "live-extent"),
    (dict(program=L.PROGRAM_CONTRACTION, extents=(), dtype=L.F32,
          structure=L.contraction_structure("bhqd", (2, 2, 3, 4), "bkd", (2, 5, 4), "bhqk")),
     L.REFUSE_UNSUPPORTED, "live-extent"),
    (dict(program=L.PROGRAM_SOFTMAX, extents=(4, 64)), L.REFUSE_UNSUPPORTED, "live-extent"),
    (dict(program=L.PROGRAM_CONTRACTION, extents=(4, 4, 0)), L.REFUSE_INVALID_ARGUMENT, None),
])
def test_live_extent_refusals(kwargs, status, rule):
    program, extents = kwargs.pop("program"), kwargs.pop("extents")
    with pytest.raises(Refusal) as e:
        realize(program, extents, flags=LIVE, **kwargs)
    assert e.value.status == status
    if rule is not None:
        assert e.value.diagnostic.startswith(rule + ":"), e.value.diagnostic


def test_live_extent_provider_offer():
    """With k live only the general MFMA form runs: the provider declines the
    skinny and staged forms by that rule and chooses the general form."""
    from tiler_amd.realize import propose
    offer = propose(L.PROGRAM_CONTRACTION, (300, 264, 192), dtype=L.BF16, variant=L.EPILOGUE_SILU,
                    permissions=RE, flags=LIVE)
    assert offer.strategies() == ["tiler.region.serial-baseline", "gfx950.contraction.mfma-general-128"]
    assert {(d.strategy, d.subject) for d in offer.declined} == {
        ("gfx950.contraction.mfma-skinny", "live-extent"),
        ("gfx950.contraction.mfma-staged-256", "live-extent"),
        ("gfx950.contraction.mfma-staged-128", "live-extent")}
    assert offer.chosen == 1
    for p in offer.proposals:
        assert p.realize().live_extents == [(0, 1, 1, 192)]


def test_moves_and_maps():
    g = realize(L.PROGRAM_GATHER, (1, 128256, 4096, 16384), variant=2)
    assert g.symbols == ["tiler_fill_u32", "tiler_gather_u128"]
    assert g.slots[3] == (L.SLOT_SCRATCH, 8)
    _check_segments(g)
    assert realize(L.PROGRAM_GATHER, (2, 50, 7, 5), variant=2).symbols[1] == "tiler_gather_u16"   # 14-byte runs
    assert realize(L.PROGRAM_GATHER, (2, 50, 8, 5), variant=2, flags=0).symbols[1] == "tiler_gather_u8"

    rows_mode = realize(L.PROGRAM_BROADCAST, (8, 4096), variant=2, rank=2, strides=(0, 1), grouping=(4096,))
    assert rows_mode.symbols == ["tiler_broadcast_rows_u16"]
    _check_segments(rows_mode)
    assert realize(L.PROGRAM_BROADCAST, (8, 3), variant=4, rank=2, strides=(0, 1), grouping=(3,)).symbols == \
        ["tiler_broadcast_u32"]

    add = realize(L.PROGRAM_POINTWISE, (1024,), variant=L.MAP_ADD)
    assert add.symbols == ["tiler_map_f32_v4_op2"] and len(add.slots) == 3
    _check_segments(add)
    # a ragged or unaligned map runs the scalar kernel over all of it (no slot offsets in a plan)
    assert realize(L.PROGRAM_POINTWISE, (1023,), variant=L.MAP_ADD).symbols == ["tiler_map_f32"]
    assert realize(L.PROGRAM_POINTWISE, (1024,), variant=L.MAP_SILU, flags=0).symbols == ["tiler_map_f32"]
    silu = realize(L.PROGRAM_POINTWISE, (4096,), variant=L.MAP_SILU)
    assert silu.symbols == ["tiler_map_f32_v4_op1"] and len(silu.slots) == 2


def test_conversion_families():
    n = realize(L.PROGRAM_CONVERT, (1 << 20,), variant=L.CONVERT_NARROW_F32_BF16)
    assert n.symbols == ["tiler_narrow_f32_bf16_v8"]
    assert n.slots == [(L.SLOT_INPUT, 4 << 20), (L.SLOT_OUTPUT, 2 << 20)]
    _check_segments(n)
    w = realize(L.PROGRAM_CONVERT, (1 << 20,), variant=L.CONVERT_WIDEN_BF16_F32)
    assert w.symbols == ["tiler_widen_bf16_f32_v8"] and w.slots[1] == (L.SLOT_OUTPUT, 4 << 20)
    assert realize(L.PROGRAM_CONVERT, (1001,), variant=L.CONVERT_WIDEN_BF16_F32).symbols == ["tiler_widen_bf16_f32"]
    assert realize(L.PROGRAM_CONVERT, (1024,), variant=L.CONVERT_NARROW_F32_BF16, flags=0).symbols == \
        ["tiler_narrow_f32_bf16"]
    with pytest.raises(Refusal):
        realize(L.PROGRAM_CONVERT, (8,), variant=7)


def test_strict_affine_u4_dequantize():
    """StrictAffineU4Dequantize (model.rs:682-696): slots [codes, scale, zero
    point, y, domain record]; aligned: the wave-block form for whole
    2048-element blocks, the vector form for whole 4-element groups, else the
    scalar form over everything; a flushing contract is realized as the
    strict one (no operand or product is subnormal)."""
    rz = realize(L.PROGRAM_DEQUANTIZE_U4, (4096,))
    assert rz.symbols == ["tiler_dequantize_u4_f32_w_slots"] and rz.dispatches[0].grid == (1, 1, 1)
    assert realize(L.PROGRAM_DEQUANTIZE_U4, (6148,)).symbols == ["tiler_dequantize_u4_f32_v4_slots"]
    assert rz.slots == [(L.SLOT_INPUT, 2048), (L.SLOT_INPUT, 4), (L.SLOT_INPUT, 1), (L.SLOT_OUTPUT, 16384),
                        (L.SLOT_SCRATCH, 4)]
    assert rz.dispatches[0].bindings == [(0, 0), (1, 16), (2, 24), (3, 32), (4, 40)]
    assert realize(L.PROGRAM_DEQUANTIZE_U4, (4097,)).symbols == ["tiler_dequantize_u4_f32_slots"]
    assert realize(L.PROGRAM_DEQUANTIZE_U4, (4096,), flags=0).symbols == ["tiler_dequantize_u4_f32_slots"]
    assert realize(L.PROGRAM_DEQUANTIZE_U4, (5,)).slots[0] == (L.SLOT_INPUT, 3)  # zero-tail carrier
    flushed = realize(L.PROGRAM_DEQUANTIZE_U4, (4096,), input_subnormals=L.SUBNORMALS_FLUSH_SIGN,
                      result_subnormals=L.SUBNORMALS_FLUSH_POSITIVE)
    assert flushed.symbols == rz.symbols
    with pytest.raises(Refusal) as e:
        realize(L.PROGRAM_DEQUANTIZE_U4, (64,), dtype=L.BF16)
    assert e.value.status == L.REFUSE_UNSUPPORTED
    assert realize(L.PROGRAM_DEQUANTIZE_U4, (0,)).raw.entry_count == 0


def test_zero_work_skips_dispatch():
    assert realize(L.PROGRAM_SOFTMAX, (0, 2048)).raw.entry_count == 0
    assert realize(L.PROGRAM_CONTRACTION, (0, 64, 64), dtype=L.BF16).raw.entry_count == 0
    assert realize(L.PROGRAM_GATHER, (1, 10, 4, 0), variant=4).raw.entry_count == 0


@pytest.mark.parametrize("kwargs,status", [
    (dict(program=L.PROGRAM_RMS_NORM, extents=(4, 64), dtype=L.F32, scalars=(0,)), L.REFUSE_INVALID_ARGUMENT),
    (dict(program=L.PROGRAM_SERIAL_SUM, extents=(2, 100), topology=L.SUM_MULTIPASS, grouping=(3, 30),
          permissions=RE), L.REFUSE_INVALID_ARGUMENT),
    (dict(program=L.PROGRAM_SERIAL_SUM, extents=(2, 100), dtype=L.BF16), L.REFUSE_UNSUPPORTED),
    (dict(program=L.PROGRAM_CONTRACTION, extents=(4, 4, 0), dtype=L.BF16), L.REFUSE_INVALID_ARGUMENT),
    (dict(program=L.PROGRAM_CONTRACTION, extents=(4, 4, 4), variant=L.EPILOGUE_SILU), L.REFUSE_UNSUPPORTED),
    (dict(program=L.PROGRAM_SOFTMAX, extents=(4, 64), dtype=L.BF16), L.REFUSE_UNSUPPORTED),
    (dict(program=L.PROGRAM_POINTWISE, extents=(64,), dtype=L.BF16, variant=L.MAP_SILU), L.REFUSE_UNSUPPORTED),
    (dict(program=L.PROGRAM_BROADCAST, extents=(4, 8), variant=4, rank=2, strides=(8, 1), grouping=(16,)),
     L.REFUSE_INVALID_ARGUMENT),
    (dict(program=99, extents=(1,)), L.REFUSE_UNSUPPORTED),
])
def test_refusals_are_typed_and_pre_commit(kwargs, status):
    program = kwargs.pop("program")
    extents = kwargs.pop("extents")
    with pytest.raises(Refusal) as e:
        realize(program, extents, **kwargs)
    assert e.value.status == status and e.value.fallback_permitted
