"""CPU: the boundary's numerical contract, the new realization programs
(expression DAGs, folds over any axis set, signed-stride reindex), the
target-environment schema, and the oracle functions that check them on the
GPU -- each pinned by something other than a restatement of itself.

Contract (tiler-ir/src/schedule/model.rs:1330-1340, 1381-1392, 1520-1531;
tiler-compiler/src/session.rs:1793-1888): a zeroed region is the strict
contract, so it must get the strict serial fold or refuse; a reassociating
realization needs permits_reassociation; a flushing subnormal mode is realized
where the kernels apply it and refused elsewhere.
"""
from __future__ import annotations

import ctypes
import struct
from fractions import Fraction

import numpy as np
import pytest

import oracle
from helpers import bits
from tiler_amd import _lib as L
from tiler_amd import runtime
from tiler_amd.realize import realize
from tiler_amd.runtime import Refusal

RE = L.PERMITS_REASSOCIATION
EPS = 0x3727C5AC


def _refuses(status, *args, **kwargs):
    with pytest.raises(Refusal) as e:
        realize(*args, **kwargs)
    assert e.value.status == status, e.value
    assert e.value.fallback_permitted
    return e.value


# --- the contract ---------------------------------------------------------------

def test_zeroed_region_is_the_strict_serial_sum():
    r = L.Region()  # every field zero
    r.program = L.PROGRAM_SERIAL_SUM
    r.extents[0], r.extents[1] = 4, 100
    out = L.Realization()
    assert L.lib().tiler_hip_realize(None, ctypes.byref(r), ctypes.byref(out), None, 0) == L.OK
    info = L.EntryInfo()
    assert L.lib().tiler_hip_payload_entry(out.entries[0].entry, ctypes.byref(info)) == L.OK
    # the strict serial fold (rows of 100 are staged through LDS, one row per
    # workgroup for 4 rows; the stand-in address is unaligned without ALIGNED16)
    assert out.entry_count == 1 and info.symbol == b"tiler_sum_f32_staged_r1_u"
    assert info.family == b"strict-serial-sum-f32/serial"
    assert L.SUM_SERIAL == 0


@pytest.mark.parametrize("topology,grouping", [(L.SUM_TREE, ()), (L.SUM_MULTIPASS, (4, 25)),
                                               (L.SUM_COOPERATIVE, (4, 5, 5))])
def test_reassociating_sums_need_the_permission(topology, grouping):
    e = _refuses(L.REFUSE_UNSUPPORTED, L.PROGRAM_SERIAL_SUM, (2, 100), topology=topology, grouping=grouping)
    assert "reassociation" in e.diagnostic
    assert realize(L.PROGRAM_SERIAL_SUM, (2, 100), topology=topology, grouping=grouping,
                   permissions=RE).raw.entry_count >= 1


def test_strict_contract_selects_the_serial_row_and_contraction_kernels():
    s = realize(L.PROGRAM_RMS_NORM, (8192, 4096), dtype=L.BF16, scalars=(EPS,),
                flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST)
    # aligned rows of at most 512 16-byte pieces, enough of them: held in registers, 8 per workgroup
    assert s.symbols == ["tiler_rms_norm_bf16_strict_rr8_p16"] and s.dispatches[0].grid == (1024, 1, 1)
    assert realize(L.PROGRAM_RMS_NORM, (8192, 2048), scalars=(EPS,), flags=L.REGION_ALIGNED16).symbols == \
        ["tiler_rms_norm_f32_strict_rr8_p16"]
    # rows of >= 64 otherwise: staged, 16 rows per workgroup at 8192 rows (512 workgroups on 256 CUs)
    st = realize(L.PROGRAM_RMS_NORM, (8192, 4104), dtype=L.BF16, scalars=(EPS,),
                 flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST)
    assert st.symbols == ["tiler_rms_norm_bf16_strict_r16"] and st.dispatches[0].grid == (512, 1, 1)
    assert realize(L.PROGRAM_RMS_NORM, (5, 20000), scalars=(EPS,)).symbols == ["tiler_rms_norm_f32_strict_r1"]
    assert realize(L.PROGRAM_RMS_NORM, (5, 40), scalars=(EPS,)).symbols == ["tiler_rms_norm_f32_strict"]
    assert realize(L.PROGRAM_SOFTMAX, (32, 131072)).symbols == ["tiler_softmax_f32_strict_r1"]
    # rows of 128..4096 aligned elements, enough of them: held in registers, 8 per workgroup
    sm = realize(L.PROGRAM_SOFTMAX, (65536, 2048))
    assert sm.symbols == ["tiler_softmax_f32_strict_rr8_p16"] and sm.dispatches[0].grid == (8192, 1, 1)
    assert sm.dispatches[0].block == (256, 1, 1)
    assert realize(L.PROGRAM_SOFTMAX, (4096, 1024)).symbols == ["tiler_softmax_f32_strict_rr8_p8"]
    assert realize(L.PROGRAM_SOFTMAX, (4096, 2052)).symbols == ["tiler_softmax_f32_strict_rr8_p32"]
    assert realize(L.PROGRAM_SOFTMAX, (4096, 4100)).symbols == ["tiler_softmax_f32_strict_r16"]
    assert realize(L.PROGRAM_SOFTMAX, (1024, 2048)).symbols == ["tiler_softmax_f32_strict_r4"]
    assert realize(L.PROGRAM_SOFTMAX, (9, 40)).symbols == ["tiler_softmax_f32_strict"]
    c = realize(L.PROGRAM_CONTRACTION, (4096, 4096, 4096), dtype=L.BF16, variant=L.EPILOGUE_SILU)
    assert c.symbols == ["tiler_contract_strict_bf16_silu_b64"] and c.dispatches[0].grid == (64, 64, 1)
    assert realize(L.PROGRAM_CONTRACTION, (40, 70, 9), dtype=L.BF16).symbols == ["tiler_contract_strict_bf16"]
    # the same regions under REASSOCIATE_F32 get the grouped forms
    assert realize(L.PROGRAM_SOFTMAX, (32, 131072), permissions=RE).symbols[-1] == "tiler_softmax_f32_rowsync_a"
    assert realize(L.PROGRAM_CONTRACTION, (4096, 4096, 4096), dtype=L.BF16, variant=L.EPILOGUE_SILU,
                   permissions=RE).symbols == ["tiler_contract_bf16_silu_t256_kf"]


@pytest.mark.parametrize("program,extents,kw", [
    (L.PROGRAM_CONVERT, (64,), {}),
    (L.PROGRAM_CONVERT, (64,), dict(variant=L.CONVERT_WIDEN_BF16_F32)),
])
@pytest.mark.parametrize("modes", [(L.SUBNORMALS_FLUSH_SIGN, 0), (0, L.SUBNORMALS_FLUSH_POSITIVE)])
def test_flushing_modes_refuse_where_not_implemented(program, extents, kw, modes):
    e = _refuses(L.REFUSE_UNSUPPORTED, program, extents, input_subnormals=modes[0],
                 result_subnormals=modes[1], **kw)
    assert "subnormal" in e.diagnostic


def test_flushing_modes_where_implemented_or_irrelevant():
    nodes = [(0, 0, 0), (0, 1, 0), (2, 0, 1)]
    rz = realize(L.PROGRAM_EXPRESSION, (64,), nodes=nodes, input_subnormals=L.SUBNORMALS_FLUSH_SIGN,
                 result_subnormals=L.SUBNORMALS_FLUSH_POSITIVE)
    seg = bytes(rz.raw.entries[0].kernargs[:rz.raw.entries[0].kernarg_bytes])
    assert struct.unpack_from("<II", seg, len(seg) - 8) == (2, 3)  # the modes reach the kernel
    # the vector form reads the modes only in its _r16f_ copy; the preserve copy compiles them out
    assert rz.symbols == ["tiler_expr_f32_r16f_i2"]
    assert realize(L.PROGRAM_EXPRESSION, (64,), nodes=nodes).symbols == ["tiler_expr_f32_r16_i2"]
    assert realize(L.PROGRAM_EXPRESSION, (64,), nodes=nodes, flags=0, input_subnormals=L.SUBNORMALS_FLUSH_SIGN
                   ).symbols == ["tiler_expr_f32_r16s_i2"]
    # byte moves perform no arithmetic
    assert realize(L.PROGRAM_GATHER, (1, 10, 4, 3), variant=4, input_subnormals=2).raw.entry_count == 2
    assert realize(L.PROGRAM_BROADCAST, (8, 4), variant=4, rank=2, strides=(0, 1), grouping=(4,),
                   result_subnormals=3).raw.entry_count == 1
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_EXPRESSION, (64,), nodes=nodes, input_subnormals=4)


FS, FP = L.SUBNORMALS_FLUSH_SIGN, L.SUBNORMALS_FLUSH_POSITIVE


@pytest.mark.parametrize("program,extents,kw,symbols", [
    # sums and folds: the rule-driven kernels (first-contributor seeds, modes at every combine)
    (L.PROGRAM_SERIAL_SUM, (2, 100), {}, ["tiler_sum_f32_staged_r1_m"]),
    (L.PROGRAM_SERIAL_SUM, (4096, 40), {}, ["tiler_sum_f32_staged_r256_m"]),
    (L.PROGRAM_SERIAL_SUM, (9, 7), {}, ["tiler_fold_f32_m"]),
    (L.PROGRAM_SERIAL_SUM, (4, 100), dict(topology=L.SUM_MULTIPASS, grouping=(10, 10), permissions=RE),
     ["tiler_sum_f32_partials_m", "tiler_fold_f32_m"]),
    (L.PROGRAM_SERIAL_SUM, (4, 6400), dict(topology=L.SUM_MULTIPASS, grouping=(80, 80), permissions=RE),
     ["tiler_sum_f32_staged_r4_m", "tiler_sum_f32_staged_r1_m"]),
    (L.PROGRAM_SERIAL_SUM, (4, 100), dict(topology=L.SUM_COOPERATIVE, grouping=(10, 5, 2), permissions=RE),
     ["tiler_sum_f32_cooperative_m"]),
    (L.PROGRAM_FOLD, (64, 16384), dict(rank=2, grouping=(2,), variant=L.FOLD_FMA, scalars=(0x3F800000, 0)),
     ["tiler_sum_f32_staged_r1_m"]),
    (L.PROGRAM_FOLD, (64, 16384), dict(rank=2, grouping=(2, 256, 64), variant=L.FOLD_FMA, scalars=(0x3F800000, 0),
                                       topology=L.SUM_COOPERATIVE, permissions=RE), ["tiler_sum_f32_cooperative_m"]),
    (L.PROGRAM_FOLD, (4, 5, 6), dict(rank=3, grouping=(5,), variant=L.FOLD_SQUARED), ["tiler_fold_f32_m"]),
    (L.PROGRAM_FOLD, (4, 5, 6), dict(rank=3, grouping=(5,), variant=L.FOLD_MAXIMUM), ["tiler_fold_maximum_f32"]),
    # rows: the serial forms that take the modes, whatever the permissions
    (L.PROGRAM_RMS_NORM, (8192, 4104), dict(scalars=(EPS,), dtype=L.BF16, permissions=RE),
     ["tiler_rms_norm_bf16_strict_r16_m"]),
    (L.PROGRAM_SOFTMAX, (2, 100), {}, ["tiler_softmax_f32_strict_r1_m"]),
    # rows the register-resident forms hold take their _m forms
    (L.PROGRAM_RMS_NORM, (8192, 4096), dict(scalars=(EPS,), dtype=L.BF16, permissions=RE),
     ["tiler_rms_norm_bf16_strict_rr8_p16_m"]),
    (L.PROGRAM_RMS_NORM, (2048, 1024), dict(scalars=(EPS,), flags=L.REGION_ALIGNED16),
     ["tiler_rms_norm_f32_strict_rr8_p8_m"]),
    (L.PROGRAM_SOFTMAX, (8192, 2048), {}, ["tiler_softmax_f32_strict_rr8_p16_m"]),
    (L.PROGRAM_SOFTMAX, (4096, 1024), {}, ["tiler_softmax_f32_strict_rr8_p8_m"]),
    # rows the staged forms take: their _m forms; rows under 64: one wave per row
    (L.PROGRAM_SOFTMAX, (1024, 2048), {}, ["tiler_softmax_f32_strict_r4_m"]),
    (L.PROGRAM_SOFTMAX, (32, 131072), {}, ["tiler_softmax_f32_strict_r1_m"]),
    (L.PROGRAM_SOFTMAX, (9, 40), {}, ["tiler_softmax_f32_strict"]),
    (L.PROGRAM_RMS_NORM, (5, 20000), dict(scalars=(EPS,)), ["tiler_rms_norm_f32_strict_r1_m"]),
    (L.PROGRAM_RMS_NORM, (5, 40), dict(scalars=(EPS,)), ["tiler_rms_norm_f32_strict"]),
    # maps: the scalar forms with the modes; bf16 expressions: the one-element form
    (L.PROGRAM_POINTWISE, (1024,), dict(variant=L.MAP_SILU), ["tiler_map_f32_m"]),
    (L.PROGRAM_POINTWISE, (1024,), dict(variant=L.MAP_ADD, dtype=L.BF16), ["tiler_map_bf16_m"]),
    (L.PROGRAM_EXPRESSION, (64,), dict(dtype=L.BF16, nodes=[(0, 0, 0), (2, 0, 0)]), ["tiler_expr_bf16_r16s_i1"]),
    # contractions: the strict fold with the modes, whatever the permissions
    (L.PROGRAM_CONTRACTION, (4, 4, 4), {}, ["tiler_contract_general_f32_m"]),
    (L.PROGRAM_CONTRACTION, (4096, 4096, 64), dict(dtype=L.BF16, variant=L.EPILOGUE_SILU, permissions=RE),
     ["tiler_contract_general_bf16_silu_m"]),
])
def test_flushing_modes_are_realized(program, extents, kw, symbols):
    """A flushing contract realizes where the kernels apply the modes; the
    modes travel in the argument segment (the last words, or the FoldRule's)."""
    rz = realize(program, extents, input_subnormals=FS, result_subnormals=FP, **kw)
    assert rz.symbols == symbols
    if program == L.PROGRAM_FOLD and kw.get("variant") == L.FOLD_MAXIMUM:
        return  # the maximum takes no mode
    seg = bytes(rz.raw.entries[0].kernargs[:rz.raw.entries[0].kernarg_bytes])
    words = struct.unpack_from(f"<{len(seg) // 4}I", seg)
    assert any(words[i:i + 2] == (FS, FP) for i in range(len(words) - 1)), words


def test_two_level_tree_refuses_a_flushing_contract():
    e = _refuses(L.REFUSE_UNSUPPORTED, L.PROGRAM_SERIAL_SUM, (4, 100), topology=L.SUM_TREE, permissions=RE,
                 input_subnormals=FS, result_subnormals=FS)
    assert "cooperative" in e.diagnostic
    # a split or workgroup fold needs the reassociation permission, and the trailing axis
    _refuses(L.REFUSE_UNSUPPORTED, L.PROGRAM_FOLD, (64, 256), rank=2, grouping=(2, 16, 16),
             topology=L.SUM_MULTIPASS)
    _refuses(L.REFUSE_UNSUPPORTED, L.PROGRAM_FOLD, (64, 256), rank=2, grouping=(1, 8, 8),
             topology=L.SUM_MULTIPASS, permissions=RE)


@pytest.mark.parametrize("topology,grouping", [(L.SUM_TREE, ()), (L.SUM_COOPERATIVE, (1, 1, 1))])
def test_rows_beyond_the_launch_grid_refuse(topology, grouping):
    _refuses(L.REFUSE_CAPACITY, L.PROGRAM_SERIAL_SUM, ((1 << 32) + 1, 1), topology=topology, grouping=grouping,
             permissions=RE)
    _refuses(L.REFUSE_CAPACITY, L.PROGRAM_SERIAL_SUM, ((1 << 31), 1), topology=topology, grouping=grouping,
             permissions=RE)


# --- expressions ------------------------------------------------------------------

def _program(rz):
    """The realization's CONSTANT slot decoded: (op, dst, a, b, imm) per instruction."""
    code = bytes(rz.raw.constant[:rz.raw.constant_bytes])
    return [struct.unpack_from("<HHHHI", code, i) for i in range(0, len(code), 12)]


def test_expression_realization_slots_and_program():
    # y = (x0 * 2 + x1) / x2: the inputs run first, one register each
    nodes = [(0, 1, 0), (1, 0x40000000, 0), (3, 0, 1), (0, 0, 0), (2, 2, 3), (0, 2, 0), (4, 4, 5)]
    rz = realize(L.PROGRAM_EXPRESSION, (1 << 26,), nodes=nodes)
    assert rz.symbols == ["tiler_expr_f32_r16_i3"]
    assert [r for r, _ in rz.slots] == [L.SLOT_INPUT] * 3 + [L.SLOT_OUTPUT, L.SLOT_CONSTANT]
    assert rz.raw.constant_slot == 4 and rz.raw.constant_bytes == 7 * 12
    prog = _program(rz)
    assert [(p[0], p[1], p[4]) for p in prog[:3]] == [(0, 0, 0), (0, 1, 1), (0, 2, 2)]  # input k -> register k
    assert [p[0] for p in prog[3:]] == [1, 3, 2, 4]
    assert max(p[1] for p in prog) < 5
    # ragged or unaligned: one element per lane; more than 4 inputs: loads in place
    assert realize(L.PROGRAM_EXPRESSION, (1001,), nodes=nodes).symbols == ["tiler_expr_f32_r16s_i3"]
    assert realize(L.PROGRAM_EXPRESSION, (1024,), nodes=nodes, flags=0).symbols == ["tiler_expr_f32_r16s_i3"]
    wide = [(0, k, 0) for k in range(6)] + [(2, 0, 1), (2, 6, 2), (2, 7, 3), (2, 8, 4), (2, 9, 5)]
    assert realize(L.PROGRAM_EXPRESSION, (1024,), nodes=wide).symbols == ["tiler_expr_f32_r16_i0"]
    bf = realize(L.PROGRAM_EXPRESSION, (1 << 20,), dtype=L.BF16, nodes=[(0, 0, 0), (1, 0x4000, 0), (3, 0, 1)])
    assert bf.symbols == ["tiler_expr_bf16_r16_i1"] and bf.slots[0] == (L.SLOT_INPUT, 2 << 20)


def test_expression_register_allocation_reuses_registers():
    # a chain of 4000 additions needs three registers; 100 values all live at
    # the end need 100 (the value-store form)
    chain = [(0, 0, 0), (1, 0x3F800000, 0)] + [(2, i + 1 if i else 0, 1) for i in range(4000)]
    rz = realize(L.PROGRAM_EXPRESSION, (4096,), nodes=chain)
    prog = _program(rz)
    assert len(prog) == 4002 and max(p[1] for p in prog) <= 2
    assert rz.symbols == ["tiler_expr_f32_r16_i1"]
    wide = [(0, 0, 0)] + [(1, 0x3F800000 + k, 0) for k in range(100)]
    acc = 0
    for k in range(100):
        wide.append((2, acc if k else 0, 1 + k))
        acc = len(wide) - 1
    # constants 1..100 are all defined before any is used: 101 live values
    mem = realize(L.PROGRAM_EXPRESSION, (4096,), nodes=wide)
    assert mem.symbols == ["tiler_expr_f32_mem"]
    assert mem.slots[-1][0] == L.SLOT_SCRATCH and mem.slots[-1][1] % (4 * 256) == 0
    regs = max(p[1] for p in _program(mem)) + 1
    assert regs >= 101 and mem.slots[-1][1] == 4 * regs * 4096


@pytest.mark.parametrize("nodes,root,status,what", [
    ([], None, L.REFUSE_INVALID_ARGUMENT, "empty"),
    ([(0, 0, 0), (2, 0, 2), (0, 1, 0)], 1, L.REFUSE_INVALID_ARGUMENT, "defined before use"),
    ([(0, 1, 0), (2, 0, 0)], None, L.REFUSE_INVALID_ARGUMENT, "dense"),        # ordinal 0 missing
    ([(0, 0, 0), (0, 0, 0), (2, 0, 1)], None, L.REFUSE_INVALID_ARGUMENT, "dense"),  # ordinal twice
    ([(0, 0, 0), (1, 5, 0), (2, 0, 0)], None, L.REFUSE_INVALID_ARGUMENT, "unreachable"),
    ([(0, 0, 0), (7, 0, 0)], None, L.REFUSE_INVALID_ARGUMENT, "vocabulary"),
    ([(1, 0, 0)], None, L.REFUSE_INVALID_ARGUMENT, "no input"),
    ([(0, 0, 0), (2, 0, 0)], 5, L.REFUSE_INVALID_ARGUMENT, "root"),
])
def test_expression_verification_refusals(nodes, root, status, what):
    e = _refuses(status, L.PROGRAM_EXPRESSION, (64,), nodes=nodes, root=root) if nodes else None
    if nodes:
        assert what in e.diagnostic
    else:
        r = L.Region()
        r.program, r.extents[0] = L.PROGRAM_EXPRESSION, 64
        out = L.Realization()
        assert L.lib().tiler_hip_realize(None, ctypes.byref(r), ctypes.byref(out), None, 0) == status


def test_expression_vocabulary_and_capacity_limits():
    # bf16 has no divide, exp or rsqrt, and 16-bit constants
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_EXPRESSION, (64,), dtype=L.BF16, nodes=[(0, 0, 0), (4, 0, 0)])
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_EXPRESSION, (64,), dtype=L.BF16,
             nodes=[(0, 0, 0), (1, 0x10000, 0), (2, 0, 1)])
    many = [(0, k, 0) for k in range(17)]
    acc = 0
    for k in range(1, 17):
        many.append((2, acc, k))
        acc = len(many) - 1
    _refuses(L.REFUSE_CAPACITY, L.PROGRAM_EXPRESSION, (64,), nodes=many)
    big = [(0, 0, 0)] + [(2, i, 0) for i in range(4096)]
    assert "4096" in _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_EXPRESSION, (64,), nodes=big).diagnostic
    at_limit = [(0, 0, 0)] + [(2, i, 0) for i in range(4095)]
    assert realize(L.PROGRAM_EXPRESSION, (64,), nodes=at_limit).raw.constant_bytes == 4096 * 12


# --- folds and reindex --------------------------------------------------------------

def test_fold_planning():
    f = realize(L.PROGRAM_FOLD, (2, 3, 4), rank=3, grouping=(0b110,))  # reduction_multi_axis golden
    assert f.symbols == ["tiler_fold_sum_f32"]
    assert f.slots == [(L.SLOT_INPUT, 96), (L.SLOT_OUTPUT, 8)]
    m = realize(L.PROGRAM_FOLD, (5, 6, 7), rank=3, grouping=(0b101,), variant=L.FOLD_MAXIMUM)
    assert m.symbols == ["tiler_fold_maximum_f32"] and m.slots[1] == (L.SLOT_OUTPUT, 24)
    # model.rs:880-906: no empty-domain value for a maximum; an empty sum commits +0
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_FOLD, (3, 0), rank=2, grouping=(0b10,), variant=L.FOLD_MAXIMUM)
    assert realize(L.PROGRAM_FOLD, (3, 0), rank=2, grouping=(0b10,)).raw.entry_count == 1
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_FOLD, (3, 4), rank=2, grouping=(0b100,))
    # SquaredSerialSumThenEpilogue: rsqrt(a / N + eps), one input, something computed
    epi = [(0, 0, 0), (1, 0x45800000, 0), (4, 0, 1), (1, EPS, 0), (2, 2, 3), (6, 4, 0)]
    e = realize(L.PROGRAM_FOLD, (16, 4096), rank=2, grouping=(0b10,), variant=L.FOLD_SQUARED, nodes=epi)
    assert e.slots[2][0] == L.SLOT_CONSTANT and e.raw.constant_slot == 2
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_FOLD, (16, 4096), rank=2, grouping=(0b10,),
             variant=L.FOLD_SQUARED, nodes=[(0, 0, 0)])


def test_reindex_planning():
    # structural_mirrored_reindex.metal: out[i] = src[(i/2)*2 + 1 - i%2] over [2, 2]
    r = realize(L.PROGRAM_REINDEX, (2, 2), rank=2, strides=(2, -1), grouping=(4, 1), variant=4)
    assert r.symbols == ["tiler_broadcast_u32"]
    seg = bytes(r.raw.entries[0].kernargs[:r.raw.entries[0].kernarg_bytes])
    dims = struct.unpack_from("<8Q", seg, 24)
    strides = struct.unpack_from("<8q", seg, 24 + 64)
    base = struct.unpack_from("<q", seg, 24 + 128 + 8)[0]
    assert dims[:2] == (2, 2) and strides[:2] == (2, -1) and base == 1
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_REINDEX, (2, 2), rank=2, strides=(2, -1), grouping=(4, 0),
             variant=4)   # reaches offset -1
    _refuses(L.REFUSE_INVALID_ARGUMENT, L.PROGRAM_REINDEX, (2, 2), rank=2, strides=(2, -1), grouping=(4, 2),
             variant=4)   # reaches offset 4


# --- target environment -------------------------------------------------------------

def _descriptor(target_id: bytes, wave: int = 64) -> bytes:
    return struct.pack(">I", len(target_id)) + target_id + struct.pack(">I", wave)


def test_target_environment_schema_and_canonical_spelling():
    s = runtime.target_environment_support()
    assert s == {"provider": "tiler.hip.target-environment", "revision": 1, "schema": (1, 0)}
    for feats in (b":sramecc+:xnack-", b":sramecc-:xnack-", b":sramecc+:xnack+", b":sramecc-:xnack+"):
        assert runtime.validate_target_environment(_descriptor(b"amdgcn-amd-amdhsa--gfx950" + feats)) is None
    bad = [
        (_descriptor(b"amdgcn-amd-amdhsa--gfx950:xnack-:sramecc+"), "canonical"),
        (_descriptor(b"amdgcn-amd-amdhsa--gfx950"), "canonical"),
        (_descriptor(b"amdgcn-amd-amdhsa--gfx942:sramecc+:xnack-"), "gfx950"),
        (_descriptor(b"amdgcn-amd-amdhsa--gfx950:sramecc+:xnack-", 32), "wavefront"),
        (_descriptor(b"amdgcn-amd-amdhsa--gfx950:sramecc+:xnack-") + b"\0", "length"),
        (b"\0\0\0", "shorter"),
    ]
    for d, why in bad:
        reason = runtime.validate_target_environment(d)
        assert reason is not None and why in reason, (d, reason)


# --- oracle pins ----------------------------------------------------------------------

def _bf16_rne_exact(q: Fraction) -> int:
    """ADR 0091 narrowing of an exact rational, by integer arithmetic."""
    if q == 0:
        return 0
    sign = 0x8000 if q < 0 else 0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    quantum = Fraction(2) ** (e - 7)
    m = a / quantum
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2):
        fl += 1
    r = fl * quantum
    if r >= Fraction(2) ** 128:
        return sign | 0x7F80
    f = np.float32(float(r))
    return sign | int(bits(np.array([f]))[0] >> 16)


def test_oracle_bf16_arithmetic_is_the_exact_rounding():
    """bf16 add/multiply: the oracle (binary128), exact rationals, and the
    binary32 shortcut the device uses agree -- on random finite pairs across
    the exponent range, ties, overflow and subnormals."""
    rng = np.random.default_rng(91)
    xs = rng.integers(0, 0x10000, 20000, dtype=np.uint32).astype(np.uint16)
    zs = rng.integers(0, 0x10000, 20000, dtype=np.uint32).astype(np.uint16)
    edge = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x0080, 0x3F80, 0x3B80, 0x3B81, 0x7F7F, 0xFF7F,
                     0x3F81, 0xBF80, 0x0100, 0x4000], dtype=np.uint16)
    xs = np.concatenate([xs, np.repeat(edge, edge.size)])
    zs = np.concatenate([zs, np.tile(edge, edge.size)])
    checked = 0
    for x, z in zip(xs.tolist(), zs.tolist()):
        fx, fz = (np.uint32(v << 16).view(np.float32) for v in (x, z))
        if not (np.isfinite(fx) and np.isfinite(fz)):
            continue
        qx, qz = Fraction(float(fx)), Fraction(float(fz))
        for op, exact, f32r in ((oracle.bf16_exact_add, qx + qz, np.float32(fx) + np.float32(fz)),
                                (oracle.bf16_exact_multiply, qx * qz, np.float32(fx) * np.float32(fz))):
            want = _bf16_rne_exact(exact)
            if exact == 0:
                want = int(oracle.bf16_narrow(np.array([f32r], np.float32))[0])  # signed zero: IEEE's sign rule
            assert op(x, z) == want, (hex(x), hex(z), op.__name__)
            assert int(oracle.bf16_narrow(np.array([f32r], np.float32))[0]) == want
            checked += 1
    assert checked > 40000


def test_oracle_f32_expression_against_ieee_binary32():
    """Add, multiply and divide nodes are single IEEE binary32 roundings
    (numpy float32 arithmetic), canonical NaN after each; exp and rsqrt nodes
    are the certified functions."""
    rng = np.random.default_rng(92)
    n = 5000
    x0 = (rng.standard_normal(n) * 10).astype(np.float32)
    x1 = (rng.standard_normal(n) * 10).astype(np.float32)
    x1[:5] = [0.0, -0.0, np.inf, np.nan, 1e-40]
    nodes = [(0, 0, 0), (0, 1, 0), (2, 0, 1), (3, 2, 0), (4, 3, 1), (1, 0x3F000000, 0), (3, 4, 5)]
    got = oracle.expression_f32(nodes, [x0, x1])
    with np.errstate(all="ignore"):
        t = (x0 + x1) * x0 / x1 * np.float32(0.5)
    t = np.where(np.isnan(t), np.uint32(0x7FC00000).view(np.float32), t)
    assert np.array_equal(bits(got), bits(t))
    e = oracle.expression_f32([(0, 0, 0), (5, 0, 0)], [x0[5:200]])
    assert np.array_equal(bits(e), bits([oracle.certified_exp_f32(float(v)) for v in x0[5:200]]))
    pos = np.abs(x1[5:200])
    r = oracle.expression_f32([(0, 0, 0), (6, 0, 0)], [pos])
    assert np.array_equal(bits(r), bits([oracle.certified_rsqrt_f32(float(v)) for v in pos]))


def test_oracle_folds_against_the_pinned_strict_sum():
    rng = np.random.default_rng(93)
    x = rng.standard_normal((3, 5, 7, 2)).astype(np.float32)
    # one trailing axis: the strict_sum the reference's operand sets pin
    assert np.array_equal(bits(oracle.fold_f32(x, x.shape, (3,))), bits(oracle.strict_sum(x, x.shape, 3)))
    # several axes: the same fold over a transposed, flattened contributor axis
    mt = np.ascontiguousarray(x.transpose(1, 3, 0, 2)).reshape(5 * 2, 21)
    assert np.array_equal(bits(oracle.fold_f32(x, x.shape, (0, 2))), bits(oracle.strict_sum(mt, mt.shape, 1)))
    # squared and scale-bias prologues: the fold over the transformed values
    sq = (x * x).astype(np.float32)
    assert np.array_equal(bits(oracle.fold_f32(x, x.shape, (2,), op=1)), bits(oracle.strict_sum(sq, sq.shape, 2)))
    sb = (x * np.float32(2.0) + np.float32(1.0)).astype(np.float32)
    assert np.array_equal(bits(oracle.fold_f32(x, x.shape, (1, 2), op=2, scale_bits=0x40000000,
                                               bias_bits=0x3F800000)),
                          bits(oracle.strict_sum(np.ascontiguousarray(sb.transpose(0, 3, 1, 2)).reshape(6, 35),
                                                 (6, 35), 1)))
    # maximum: order-insensitive, so numpy's reduction gives the same value
    mx = oracle.fold_f32(x, x.shape, (1, 3), op=3)
    assert np.array_equal(mx, x.max(axis=(1, 3)).reshape(-1))
    z = np.array([-0.0, 0.0, -0.0], np.float32)
    assert bits(oracle.fold_f32(z, (3,), (0,), op=3))[0] == 0
    assert bits(oracle.fold_f32(np.array([1.0, np.nan, 2.0], np.float32), (3,), (0,), op=3))[0] == 0x7FC00000
    assert oracle.fold_f32(np.zeros((2, 0), np.float32), (2, 0), (1,)).tolist() == [0.0, 0.0]
