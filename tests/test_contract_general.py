"""CPU: contractions over general index structures (ADR 0087).

The oracle's general fold (oracle.contract_general, restating
tiler-reference/src/contraction.rs:346-715) is pinned by
* the td,od->to oracle, itself pinned by the reference's SHA-256 digests of
  the L3 profile cells (tests/test_oracle.py): bit-identical results;
* the two attention goldens' own index arithmetic
  (tiler-metal/goldens/contraction_attention_{score,value}.metal): the
  emitted kernels' per-invocation operand offsets, transcribed below as
  data, folded in the goldens' order -- which is what the reference's
  lowering of bhqd,bkd->bhqk and bhqk,bkd->bhqd computes;
* the strict serial sum (pinned by the reference's operand sets): a scalar
  contraction over two summed indices folds their products in ascending
  label order, whatever the operands' axis order;
and the planner's structural refusals and form selection are checked here.
"""
import numpy as np
import pytest

import oracle
from tiler_amd import _lib as L
from tiler_amd.realize import Refusal, realize

S = L.contraction_structure
RE = L.PERMITS_REASSOCIATION


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_general_oracle_is_the_strict_td_od_to_fold():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((37, 53)).astype(np.float32)
    b = rng.standard_normal((29, 53)).astype(np.float32)
    got = oracle.contract_general(a, "td", b, "od", "to")
    assert np.array_equal(bits(got), bits(oracle.contract_strict_f32(a, b, 37, 29, 53)))
    # storing the left operand [k, m] changes no contributor sequence
    assert np.array_equal(bits(oracle.contract_general(np.ascontiguousarray(a.T), "dt", b, "od", "to")), bits(got))


def test_general_oracle_folds_summed_indices_in_label_order():
    rng = np.random.default_rng(2)
    # +-2^25 adjacent in row-major order and 7 apart in column-major order:
    # the ones between them are absorbed in one order only (75 against 69)
    x = np.ones((7, 11), np.float32)
    x[0, 0], x[0, 1] = 2.0 ** 25, -(2.0 ** 25)
    y = np.where(rng.random((7, 11)) < 2, 1.0, 0.0).astype(np.float32)
    prod = (x * y).astype(np.float32)
    # labels a < b: a-major, the row-major order of [7, 11]
    want = oracle.strict_sum(prod.reshape(-1), (77,), 0)
    assert bits(oracle.contract_general(x, "ab", y, "ab", "")).item() == bits(want).item()
    # the same operands read as [b][a]: the fold is still a-major, i.e. column-major here
    want_t = oracle.strict_sum(np.ascontiguousarray(prod.T).reshape(-1), (77,), 0)
    assert bits(oracle.contract_general(x, "ba", y, "ba", "")).item() == bits(want_t).item()
    assert bits(want_t).item() != bits(want).item()  # the order is observable on these values


def test_general_oracle_reproduces_the_attention_goldens():
    rng = np.random.default_rng(3)
    # contraction_attention_score.metal: b0 48 elements, b1 40, b2 60; v0 < 60,
    # b0[(v0/30)*24 + ((v0/15)%2)*12 + ((v0/5)%3)*4 + d], b1[(v0/30)*20 + (v0%5)*4 + d], d in [0, 4)
    q = rng.standard_normal(48).astype(np.float32)
    k = rng.standard_normal(40).astype(np.float32)
    want = np.empty(60, np.float32)
    for v0 in range(60):
        acc = None
        for d in range(4):
            p = np.float32(q[(v0 // 30) * 24 + ((v0 // 15) % 2) * 12 + ((v0 // 5) % 3) * 4 + d] *
                           k[(v0 // 30) * 20 + (v0 % 5) * 4 + d])
            acc = p if acc is None else np.float32(acc + p)
        want[v0] = acc
    got = oracle.contract_general(q.reshape(2, 2, 3, 4), "bhqd", k.reshape(2, 5, 4), "bkd", "bhqk")
    assert got.shape == (2, 2, 3, 5) and np.array_equal(bits(got).reshape(-1), bits(want))
    # contraction_attention_value.metal: b0 60, b1 40, b2 48; v0 < 48,
    # b0[(v0/24)*30 + ((v0/12)%2)*15 + ((v0/4)%3)*5 + j], b1[(v0/24)*20 + j*4 + v0%4], j in [0, 5)
    pr = rng.standard_normal(60).astype(np.float32)
    v = rng.standard_normal(40).astype(np.float32)
    want = np.empty(48, np.float32)
    for v0 in range(48):
        acc = None
        for j in range(5):
            p = np.float32(pr[(v0 // 24) * 30 + ((v0 // 12) % 2) * 15 + ((v0 // 4) % 3) * 5 + j] *
                           v[(v0 // 24) * 20 + j * 4 + v0 % 4])
            acc = p if acc is None else np.float32(acc + p)
        want[v0] = acc
    got = oracle.contract_general(pr.reshape(2, 2, 3, 5), "bhqk", v.reshape(2, 5, 4), "bkd", "bhqd")
    assert got.shape == (2, 2, 3, 4) and np.array_equal(bits(got).reshape(-1), bits(want))


def test_general_oracle_bf16_is_the_widened_f32_fold_narrowed_once():
    rng = np.random.default_rng(4)
    a = oracle.bf16_narrow(rng.standard_normal((3, 5, 24)).astype(np.float32))
    b = oracle.bf16_narrow(rng.standard_normal((3, 7, 24)).astype(np.float32))
    wide = oracle.contract_general(oracle.bf16_widen(a), "bmk", oracle.bf16_widen(b), "bnk", "bmn")
    assert np.array_equal(oracle.contract_general(a, "bmk", b, "bnk", "bmn"), oracle.bf16_narrow(wide))
    silu = oracle.contract_general(a, "bmk", b, "bnk", "bmn", silu=True)
    assert np.array_equal(silu, oracle.bf16_narrow(oracle.silu_f32(wide)))


@pytest.mark.parametrize("structure,why", [
    (S("ab", (2, 3), "cb", (4, 3), "ad"), "an output index in no operand"),
    (S("ab", (2, 3), "cd", (4, 5), "ac"), "a summed index in one operand"),
    (S("aa", (2, 2), "ab", (2, 3), "b"), "an index repeated within an operand"),
    (S("ab", (2, 3), "cb", (4, 3), "aa"), "a duplicate output index"),
    (S("ab", (2, 3), "ab", (2, 3), "ab"), "no summed index"),
    (S("ab", (2, 3), "cb", (4, 4), "ac"), "one index with two extents"),
    (S("ab", (2, 0), "cb", (4, 0), "ac"), "empty contracted domain"),
])
def test_structural_rules_refuse(structure, why):
    for dtype in (L.F32, L.BF16):
        with pytest.raises(Refusal) as e:
            realize(L.PROGRAM_CONTRACTION, (), dtype=dtype, structure=structure, permissions=RE)
        assert e.value.status == L.REFUSE_INVALID_ARGUMENT and why in str(e.value)
    with pytest.raises(Refusal):
        oracle_structure = structure  # the oracle refuses the same structures
        li = [chr(c) for c in oracle_structure.operand_indices[0][:oracle_structure.operand_rank[0]]]
        ri = [chr(c) for c in oracle_structure.operand_indices[1][:oracle_structure.operand_rank[1]]]
        oi = [chr(c) for c in oracle_structure.output_indices[:oracle_structure.output_rank]]
        ld = tuple(oracle_structure.operand_dims[0][:len(li)])
        rd = tuple(oracle_structure.operand_dims[1][:len(ri)])
        try:
            oracle.contract_general(np.zeros(ld, np.float32), "".join(li), np.zeros(rd, np.float32), "".join(ri),
                                    "".join(oi))
        except RuntimeError as err:
            raise Refusal(L.REFUSE_INVALID_ARGUMENT, "oracle", str(err))


def test_other_refusals():
    sc = S("mk", (4, 8), "nk", (5, 8), "mn")
    with pytest.raises(Refusal):  # the f32 family has no epilogue
        realize(L.PROGRAM_CONTRACTION, (), dtype=L.F32, structure=sc, variant=L.EPILOGUE_SILU)
    sc.reserved = 1
    with pytest.raises(Refusal):
        realize(L.PROGRAM_CONTRACTION, (), dtype=L.F32, structure=sc)
    wide = S("abcdefgh", (1,) * 8, "h", (1,), "a")
    wide.operand_rank[0] = 9  # more axes than a tuple holds
    with pytest.raises(Refusal):
        realize(L.PROGRAM_CONTRACTION, (), dtype=L.F32, structure=wide)


def test_form_selection():
    def symbols(structure, dtype=L.BF16, permissions=RE, **kw):
        return realize(L.PROGRAM_CONTRACTION, (), dtype=dtype, structure=structure, permissions=permissions,
                       **kw).symbols
    score = S("bhqd", (2, 32, 1024, 128), "bkd", (2, 1024, 128), "bhqk")
    value = S("bhqk", (2, 32, 1024, 1024), "bkd", (2, 1024, 128), "bhqd")
    # the strict fold: f32, and bf16 without the reassociation permission
    assert symbols(score, L.F32, 0) == ["tiler_contract_general_f32"]
    assert symbols(score, L.F32) == ["tiler_contract_general_f32"]  # f32 has no MFMA form
    assert symbols(score, permissions=0) == ["tiler_contract_general_bf16"]
    assert symbols(score, permissions=0, variant=L.EPILOGUE_SILU) == ["tiler_contract_general_bf16_silu"]
    # MFMA: K shared across heads (batch stride 0); V stored [k, n] transposed first
    rz = realize(L.PROGRAM_CONTRACTION, (), dtype=L.BF16, structure=score, permissions=RE)
    assert rz.symbols == ["tiler_contract_bf16_t256_b"] and rz.dispatches[0].grid[:2] == (16, 64)
    rz = realize(L.PROGRAM_CONTRACTION, (), dtype=L.BF16, structure=value, permissions=RE)
    assert rz.symbols == ["tiler_transpose_bf16", "tiler_contract_bf16_t128_b"]
    assert rz.slots[3] == (L.SLOT_SCRATCH, 2 * 1024 * 128 * 2)
    assert symbols(S("bhqd", (1, 32, 1, 128), "bkd", (1, 4096, 128), "bhqk")) == ["tiler_contract_bf16_skinny1_b"]
    assert symbols(S("bhqd", (2, 3, 5, 7), "bkd", (2, 9, 7), "bhqk")) == ["tiler_contract_bf16_g128_k_b"]
    assert symbols(S("bmk", (3, 300, 64), "bnk", (3, 200, 64), "bmn"),
                   variant=L.EPILOGUE_SILU) == ["tiler_contract_bf16_silu_t128_b"]
    # not [.., m, k] x [.., n|k, k|n] -> [.., m, n]: the strict fold
    assert symbols(S("km", (64, 32), "nk", (16, 64), "mn")) == ["tiler_contract_general_bf16"]
    assert symbols(S("mk", (32, 64), "nk", (16, 64), "nm")) == ["tiler_contract_general_bf16"]
    assert symbols(S("abk", (4, 5, 6), "bk", (5, 6), "a")) == ["tiler_contract_general_bf16"]
    # more batches than the launch grid's second dimension: the strict fold
    assert symbols(S("bmk", (70000, 2, 8), "bnk", (70000, 2, 8), "bmn")) == ["tiler_contract_general_bf16"]
    # the strict form's geometry travels in a constant slot
    rz = realize(L.PROGRAM_CONTRACTION, (), dtype=L.F32, structure=score)
    assert rz.slots[3][0] == L.SLOT_CONSTANT and rz.raw.constant_bytes == rz.slots[3][1]


def test_contraction_under_modes_closed_forms():
    """contraction.rs:600-625 under the modes, on closed forms: a subnormal
    product of normal factors (only the result mode reaches it); a subnormal
    factor (the input mode); products that cancel to a subnormal sum; the
    seed is the first product, which a flushing result mode still meets."""
    PRE, FS, FP = oracle.PRESERVE, oracle.FLUSH_SIGN_PRESERVING, oracle.FLUSH_POSITIVE_ZERO
    t = np.float32(2.0 ** -70)
    a = np.array([[t]], np.float32)
    b = np.array([[-t]], np.float32)
    got = lambda im, rm: int(bits(oracle.contract_general(a, "mk", b, "nk", "mn", input_mode=im, result_mode=rm))[0])
    assert got(PRE, PRE) == 0x80000200            # -2^-140 = -(2^9 quanta): a subnormal product
    assert got(FS, PRE) == 0x80000200             # no factor is subnormal
    assert got(PRE, FS) == 0x80000000 and got(PRE, FP) == 0x00000000
    sub = np.array([[np.uint32(0x00000100).view(np.float32)]], np.float32)
    two = np.array([[2.0]], np.float32)
    assert int(bits(oracle.contract_general(sub, "mk", two, "nk", "mn"))[0]) == 0x00000200
    assert int(bits(oracle.contract_general(sub, "mk", two, "nk", "mn", input_mode=FS))[0]) == 0
    # (2^-126 (1 + 2^-23)) * 1 + (-2^-126) * 1: a normal seed, a Sterbenz difference 2^-149
    a2 = np.array([[np.uint32(0x00800001).view(np.float32), np.uint32(0x80800000).view(np.float32)]], np.float32)
    one = np.ones((1, 2), np.float32)
    assert int(bits(oracle.contract_general(a2, "mk", one, "nk", "mn"))[0]) == 0x00000001
    assert int(bits(oracle.contract_general(a2, "mk", one, "nk", "mn", result_mode=FS))[0]) == 0x00000000
    # the same bits as the strict f32 oracle under the preserving modes
    rng = np.random.default_rng(9)
    x, y = rng.standard_normal((5, 7)).astype(np.float32), rng.standard_normal((6, 7)).astype(np.float32)
    assert np.array_equal(bits(oracle.contract_general(x, "mk", y, "nk", "mn")),
                          bits(oracle.contract_strict_f32(x, y, 5, 6, 7)))
