"""Pins the CPU oracle (oracle/tiler_oracle.c) before anything is compared to it.

Every family is checked against the reference's own golden vectors
(tests/golden/reference_vectors.json) and, where those leave a function open,
against what the mathematics fixes: exact integer midpoint tests for the
reciprocal square root, a 60-digit decimal exponential, exact rational sums,
brute-force groupings.  Each check is chosen so a plausible mistake (a dropped
term, a swapped association, division instead of reciprocal multiply, a
number-preferring maximum, FMA contraction) fails it.
"""
from __future__ import annotations

import decimal
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from helpers import (bits, expected_bits, f32, golden, hexbits, sha256_le_f32,
                     splitmix_operands, splitmix_scalar, values_of)

G = golden()


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


# -- rms_norm ---------------------------------------------------------------------

@pytest.mark.parametrize("case", G["rms_norm"]["cases"], ids=lambda c: c["name"])
def test_rms_norm_golden(case):
    x = values_of(case, "x")
    w = values_of(case, "w")
    eps = hexbits(G["rms_norm"]["eps_bits"])
    y = oracle.rms_norm_f32(x, w, case["shape"], case["axis"], eps)
    assert list(bits(y)) == list(expected_bits(case))


def test_rms_norm_worked_example_intermediates():
    case = G["rms_norm"]["cases"][0]
    inter = case["intermediates"]
    sq = np.float32(3.0) * np.float32(3.0), np.float32(4.0) * np.float32(4.0)
    total = np.float32(sq[0] + sq[1])
    assert bits([total])[0] == hexbits(inter["total"])
    mean = np.float32(total / np.float32(2.0))
    arg = np.float32(mean + f32([G["rms_norm"]["eps_bits"]])[0])
    assert bits([arg])[0] == hexbits(inter["argument"])
    assert bits([oracle.certified_rsqrt_f32(arg)])[0] == hexbits(inter["scale"])


def test_rms_norm_holed_rows_and_extents():
    hr = G["rms_norm"]["holed_rows"]
    eps = hexbits(G["rms_norm"]["eps_bits"])
    for key in ("extent_1024", "extent_128"):
        n = int(key.split("_")[1])
        x = np.full(n, hr[key]["fill"], np.float32)
        y_uniform = oracle.rms_norm_f32(x, np.ones(n, np.float32), (1, n), 1, eps)
        assert np.all(bits(y_uniform) == 0x3F800000)
        x[hr[key]["hole"]] = 0.0
        y = oracle.rms_norm_f32(x, np.ones(n, np.float32), (1, n), 1, eps)
        assert bits(y)[0] == hexbits(hr[key]["first_bits"])
        assert bits(y)[hr[key]["hole"]] == 0


def test_rms_norm_weight_after_normalize_discriminates():
    case = G["rms_norm"]["weight_after_normalize"]
    x = np.asarray(case["x"], np.float32)
    w = np.asarray(case["w"], np.float32)
    eps = hexbits(G["rms_norm"]["eps_bits"])
    y = oracle.rms_norm_f32(x, w, (1, 2), 1, eps)
    total = np.float32(np.float32(9.0) + np.float32(16.0))
    s = oracle.certified_rsqrt_f32(np.float32(total / np.float32(2.0) + f32([eps])[0]))
    want = [np.float32(w[i] * np.float32(x[i] * s)) for i in range(2)]
    other = [np.float32(np.float32(w[i] * x[i]) * s) for i in range(2)]
    assert list(bits(y)) == list(bits(want))
    assert list(bits(want)) != list(bits(other)), "the corpus must separate the associations"


def test_rms_norm_axis_and_refusals():
    eps = hexbits(G["rms_norm"]["eps_bits"])
    v = np.arange(1, 7, dtype=np.float32)
    rows = oracle.rms_norm_f32(v, np.ones(6, np.float32), (2, 3), 1, eps)
    cols = oracle.rms_norm_f32(v, np.ones(6, np.float32), (2, 3), 0, eps)
    assert list(bits(rows)) != list(bits(cols))
    for bad in G["rms_norm"]["bad_eps_bits"]:
        with pytest.raises(oracle.OracleError):
            oracle.rms_norm_f32([1.0, 2.0], [1.0, 1.0], (1, 2), 1, hexbits(bad))


# -- certified rsqrt, pinned by exact integer arithmetic ------------------------------

def _exact_rsqrt_rounds_to(t: float, c: float) -> bool:
    """True iff c is the correctly rounded binary32 of 1/sqrt(t), decided with
    exact rationals: m^2 * t compared with 1 at both neighbouring midpoints."""
    ft = Fraction(float(t))
    cb = int(bits([c])[0])
    lo = Fraction(float(f32([cb - 1])[0]))
    hi = Fraction(float(f32([cb + 1])[0]))
    fc = Fraction(float(c))
    m_lo, m_hi = (fc + lo) / 2, (fc + hi) / 2
    # 1/sqrt(t) > m  <=>  m^2 * t < 1
    return m_lo * m_lo * ft < 1 < m_hi * m_hi * ft


def test_rsqrt_golden_rows():
    g = G["rsqrt"]
    eps = f32([G["rms_norm"]["eps_bits"]])[0]
    assert bits([oracle.certified_rsqrt_f32(eps)])[0] == hexbits(g["eps_bits_to"])
    composed = np.float32(np.float32(1.0) / np.sqrt(eps))
    assert bits([composed])[0] == hexbits(g["two_rounding_composition_at_eps"])
    for a, b in g["exact"]:
        av = f32([a])[0] if a.startswith("0x") else np.float32(float(a))
        bv = f32([b])[0] if b.startswith("0x") else np.float32(float(b))
        assert bits([oracle.certified_rsqrt_f32(av)])[0] == bits([bv])[0]
    assert math.isnan(oracle.certified_rsqrt_f32(np.float32("nan")))
    assert bits([oracle.certified_rsqrt_f32(np.float32("inf"))])[0] == 0
    assert bits([oracle.certified_rsqrt_f32(np.float32(0.0))])[0] == 0x7F800000
    assert bits([oracle.certified_rsqrt_f32(np.float32(-0.0))])[0] == 0xFF800000
    assert math.isnan(oracle.certified_rsqrt_f32(np.float32(-1.0)))


def test_rsqrt_matches_exact_midpoint_decision_on_a_sweep():
    rng = np.random.default_rng(7)
    sweep = list(range(0x3F800000, 0x3F800000 + 512))          # rms_norm/tests.rs:136-158 band
    sweep += list(rng.integers(0x00000001, 0x7F7FFFFF, 3000))   # all finite positive classes
    for b in sweep:
        t = f32([b])[0]
        c = oracle.certified_rsqrt_f32(t)
        assert _exact_rsqrt_rounds_to(t, c), hex(b)


# -- certified exp / silu, pinned by a 60-digit decimal exponential -------------------

def _decimal_exp_rounds_to(t: float, c: float) -> bool:
    with decimal.localcontext() as dc:
        dc.prec = 60
        e = decimal.Decimal(float(t)).exp()
        cb = int(bits([c])[0])
        fc = decimal.Decimal(float(c))
        if c == 0:
            lo_mid = decimal.Decimal(0)
        else:
            lo_mid = (fc + decimal.Decimal(float(f32([cb - 1])[0]))) / 2
        hi_mid = (fc + decimal.Decimal(float(f32([cb + 1])[0]))) / 2
        return lo_mid < e < hi_mid or (c == 0 and e < hi_mid)


def test_exp_matches_decimal_reference_on_a_sweep():
    rng = np.random.default_rng(11)
    args = rng.uniform(-103.9, 88.7, 2500).astype(np.float32)
    args = np.concatenate([args, rng.uniform(-1, 1, 500).astype(np.float32),
                           f32(["0xc2cff1b5", "0xc2aeac50", "0x42b17217", "0xc2b00000"])])
    for t in args:
        c = oracle.certified_exp_f32(t)
        assert _decimal_exp_rounds_to(t, c), hex(int(bits([t])[0]))


def test_exp_guards_and_golden_values():
    assert oracle.certified_exp_f32(np.float32(89.0)) == np.inf
    assert bits([oracle.certified_exp_f32(np.float32(-104.0))])[0] == 0
    assert bits([oracle.certified_exp_f32(np.float32(0.0))])[0] == 0x3F800000
    assert bits([oracle.certified_exp_f32(np.float32(-0.0))])[0] == 0x3F800000
    th = G["softmax"]["thresholds"]
    assert bits([oracle.certified_exp_f32(f32([th["exp_zero_at"]])[0])])[0] == 0
    sub = oracle.certified_exp_f32(f32([th["exp_subnormal_at"]])[0])
    assert 0 < bits([sub])[0] < 0x00800000
    ex = G["softmax"]["cases"][0]["intermediates"]["exp"]
    for t, want in zip([-2.0, -1.0, 0.0], ex):
        assert bits([oracle.certified_exp_f32(np.float32(t))])[0] == hexbits(want)


def test_silu_boundary_corpus():
    corpus = G["silu"]["corpus"]
    x = f32([a for a, _ in corpus])
    y = oracle.silu_f32(x)
    assert [int(v) for v in bits(y)] == [hexbits(b) for _, b in corpus]


# -- softmax -----------------------------------------------------------------------

@pytest.mark.parametrize("case", G["softmax"]["cases"], ids=lambda c: c["name"])
def test_softmax_golden(case):
    x = values_of(case, "x")
    axis = case.get("axis", 1)
    y = oracle.softmax_f32(x, case["shape"], axis)
    assert list(bits(y)) == list(expected_bits(case))


def test_softmax_reciprocal_form_not_division():
    y = oracle.softmax_f32([0.0, 2.0], (1, 2), 1)
    e = [oracle.certified_exp_f32(np.float32(-2.0)), oracle.certified_exp_f32(np.float32(0.0))]
    d = np.float32(e[0] + e[1])
    r = np.float32(np.float32(1.0) / d)
    assert list(bits(y)) == list(bits([np.float32(v * r) for v in e]))
    assert any(bits([np.float32(v / d)])[0] != bits([np.float32(v * r)])[0] for v in e)


def test_maximum_rows_and_family():
    for a, b, want in G["softmax"]["maximum"]["rows"]:
        assert bits([oracle.maximum_f32(f32([a])[0], f32([b])[0])])[0] == hexbits(want)
    assert math.isnan(oracle.maximum_f32(np.float32("nan"), np.float32(1.0)))
    assert math.isnan(oracle.maximum_f32(np.float32(1.0), np.float32("nan")))


def test_softmax_empty_rows():
    assert oracle.softmax_f32(np.zeros(0, np.float32), (2, 0), 1).size == 0
    assert oracle.softmax_f32(np.zeros(0, np.float32), (0, 4), 1).size == 0


# -- sums ---------------------------------------------------------------------------

def test_serial_sum_operand_sets():
    s = G["serial_sum"]
    assert bits(oracle.strict_sum(f32(s["parallel_operands"]), (4,), 0))[0] == hexbits(s["parallel_sum"])
    gs = f32(s["grouping_sensitive_operands"])
    assert bits(oracle.strict_sum(gs, (4,), 0))[0] == hexbits(s["grouping_sensitive_serial"])
    assert bits(oracle.strict_partitioned_sum(gs, 1, 4, 2, 2))[0] == hexbits(s["grouping_sensitive_pairwise"])
    sep = f32(s["separating_operands"])
    assert bits(oracle.strict_partitioned_sum(sep, 1, 12, 6, 2))[0] == hexbits(s["separating_tree_6x2"])
    assert bits(oracle.strict_partitioned_sum(sep, 1, 12, 4, 3))[0] == hexbits(s["separating_split_4x3"])
    ex = f32(s["separating_exact_operands"])
    for p, c in [(1, 12), (2, 6), (3, 4), (4, 3), (6, 2), (12, 1)]:
        assert bits(oracle.strict_partitioned_sum(ex, 1, 12, p, c))[0] == hexbits(s["separating_exact_sum"])


def test_partitioned_sum_refuses_inexact_cover_and_matches_cooperative_single_round():
    x = np.arange(12, dtype=np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.strict_partitioned_sum(x, 1, 12, 5, 2)
    sep = f32(G["serial_sum"]["separating_operands"])
    a = oracle.strict_partitioned_sum(sep, 1, 12, 6, 2)
    b = oracle.cooperative_grouped_sum(sep, 1, 12, 6, 2, 1)
    assert bits(a)[0] == bits(b)[0]  # evaluate.rs:526-528


def test_cooperative_layouts_separate():
    # RoundMajor and ParticipantMajor fold the same cells in different orders.
    rng = np.random.default_rng(3)
    x = rng.standard_normal(2 * 3 * 4).astype(np.float32) * np.float32(1e3)
    x[0] = np.float32(1e8)
    rm = oracle.cooperative_grouped_sum(x, 1, 24, 3, 2, 4, oracle.ROUND_MAJOR)
    pm = oracle.cooperative_grouped_sum(x, 1, 24, 3, 2, 4, oracle.PARTICIPANT_MAJOR)
    exact = float(sum(Fraction(float(v)) for v in x))
    assert abs(float(rm[0]) - exact) < 64 and abs(float(pm[0]) - exact) < 64
    # brute force the declared RoundMajor order
    acc = None
    for r in range(4):
        staged = None
        for p in range(3):
            cell = r * 3 + p
            part = x[cell * 2]
            part = np.float32(part + x[cell * 2 + 1])
            staged = part if staged is None else np.float32(staged + part)
        acc = staged if acc is None else np.float32(acc + staged)
    assert bits([acc])[0] == bits(rm)[0]


def test_flush_example_under_modes():
    fe = G["serial_sum"]["flush_example"]
    x = f32(fe["operands"])
    keep = oracle.strict_partial_sums(x, 1, 4, 2, 2)
    flush = oracle.strict_partial_sums(x, 1, 4, 2, 2, result_mode=oracle.FLUSH_SIGN_PRESERVING)
    assert [hex(v) for v in bits(keep)] == [hex(hexbits(v)) for v in fe["preserve_2x2"]]
    assert [hex(v) for v in bits(flush)] == [hex(hexbits(v)) for v in fe["flush_2x2"]]
    assert list(bits(oracle.strict_partial_sums(x, 1, 4, 4, 1))) == [hexbits(v) for v in fe["operands"]]


def test_row_patterns_strict_sum_canonicalizes_nan():
    rows = G["serial_sum"]["row_patterns"]
    x = f32([b for r in rows for b in r])
    s = bits(oracle.strict_sum(x, (4, 3), 1))
    assert s[0] == 0x40C00000  # 6.0
    assert s[1] == 0x3F800000  # -0 + least subnormal + 1 = 1
    assert s[2] == 0x7FC00000  # non-canonical NaN -> canonical
    assert s[3] == 0x7F800000  # inf + 1 - 1


def test_empty_sum_is_positive_zero():
    assert bits(oracle.strict_sum(np.zeros(0, np.float32), (3, 0), 1)).tolist() == [0, 0, 0]


# -- grouped restatements of the device kernels --------------------------------------

def test_row_grouping_on_exact_sets_and_separating_set():
    ex = f32(G["serial_sum"]["separating_exact_operands"])
    for vec, waves in [(1, 1), (4, 1), (8, 1), (4, 4)]:
        assert bits(oracle.row_grouped_sum(ex, 1, 12, vec, waves))[0] == 0x457FF000
    # vec 2, one wave: lanes hold pairs (a0+a1), (a2+a3): the pairwise value
    gs = f32(G["serial_sum"]["grouping_sensitive_operands"])
    assert bits(oracle.row_grouped_sum(gs, 1, 4, 2, 1))[0] == 0x3F800001
    # vec 4: one lane folds all four serially: the strict value
    assert bits(oracle.row_grouped_sum(gs, 1, 4, 4, 1))[0] == 0x3F800000


def test_row_grouping_brute_force():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(777) * 1e4).astype(np.float32)
    vec, waves = 4, 1
    part = [np.float32(-0.0)] * 64
    for p in range(777):
        t = (p // vec) % 64
        part[t] = np.float32(part[t] + x[p])
    v = list(part)
    for o in (32, 16, 8, 4, 2, 1):
        v = [np.float32(v[l] + v[l ^ o]) for l in range(64)]
    assert bits([v[0]])[0] == bits(oracle.row_grouped_sum(x, 1, 777, vec, waves))[0]


def test_grid_tree_sum_exact_on_integers_and_close_to_f64():
    x = np.arange(1, 100001, dtype=np.float32) % np.float32(97)
    exact = float(np.sum(x.astype(np.float64)))
    for blocks in (1, 3, 64, 1024):
        assert float(oracle.grid_tree_sum(x, blocks)) == exact
    rng = np.random.default_rng(1)
    y = rng.uniform(-1, 1, 1 << 20).astype(np.float32)
    ref = float(np.sum(y.astype(np.float64)))
    got = float(oracle.grid_tree_sum(y, 1024))
    assert abs(got - ref) <= 1e-5 * abs(ref)


def test_grouped_rms_and_softmax_agree_with_strict_on_exact_inputs():
    eps = hexbits(G["rms_norm"]["eps_bits"])
    x = np.full(1024, 32.0, np.float32)
    y = oracle.rms_norm_grouped(x, np.ones(1024, np.float32), 1, 1024, eps, True, 8, 1)
    assert np.all(bits(y) == 0x3F800000)
    x = np.full(10 * 16, np.float32(0.25))
    y = oracle.softmax_grouped(x, 16, 10, 4, 1)
    assert np.all(bits(y) == 0x3DCCCCCD)


def test_segmented_softmax_composes_the_pinned_fold():
    # Each segment's partial is the pinned row-grouped fold of its exponents;
    # the row total is their left fold; the scaling is softmax.rs's.
    rng = np.random.default_rng(17)
    rows, extent, seg = 2, 20000, 8192
    x = (rng.standard_normal((rows, extent)) * 3).astype(np.float32)
    got = oracle.softmax_grouped(x, rows, extent, 4, 4, seg).reshape(rows, extent)
    for r in range(rows):
        m = x[r, 0]
        for v in x[r, 1:]:
            m = oracle.maximum_f32(m, v)
        e = np.array([oracle.certified_exp_f32(np.float32(v - np.float32(m))) for v in x[r]], np.float32)
        d = None
        for s0 in range(0, extent, seg):
            part = oracle.row_grouped_sum(e[s0:s0 + seg], 1, min(seg, extent - s0), 4, 4)[0]
            d = part if d is None else np.float32(d + part)
        want = e * (np.float32(1.0) / d)
        assert np.array_equal(bits(got[r]), bits(want))


def test_segmented_softmax_special_cases():
    rng = np.random.default_rng(18)
    x = (rng.standard_normal((3, 9000)) * 4).astype(np.float32)
    whole = oracle.softmax_grouped(x, 3, 9000, 4, 4)
    # a segment at least the row, or 0, is the unsegmented fold
    assert np.array_equal(bits(oracle.softmax_grouped(x, 3, 9000, 4, 4, 9000)), bits(whole))
    assert np.array_equal(bits(oracle.softmax_grouped(x, 3, 9000, 4, 4, 1 << 20)), bits(whole))
    assert np.array_equal(bits(oracle.softmax_grouped(x, 3, 9000, 4, 4, 0)), bits(whole))
    # and a real split changes the association (on these seeds, some bit)
    split = oracle.softmax_grouped(x, 3, 9000, 4, 4, 4096)
    assert not np.array_equal(bits(split), bits(whole))
    assert np.max(np.abs(split.astype(np.float64) - whole) / whole) < 1e-5
    # exact inputs: every grouping gives the exact quotient
    c = np.full((2, 20000), np.float32(0.5))
    assert np.all(bits(oracle.softmax_grouped(c, 2, 20000, 4, 4, 8192)) == bits(np.float32(1 / 20000))[()])


# -- gather ---------------------------------------------------------------------------

def _geometry(shape, axis):
    outer = int(np.prod(shape[:axis])) if axis else 1
    inner = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
    return outer, shape[axis], inner


@pytest.mark.parametrize("case", G["gather"]["cases"], ids=lambda c: c["name"])
def test_gather_golden(case):
    shape = case["source_shape"]
    src = np.arange(int(np.prod(shape)), dtype=np.uint32)
    outer, gathered, inner = _geometry(shape, case["axis"])
    out, err = oracle.gather(src, outer, gathered, inner, np.asarray(case["index"], np.uint32))
    assert err is None
    assert out.tolist() == case["result"]


@pytest.mark.parametrize("ref", G["gather"]["refusals"], ids=lambda r: str(r["index"]))
def test_gather_refusals(ref):
    src = np.arange(15, dtype=np.uint32)
    out, err = oracle.gather(src, 1, 5, 3, np.asarray(ref["index"], np.uint32))
    assert out is None and err == (ref["position"], ref["value"])


def test_gather_signed_index_refuses_negative_and_preserves_payloads():
    src = np.arange(15, dtype=np.uint32)
    out, err = oracle.gather(src, 1, 5, 3, np.asarray([1, -1], np.int32).view(np.uint32),
                             index_signed=True)
    assert out is None and err == (1, -1)
    p = G["gather"]["payloads"]
    srcb = np.asarray([hexbits(b) for b in p["source_bits"]], np.uint32)
    out, err = oracle.gather(srcb, 1, 4, 1, np.asarray(p["index"], np.uint32))
    assert [int(v) for v in out] == [hexbits(b) for b in p["result_bits"]]


# -- strict contraction, pinned by the reference's six device digests ----------------

def test_sha256_helper_vectors():
    import hashlib
    for msg, digest in G["contraction"]["sha256_vectors"].items():
        assert hashlib.sha256(msg.encode()).hexdigest() == digest


def test_splitmix_stream_matches_scalar_definition():
    seed = hexbits(G["contraction"]["workload_seed"])
    v = splitmix_operands(seed, 64)
    for i in (0, 1, 5, 63):
        assert float(v[i]) == splitmix_scalar(seed, i)


@pytest.mark.parametrize("cell", G["contraction"]["cells"], ids=lambda c: c["id"])
def test_strict_contraction_reproduces_reference_digests(cell):
    seed = hexbits(G["contraction"]["workload_seed"])
    mask = hexbits(G["contraction"]["right_seed_mask"])
    a = splitmix_operands(seed, cell["m"] * cell["k"])
    b = splitmix_operands(seed ^ mask, cell["n"] * cell["k"])
    c = oracle.contract_strict_f32(a, b, cell["m"], cell["n"], cell["k"])
    assert sha256_le_f32(c) == cell["sha256"]


def test_strict_contraction_is_not_fma_and_seeds_at_first_product():
    # A perturbed oracle (FMA, or a +0.0 seed) would change these values.
    a = np.asarray([[1.0 + 2 ** -12, -0.0]], np.float32)
    b = np.asarray([[1.0 - 2 ** -12, -0.0], [-0.0, 0.0]], np.float32)
    c = oracle.contract_strict_f32(a, b, 1, 2, 2)
    p = np.float32(np.float32(a[0, 0]) * np.float32(b[0, 0]))
    assert bits(c)[0, 0] == bits([np.float32(p + np.float32(0.0))])[0]
    # products (1+2^-12)*-0 = -0 and -0*0 = -0: first-product seeding keeps -0,
    # a +0.0 seed would give +0
    assert bits(c)[0, 1] == 0x80000000
    c2 = oracle.contract_strict_f32(np.asarray([[-0.0]], np.float32),
                                    np.asarray([[1.0]], np.float32), 1, 1, 1)
    assert bits(c2)[0, 0] == 0x80000000  # first-product seed keeps -0


# -- bf16 narrowing (ADR 0091 decision 2), checked against exact rational rounding ------

def _rne_bf16_exact(v: float) -> int:
    if math.isnan(v):
        return 0x7FC0
    if math.isinf(v):
        return 0x7F80 if v > 0 else 0xFF80
    sign = 0x8000 if math.copysign(1.0, v) < 0 else 0
    fv = Fraction(abs(v))
    if fv == 0:
        return sign
    best = None
    # candidates: bf16 values around v
    b32 = int(bits([np.float32(abs(v))])[0])
    for cand in range((b32 >> 16) - 1, (b32 >> 16) + 2):
        if cand < 0 or cand > 0x7F80:
            continue
        cv = Fraction(float(f32([cand << 16])[0])) if cand < 0x7F80 else None
        if cv is None:
            continue
        d = abs(cv - fv)
        if best is None or d < best[0] or (d == best[0] and cand % 2 == 0):
            best = (d, cand)
    # overflow: at or above the midpoint between max finite and 2^128
    maxf = Fraction(float(f32([0x7F7F0000])[0]))
    if fv >= maxf + (Fraction(2) ** 128 - maxf) / 2:
        return sign | 0x7F80
    return sign | best[1]


def test_bf16_narrowing_matches_exact_rounding():
    rng = np.random.default_rng(9)
    pats = list(rng.integers(0, 1 << 32, 4000, dtype=np.uint64).astype(np.uint32))
    pats += [0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7F8000, 0x7F7F7FFF, 0x7F7FFFFF,
             0x00008000, 0x00018000, 0x0000FFFF, 0x80008000, 0x7FC01234, 0xFF800001, 0x80000000]
    vals = f32(pats)
    got = oracle.bf16_narrow(vals)
    for p, v, g in zip(pats, vals, got):
        assert int(g) == _rne_bf16_exact(float(v)), hex(int(p))
    assert np.array_equal(bits(oracle.bf16_widen(got)), np.asarray([int(g) << 16 for g in got], np.uint32))


# --- strict-affine U4 dequantization ------------------------------------------

def test_dequantize_u4_reference_rows():
    g = golden()["strict_affine_u4"]
    for row in g["dequantize_one"]:
        packed = oracle.pack_u4([row["code"]])
        got = oracle.dequantize_u4(packed, 1, int(row["scale_bits"], 16), row["zero_point"])
        assert int(bits(got)[0]) == hexbits(row["value_bits"]), row["source"]


def test_dequantize_u4_scale_and_zero_point_domain():
    g = golden()["strict_affine_u4"]
    packed = oracle.pack_u4([7, 8])
    for b in g["invalid_scale_bits"]["bits"]:
        assert oracle.strict_affine_domain(int(b, 16), 8) == 1, b
        with pytest.raises(ValueError):
            oracle.dequantize_u4(packed, 2, int(b, 16), 8)
    assert oracle.strict_affine_domain(int(g["smallest_normal_scale_bits"]["bits"], 16), 8) == 0
    assert oracle.strict_affine_domain(0x3F000000, 15) == 0
    assert oracle.strict_affine_domain(0x3F000000, 16) == 2
    assert oracle.strict_affine_domain(0x7F7FFFFF, 0) == 0  # the largest finite scale is normal


def test_dequantize_u4_packing_is_lsb_first_with_a_zero_tail():
    g = golden()["strict_affine_u4"]["packing"]
    carriers = np.array([int(c, 16) for c in g["carriers"]], np.uint8)
    assert np.array_equal(oracle.pack_u4(g["codes"]), carriers)
    got = oracle.dequantize_u4(carriers, 3, 0x3F800000, 0)
    assert got.tolist() == [float(c) for c in g["codes"]]


@pytest.mark.parametrize("scale_bits", [0x00800000, 0x3F000000, 0x3DCCCCCD, 0x7F7FFFFF, 0x7E800001, 0x0E5A3C11])
def test_dequantize_u4_every_code_and_zero_point_is_one_rounding(scale_bits):
    """All 16 codes x 16 zero points: the difference is an exact integer, its
    product with the scale is exact in binary64 (5 + 24 significant bits), so
    one rounding of that product to binary32 is the IEEE product; the zero
    point's own code is +0.0; at the smallest normal scale every value is +0.0
    or normal (quantization.rs:687-703)."""
    scale = np.uint32(scale_bits).view(np.float32)
    codes = np.tile(np.arange(16, dtype=np.uint8), 1)
    for zp in range(16):
        got = oracle.dequantize_u4(oracle.pack_u4(codes), 16, scale_bits, zp)
        diff = codes.astype(np.int64) - zp
        with np.errstate(over="ignore"):
            want = (diff.astype(np.float64) * np.float64(scale)).astype(np.float32)
        want[diff == 0] = np.float32(0.0)  # +0.0, never -0.0
        assert np.array_equal(bits(got), bits(want)), (hex(scale_bits), zp)
        if scale_bits == 0x00800000:
            assert all(v == 0 or (np.isfinite(v) and abs(v) >= np.finfo(np.float32).tiny) for v in got)


def test_dequantize_u4_a_planted_mistake_fails_the_exhaustive_check():
    """The independent formula of the exhaustive check separates the
    reference's decode from two plausible mistakes: the high nibble taken
    first, and (zero point - code) for (code - zero point)."""
    codes = np.arange(16, dtype=np.uint8)
    packed = oracle.pack_u4(codes)
    got = oracle.dequantize_u4(packed, 16, 0x3F800000, 3)
    high_first = np.concatenate([[(p >> 4) & 15, p & 15] for p in packed]).astype(np.float32) - 3
    negated = (3 - codes.astype(np.int64)).astype(np.float32)
    want = (codes.astype(np.int64) - 3).astype(np.float32)
    assert np.array_equal(bits(got), bits(want))
    assert not np.array_equal(bits(got), bits(high_first))
    assert not np.array_equal(bits(got), bits(negated))


# --- the declared subnormal modes ----------------------------------------------

READINGS = [(oracle.PRESERVE, oracle.PRESERVE), (oracle.FLUSH_SIGN_PRESERVING, oracle.PRESERVE),
            (oracle.PRESERVE, oracle.FLUSH_SIGN_PRESERVING),
            (oracle.FLUSH_SIGN_PRESERVING, oracle.FLUSH_SIGN_PRESERVING)]
NODE_OP = {"add": 2, "multiply": 3}


def test_f32_sites_under_each_reading():
    """The evaluator's five occurrences (tests.rs:786-859) as one-node
    expressions: each reading lands where the reference says."""
    for case in G["subnormal_modes"]["f32_sites"]["cases"]:
        l, r = f32([case["left"]]), f32([case["right"]])
        nodes = [(0, 0, 0), (0, 1, 0), (NODE_OP[case["op"]], 0, 1)]
        for (im, rm), want in zip(READINGS, case["readings"]):
            got = oracle.expression_f32(nodes, [l, r], input_mode=im, result_mode=rm)
            assert int(bits(got)[0]) == hexbits(want), (case["name"], im, rm)


def test_split_and_modes_are_answered_independently():
    for row in G["subnormal_modes"]["f32_split"]["rows"]:
        x = f32(row["contributors"])
        for (im, rm), want in zip(READINGS, row["readings"]):
            part = oracle.strict_partial_sums(x, 1, 4, 2, 2, input_mode=im, result_mode=rm)
            assert [int(v) for v in bits(part)] == [hexbits(v) for v in want["partials_2x2"]], (row["name"], im, rm)
            t22 = oracle.strict_partitioned_sum(x, 1, 4, 2, 2, input_mode=im, result_mode=rm)
            t41 = oracle.strict_partitioned_sum(x, 1, 4, 4, 1, input_mode=im, result_mode=rm)
            assert int(bits(t22)[0]) == hexbits(want["total_2x2"]), (row["name"], im, rm)
            assert int(bits(t41)[0]) == hexbits(want["total_4x1"]), (row["name"], im, rm)
            # a one-contributor partition transports its operand under every reading
            assert [int(v) for v in bits(oracle.strict_partial_sums(x, 1, 4, 4, 1, input_mode=im, result_mode=rm))] \
                == [hexbits(v) for v in row["contributors"]]


def test_bf16_counterexamples_under_each_reading():
    """bf16.rs's seven counterexamples, each reading: the input mode replaces
    operand encodings, the result mode the rounded encoding; under the
    always-positive flush the negated rows give +0 on both dimensions."""
    g = G["subnormal_modes"]["bf16_counterexamples"]
    for case in g["cases"]:
        l = np.array([hexbits(case["left"])], np.uint16)
        r = np.array([hexbits(case["right"])], np.uint16)
        nodes = [(0, 0, 0), (0, 1, 0), (NODE_OP[case["op"]], 0, 1)]
        for (im, rm), want in zip(READINGS, case["readings"]):
            got = oracle.expression_bf16(nodes, [l, r], input_mode=im, result_mode=rm)
            assert int(got[0]) == hexbits(want), (case, im, rm)
    pos = oracle.FLUSH_POSITIVE_ZERO
    for left, right in (("0x8040", "0x4000"), ("0x8080", "0x3f00")):
        got = oracle.expression_bf16([(0, 0, 0), (0, 1, 0), (3, 0, 1)],
                                     [np.array([hexbits(left)], np.uint16), np.array([hexbits(right)], np.uint16)],
                                     input_mode=pos, result_mode=pos)
        assert int(got[0]) == 0x0000, (left, right)


def test_fold_under_modes_seeds_at_the_first_contributor():
    """A lone subnormal contributor is transported (no addition happens), and
    with a flushing result mode two subnormals summing to a normal keep it
    (an identity-seeded fold would flush the first one)."""
    x = f32(["0x00400000"])
    for im, rm in READINGS:
        assert int(bits(oracle.strict_sum(x, (1, 1), 1, input_mode=im, result_mode=rm))[0]) == 0x00400000
    y = f32(["0x00400000", "0x00400000"])
    got = oracle.strict_sum(y, (1, 2), 1, input_mode=oracle.PRESERVE, result_mode=oracle.FLUSH_SIGN_PRESERVING)
    assert int(bits(got)[0]) == 0x00800000
    fold = oracle.fold_f32(y, (1, 2), (1,), input_mode=oracle.PRESERVE, result_mode=oracle.FLUSH_SIGN_PRESERVING)
    assert int(bits(fold)[0]) == 0x00800000
