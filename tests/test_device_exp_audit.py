"""The device's binary32 exp is correctly rounded on every input.

tiler::exp_f32_cr (softmax and SiLU) evaluates e^s in binary64 and rounds
once.  oracle/device_exp_audit.c restates that evaluation bit for bit and
scans every binary32 input in (-104, 89): each input whose binary64 value
lies within 2^-48 of a binary32 rounding boundary is compared with the
certified exp (tiler-reference/src/silu.rs:189-229); every other input rounds
correctly by the error bound stated there (< 2^-50.7).  The near-boundary
inputs are kept in tests/golden/device_exp_hard_cases.json, which the GPU
test drives through the device's SiLU and softmax.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "device_exp_hard_cases.json")
# binary32 bit patterns in [+0, 89) and in (-104, -0]
SCANNED = 0x42B20000 + (0xC2D00000 - 0x80000000)
THREADS = max(1, min(16, os.cpu_count() or 1))


def _fixture():
    with open(FIXTURE) as f:
        return json.load(f)


def test_exhaustive_audit_finds_every_input_correctly_rounded():
    r = oracle.audit_device_exp(margin_log2=-48, threads=THREADS)
    assert r["checked"] == SCANNED
    assert r["mismatches"] == 0, f"first misrounded input {r['first_mismatch']!r}"
    fx = _fixture()
    assert fx["scanned"] == SCANNED
    assert [f"0x{int(b):08x}" for b in r["hard"].view(np.uint32)] == fx["inputs"]


def test_a_perturbation_inside_the_margin_is_caught():
    """Planted mistake: scaling the device value by (1 + 2^-49) before the
    rounding must produce misrounded near-boundary inputs."""
    r = oracle.audit_device_exp(margin_log2=-48, threads=THREADS, planted_log2=-49)
    assert r["mismatches"] > 0


def test_fixture_values_are_the_certified_and_the_restated_device_exp():
    fx = _fixture()
    for inp, want in zip(fx["inputs"], fx["certified_exp"]):
        s = np.uint32(int(inp, 16)).view(np.float32)
        assert int(np.float32(oracle.certified_exp_f32(float(s))).view(np.uint32)) == int(want, 16)
        assert int(np.float32(oracle.device_exp_f32(float(s))).view(np.uint32)) == int(want, 16)


@pytest.mark.parametrize("s", [0.0, -0.0, 1e-30, -1e-30, 88.72, 88.7228, -87.33, -103.97, -103.2])
def test_restated_device_exp_matches_certified_at_boundaries(s):
    s = float(np.float32(s))
    assert np.float32(oracle.device_exp_f32(s)).view(np.uint32) == \
        np.float32(oracle.certified_exp_f32(s)).view(np.uint32)


def test_nonpositive_exp_reduction_is_the_audited_rint():
    """tiler::exp_f32_cr_nonpositive forms k as fl(s * 64/ln2) + 1.5 * 2^52
    minus 1.5 * 2^52 and reads k from the sum's low word, where exp_f32_cr
    (the audited evaluation) takes rint of the same product and converts it.
    Every binary32 s in (-104, 0] gives the same binary64 k and the same
    integer (so the rest of the evaluation is the audited one): checked on
    every 97th input of the range and on products planted at halfway points
    (ties round to even in both)."""
    c = float.fromhex("0x1.71547652b82fep+6")  # TILER_64_OVER_LN2, exp_table.h
    lo, hi = 0x80000000, 0xC2D00000            # -0 .. -104
    u = np.arange(lo, hi, 97, dtype=np.uint64).astype(np.uint32)
    s = u.view(np.float32).astype(np.float64)
    s = s[s > -104.0]
    y = s * c
    magic = float.fromhex("0x1.8p52")
    shifted = y + magic
    kd = shifted - magic
    assert np.array_equal(kd, np.rint(y))
    low = (shifted.view(np.uint64) & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.int32)
    assert np.array_equal(low.astype(np.int64), np.rint(y).astype(np.int64))
    ties = -np.arange(1, 6600, dtype=np.float64) - 0.5  # k + 0.5 for every k the domain reaches
    assert np.array_equal((ties + magic) - magic, np.rint(ties))
