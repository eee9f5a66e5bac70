"""The HIP conformance vertical (`tiler_amd.conformance`), after
tiler-conformance/src/measurement.rs: the three outcomes and the rule that turns
them into a verdict, on the CPU; the pinned expectations it carries against
the committed golden fixture; and, on the GPU, every vertical measured and
matching.
"""
from __future__ import annotations

import io

import numpy as np
import pytest

from helpers import golden, hexbits, splitmix_operands
from tiler_amd import conformance as C

G = golden()


def test_the_pinned_expectations_are_the_reference_records():
    cells = {c["id"]: c for c in G["contraction"]["cells"]}
    assert {cid for cid, *_ in C.CONTRACTION_CELLS} == set(cells)
    for cid, m, n, k, digest in C.CONTRACTION_CELLS:
        assert (m, n, k, digest) == (cells[cid]["m"], cells[cid]["n"], cells[cid]["k"], cells[cid]["sha256"])
    assert C.WORKLOAD_SEED == hexbits(G["contraction"]["workload_seed"])
    assert C.RIGHT_SEED_MASK == hexbits(G["contraction"]["right_seed_mask"])
    s = G["serial_sum"]
    by_name = {name: (ops, want) for name, ops, _, _, want in C.SERIAL_SUM_CELLS}
    for name, key, want_key in [("parallel/serial", "parallel_operands", "parallel_sum"),
                                ("grouping-sensitive/serial", "grouping_sensitive_operands", "grouping_sensitive_serial"),
                                ("separating/tree-6x2", "separating_operands", "separating_tree_6x2"),
                                ("separating/split-4x3", "separating_operands", "separating_split_4x3"),
                                ("separating-exact/serial", "separating_exact_operands", "separating_exact_sum")]:
        ops, want = by_name[name]
        assert list(ops) == [hexbits(v) for v in s[key]] and want == hexbits(s[want_key])


def test_the_row_examples_are_the_reference_records():
    r = next(c for c in G["rms_norm"]["cases"] if c["name"] == "worked example")
    sm = next(c for c in G["softmax"]["cases"] if c["name"] == "worked example")
    cells = {name: (xs, ws, eps, want) for name, _, xs, ws, eps, want in C.ROW_CELLS}
    xs, ws, eps, want = cells["rms-norm/worked-example"]
    assert list(np.asarray(xs, np.uint32).view(np.float32)) == r["x"]
    assert list(np.asarray(ws, np.uint32).view(np.float32)) == r["w"]
    assert eps == hexbits(G["rms_norm"]["eps_bits"]) and list(want) == [hexbits(v) for v in r["y_bits"]]
    xs, _, _, want = cells["softmax/worked-example"]
    assert list(xs) == [hexbits(v) for v in sm["x_bits"]] and list(want) == [hexbits(v) for v in sm["y_bits"]]


def test_operands_match_the_test_side_generator():
    for seed in (C.WORKLOAD_SEED, C.WORKLOAD_SEED ^ C.RIGHT_SEED_MASK):
        assert np.array_equal(C.splitmix_operands(seed, 5000), splitmix_operands(seed, 5000))


def test_require_or_report_outcomes(monkeypatch):
    monkeypatch.delenv(C.REQUIRE_MEASUREMENT, raising=False)
    out = io.StringIO()
    assert C.require_or_report("v", C.Measured.unavailable("no device"), out) is None
    assert "MEASUREMENT BOUNDARY UNAVAILABLE -- no device" in out.getvalue()
    monkeypatch.setenv(C.REQUIRE_MEASUREMENT, "1")
    with pytest.raises(C.ConformanceFailure):
        C.require_or_report("v", C.Measured.unavailable("no device"), io.StringIO())
    monkeypatch.delenv(C.REQUIRE_MEASUREMENT)
    with pytest.raises(C.ConformanceFailure):  # a reached environment that refused is a defect
        C.require_or_report("v", C.Measured.failed("dispatch refused"), io.StringIO())
    b = C.MeasurementBoundary("Linux", "6", "x86_64", "dev", "gfx950", 256, 1, 2, "clang", "key", "tgt", 10, "ab" * 32)
    out = io.StringIO()
    assert C.require_or_report("v", C.Measured.ran(b, [{"cell": "c", "match": True}]), out) == [
        {"cell": "c", "match": True}]
    assert "gfx950" in out.getvalue()


def test_deterministic_half_runs_everywhere():
    d = C.deterministic_half()
    assert len(d) == len(C.CONTRACTION_CELLS) + len(C.SERIAL_SUM_CELLS) + len(C.ROW_CELLS)


def test_a_host_without_the_device_reports_unavailable(monkeypatch):
    # Forced from the host: binding reports what is missing, and every
    # vertical carries that reason; nothing claims a device result.
    monkeypatch.setattr(C, "_bind", lambda: (None, C.Measured.unavailable("no gfx950 device to bind")))
    outcomes = C.run()
    assert [label for label, _ in outcomes] == [label for label, _ in C.VERTICALS]
    assert all(o.kind == "unavailable" and "gfx950" in o.reason for _, o in outcomes)
    monkeypatch.delenv(C.REQUIRE_MEASUREMENT, raising=False)
    assert C.main() == 0
    monkeypatch.setenv(C.REQUIRE_MEASUREMENT, "1")
    assert C.main() == 1


@pytest.mark.gpu
def test_every_vertical_is_measured_and_matches():
    outcomes = C.run()
    for label, outcome in outcomes:
        assert outcome.kind == "ran", (label, outcome.reason)
        assert outcome.boundary.gcn_arch.startswith("gfx950")
        assert outcome.observed and all(row["match"] for row in outcome.observed), (label, outcome.observed)
