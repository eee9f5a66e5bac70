"""CPU: the ctypes mirror of include/tiler_hip.h has the header's layout.

Every struct the Python host side passes through the C ABI is declared
twice: once in the header (the boundary a foreign binding would use) and once
as a ctypes.Structure in tiler_amd/_lib.py.  A field added to one and not the
other shifts every later field without any error at the call.  This test
compiles a small C program against the header with gcc that prints sizeof and
every field's offsetof, and requires the ctypes declarations to agree on
each.
"""
from __future__ import annotations

import ctypes
import os
import shutil
import subprocess

import pytest

from tiler_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# ctypes mirror -> the header's typedef
STRUCTS = {
    L.TargetProfile: "tiler_hip_target_profile",
    L.PayloadView: "tiler_hip_payload_view",
    L.EntryInfo: "tiler_hip_entry_info",
    L.ExecutionEnvironment: "tiler_hip_execution_environment",
    L.RoutedEntry: "tiler_hip_routed_entry",
    L.DispatchEntry: "tiler_hip_dispatch_entry",
    L.LiveExtent: "tiler_hip_live_extent",
    L.DispatchPlan: "tiler_hip_dispatch_plan",
    L.TargetEnvironmentSchema: "tiler_hip_target_environment_schema",
    L.SumPlan: "tiler_hip_sum_plan",
    L.ExpressionNode: "tiler_hip_expression_node",
    L.ContractionStructure: "tiler_hip_contraction_structure",
    L.Region: "tiler_hip_region",
    L.Proposal: "tiler_hip_proposal",
    L.DeclinedStrategy: "tiler_hip_declined_strategy",
    L.ProviderOffer: "tiler_hip_provider_offer",
    L.RealizedEntry: "tiler_hip_realized_entry",
    L.Realization: "tiler_hip_realization",
    L.EnvelopePayload: "tiler_hip_envelope_payload",
    L.Envelope: "tiler_hip_envelope",
    L.PayloadMapping: "tiler_hip_payload_mapping",
    L.PayloadSubject: "tiler_hip_payload_subject",
}


def _program() -> str:
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "tiler_hip.h"', "int main(void) {"]
    for cls, name in STRUCTS.items():
        lines.append(f'  printf("{name} sizeof %zu\\n", sizeof({name}));')
        for field, *_ in cls._fields_:
            lines.append(f'  printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    lines += ["  return 0;", "}"]
    return "\n".join(lines) + "\n"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_ctypes_mirror_matches_the_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(_program())
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{os.path.join(ROOT, 'include')}", str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        name, field, value = line.split()
        got[(name, field)] = int(value)
    wrong = []
    for cls, name in STRUCTS.items():
        if got[(name, "sizeof")] != ctypes.sizeof(cls):
            wrong.append(f"sizeof {name}: header {got[(name, 'sizeof')]}, ctypes {ctypes.sizeof(cls)}")
        for field, *_ in cls._fields_:
            off = getattr(cls, field).offset
            if got[(name, field)] != off:
                wrong.append(f"{name}.{field}: header {got[(name, field)]}, ctypes {off}")
    assert not wrong, "\n".join(wrong)
