"""Writes device_exp_hard_cases.json: every binary32 input in (-104, 89) whose
device exp value (binary64, before the one rounding to binary32) lies within
2^-48 of a binary32 rounding boundary, with the certified exp of each
(oracle.certified_exp_f32, tiler-reference/src/silu.rs:189-229).

Run from the repository root: python tests/golden/make_device_exp_hard_cases.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402


def main():
    oracle.build()
    r = oracle.audit_device_exp(margin_log2=-48, threads=min(16, os.cpu_count() or 1))
    assert r["mismatches"] == 0 and r["hard_count"] == len(r["hard"])
    inputs = [f"0x{int(b):08x}" for b in r["hard"].view(np.uint32)]
    certified = [f"0x{int(np.float32(oracle.certified_exp_f32(float(s))).view(np.uint32)):08x}"
                 for s in r["hard"]]
    out = {"margin_log2": -48, "scanned": r["checked"], "inputs": inputs, "certified_exp": certified}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "device_exp_hard_cases.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(f"{len(inputs)} near-boundary inputs of {r['checked']} scanned")


if __name__ == "__main__":
    main()
