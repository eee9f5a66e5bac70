"""Builds the test-only device code objects under tests/native (*.hip) into
tests/_build/<name>.hsaco with the product's own device flags.

Test infrastructure: these kernels audit device helpers exhaustively (e.g.
tests/native/silu_epilogue_audit.hip).  The GPU tests load them through the
adapter's tiler_hip_prepare_entries, like any routed payload; the product
library never contains or loads them.  __graft_entry__.build() calls build(),
so the objects exist before any GPU run (nothing compiles on the GPU box).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(ROOT, "tests", "_build")


def object_path(name: str) -> str:
    return os.path.join(OUT, name + ".hsaco")


def build(verbose: bool = False) -> list:
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from tiler_amd import build as tb

    os.makedirs(OUT, exist_ok=True)
    built = []
    for src in sorted(f for f in os.listdir(HERE) if f.endswith(".hip")):
        dst = object_path(src[:-4])
        subprocess.run([tb.CLANG, *tb.DEVICE_FLAGS, "-o", dst + ".tmp", os.path.join(HERE, src)], check=True)
        os.replace(dst + ".tmp", dst)
        built.append(dst)
        if verbose:
            print(f"built {dst}")
    return built


if __name__ == "__main__":
    build(verbose=True)
