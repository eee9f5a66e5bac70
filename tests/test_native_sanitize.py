"""The host-side planners, the governed digest and the envelope reader under
AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

Builds tests/native/planner_sanitize.cpp against the runtime's own
program.cpp and digest.cpp with g++ -fsanitize=address,undefined (no device
code, no HIP runtime). It runs every planner over random and edge-case
requests (zero, huge and overflowing extents, unaligned addresses, invalid
enums), the expression compiler over random and malformed node arrays (then
the expression and fold-epilogue planners over what compiles), folds and
signed-stride reindexes over random axis sets, general contractions over
random index structures, and the digest over random splits. The run must finish clean: no
sanitizer report, no argument segment overflow, every binding inside its
segment and naming a declared slot.

tests/native/envelope_sanitize.cpp reads 120,000 mutants of one envelope and
one payload-metadata record: flipped bytes, overwritten lengths and counts,
truncations and insertions. Manifest mutants are resealed, so they reach the
parser rather than stopping at the manifest digest.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RT = os.path.join(ROOT, "tiler_amd", "csrc", "runtime")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_planners_and_digest_are_sanitizer_clean(tmp_path):
    exe = tmp_path / "planner_sanitize"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    f"-I{os.path.join(ROOT, 'include')}", f"-I{RT}",
                    os.path.join(ROOT, "tests", "native", "planner_sanitize.cpp"),
                    os.path.join(RT, "program.cpp"), os.path.join(RT, "digest.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "planner-sanitize ok" in r.stdout and "runtime error" not in r.stderr


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_envelope_reader_is_sanitizer_clean(tmp_path):
    sys.path.insert(0, os.path.dirname(__file__))
    import envelope_fixture as F
    md = F.payload_metadata(entries=[(b"tiler_map_f32", "tiler_map_f32", [0, 1, 2])])
    envelope = F.Artifact(payloads=[F.Payload(metadata=md, code=b"\x7fELF code object")],
                          kernel_programs=[b"program a", b"program b"],
                          interior=F.u64(2) + bytes(range(64)) + F.framed(b"realization")).encode()
    (tmp_path / "envelope.bin").write_bytes(envelope)
    (tmp_path / "metadata.bin").write_bytes(md)
    exe = tmp_path / "envelope_sanitize"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    f"-I{RT}", os.path.join(ROOT, "tests", "native", "envelope_sanitize.cpp"),
                    os.path.join(RT, "envelope.cpp"), os.path.join(RT, "digest.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), str(tmp_path / "envelope.bin"), str(tmp_path / "metadata.bin")],
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "envelope-sanitize ok" in r.stdout and "runtime error" not in r.stderr
