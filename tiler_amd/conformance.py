"""The HIP conformance vertical: the measured half of a conformance run, and
the environment row it is bounded to (after tiler-conformance/src/
measurement.rs:1-200).

A run has two halves that fail for unrelated reasons:
- The deterministic half generates each cell's operands. It carries the
  expected results as data, restated from the reference's own records. It
  needs nothing else.
- The measured half needs this library and a gfx950 device.

A host without the device reports the measured half as `Unavailable` and
names what is missing. It never skips silently. A host that reached the
device and was refused reports `Failed`, which is a defect, not a boundary.
`require_or_report` turns the three outcomes into a verdict in one place. With
`TILER_REQUIRE_HIP_CONFORMANCE` set, `Unavailable` is a failure too; the
variable can only make a run stricter.

Verticals:
- `contraction-profile-cells`: the strict f32 contraction over SplitMix64
  operands, checked by the SHA-256 of each result against the six digests of
  tiler-reference/tests/contraction_profile_cells.rs:148-300.
- `serial-sum-cells`: the serial, multi-pass and tree sums over the operand
  sets of tiler-conformance/src/serial_sum.rs:202-368, checked bit for bit
  against the results those records state.
- `row-worked-examples`: the RMSNorm and softmax worked examples whose every
  bit the reference's tests fix.

`python -m tiler_amd.conformance` prints the boundary and every vertical's
outcome. It exits non-zero on a failure, or on an unavailable measurement
under the variable.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import platform
import sys
import time
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L

REQUIRE_MEASUREMENT = "TILER_REQUIRE_HIP_CONFORMANCE"

# tiler-reference/tests/contraction_profile_cells.rs:148-300: td,od->to
# (A[m,k] x B[n,k] -> C[m,n]); operands prng_value(seed, i) = m * 2^-24 with
# m the top 24 bits of SplitMix64(seed + i * 0x2545F4914F6CDD1D), centred; the
# right operand's seed is XOR-ed with 0xA5A5A5A5A5A5A5A5; the digest is the
# SHA-256 of the little-endian f32 result.
WORKLOAD_SEED = 0x5445524D
RIGHT_SEED_MASK = 0xA5A5A5A5A5A5A5A5
CONTRACTION_CELLS = (
    ("w_decode_kv", 1, 1024, 1024, "79810ce471cbd6cd05e5c0c30ea6023e74b997bd5b349212b71cd4a23fe8701f"),
    ("w_prefill_q", 10, 2048, 1024, "1c54f5cd7265ee288ec79bcd9254243b78a95d57c3c489e5ea90bcc4298073c0"),
    ("w_prefill_mlp_in", 128, 3072, 1024, "eb382840ac9e533f57e51a0ffed2d61608664ecc5869aaa9f93afa3c312696a0"),
    ("w_prefill_mlp_out", 128, 1024, 3072, "124571de47ebff2f152b120afc9944b3465bffe94d8ac283a077677f61feb5f5"),
    ("w_prefill_o", 128, 1024, 2048, "b99eff9042d9e4b25e3844ff0462e5e6303e57b146aa79400622885bffc5f2f6"),
    ("w_vocab_slice", 1, 8192, 1024, "88b01ae776f42bdb2f2d1092ddfd039e20e652d28393a6e2ec19e5cc1d9803c8"),
)

# tiler-conformance/src/serial_sum.rs:202-368: operand sets (f32 bits) and the
# result each topology must produce.
_GROUPING = (0x3F400000, 0x3E800000, 0x33400000, 0x33000000)
SERIAL_SUM_CELLS = (
    # (name, operands, topology, (partitions, per_partition), expected bits)
    ("parallel/serial", (0x3F800000, 0x40000000, 0x40800000, 0x41000000), "serial", None, 0x41700000),
    ("grouping-sensitive/serial", _GROUPING, "serial", None, 0x3F800000),
    ("separating/tree-6x2", _GROUPING + (0,) * 8, "multipass", (6, 2), 0x3F800001),
    ("separating/split-4x3", _GROUPING + (0,) * 8, "multipass", (4, 3), 0x3F800000),
    ("separating-exact/serial", tuple(0x3F800000 + (i << 23) for i in range(12)), "serial", None, 0x457FF000),
    ("separating-exact/tree", tuple(0x3F800000 + (i << 23) for i in range(12)), "tree", None, 0x457FF000),
)


# Worked examples whose every bit the reference's tests fix.
# tiler-reference/src/rms_norm/tests.rs:253-276 (f32, eps bits 0x358637bd);
# tiler-reference/src/softmax/tests.rs:362-455 (the last score is the most
# negative finite f32, a masked contributor).
ROW_CELLS = (
    ("rms-norm/worked-example", "rms_norm", (0x40400000, 0x40800000), (0x3F800000, 0x40000000), 0x358637BD,
     (0x3F593923, 0x4010D0C2)),
    ("softmax/worked-example", "softmax", (0x3F800000, 0x40000000, 0x40400000, 0xFF7FFFFF), None, None,
     (0x3DB861F3, 0x3E7A9A1A, 0x3F2A4D3B, 0x00000000)),
)


@dataclass
class MeasurementBoundary:
    """The environment row one measured result is bounded to; every field is
    observed on the host that ran."""
    os_family: str
    os_release: str
    architecture: str
    device_name: str
    gcn_arch: str
    compute_units: int
    runtime_version: int
    driver_version: int
    toolchain: str
    profile_key: str
    target: str
    code_object_bytes: int
    payload_identity: str

    def __str__(self) -> str:
        return (f"  host:      {self.os_family} {self.os_release} on {self.architecture}\n"
                f"  device:    {self.device_name} ({self.gcn_arch}, {self.compute_units} CUs), "
                f"runtime {self.runtime_version}, driver {self.driver_version}\n"
                f"  toolchain: {self.toolchain}\n"
                f"  compiled:  {self.profile_key} for {self.target} "
                f"({self.code_object_bytes} code-object bytes, payload {self.payload_identity[:16]}...)")


@dataclass
class Measured:
    """Ran (with its boundary and what it observed), Unavailable (with what
    is missing) or Failed (with what refused)."""
    kind: str
    boundary: MeasurementBoundary | None = None
    observed: list = field(default_factory=list)
    reason: str = ""

    @staticmethod
    def ran(boundary, observed):
        return Measured("ran", boundary, observed)

    @staticmethod
    def unavailable(reason):
        return Measured("unavailable", reason=reason)

    @staticmethod
    def failed(detail):
        return Measured("failed", reason=detail)


class ConformanceFailure(AssertionError):
    pass


def require_or_report(label: str, outcome: Measured, out=sys.stderr):
    """Reports one measured half and returns what it observed (None when it
    did not run).  Raises ConformanceFailure when the half failed, and when
    it was unavailable under TILER_REQUIRE_HIP_CONFORMANCE."""
    if outcome.kind == "ran":
        print(f"{label}: measured on this row:\n{outcome.boundary}", file=out)
        return outcome.observed
    if outcome.kind == "unavailable":
        if os.environ.get(REQUIRE_MEASUREMENT):
            raise ConformanceFailure(f"{REQUIRE_MEASUREMENT} is set and the measured half is unavailable: "
                                     f"{outcome.reason}")
        print(f"{label}: MEASUREMENT BOUNDARY UNAVAILABLE -- {outcome.reason}. The deterministic half (the "
              "pinned expectations and the operands) ran; nothing here claims a device result.", file=out)
        return None
    raise ConformanceFailure(f"{label}: the measured half reached its environment and refused: {outcome.reason}")


def splitmix_operands(seed: int, count: int) -> np.ndarray:
    idx = np.arange(count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = np.uint64(seed) + idx * np.uint64(0x2545F4914F6CDD1D) + np.uint64(0x9E3779B97F4A7C15)
        z = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    field_ = ((z >> np.uint64(40)) & np.uint64(0xFFFFFF)).astype(np.int64)
    return (field_ - 8388608).astype(np.float32) * np.float32(1.0 / 16777216.0)


def _bind():
    """(context, boundary) or a Measured.unavailable naming what is missing."""
    try:
        lib = L.lib()
    except L.LibraryMissing as e:
        return None, Measured.unavailable(f"the tiler-hip library is not built ({e})")
    from .runtime import Context, Refusal
    try:
        ctx = Context(0)
    except Refusal as r:
        return None, Measured.unavailable(f"no gfx950 device to bind: {r}")
    view = L.PayloadView()
    lib.tiler_hip_payload(ctypes.byref(view))
    profile = L.TargetProfile()
    lib.tiler_hip_profile_declare(ctypes.byref(profile))
    ident = (ctypes.c_uint8 * 32)()
    lib.tiler_hip_payload_identity(ident)
    env = ctx.environment
    boundary = MeasurementBoundary(
        platform.system(), platform.release(), platform.machine(), env["device_name"], env["gcn_arch_name"],
        env["compute_units"], env["runtime_version"], env["driver_version"],
        view.toolchain.decode(), profile.profile_key.decode(), view.target.decode(), view.code_bytes,
        bytes(ident).hex())
    return ctx, boundary


def _time_us(ctx, fn, repeats: int = 5) -> float:
    fn()
    ctx.synchronize()
    t = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        ctx.synchronize()
        t.append(time.perf_counter() - t0)
    return float(np.median(t) * 1e6)


def contraction_profile_cells(ctx, boundary) -> Measured:
    observed = []
    try:
        for cid, m, n, k, digest in CONTRACTION_CELLS:
            a = splitmix_operands(WORKLOAD_SEED, m * k)
            b = splitmix_operands(WORKLOAD_SEED ^ RIGHT_SEED_MASK, n * k)
            da, db, dc = ctx.to_device(a), ctx.to_device(b), ctx.alloc(m * n * 4)
            try:
                us = _time_us(ctx, lambda: ctx.contract_strict_f32(da, db, m, n, k, dc))
                c = dc.download(np.float32, (m, n))
            finally:
                da.free(); db.free(); dc.free()
            got = hashlib.sha256(np.ascontiguousarray(c, dtype="<f4").tobytes()).hexdigest()
            observed.append({"cell": cid, "m": m, "n": n, "k": k, "match": got == digest, "sha256": got,
                             "us": us})
    except Exception as e:  # a reached device that refused: a defect
        return Measured.failed(f"{type(e).__name__}: {e}")
    return Measured.ran(boundary, observed)


def serial_sum_cells(ctx, boundary) -> Measured:
    topo = {"serial": L.SUM_SERIAL, "multipass": L.SUM_MULTIPASS, "tree": L.SUM_TREE}
    observed = []
    try:
        for name, operands, topology, grouping, want in SERIAL_SUM_CELLS:
            x = np.asarray(operands, dtype=np.uint32).view(np.float32)
            dx, dy = ctx.to_device(x), ctx.alloc(4)
            try:
                kw = {} if grouping is None else {"partitions": grouping[0], "per_partition": grouping[1]}
                ctx.sum_f32(dx, 1, x.size, dy, topology=topo[topology], **kw)
                got = int(dy.download(np.float32, (1,)).view(np.uint32)[0])
            finally:
                dx.free(); dy.free()
            observed.append({"cell": name, "match": got == want, "bits": f"0x{got:08x}",
                             "expected": f"0x{want:08x}"})
    except Exception as e:
        return Measured.failed(f"{type(e).__name__}: {e}")
    return Measured.ran(boundary, observed)


def row_worked_examples(ctx, boundary) -> Measured:
    observed = []
    try:
        for name, family, xs, ws, eps, want in ROW_CELLS:
            x = np.asarray(xs, dtype=np.uint32).view(np.float32)
            dx, dy = ctx.to_device(x), ctx.alloc(x.nbytes)
            dw = ctx.to_device(np.asarray(ws, dtype=np.uint32).view(np.float32)) if ws is not None else None
            try:
                if family == "rms_norm":
                    ctx.rms_norm(L.F32, dx, dw, 1, x.size, eps, dy, weight_broadcast=True)
                else:
                    ctx.softmax_f32(dx, 1, x.size, dy)
                got = [int(v) for v in dy.download(np.float32, (x.size,)).view(np.uint32)]
            finally:
                for b in (dx, dy, dw):
                    if b is not None:
                        b.free()
            observed.append({"cell": name, "match": got == list(want), "bits": [f"0x{v:08x}" for v in got]})
    except Exception as e:
        return Measured.failed(f"{type(e).__name__}: {e}")
    return Measured.ran(boundary, observed)


VERTICALS = (("contraction-profile-cells", contraction_profile_cells), ("serial-sum-cells", serial_sum_cells),
             ("row-worked-examples", row_worked_examples))


def deterministic_half() -> dict:
    """What runs on every host: each cell's operands, generated and
    fingerprinted, with the pinned result it must reproduce."""
    out = {}
    for cid, m, n, k, digest in CONTRACTION_CELLS:
        a = splitmix_operands(WORKLOAD_SEED, m * k)
        b = splitmix_operands(WORKLOAD_SEED ^ RIGHT_SEED_MASK, n * k)
        out[cid] = {"operands_sha256": hashlib.sha256(a.tobytes() + b.tobytes()).hexdigest(), "expected": digest}
    for name, operands, topology, grouping, want in SERIAL_SUM_CELLS:
        out[name] = {"operands": len(operands), "topology": topology, "expected": f"0x{want:08x}"}
    for name, family, xs, ws, eps, want in ROW_CELLS:
        out[name] = {"family": family, "expected": [f"0x{v:08x}" for v in want]}
    return out


def run() -> list:
    """[(label, Measured)] for every vertical.  The deterministic half runs
    first, on every host.  Binding happens once; an unavailable device makes
    every vertical unavailable with the same reason."""
    deterministic_half()
    ctx, boundary_or_outcome = _bind()
    if ctx is None:
        return [(label, boundary_or_outcome) for label, _ in VERTICALS]
    try:
        return [(label, fn(ctx, boundary_or_outcome)) for label, fn in VERTICALS]
    finally:
        ctx.close()


def main(argv=None) -> int:
    failures = 0
    for label, outcome in run():
        try:
            observed = require_or_report(label, outcome)
        except ConformanceFailure as e:
            print(f"{label}: FAILED -- {e}", file=sys.stderr)
            failures += 1
            continue
        for row in observed or []:
            ok = row["match"]
            failures += 0 if ok else 1
            extra = f"  {row['us']:.1f} us" if "us" in row else ""
            print(f"  {label} {row['cell']}: {'ok' if ok else 'MISMATCH'}{extra}", file=sys.stderr)
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
