"""GPU: realizations routed through a code object carried in an artifact
envelope.

The envelope carries this build's own payload:
- its metadata section is `tiler_hip_payload_metadata`;
- its code section is the gfx950 code object;
- its descriptor digest is the payload identity.
`select_payload` picks it, and `route(..., payload=...)` prepares every
dispatched symbol from the carried code bytes. A symbol the payload's
PayloadEntryMappings do not name is refused before anything is committed.
Results are compared bit for bit with the family entry points, which run the
library's built-in code object.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np
import pytest

import oracle
from tiler_amd import _lib as L
from tiler_amd import envelope as E
from tiler_amd import families
from tiler_amd.realize import realize, route
from tiler_amd.runtime import Refusal

sys.path.insert(0, os.path.dirname(__file__))
import envelope_fixture as F  # noqa: E402

pytestmark = pytest.mark.gpu

EPS = 0x3727C5AC


def _built_payload():
    lib = L.lib()
    need = ctypes.c_uint64()
    assert lib.tiler_hip_payload_metadata(None, 0, ctypes.byref(need)) == L.OK
    md = ctypes.create_string_buffer(need.value)
    assert lib.tiler_hip_payload_metadata(md, need.value, ctypes.byref(need)) == L.OK
    view = L.PayloadView()
    assert lib.tiler_hip_payload(ctypes.byref(view)) == L.OK
    return md.raw, ctypes.string_at(view.code, view.code_bytes)


@pytest.fixture(scope="module")
def carried():
    md, code = _built_payload()
    data = F.Artifact(payloads=[F.Payload(metadata=md, code=code)]).encode()
    chosen = E.select_payload(E.read_envelope(data))
    assert chosen.code == code and chosen.subject.target == "amdgcn-amd-amdhsa--gfx950"
    return chosen


def _routed(ctx, rz, inputs, outputs, payload):
    dev_in = [ctx.to_device(a) for a in inputs]
    dev_out = [ctx.alloc(max(1, int(np.prod(shape)) * np.dtype(dt).itemsize)) for dt, shape in outputs]
    storage, i_in, i_out = [], 0, 0
    for role, _ in rz.slots:
        if role == L.SLOT_INPUT:
            storage.append(dev_in[i_in]); i_in += 1
        elif role == L.SLOT_OUTPUT:
            storage.append(dev_out[i_out]); i_out += 1
        else:
            storage.append(None)
    try:
        route(ctx, rz, storage, payload=payload)
        return [b.download(dt, shape) for b, (dt, shape) in zip(dev_out, outputs)]
    finally:
        for b in dev_in + dev_out:
            b.free()


def test_rms_norm_through_the_carried_payload(ctx, carried):
    print("envelope route: rms_norm bf16 64x4096", flush=True)
    rows, extent = 64, 4096
    rng = np.random.default_rng(5)
    x = oracle.bf16_narrow(rng.standard_normal((rows, extent)).astype(np.float32))
    w = oracle.bf16_narrow(rng.normal(1.0, 0.1, extent).astype(np.float32))
    rz = realize(L.PROGRAM_RMS_NORM, (rows, extent), dtype=L.BF16, scalars=(EPS,),
                 flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [x, w], [(np.uint16, (rows, extent))], carried)
    dx, dw, dy = ctx.to_device(x), ctx.to_device(w), ctx.alloc(x.nbytes)
    try:
        ctx.rms_norm(L.BF16, dx, dw, rows, extent, EPS, dy, weight_broadcast=True)
        want = dy.download(np.uint16, (rows, extent))
    finally:
        dx.free(); dw.free(); dy.free()
    assert np.array_equal(got, want)


def test_tree_sum_through_the_carried_payload(ctx, carried):
    print("envelope route: tree sum 3 x 2^20+5", flush=True)
    rows, extent = 3, (1 << 20) + 5
    x = np.random.default_rng(6).uniform(-1, 1, (rows, extent)).astype(np.float32)
    rz = realize(L.PROGRAM_SERIAL_SUM, (rows, extent), topology=L.SUM_TREE, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [x], [(np.float32, (rows,))], carried)
    want = families.tree_sum(x, (rows, extent), 1, ctx=ctx)
    assert np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).reshape(-1).view(np.uint32))


def test_bf16_contraction_through_the_carried_payload(ctx, carried):
    print("envelope route: contraction bf16 512x512x256 + silu", flush=True)
    m, n, k = 512, 512, 256
    rng = np.random.default_rng(7)
    a = oracle.bf16_narrow((rng.standard_normal((m, k)) / 16).astype(np.float32))
    b = oracle.bf16_narrow((rng.standard_normal((n, k)) / 16).astype(np.float32))
    rz = realize(L.PROGRAM_CONTRACTION, (m, n, k), dtype=L.BF16, variant=L.EPILOGUE_SILU, permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    (got,) = _routed(ctx, rz, [a, b], [(np.uint16, (m, n))], carried)
    assert np.array_equal(got, families.contract_bf16(a, b, L.EPILOGUE_SILU, ctx=ctx))


def test_a_symbol_the_payload_does_not_map_is_refused(ctx):
    md_full, code = _built_payload()
    only = F.payload_metadata(entries=[(b"tiler_map_f32", "tiler_map_f32", [0, 1, 2])])
    data = F.Artifact(payloads=[F.Payload(metadata=only, code=code)]).encode()
    chosen = E.select_payload(E.read_envelope(data))
    rz = realize(L.PROGRAM_SOFTMAX, (4, 256), permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    x, y = ctx.alloc(4 * 256 * 4), ctx.alloc(4 * 256 * 4)
    try:
        with pytest.raises(Refusal) as r:
            route(ctx, rz, [x, y], payload=chosen)
        assert r.value.status == L.REFUSE_ABSENT_SYMBOL
    finally:
        x.free(); y.free()
