"""GPU: the reference's emitter goldens that no other GPU test names, run on
the device through the realize route at the goldens' own shapes and checked
bit for bit against their kernels' arithmetic, transcribed in
tests/test_goldens.py: contraction_strict_tensor (2 x 3, K = 4),
contraction_tiled_cooperative (10 x 32, K = 32), cooperative_workgroup_reduction
(2 outputs of 6, 3 participants of 2), reduction_single_axis (2 x 3) and
structural_widening_broadcast ([2] -> [4]).
"""
from __future__ import annotations

import numpy as np
import pytest

from test_goldens import (golden_cooperative, golden_single_axis, golden_strict_tensor, golden_tiled_cooperative,
                          golden_widening_broadcast)
from tiler_amd import _lib as L
from tiler_amd.realize import realize, route

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _run(ctx, rz, inputs, out_elems):
    dev = [ctx.to_device(x) for x in inputs]
    out = ctx.alloc(4 * out_elems)
    try:
        route(ctx, rz, dev + [out])
        return out.download(np.float32, (out_elems,))
    finally:
        for b in dev + [out]:
            b.free()


@pytest.mark.parametrize("seed", range(2))
def test_goldens_on_the_device(ctx, seed):
    rng = np.random.default_rng(40 + seed)
    a = rng.standard_normal(8).astype(np.float32)
    b = rng.standard_normal(12).astype(np.float32)
    print("[golden] contraction_strict_tensor", flush=True)
    got = _run(ctx, realize(L.PROGRAM_CONTRACTION, (2, 3, 4), ctx=ctx), [a, b], 6)
    assert np.array_equal(_bits(got), _bits(golden_strict_tensor(a, b)))
    a = rng.standard_normal(320).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    print("[golden] contraction_tiled_cooperative", flush=True)
    got = _run(ctx, realize(L.PROGRAM_CONTRACTION, (10, 32, 32), ctx=ctx), [a, b], 320)
    assert np.array_equal(_bits(got), _bits(golden_tiled_cooperative(a, b)))
    x = (rng.standard_normal(12) * np.exp2(rng.integers(-20, 20, 12))).astype(np.float32)
    print("[golden] cooperative_workgroup_reduction", flush=True)
    rz = realize(L.PROGRAM_SERIAL_SUM, (2, 6), topology=L.SUM_COOPERATIVE, grouping=(3, 2, 1),
                 permissions=L.PERMITS_REASSOCIATION, ctx=ctx)
    assert np.array_equal(_bits(_run(ctx, rz, [x], 2)), _bits(golden_cooperative(x)))
    y = (rng.standard_normal(6) * np.exp2(rng.integers(-20, 20, 6))).astype(np.float32)
    print("[golden] reduction_single_axis", flush=True)
    got = _run(ctx, realize(L.PROGRAM_SERIAL_SUM, (2, 3), ctx=ctx), [y], 2)
    assert np.array_equal(_bits(got), _bits(golden_single_axis(y)))
    z = rng.standard_normal(2).astype(np.float32)
    print("[golden] structural_widening_broadcast", flush=True)
    rz = realize(L.PROGRAM_BROADCAST, (2, 2), rank=2, strides=(0, 1), grouping=(2,), variant=4, ctx=ctx)
    assert np.array_equal(_bits(_run(ctx, rz, [z], 4)), _bits(golden_widening_broadcast(z)))
