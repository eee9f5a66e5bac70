"""GPU: contractions over general index structures, against the oracle.

* strict (f32; bf16 with and without SiLU): bit-exact with
  oracle.contract_general (contraction.rs:346-715), on the attention
  goldens' own shapes (tiler-metal/goldens/contraction_attention_{score,
  value}.metal), larger attention shapes, two summed indices whose label
  order differs from the operands' axis order, a scalar result, a left
  operand stored [k, m], and a right operand shared across a batch axis;
* the batched MFMA forms (bf16 under PERMITS_REASSOCIATION): attention
  scores with K shared across heads, attention values with V stored [k, n]
  (transposed first), decode (one query row), odd extents, 256-tiles,
  with and without SiLU -- each batch within the bf16 contraction's
  relative Frobenius bound of 1e-2 against the strict f32 fold of the
  widened operands (then the reference SiLU);
* the adapter route (realize -> route) for the strict form (geometry in a
  constant slot) and the MFMA form with its transpose workspace.
"""
import numpy as np
import pytest

import oracle
from tiler_amd import _lib as L
from tiler_amd.realize import realize, route

pytestmark = pytest.mark.gpu

S = L.contraction_structure
RE = L.PERMITS_REASSOCIATION


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _operands(rng, ld, rd, bf16):
    a = rng.standard_normal(ld).astype(np.float32)
    b = rng.standard_normal(rd).astype(np.float32)
    if bf16:
        return oracle.bf16_narrow(a), oracle.bf16_narrow(b)
    return a, b


def _device(ctx, dtype, li, a, ri, b, oi, epilogue=L.EPILOGUE_NONE, permissions=0):
    s = S(li, a.shape, ri, b.shape, oi)
    extent = {}
    for lab, d in list(zip(li, a.shape)) + list(zip(ri, b.shape)):
        extent.setdefault(lab, d)
    shape = tuple(extent[lab] for lab in oi)
    da, db = ctx.to_device(a), ctx.to_device(b)
    count = int(np.prod(shape)) if shape else 1
    dy = ctx.alloc(max(1, count * a.itemsize))
    try:
        ctx.contract(dtype, s, da, db, dy, epilogue=epilogue, permissions=permissions)
        ctx.synchronize()
        return dy.download(a.dtype, shape)
    finally:
        for buf in (da, db, dy):
            buf.free()


STRICT_CASES = [
    ("bhqd", (2, 2, 3, 4), "bkd", (2, 5, 4), "bhqk"),        # contraction_attention_score.metal
    ("bhqk", (2, 2, 3, 5), "bkd", (2, 5, 4), "bhqd"),        # contraction_attention_value.metal
    ("bhqd", (2, 4, 33, 40), "bkd", (2, 70, 40), "bhqk"),
    ("bhqk", (2, 4, 33, 70), "bkd", (2, 70, 40), "bhqd"),
    ("acbd", (3, 5, 4, 6), "cbe", (5, 4, 7), "ade"),          # summed b < c, stored c-major in the left
    ("ab", (64, 33), "ab", (64, 33), ""),                    # a scalar
    ("kt", (50, 17), "ok", (13, 50), "to"),                  # the left operand stored [k, m]
    ("bij", (3, 9, 11), "jk", (11, 5), "bik"),               # the right operand shared across b
]


@pytest.mark.parametrize("case", STRICT_CASES, ids=lambda c: f"{c[0]},{c[2]}->{c[4]}:{'x'.join(map(str, c[1]))}")
def test_strict_f32_general_is_bit_exact(ctx, case):
    li, ld, ri, rd, oi = case
    print(f"[contract general f32] {li}{ld},{ri}{rd}->{oi}", flush=True)
    a, b = _operands(np.random.default_rng(len(li) * 7 + sum(ld)), ld, rd, False)
    if a.size > 8:
        a.flat[0] = np.nan  # a NaN product commits the canonical NaN
    want = oracle.contract_general(a, li, b, ri, oi)
    got = _device(ctx, L.F32, li, a, ri, b, oi)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("case", STRICT_CASES[:5], ids=lambda c: f"{c[0]},{c[2]}->{c[4]}")
def test_strict_bf16_general_is_bit_exact(ctx, case, silu):
    li, ld, ri, rd, oi = case
    print(f"[contract general bf16 silu={silu}] {li}{ld},{ri}{rd}->{oi}", flush=True)
    a, b = _operands(np.random.default_rng(sum(rd)), ld, rd, True)
    want = oracle.contract_general(a, li, b, ri, oi, silu=silu)
    got = _device(ctx, L.BF16, li, a, ri, b, oi, L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE)
    assert np.array_equal(got, want)


MFMA_CASES = [
    ("bhqd", (2, 8, 256, 64), "bkd", (2, 256, 64), "bhqk", "tiler_contract_bf16_t128_b"),
    ("bhqk", (2, 8, 256, 256), "bkd", (2, 256, 64), "bhqd", "tiler_contract_bf16_t128_b"),
    ("bhqd", (2, 8, 1, 128), "bkd", (2, 512, 128), "bhqk", "tiler_contract_bf16_skinny1_b"),
    ("bhqd", (2, 3, 37, 20), "bkd", (2, 45, 20), "bhqk", "tiler_contract_bf16_g128_k_b"),
    ("bhqd", (2, 32, 512, 64), "bkd", (2, 512, 64), "bhqk", "tiler_contract_bf16_t256_b"),
]


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("case", MFMA_CASES, ids=lambda c: c[5])
def test_mfma_batched_within_frobenius_bound(ctx, case, silu):
    li, ld, ri, rd, oi, kernel = case
    structure = S(li, ld, ri, rd, oi)
    symbols = realize(L.PROGRAM_CONTRACTION, (), dtype=L.BF16, structure=structure, permissions=RE,
                      variant=L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE, ctx=ctx).symbols
    assert symbols[-1] == (kernel.replace("bf16_", "bf16_silu_") if silu else kernel)
    print(f"[contract mfma silu={silu}] {li}{ld},{ri}{rd}->{oi} {symbols}", flush=True)
    a, b = _operands(np.random.default_rng(sum(ld) + sum(rd)), ld, rd, True)
    got = oracle.bf16_widen(_device(ctx, L.BF16, li, a, ri, b, oi, L.EPILOGUE_SILU if silu else L.EPILOGUE_NONE,
                                    RE)).astype(np.float64)
    want = oracle.contract_general(oracle.bf16_widen(a), li, oracle.bf16_widen(b), ri, oi)
    if silu:
        want = oracle.silu_f32(want.reshape(-1)).reshape(want.shape)
    want = want.astype(np.float64)
    per = want.shape[-2] * want.shape[-1]
    g, w = got.reshape(-1, per), want.reshape(-1, per)
    err = np.linalg.norm(g - w, axis=1) / np.maximum(np.linalg.norm(w, axis=1), 1e-30)
    assert err.max() <= 1e-2, err.max()


def test_general_contractions_through_the_route(ctx):
    rng = np.random.default_rng(9)
    # the strict form: its geometry rides in the constant slot
    a, b = _operands(rng, (2, 3, 5, 8), (2, 7, 8), False)
    rz = realize(L.PROGRAM_CONTRACTION, (), dtype=L.F32, structure=S("bhqd", a.shape, "bkd", b.shape, "bhqk"),
                 ctx=ctx)
    assert rz.slots[3][0] == L.SLOT_CONSTANT
    da, db, dy = ctx.to_device(a), ctx.to_device(b), ctx.alloc(2 * 3 * 5 * 7 * 4)
    try:
        route(ctx, rz, [da, db, dy, None])
        got = dy.download(np.float32, (2, 3, 5, 7))
    finally:
        for buf in (da, db, dy):
            buf.free()
    assert np.array_equal(bits(got), bits(oracle.contract_general(a, "bhqd", b, "bkd", "bhqk")))
    # the MFMA form with V stored [k, n]: the transpose workspace is a scratch slot
    p, v = _operands(rng, (2, 4, 64, 96), (2, 96, 32), True)
    rz = realize(L.PROGRAM_CONTRACTION, (), dtype=L.BF16, structure=S("bhqk", p.shape, "bkd", v.shape, "bhqd"),
                 permissions=RE, ctx=ctx)
    assert rz.symbols[0] == "tiler_transpose_bf16" and rz.slots[3][0] == L.SLOT_SCRATCH
    dp, dv, dy = ctx.to_device(p), ctx.to_device(v), ctx.alloc(2 * 4 * 64 * 32 * 2)
    try:
        route(ctx, rz, [dp, dv, dy, None])
        got = oracle.bf16_widen(dy.download(np.uint16, (2, 4, 64, 32))).astype(np.float64)
    finally:
        for buf in (dp, dv, dy):
            buf.free()
    want = oracle.contract_general(oracle.bf16_widen(p), "bhqk", oracle.bf16_widen(v), "bkd", "bhqd").astype(np.float64)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-2
