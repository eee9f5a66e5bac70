"""GPU parity for the strict-affine U4 dequantization
(ScalarProgram::StrictAffineU4Dequantize, tiler-ir/src/schedule/model.rs:682-696;
tiler-reference/src/quantization.rs:218-246, :409-419):

* the direct entry point over every (code, zero point) pair at boundary
  scales, random tensors with ragged tails, and unaligned storage -- bit for
  bit with oracle.dequantize_u4;
* its pre-commit refusals for a scale outside positive-normal-f32 and a zero
  point above 15 (the value contract, quantization.rs:318-370);
* the realized region through the RuntimeAdapter stages, both kernel forms,
  and the device-side domain verdict for operands read from slots.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import bits, golden
from tiler_amd import _lib as L
from tiler_amd import families
from tiler_amd.realize import realize, route
from tiler_amd.runtime import Failure, Refusal

pytestmark = pytest.mark.gpu

G = golden()["strict_affine_u4"]
SCALES = [0x00800000, 0x3F000000, 0x3DCCCCCD, 0x7F7FFFFF, 0x7E800001, 0x0E5A3C11]


@pytest.mark.parametrize("scale_bits", SCALES)
def test_every_code_and_zero_point(ctx, scale_bits):
    codes = np.tile(np.arange(16, dtype=np.uint8), 4)  # 64 codes: the vector form
    packed = oracle.pack_u4(codes)
    for zp in range(16):
        got = families.dequantize_u4(packed, codes.size, scale_bits, zp, ctx=ctx)
        want = oracle.dequantize_u4(packed, codes.size, scale_bits, zp)
        assert np.array_equal(bits(got), bits(want)), (hex(scale_bits), zp)


def test_reference_rows(ctx):
    for row in G["dequantize_one"]:
        got = families.dequantize_u4(oracle.pack_u4([row["code"]]), 1, int(row["scale_bits"], 16),
                                     row["zero_point"], ctx=ctx)
        assert int(bits(got)[0]) == int(row["value_bits"], 16), row["source"]


@pytest.mark.parametrize("n", [1, 15, 16, 17, 1000, 4096, 2048 * 3 + 1030, (1 << 22) + 5, 1 << 24])
def test_random_codes_with_ragged_tails(ctx, n):
    """Whole 2048-element wave blocks (tiler_dequantize_u4_f32_w), then
    4-element chunks (_v4) and single elements for the rest."""
    rng = np.random.default_rng(n)
    codes = rng.integers(0, 16, n, dtype=np.uint8)
    packed = oracle.pack_u4(codes)
    scale = int(np.float32(rng.uniform(1e-3, 4.0)).view(np.uint32))
    zp = int(rng.integers(0, 16))
    print(f"[dequantize] n={n} scale=0x{scale:08x} zp={zp}", flush=True)
    got = families.dequantize_u4(packed, n, scale, zp, ctx=ctx)
    assert np.array_equal(bits(got), bits(oracle.dequantize_u4(packed, n, scale, zp)))


def test_unaligned_storage_takes_the_scalar_form(ctx):
    """Codes and output one byte / four bytes past 16-byte alignment: the
    scalar kernel serves the whole tensor, with the same bits."""
    n = 4099
    rng = np.random.default_rng(7)
    codes = rng.integers(0, 16, n, dtype=np.uint8)
    packed = oracle.pack_u4(codes)
    dc = ctx.alloc(packed.size + 16)
    dy = ctx.alloc(4 * n + 16)
    try:
        dc.offset(1).upload(packed)
        ctx.fill_u32(dy, 0x7FC00001, n + 4)
        ctx.dequantize_u4(dc.offset(1), n, 0x3F400000, 5, dy.offset(4))
        ctx.synchronize()
        raw = dy.download(np.uint32, (n + 4,))
        assert raw[0] == 0x7FC00001 and (raw[n + 1:] == 0x7FC00001).all()  # nothing outside y
        want = oracle.dequantize_u4(packed, n, 0x3F400000, 5)
        assert np.array_equal(raw[1:n + 1], bits(want))
    finally:
        dc.free()
        dy.free()


def test_out_of_domain_operands_refuse_before_commit(ctx):
    packed = oracle.pack_u4([7, 8])
    for b in G["invalid_scale_bits"]["bits"]:
        with pytest.raises(Refusal) as e:
            families.dequantize_u4(packed, 2, int(b, 16), 8, ctx=ctx)
        assert e.value.status == L.REFUSE_INVALID_ARGUMENT, b
    with pytest.raises(Refusal):
        families.dequantize_u4(packed, 2, 0x3F000000, 16, ctx=ctx)
    ok = families.dequantize_u4(packed, 2, int(G["smallest_normal_scale_bits"]["bits"], 16), 8, ctx=ctx)
    assert bits(ok).tolist() == bits(oracle.dequantize_u4(packed, 2, 0x00800000, 8)).tolist()


@pytest.mark.parametrize("n,form", [(4096, "tiler_dequantize_u4_f32_w_slots"),
                                    (6148, "tiler_dequantize_u4_f32_v4_slots"),
                                    (4097, "tiler_dequantize_u4_f32_slots")])
def test_realized_region(ctx, n, form):
    rng = np.random.default_rng(n + 3)
    codes = rng.integers(0, 16, n, dtype=np.uint8)
    packed = oracle.pack_u4(codes)
    rz = realize(L.PROGRAM_DEQUANTIZE_U4, (n,), flags=L.REGION_ALIGNED16, ctx=ctx)
    assert rz.symbols == [form], rz.symbols
    scale = np.array([0x3E99999A], np.uint32)
    bufs = [ctx.to_device(packed), ctx.to_device(scale), ctx.to_device(np.array([3], np.uint8)),
            ctx.alloc(4 * n), None]
    try:
        route(ctx, rz, bufs)
        got = bufs[3].download(np.float32, (n,))
        assert np.array_equal(bits(got), bits(oracle.dequantize_u4(packed, n, 0x3E99999A, 3)))
        # operands outside their domain, read from the slots: a post-commit
        # failure, and the output keeps what it held
        for scale_bits, zp, what in ((0x00000001, 3, "scale"), (0x3F800000, 16, "zero point")):
            bufs[1].upload(np.array([scale_bits], np.uint32))
            bufs[2].upload(np.array([zp], np.uint8))
            ctx.fill_u32(bufs[3], 0x7FC00001, n)
            ctx.synchronize()
            with pytest.raises(Failure) as e:
                route(ctx, rz, bufs)
            assert e.value.status == L.FAIL_VALUE_DOMAIN and what in str(e.value), str(e.value)
            assert (bufs[3].download(np.uint32, (n,)) == 0x7FC00001).all()
    finally:
        for b in bufs:
            if b is not None:
                b.free()
