"""CPU: every kernel of the reference's emitter goldens has a realization.

tiler-metal/goldens/*.metal are the thirteen VerifiedKernel shapes the
reference's emitter is pinned on (tiler-metal/src/emit.rs:647-840 writes
them).  Each one is a region here -- its ScalarProgram, topology and the
golden's own extents -- and tiler_hip_realize must realize it.  The goldens'
index arithmetic is transcribed below (as loops over the golden's own
buffers) for the five that no other test names, and the oracle must agree
with the transcription bit for bit; tests/test_gpu_goldens.py runs the same
regions on the device.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tiler_amd import _lib as L
from tiler_amd.realize import realize

RE = L.PERMITS_REASSOCIATION
S = L.contraction_structure

# (golden, region keywords, the realized symbols)
GOLDENS = [
    ("contraction_attention_score", dict(program=L.PROGRAM_CONTRACTION, extents=(),
                                         structure=S("bhqd", (2, 2, 3, 4), "bkd", (2, 5, 4), "bhqk")),
     ["tiler_contract_general_f32"]),
    ("contraction_attention_value", dict(program=L.PROGRAM_CONTRACTION, extents=(),
                                         structure=S("bhqk", (2, 2, 3, 5), "bkd", (2, 5, 4), "bhqd")),
     ["tiler_contract_general_f32"]),
    ("contraction_strict_tensor", dict(program=L.PROGRAM_CONTRACTION, extents=(2, 3, 4)),
     ["tiler_contract_strict_f32"]),
    ("contraction_tiled_cooperative", dict(program=L.PROGRAM_CONTRACTION, extents=(10, 32, 32)),
     ["tiler_contract_strict_f32"]),
    ("cooperative_workgroup_reduction", dict(program=L.PROGRAM_SERIAL_SUM, extents=(2, 6), topology=L.SUM_COOPERATIVE,
                                             grouping=(3, 2, 1), permissions=RE),
     ["tiler_sum_f32_cooperative"]),
    ("elementary_silu_activation", dict(program=L.PROGRAM_POINTWISE, extents=(1024,), variant=L.MAP_SILU),
     ["tiler_map_f32_v4_op1"]),
    ("pointwise_scale_bias", dict(program=L.PROGRAM_EXPRESSION, extents=(1024,),
                                  nodes=[(0, 0, 0), (1, 0x40000000, 0), (3, 0, 1), (1, 0x3F800000, 0), (2, 2, 3)]),
     ["tiler_expr_f32_r16_i1"]),
    ("pointwise_scale_bias_bf16", dict(program=L.PROGRAM_EXPRESSION, extents=(1024,), dtype=L.BF16,
                                       nodes=[(0, 0, 0), (1, 0x4000, 0), (3, 0, 1), (1, 0x3F80, 0), (2, 2, 3)]),
     ["tiler_expr_bf16_r16_i1"]),
    ("reduction_fused_multiply_add", dict(program=L.PROGRAM_FOLD, extents=(2, 3), rank=2, grouping=(0b10,),
                                          variant=L.FOLD_FMA, scalars=(0x40000000, 0x3F800000)),
     ["tiler_fold_fma_f32"]),
    ("reduction_multi_axis", dict(program=L.PROGRAM_FOLD, extents=(2, 3, 4), rank=3, grouping=(0b110,)),
     ["tiler_fold_sum_f32"]),
    ("reduction_single_axis", dict(program=L.PROGRAM_SERIAL_SUM, extents=(2, 3)),
     ["tiler_sum_f32_serial"]),
    ("structural_mirrored_reindex", dict(program=L.PROGRAM_REINDEX, extents=(2, 2), rank=2, strides=(2, -1),
                                         grouping=(4, 1), variant=4),
     ["tiler_broadcast_u32"]),
    ("structural_widening_broadcast", dict(program=L.PROGRAM_BROADCAST, extents=(2, 2), rank=2, strides=(0, 1),
                                           grouping=(2,), variant=4),
     None),
]


def test_every_golden_is_realized():
    assert len({g for g, _, _ in GOLDENS}) == 13  # the reference's whole golden set
    for name, kw, symbols in GOLDENS:
        kw = dict(kw)
        program, extents = kw.pop("program"), kw.pop("extents")
        rz = realize(program, extents, **kw)
        assert rz.dispatches, name
        if symbols is not None:
            assert rz.symbols == symbols, (name, rz.symbols)


# The goldens' arithmetic, transcribed from their kernels: f32 products and
# sums one rounding each, in the loop order the kernel runs.

def golden_strict_tensor(b0, b1):
    # contraction_strict_tensor.metal: v0 < 6; b0[(v0/3)*4 + k] * b1[(v0%3)*4 + k], k = 0..3, seeded by k = 0
    out = np.empty(6, np.float32)
    for v0 in range(6):
        acc = np.float32(b0[(v0 // 3) * 4] * b1[(v0 % 3) * 4])
        for k in range(1, 4):
            acc = np.float32(acc + np.float32(b0[(v0 // 3) * 4 + k] * b1[(v0 % 3) * 4 + k]))
        out[v0] = acc
    return out


def golden_tiled_cooperative(b0, b1):
    # contraction_tiled_cooperative.metal: 16 x 16 tiles over a 10 x 32 output, K = 32 in two rounds of 16;
    # thread (row v15, column v16) folds tg0[row][k] * tg1[col][k] in ascending k, the first product the seed;
    # b0 is [10][32], b1 [32][32] (both k-contiguous), guarded loads zero-fill outside the output
    out = np.empty((10, 32), np.float32)
    for m in range(10):
        for n in range(32):
            acc = np.float32(b0[m * 32] * b1[n * 32])
            for k in range(1, 32):
                acc = np.float32(acc + np.float32(b0[m * 32 + k] * b1[n * 32 + k]))
            out[m, n] = acc
    return out.reshape(-1)


def golden_cooperative(b0):
    # cooperative_workgroup_reduction.metal: 2 outputs of 6; participant p (< 3) folds b0[o*6 + p*2 + j], j < 2;
    # participant 0 folds the three staged partials in ascending order
    out = np.empty(2, np.float32)
    for o in range(2):
        staged = []
        for p in range(3):
            acc = np.float32(b0[o * 6 + p * 2])
            acc = np.float32(acc + b0[o * 6 + p * 2 + 1])
            staged.append(acc)
        acc = staged[0]
        for p in range(1, 3):
            acc = np.float32(acc + staged[p])
        out[o] = acc
    return out


def golden_single_axis(b0):
    # reduction_single_axis.metal: v0 < 2; b0[v0*3] seeds, + b0[v0*3 + j], j = 1, 2
    out = np.empty(2, np.float32)
    for v0 in range(2):
        acc = np.float32(b0[v0 * 3])
        for j in range(1, 3):
            acc = np.float32(acc + b0[v0 * 3 + j])
        out[v0] = acc
    return out


def golden_widening_broadcast(b0):
    # structural_widening_broadcast.metal: v0 < 4; b1[v0] = b0[v0 % 2]
    return np.array([b0[v0 % 2] for v0 in range(4)], np.float32)


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("seed", range(3))
def test_oracle_matches_the_transcribed_goldens(seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(8).astype(np.float32)
    b = rng.standard_normal(12).astype(np.float32)
    assert np.array_equal(_bits(golden_strict_tensor(a, b)), _bits(oracle.contract_strict_f32(a, b, 2, 3, 4).reshape(-1)))
    a = rng.standard_normal(320).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    assert np.array_equal(_bits(golden_tiled_cooperative(a, b)),
                          _bits(oracle.contract_strict_f32(a, b, 10, 32, 32).reshape(-1)))
    x = (rng.standard_normal(12) * np.exp2(rng.integers(-20, 20, 12))).astype(np.float32)
    assert np.array_equal(_bits(golden_cooperative(x)), _bits(oracle.cooperative_grouped_sum(x, 2, 6, 3, 2, 1)))
    y = (rng.standard_normal(6) * np.exp2(rng.integers(-20, 20, 6))).astype(np.float32)
    assert np.array_equal(_bits(golden_single_axis(y)), _bits(oracle.strict_sum(y, (2, 3), 1)))
    # the cooperative grouping differs from the serial fold on values where order matters
    big = np.array([2.0 ** 25, 1, -(2.0 ** 25), 1, 1, 1] * 2, np.float32)
    assert not np.array_equal(_bits(golden_cooperative(big)), _bits(oracle.strict_sum(big, (2, 6), 1)))
