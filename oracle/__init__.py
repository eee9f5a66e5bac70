"""CPU restatement of ``tiler-reference`` for the tiler-hip hot path.

TEST INFRASTRUCTURE ONLY. This package is the parity checker: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. The product (``libtiler_hip.so`` and the ``tiler_amd`` package) never
imports, links or executes anything here.

The reference (``/root/reference/crates/tiler-reference``) is Rust and no Rust
toolchain exists in this image, so ``oracle/_ref`` is never built; the
restatement in ``tiler_oracle.c`` is pinned by the reference's own golden
vectors (``tests/golden``) and by independent mathematical checks (see the
header of ``tiler_oracle.c`` for which check pins which function).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(BUILD_DIR, "libtiler_oracle.so")

OK = 0
INVALID_APPLICATION = 1
UNDECIDED = 2
GATHER_INDEX_OUT_OF_BOUNDS = 3

PRESERVE = 0
FLUSH_SIGN_PRESERVING = 1
FLUSH_POSITIVE_ZERO = 2

ROUND_MAJOR = 0
PARTICIPANT_MAJOR = 1

CANONICAL_F32_NAN = 0x7FC00000


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: oracle status {status}")
        self.status = status


def build() -> str:
    """Compiles the restatement with strict binary32 arithmetic (no FMA)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = f"{LIB_PATH}.{os.getpid()}.tmp"  # one per process: parallel test workers build at once
    cmd = [
        "gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
        "-Wall", "-o", tmp, os.path.join(HERE, "tiler_oracle.c"),
        os.path.join(HERE, "device_exp_audit.c"),
        "-lquadmath", "-lm", "-lpthread",
    ]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


_lib = None

_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
_SIGS = {
    "tiler_oracle_canonical_nan_bits": (_U32, []),
    "tiler_oracle_apply_subnormal_mode": (ctypes.c_float, [_I32, ctypes.c_float]),
    "tiler_oracle_maximum_f32": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
    "tiler_oracle_bf16_narrow": (ctypes.c_uint16, [ctypes.c_float]),
    "tiler_oracle_bf16_widen": (ctypes.c_float, [ctypes.c_uint16]),
    "tiler_oracle_bf16_narrow_array": (None, [_P, _U64, _P]),
    "tiler_oracle_bf16_widen_array": (None, [_P, _U64, _P]),
    "tiler_oracle_strict_sum_f32": (_I32, [_P, _U64, _U64, _U64, _P, _I32, _I32]),
    "tiler_oracle_strict_partial_sums_f32": (_I32, [_P, _U64, _U64, _U64, _U64, _P, _I32, _I32]),
    "tiler_oracle_strict_partitioned_sum_f32": (_I32, [_P, _U64, _U64, _U64, _U64, _P, _I32, _I32]),
    "tiler_oracle_cooperative_grouped_sum_f32": (
        _I32, [_P, _U64, _U64, _U64, _U64, _U64, _I32, _P, _I32, _I32]),
    "tiler_oracle_certified_exp_f32": (_I32, [ctypes.c_float, _P]),
    "tiler_oracle_device_exp_f32": (ctypes.c_float, [ctypes.c_float]),
    "tiler_oracle_audit_device_exp": (_I32, [_I32, _I32, _U32, _P, _U64, _P, _P, _P, _P]),
    "tiler_oracle_certified_rsqrt_f32": (_I32, [ctypes.c_float, _P]),
    "tiler_oracle_silu_f32": (_I32, [_P, _U64, _P, _I32, _I32]),
    "tiler_oracle_softmax_f32": (_I32, [_P, _U64, _U64, _U64, _P, _I32, _I32]),
    "tiler_oracle_rms_norm_f32": (_I32, [_P, _P, _U64, _U64, _U64, _U32, _P, _I32, _I32]),
    "tiler_oracle_gather": (_I32, [_P, _U64, _U64, _U64, _U32, _P, _U64, _I32, _P, _P, _P]),
    "tiler_oracle_dequantize_u4": (_I32, [_P, _U64, _U32, ctypes.c_uint8, _P]),
    "tiler_oracle_strict_affine_domain": (_I32, [_U32, ctypes.c_uint8]),
    "tiler_oracle_contract_strict_f32": (_I32, [_P, _P, _U64, _U64, _U64, _P, _U64, _U64, _U32]),
    "tiler_oracle_contract_general": (_I32, [_U32, _I32, _U32, _P, _P, _U32, _P, _P, _U32, _P, _P, _P, _P,
                                             _U32, _I32, _I32]),
    "tiler_oracle_row_grouped_sum_f32": (_I32, [_P, _U64, _U64, _U32, _U32, _P]),
    "tiler_oracle_grid_tree_sum_f32": (_I32, [_P, _U64, _U32, _P]),
    "tiler_oracle_rms_norm_grouped_f32": (_I32, [_P, _P, _U64, _U64, _U32, _I32, _U32, _U32, _P]),
    "tiler_oracle_softmax_grouped_f32": (_I32, [_P, _U64, _U64, _U32, _U32, _P]),
    "tiler_oracle_softmax_segmented_f32": (_I32, [_P, _U64, _U64, _U64, _U32, _U32, _P]),
    "tiler_oracle_expression_f32": (_I32, [_P, _P, _P, _U32, _U32, _P, _U64, _P, _I32, _I32]),
    "tiler_oracle_expression_bf16": (_I32, [_P, _P, _P, _U32, _U32, _P, _U64, _P, _I32, _I32]),
    "tiler_oracle_bf16_exact_add": (ctypes.c_uint16, [ctypes.c_uint16, ctypes.c_uint16]),
    "tiler_oracle_bf16_exact_multiply": (ctypes.c_uint16, [ctypes.c_uint16, ctypes.c_uint16]),
    "tiler_oracle_fold_f32": (_I32, [_P, _U32, _P, _U64, _U32, _U32, _U32, _P, _I32, _I32]),
}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _check(st: int, what: str):
    if st != OK:
        raise OracleError(st, what)


def f32_from_bits(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


def bits_of(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32)


# --- scalar helpers ----------------------------------------------------------

def maximum_f32(a: float, b: float) -> float:
    return lib().tiler_oracle_maximum_f32(a, b)


def certified_exp_f32(x: float) -> float:
    out = np.zeros(1, np.float32)
    _check(lib().tiler_oracle_certified_exp_f32(float(np.float32(x)), _ptr(out)), "certified_exp_f32")
    return out[0]


def certified_rsqrt_f32(x: float) -> float:
    out = np.zeros(1, np.float32)
    _check(lib().tiler_oracle_certified_rsqrt_f32(float(np.float32(x)), _ptr(out)),
           "certified_rsqrt_f32")
    return out[0]


def bf16_narrow(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    lib().tiler_oracle_bf16_narrow_array(_ptr(a), a.size, _ptr(out))
    return out


def bf16_widen(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.uint16))
    out = np.empty(a.shape, np.float32)
    lib().tiler_oracle_bf16_widen_array(_ptr(a), a.size, _ptr(out))
    return out


# --- families ----------------------------------------------------------------

def _geometry(shape, axis):
    shape = tuple(int(s) for s in shape)
    if not 0 <= axis < len(shape):
        raise OracleError(INVALID_APPLICATION, "axis outside the shape")
    outer = int(np.prod(shape[:axis], dtype=np.int64)) if axis else 1
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64)) if axis + 1 < len(shape) else 1
    return outer, shape[axis], inner


def strict_sum(values, shape, axis, input_mode=PRESERVE, result_mode=PRESERVE) -> np.ndarray:
    x = _f32(values).reshape(-1)
    outer, extent, inner = _geometry(shape, axis)
    if x.size != outer * extent * inner:
        raise OracleError(INVALID_APPLICATION, "payload length")
    out = np.empty(outer * inner, np.float32)
    _check(lib().tiler_oracle_strict_sum_f32(_ptr(x), outer, extent, inner, _ptr(out),
                                             input_mode, result_mode), "strict_sum")
    return out


def strict_partial_sums(values, rows, extent, partitions, per_partition,
                        input_mode=PRESERVE, result_mode=PRESERVE) -> np.ndarray:
    x = _f32(values).reshape(-1)
    out = np.empty(rows * partitions, np.float32)
    _check(lib().tiler_oracle_strict_partial_sums_f32(_ptr(x), rows, extent, partitions,
                                                      per_partition, _ptr(out), input_mode,
                                                      result_mode), "strict_partial_sums")
    return out


def strict_partitioned_sum(values, rows, extent, partitions, per_partition,
                           input_mode=PRESERVE, result_mode=PRESERVE) -> np.ndarray:
    x = _f32(values).reshape(-1)
    out = np.empty(rows, np.float32)
    _check(lib().tiler_oracle_strict_partitioned_sum_f32(_ptr(x), rows, extent, partitions,
                                                         per_partition, _ptr(out), input_mode,
                                                         result_mode), "strict_partitioned_sum")
    return out


def cooperative_grouped_sum(values, rows, extent, participants, per_partition, rounds,
                            layout=ROUND_MAJOR, input_mode=PRESERVE,
                            result_mode=PRESERVE) -> np.ndarray:
    x = _f32(values).reshape(-1)
    out = np.empty(rows, np.float32)
    _check(lib().tiler_oracle_cooperative_grouped_sum_f32(
        _ptr(x), rows, extent, participants, per_partition, rounds, layout, _ptr(out),
        input_mode, result_mode), "cooperative_grouped_sum")
    return out


def silu_f32(values, input_mode=PRESERVE, result_mode=PRESERVE) -> np.ndarray:
    x = _f32(values)
    out = np.empty(x.shape, np.float32)
    _check(lib().tiler_oracle_silu_f32(_ptr(x), x.size, _ptr(out), input_mode, result_mode),
           "silu_f32")
    return out


def softmax_f32(values, shape, axis, input_mode=PRESERVE, result_mode=PRESERVE) -> np.ndarray:
    x = _f32(values).reshape(-1)
    outer, extent, inner = _geometry(shape, axis)
    if x.size != outer * extent * inner:
        raise OracleError(INVALID_APPLICATION, "payload length")
    out = np.empty(x.size, np.float32)
    _check(lib().tiler_oracle_softmax_f32(_ptr(x), outer, extent, inner, _ptr(out), input_mode,
                                          result_mode), "softmax_f32")
    return out


def rms_norm_f32(values, weights, shape, axis, eps_bits, input_mode=PRESERVE,
                 result_mode=PRESERVE) -> np.ndarray:
    x = _f32(values).reshape(-1)
    w = _f32(weights).reshape(-1)
    outer, extent, inner = _geometry(shape, axis)
    if x.size != outer * extent * inner or w.size != x.size:
        raise OracleError(INVALID_APPLICATION, "payload length")
    out = np.empty(x.size, np.float32)
    _check(lib().tiler_oracle_rms_norm_f32(_ptr(x), _ptr(w), outer, extent, inner, eps_bits,
                                           _ptr(out), input_mode, result_mode), "rms_norm_f32")
    return out


def pack_u4(codes) -> np.ndarray:
    """U4 codes (values 0..15) packed LSB-first into U8 carriers with a zero
    tail (schedule/model.rs:682-696): element i is nibble i % 2 of byte i / 2."""
    c = np.asarray(codes, dtype=np.uint8).reshape(-1)
    if c.size and int(c.max()) > 15:
        raise ValueError("a U4 code above 15")
    padded = np.zeros(c.size + (c.size & 1), np.uint8)
    padded[:c.size] = c
    return (padded[0::2] | (padded[1::2] << 4)).astype(np.uint8)


def dequantize_u4(packed, n: int, scale_bits: int, zero_point: int) -> np.ndarray:
    """quantization.rs:218-246, :409-419 over n packed U4 codes; raises
    ValueError for a scale outside positive-normal-f32 or a zero point above
    15 (the value contract, quantization.rs:318-370)."""
    p = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    if p.size < (n + 1) // 2:
        raise ValueError("fewer carriers than codes")
    out = np.empty(n, np.float32)
    if lib().tiler_oracle_dequantize_u4(_ptr(p), n, scale_bits & 0xFFFFFFFF, zero_point & 0xFF, _ptr(out)) != OK:
        raise ValueError("strict-affine value outside its domain")
    return out


def strict_affine_domain(scale_bits: int, zero_point: int) -> int:
    """0 valid, 1 scale outside positive-normal-f32, 2 zero point above 15."""
    return lib().tiler_oracle_strict_affine_domain(scale_bits & 0xFFFFFFFF, zero_point & 0xFF)


def gather(source: np.ndarray, outer: int, gathered: int, inner: int, index,
           index_signed: bool = False):
    """Byte-exact gather; returns (output bytes, None) or (None, (position, value))."""
    src = np.ascontiguousarray(source)
    elem = src.dtype.itemsize
    idx = np.ascontiguousarray(np.asarray(index).astype(np.int64).astype(np.uint32)
                               if np.asarray(index).dtype != np.uint32 else np.asarray(index))
    count = idx.size
    out = np.empty(outer * count * inner, src.dtype)
    pos = ctypes.c_uint64(0)
    val = ctypes.c_int64(0)
    st = lib().tiler_oracle_gather(_ptr(src), outer, gathered, inner, elem, _ptr(idx), count,
                                   1 if index_signed else 0, _ptr(out), ctypes.byref(pos),
                                   ctypes.byref(val))
    if st == GATHER_INDEX_OUT_OF_BOUNDS:
        return None, (pos.value, val.value)
    _check(st, "gather")
    return out, None


def contract_strict_f32(a, b, m, n, k, row_begin=0, row_end=None, threads=None) -> np.ndarray:
    """``td,od->to``: C[m, n] from A[m, k] and B[n, k]; rows [row_begin, row_end)."""
    a = _f32(a).reshape(-1)
    b = _f32(b).reshape(-1)
    row_end = m if row_end is None else row_end
    c = np.zeros(m * n, np.float32)
    threads = threads or max(1, min(os.cpu_count() or 1, 16))
    _check(lib().tiler_oracle_contract_strict_f32(_ptr(a), _ptr(b), m, n, k, _ptr(c), row_begin,
                                                  row_end, threads), "contract_strict_f32")
    return c.reshape(m, n)


def contract_general(left, left_idx, right, right_idx, out_idx, silu=False, threads=None, input_mode=PRESERVE,
                     result_mode=PRESERVE) -> np.ndarray:
    """A binary contraction by index labels (ADR 0087), e.g. attention scores
    ``contract_general(q, "bhqd", k, "bkd", "bhqk")``: labels are strings of
    single characters or sequences of ints.  f32 operands give an f32 result;
    uint16 (bf16 bit patterns) operands give bf16 bits, optionally through
    the reference SiLU.  Shapes come from the operand arrays."""
    def labels(x):
        return np.array([ord(c) for c in x] if isinstance(x, str) else list(x), np.uint32)
    bf16 = left.dtype == np.uint16
    left = np.ascontiguousarray(left, np.uint16 if bf16 else np.float32)
    right = np.ascontiguousarray(right, np.uint16 if bf16 else np.float32)
    li, ri, oi = labels(left_idx), labels(right_idx), labels(out_idx)
    ld = np.array(left.shape, np.uint64)
    rd = np.array(right.shape, np.uint64)
    extent = {}
    for lab, d in list(zip(li, left.shape)) + list(zip(ri, right.shape)):
        extent.setdefault(int(lab), d)
    shape = tuple(extent.get(int(lab), 0) for lab in oi)
    out = np.zeros(shape, np.uint16 if bf16 else np.float32)
    threads = threads or max(1, min(os.cpu_count() or 1, 16))
    _check(lib().tiler_oracle_contract_general(1 if bf16 else 0, 1 if silu else 0, li.size, _ptr(li), _ptr(ld),
                                               ri.size, _ptr(ri), _ptr(rd), oi.size, _ptr(oi), _ptr(left),
                                               _ptr(right), _ptr(out), threads, input_mode, result_mode),
           "contract_general")
    return out


def row_grouped_sum(contributors, rows, extent, vec, waves) -> np.ndarray:
    x = _f32(contributors).reshape(-1)
    out = np.empty(rows, np.float32)
    _check(lib().tiler_oracle_row_grouped_sum_f32(_ptr(x), rows, extent, vec, waves, _ptr(out)),
           "row_grouped_sum")
    return out


def grid_tree_sum(values, blocks) -> float:
    x = _f32(values).reshape(-1)
    out = np.empty(1, np.float32)
    _check(lib().tiler_oracle_grid_tree_sum_f32(_ptr(x), x.size, blocks, _ptr(out)),
           "grid_tree_sum")
    return out[0]


def rms_norm_grouped(values, weights, rows, extent, eps_bits, weight_broadcast, vec,
                     waves) -> np.ndarray:
    x = _f32(values).reshape(-1)
    w = _f32(weights).reshape(-1)
    out = np.empty(rows * extent, np.float32)
    _check(lib().tiler_oracle_rms_norm_grouped_f32(_ptr(x), _ptr(w), rows, extent, eps_bits,
                                                   1 if weight_broadcast else 0, vec, waves,
                                                   _ptr(out)), "rms_norm_grouped")
    return out


def softmax_grouped(values, rows, extent, vec, waves, segment=0) -> np.ndarray:
    """Softmax whose exponent sum folds segments of `segment` elements (0: the
    whole row) by the (vec, waves) grouping, partials left-folded."""
    x = _f32(values).reshape(-1)
    out = np.empty(rows * extent, np.float32)
    _check(lib().tiler_oracle_softmax_segmented_f32(_ptr(x), rows, extent, segment, vec, waves,
                                                    _ptr(out)), "softmax_grouped")
    return out


def audit_device_exp(margin_log2: int = -48, threads: int = 8, cap: int = 1 << 16,
                     planted_log2: int = 0) -> dict:
    """Exhaustive audit of the device's binary32 exp (device_exp_audit.c):
    returns the inputs near a rounding boundary (sorted), how many inputs were
    scanned, and how many of the near-boundary ones differ from the certified
    exp."""
    hard = np.zeros(cap, dtype=np.float32)
    nh, nc, nm = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    first = ctypes.c_float()
    _check(lib().tiler_oracle_audit_device_exp(margin_log2, planted_log2, threads, _ptr(hard), cap,
                                               ctypes.byref(nh), ctypes.byref(nc),
                                               ctypes.byref(nm), ctypes.byref(first)),
           "audit_device_exp")
    kept = np.sort(hard[:min(nh.value, cap)])
    return {"hard": kept, "hard_count": nh.value, "checked": nc.value,
            "mismatches": nm.value, "first_mismatch": first.value}


def device_exp_f32(s: float) -> float:
    """The device's binary32 exp, restated (see audit_device_exp)."""
    return float(lib().tiler_oracle_device_exp_f32(s))


def _node_arrays(nodes):
    ops = np.array([nd[0] for nd in nodes], dtype=np.uint32)
    a = np.array([nd[1] for nd in nodes], dtype=np.uint32)
    b = np.array([nd[2] if len(nd) > 2 else 0 for nd in nodes], dtype=np.uint32)
    return ops, a, b


def expression_f32(nodes, inputs, root=None, input_mode=PRESERVE, result_mode=PRESERVE) -> np.ndarray:
    """A pointwise f32 expression DAG (pointwise.rs:74-140): `nodes` are
    (op, a, b) triples (0 input, 1 constant, 2 add, 3 multiply, 4 divide,
    5 exp, 6 rsqrt), `inputs` one array per access ordinal."""
    ops, a, b = _node_arrays(nodes)
    ins = [_f32(x).reshape(-1) for x in inputs]
    n = ins[0].size if ins else 0
    ptrs = (ctypes.c_void_p * max(1, len(ins)))(*[x.ctypes.data for x in ins])
    y = np.empty(n, np.float32)
    root = len(nodes) - 1 if root is None else root
    _check(lib().tiler_oracle_expression_f32(_ptr(ops), _ptr(a), _ptr(b), len(nodes), root, ptrs, n, _ptr(y),
                                             input_mode, result_mode), "expression_f32")
    return y


def expression_bf16(nodes, inputs, root=None, input_mode=PRESERVE, result_mode=PRESERVE) -> np.ndarray:
    """A pointwise bf16 expression DAG (pointwise_bf16.rs): inputs and result
    as bf16 bit patterns (uint16); the subnormal modes act on operand and
    rounded-result encodings (bf16.rs:517-533)."""
    ops, a, b = _node_arrays(nodes)
    ins = [np.ascontiguousarray(x, dtype=np.uint16).reshape(-1) for x in inputs]
    n = ins[0].size if ins else 0
    ptrs = (ctypes.c_void_p * max(1, len(ins)))(*[x.ctypes.data for x in ins])
    y = np.empty(n, np.uint16)
    root = len(nodes) - 1 if root is None else root
    _check(lib().tiler_oracle_expression_bf16(_ptr(ops), _ptr(a), _ptr(b), len(nodes), root, ptrs, n, _ptr(y),
                                              input_mode, result_mode), "expression_bf16")
    return y


def bf16_exact_add(x: int, z: int) -> int:
    return int(lib().tiler_oracle_bf16_exact_add(x, z))


def bf16_exact_multiply(x: int, z: int) -> int:
    return int(lib().tiler_oracle_bf16_exact_multiply(x, z))


def fold_f32(values, dims, reduced_axes, op=0, scale_bits=0, bias_bits=0, input_mode=PRESERVE,
             result_mode=PRESERVE) -> np.ndarray:
    """The strict serial fold of a dense tensor over `reduced_axes` (op 0 sum,
    1 squared, 2 scale-bias, 3 maximum); the kept axes in order."""
    x = _f32(values).reshape(-1)
    d = np.ascontiguousarray(dims, dtype=np.uint64)
    mask = sum(1 << ax for ax in reduced_axes)
    outputs = int(np.prod([dims[i] for i in range(len(dims)) if not (mask >> i) & 1], dtype=np.int64))
    out = np.empty(outputs, np.float32)
    _check(lib().tiler_oracle_fold_f32(_ptr(x), len(dims), _ptr(d), mask, op, scale_bits, bias_bits, _ptr(out),
                                       input_mode, result_mode), "fold_f32")
    return out
