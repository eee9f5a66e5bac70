"""Shared test helpers: golden-vector loading, bit views, the reference's
SplitMix64 operand stream, and f64 comparators."""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name: str = "reference_vectors.json") -> dict:
    with open(os.path.join(GOLDEN, name)) as fh:
        return json.load(fh)


def hexbits(v) -> int:
    return int(v, 16) if isinstance(v, str) else int(v)


def f32(bits) -> np.ndarray:
    return np.asarray([hexbits(b) for b in bits], dtype=np.uint32).view(np.float32)


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32)


def values_of(case: dict, key: str) -> np.ndarray:
    """A case's operand either as decimal values (`key`) or bit patterns (`key_bits`)."""
    if key + "_bits" in case:
        return f32(case[key + "_bits"])
    if key + "_fill_bits" in case:
        n = int(np.prod(case["shape"]))
        return f32([case[key + "_fill_bits"]] * n)
    if key + "_fill" in case:
        n = int(np.prod(case["shape"]))
        return np.full(n, case[key + "_fill"], dtype=np.float32)
    return np.asarray(case[key], dtype=np.float32)


def expected_bits(case: dict, key: str = "y") -> np.ndarray:
    if key + "_bits" in case:
        return np.asarray([hexbits(b) for b in case[key + "_bits"]], dtype=np.uint32)
    n = int(np.prod(case["shape"]))
    return np.full(n, hexbits(case[key + "_fill_bits"]), dtype=np.uint32)


# -- tiler-reference/tests/contraction_profile_cells.rs:260-290 operand stream --
def splitmix_operands(seed: int, count: int) -> np.ndarray:
    """prng_value(seed, i) for i < count: m * 2^-24, m in [-2^23, 2^23)."""
    idx = np.arange(count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = np.uint64(seed) + idx * np.uint64(0x2545F4914F6CDD1D)
        x = x + np.uint64(0x9E3779B97F4A7C15)
        z = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    field = ((z >> np.uint64(40)) & np.uint64(0xFFFFFF)).astype(np.int64)
    return (field - 8388608).astype(np.float32) * np.float32(1.0 / 16777216.0)


def splitmix_scalar(seed: int, index: int) -> float:
    m64 = (1 << 64) - 1
    x = (seed + index * 0x2545F4914F6CDD1D) & m64
    x = (x + 0x9E3779B97F4A7C15) & m64
    z = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & m64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m64
    z ^= z >> 31
    return float(np.float32(((z >> 40) & 0xFFFFFF) - 8388608) * np.float32(1.0 / 16777216.0))


def sha256_le_f32(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<f4").tobytes()).hexdigest()


# -- bf16 helpers (numpy; test side) --
def bf16_widen(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << np.uint32(16)).view(np.float32)


def bf16_ulp_distance(got_bits: np.ndarray, ref64: np.ndarray) -> np.ndarray:
    """|got - ref| in units of the bf16 ulp at ref (exponent of |ref|)."""
    got = bf16_widen(got_bits).astype(np.float64)
    ref = np.asarray(ref64, dtype=np.float64)
    mag = np.abs(ref)
    e = np.floor(np.log2(np.where(mag > 0, mag, 1.0)))
    e = np.maximum(e, -126.0)  # below 2^-126 the bf16 quantum stays 2^-133
    ulp = np.exp2(e - 7.0)
    return np.abs(got - ref) / ulp
