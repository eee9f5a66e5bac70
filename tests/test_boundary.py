"""The C-ABI boundary without a GPU: the library loads, exports every symbol
include/tiler_hip.h declares, and its device-free stages behave (target
profile, payload view and entry mapping, validate-from-bytes refusals, the
pre-commit gather bound, binding without a device)."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

import tiler_amd
from tiler_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tiler_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tiler_hip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the whole header too
    assert not [n for n in names if n not in L.SIGNATURES]


def test_target_profile_is_the_gfx950_profile():
    p = tiler_amd.profile()
    assert p["profile_key"] == "tiler.hip.gfx950.profile-v1"
    assert p["target_triple"] == "amdgcn-amd-amdhsa--gfx950"
    assert p["wavefront_size"] == 64 and p["subgroup_width"] == 64
    assert p["compute_units"] == 256 and p["xcds"] == 8
    assert p["lds_bytes_per_workgroup"] == 160 * 1024
    assert p["hbm_bytes_per_second"] == 8.0e12
    assert p["mfma_bf16_dense_flops"] == 2.5e15
    assert p["f32_subnormals_preserved"] == 1


def _payload():
    v = L.PayloadView()
    assert L.lib().tiler_hip_payload(ctypes.byref(v)) == L.OK
    return v, ctypes.string_at(v.code, v.code_bytes)


def test_payload_view_and_entry_mapping():
    v, code = _payload()
    assert v.backend == b"tiler.hip"
    assert v.representation == b"tiler.hip.gfx950.code-object-v1"
    assert v.target == b"amdgcn-amd-amdhsa--gfx950"
    assert b"clang" in v.toolchain and b"gfx950" in v.flags and b"-ffp-contract=off" in v.flags
    assert code[:4] == b"\x7fELF"
    seen = set()
    for i in range(v.entry_count):
        e = L.EntryInfo()
        assert L.lib().tiler_hip_payload_entry(i, ctypes.byref(e)) == L.OK
        assert e.symbol not in seen
        seen.add(e.symbol)
        assert e.kernarg_bytes > 0 and e.buffer_bindings >= 1
        d = ctypes.create_string_buffer(256)
        assert L.lib().tiler_hip_validate_payload(code, len(code), e.symbol, e.kernarg_bytes, d,
                                                  256) == L.OK, d.value
    e = L.EntryInfo()
    assert L.lib().tiler_hip_payload_entry(v.entry_count, ctypes.byref(e)) == L.REFUSE_INVALID_ARGUMENT


@pytest.mark.parametrize("mutation,status", [
    ("truncate", L.REFUSE_MALFORMED_PAYLOAD),
    ("magic", L.REFUSE_MALFORMED_PAYLOAD),
    ("machine", L.REFUSE_MALFORMED_PAYLOAD),
    ("foreign-arch", L.REFUSE_MALFORMED_PAYLOAD),
    ("absent-symbol", L.REFUSE_ABSENT_SYMBOL),
    ("kernarg-mismatch", L.REFUSE_BINDING_MISMATCH),
])
def test_validate_payload_refuses_from_bytes(mutation, status):
    _, code = _payload()
    b = bytearray(code)
    sym, ka = b"tiler_softmax_f32_ch8", 0
    if mutation == "truncate":
        b = b[:200]
    elif mutation == "magic":
        b[1] = ord("X")
    elif mutation == "machine":
        b[18] = 62  # EM_X86_64
    elif mutation == "foreign-arch":
        b[48] = 0x4C  # gfx942
    elif mutation == "absent-symbol":
        sym = b"tiler_kernel_that_does_not_exist"
    elif mutation == "kernarg-mismatch":
        ka = 12345
    d = ctypes.create_string_buffer(256)
    buf = bytes(b)
    assert L.lib().tiler_hip_validate_payload(buf, len(buf), sym, ka, d, 256) == status
    assert d.value  # the first disagreeing fact is named


def test_pre_commit_gather_bound_names_first_position():
    with pytest.raises(tiler_amd.GatherIndexOutOfBounds) as err:
        tiler_amd.validate_gather_index(np.asarray([1, 2, 9, 3], np.uint32), 5, False)
    assert err.value.position == 2 and err.value.value == 9 and err.value.fallback_permitted
    with pytest.raises(tiler_amd.GatherIndexOutOfBounds) as err:
        tiler_amd.validate_gather_index(np.asarray([0, -1], np.int32).view(np.uint32), 5, True)
    assert err.value.position == 1 and err.value.value == -1
    tiler_amd.validate_gather_index(np.asarray([0, 4], np.uint32), 5, False)
    tiler_amd.validate_gather_index(np.zeros(0, np.uint32), 5, False)


def test_row_grouping_is_declared_device_free():
    import tiler_amd
    assert tiler_amd.row_grouping(L.ROWS_RMS_NORM, L.BF16, 4096) == (8, 1, 0)
    assert tiler_amd.row_grouping(L.ROWS_RMS_NORM, L.BF16, 8192) == (8, 1, 0)
    assert tiler_amd.row_grouping(L.ROWS_RMS_NORM, L.BF16, 8193) == (8, 16, 0)
    assert tiler_amd.row_grouping(L.ROWS_RMS_NORM, L.F32, 100000) == (4, 16, 0)
    assert tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.F32, 2048) == (4, 1, 0)
    assert tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.F32, 8192) == (4, 1, 0)
    assert tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.F32, 8193) == (4, 4, 8192)
    assert tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.F32, 131072) == (4, 4, 8192)
    assert tiler_amd.row_grouping(L.ROWS_SUM, L.F32, 10) == (4, 4, 0)
    with pytest.raises(tiler_amd.Refusal):
        tiler_amd.row_grouping(L.ROWS_SOFTMAX, L.BF16, 2048)
    with pytest.raises(tiler_amd.Refusal):
        tiler_amd.row_grouping(7, L.F32, 2048)


def test_bind_refuses_without_a_device_here():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present; covered by the gpu tests")
    with pytest.raises(tiler_amd.Refusal) as err:
        tiler_amd.Context(0)
    assert err.value.status == L.REFUSE_NO_DEVICE and err.value.fallback_permitted


def test_status_classes():
    refusal = tiler_amd.Refusal(L.REFUSE_CAPACITY, "x")
    failure = tiler_amd.Failure(L.FAIL_LAUNCH, "y")
    assert refusal.fallback_permitted and not failure.fallback_permitted
