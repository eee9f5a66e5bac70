"""The governed digest and the payload's compilation subject, device-free.

`tiler_hip_digest` is FIPS 180-4 SHA-256 over a domain, fixed-width
qualifiers and one trailing run (tiler-digest/src/lib.rs:168-240). It is
pinned three ways:
- by the standard's published vectors;
- by the reference's own digest-of-digests over every message length
  0..192, a value Python's hashlib produced for the reference
  (tiler-digest/src/lib.rs:566-596; committed in tests/golden);
- by hashlib here, on random runs and on every padding branch.

`tiler_hip_payload_metadata` is checked by decoding it field by field in the
order of the reference's encoder (tiler-artifact/src/program/codec/
payload.rs:477-580). Every field is checked against what the build says it
compiled: the source bundle of the files on disk, the ordered flags, the
entry table. The reference holds no encoded PayloadMetadata to compare
against, so the encoding itself is parity unpinned beyond this structural
check. `tiler_hip_payload_identity` is its governed digest under the
reference's identity domain, recomputed here with hashlib.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import os

import numpy as np

from tiler_amd import _lib as L
from tiler_amd import build as B

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")))


def digest(domain: bytes, body: bytes, qualifiers=()) -> bytes:
    out = (ctypes.c_uint8 * 32)()
    qs = [ctypes.create_string_buffer(q, max(1, len(q))) for q in qualifiers]
    qp = (ctypes.c_void_p * max(1, len(qs)))(*[ctypes.cast(q, ctypes.c_void_p) for q in qs])
    ql = (ctypes.c_uint64 * max(1, len(qs)))(*[len(q) for q in qualifiers])
    st = L.lib().tiler_hip_digest(domain, len(domain), qp, ql, len(qs), body, len(body), out)
    assert st == L.OK
    return bytes(out)


def test_fips_180_4_published_vectors():
    v = GOLDEN["contraction"]["sha256_vectors"]
    assert digest(b"", b"").hex() == v[""]
    assert digest(b"", b"abc").hex() == v["abc"]
    assert digest(b"", b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq").hex() == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    assert digest(b"", b"a" * 1000000).hex() == \
        "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"


def test_reference_digest_of_every_padding_residue():
    g = GOLDEN["digest"]
    dom, byte = bytes.fromhex(g["domain_hex"]), bytes.fromhex(g["message_byte_hex"])
    acc = b"".join(digest(dom, byte * n) for n in range(g["max_length"] + 1))
    assert digest(b"", acc).hex() == g["digest_of_digests"]


def test_agrees_with_hashlib_on_random_runs_and_qualifiers():
    rng = np.random.default_rng(91)
    for n in list(range(0, 200)) + [1000, 4095, 4096, 4097, 100003]:
        body = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        dom = b"tiler.hip.test\0"
        q = [rng.integers(0, 256, int(rng.integers(1, 70)), dtype=np.uint8).tobytes() for _ in range(int(rng.integers(0, 4)))]
        assert digest(dom, body, q) == hashlib.sha256(dom + b"".join(q) + body).digest(), n


def test_qualifiers_are_plain_concatenation_and_separate_subjects():
    # a qualified digest with no qualifiers is the plain digest (lib.rs:598-615)
    assert digest(b"tiler.a\0", b"payload", []) == digest(b"tiler.a\0", b"payload")
    # the domain and a qualifier each separate subjects sharing a body (lib.rs:589-634)
    assert digest(b"tiler.a\0", b"payload") != digest(b"tiler.b\0", b"payload")
    assert digest(b"tiler.a\0", b"payload", [b"\x01"]) != digest(b"tiler.a\0", b"payload", [b"\x02"])
    # every padding branch: chunked and single-shot agree (lib.rs:546-560)
    for n in (54, 55, 56, 63, 64, 65, 119, 120, 127, 128):
        m = b"\x5a" * n
        assert digest(b"", m[n // 2:], [m[:n // 2]]) == hashlib.sha256(m).digest()


class _Cursor:
    def __init__(self, b: bytes):
        self.b, self.i = b, 0

    def take(self, n: int) -> bytes:
        assert self.i + n <= len(self.b), "ran past the end"
        out = self.b[self.i:self.i + n]
        self.i += n
        return out

    def u(self, width: int) -> int:
        return int.from_bytes(self.take(width), "big")

    def run(self) -> bytes:
        return self.take(self.u(8))

    def text(self) -> str:
        return self.run().decode()


def _metadata() -> bytes:
    need = ctypes.c_uint64()
    assert L.lib().tiler_hip_payload_metadata(None, 0, ctypes.byref(need)) == L.OK
    buf = ctypes.create_string_buffer(need.value)
    assert L.lib().tiler_hip_payload_metadata(buf, need.value - 1, ctypes.byref(need)) == L.REFUSE_CAPACITY
    assert L.lib().tiler_hip_payload_metadata(buf, need.value, ctypes.byref(need)) == L.OK
    return buf.raw[:need.value]


def _entries():
    out = []
    for i in range(10000):
        e = L.EntryInfo()
        if L.lib().tiler_hip_payload_entry(i, ctypes.byref(e)) != L.OK:
            break
        out.append((e.symbol.decode(), e.buffer_bindings))
    return out


def test_payload_metadata_decodes_to_what_was_compiled():
    c = _Cursor(_metadata())
    domain = b"tiler.artifact-envelope.payload-metadata.v1\0"
    assert c.take(len(domain)) == domain
    assert (c.u(2), c.u(2)) == (1, 0)                         # schema
    assert c.text() == "tiler.hip.source-bundle.v1"
    source = c.run()
    assert source == B.source_bundle()                         # the sources on disk, as built
    v = L.PayloadView()
    assert L.lib().tiler_hip_payload(ctypes.byref(v)) == L.OK
    assert ctypes.string_at(v.source, v.source_bytes) == source
    assert c.text() == "tiler.hip.rocm-clang"
    assert c.text() == v.target.decode() == "amdgcn-amd-amdhsa--gfx950"
    assert c.text() == v.backend.decode()
    assert c.text() == "hip-c++17"
    assert (c.u(2), c.u(2)) == (0, 0)                         # no deployment minimum
    assert c.u(8) == 1 and c.text() == "compiler" and c.text() == v.toolchain.decode()
    assert [c.text(), c.text(), c.text()] == ["", "", ""]     # no SDK
    flags = [c.text() for _ in range(c.u(8))]
    assert flags == B.DEVICE_FLAGS
    assert c.u(8) == 0                                          # no link flags
    entries = _entries()
    n = c.u(8)
    assert n == len(entries)
    decoded = []
    for _ in range(n):
        key, sym = c.text(), c.text()
        transports = [c.u(4) for _ in range(c.u(8))]
        assert key == sym
        decoded.append((sym, transports))
    assert [s for s, _ in decoded] == sorted(s for s, _ in entries)   # canonical key order
    buffers = dict(entries)
    assert all(t == list(range(buffers[s])) for s, t in decoded)
    obligations = [(c.text(), c.text()) for _ in range(c.u(8))]
    assert obligations == sorted(obligations) and ("tiler.hip.target-arch", "gfx950") in obligations
    assert c.take(1) == b"\x00"                                 # PayloadPlatform::Unversioned
    assert c.i == len(c.b)                                      # no trailing bytes


def test_payload_identity_is_the_governed_digest_of_the_metadata():
    out = (ctypes.c_uint8 * 32)()
    assert L.lib().tiler_hip_payload_identity(out) == L.OK
    want = hashlib.sha256(b"tiler.artifact-envelope.payload-identity.v1\0" + _metadata()).digest()
    assert bytes(out) == want


def test_bundle_lists_every_kernel_source_in_order():
    c = _Cursor(B.source_bundle())
    names = []
    for _ in range(c.u(8)):
        names.append(c.text())
        c.run()
    assert c.i == len(c.b) and names == sorted(names) and "tiler_kernels.hip" in names and "contract.hip" in names


def test_digest_refuses_missing_pointers():
    out = (ctypes.c_uint8 * 32)()
    assert L.lib().tiler_hip_digest(None, 4, None, None, 0, b"x", 1, out) == L.REFUSE_INVALID_ARGUMENT
    assert L.lib().tiler_hip_digest(b"d", 1, None, None, 1, b"x", 1, out) == L.REFUSE_INVALID_ARGUMENT


def _own_fields() -> dict:
    """This library's PayloadMetadata decoded into the test-side encoder's
    keywords (tests/envelope_fixture.payload_metadata)."""
    c = _Cursor(_metadata())
    c.take(len(b"tiler.artifact-envelope.payload-metadata.v1\0"))
    f = {"schema": (c.u(2), c.u(2)), "source_representation": c.text(), "source": c.run(), "toolchain": c.text(),
         "target": c.text(), "family": c.text(), "language": c.text(), "deployment": (c.u(2), c.u(2))}
    f["components"] = tuple((c.text(), c.text()) for _ in range(c.u(8)))
    f["sdk"] = (c.text(), c.text(), c.text())
    f["flags"] = tuple(c.text() for _ in range(c.u(8)))
    f["link_flags"] = tuple(c.text() for _ in range(c.u(8)))
    entries = []
    for _ in range(c.u(8)):
        key, sym = c.run(), c.text()
        entries.append((key, sym, tuple(c.u(4) for _ in range(c.u(8)))))
    f["entries"] = tuple(entries)
    f["obligations"] = tuple((c.text(), c.text()) for _ in range(c.u(8)))
    f["platform_tag"] = c.take(1)
    assert c.i == len(c.b)
    return f


def _correspondence(md: bytes):
    fact = ctypes.create_string_buffer(256)
    st = L.lib().tiler_hip_payload_correspondence(md, len(md), fact, 256)
    return st, fact.value.decode()


def test_payload_correspondence_names_the_first_disagreeing_fact():
    import envelope_fixture as F
    own = _own_fields()
    assert F.payload_metadata(**own) == _metadata()   # the test-side encoder reproduces the record exactly
    assert _correspondence(_metadata()) == (L.OK, "")
    variants = [
        ("source-representation", {"source_representation": "tiler.hip.source-bundle.v2"}),
        ("source", {"source": own["source"] + b" "}),
        ("toolchain", {"toolchain": "tiler.hip.other-clang"}),
        ("target", {"target": "amdgcn-amd-amdhsa--gfx942"}),
        ("components", {"components": (("compiler", "another clang"),)}),
        ("flags", {"flags": own["flags"][:-1]}),
        ("flags", {"link_flags": ("-shared",)}),
        ("entries", {"entries": own["entries"][:-1]}),
    ]
    for fact, change in variants:
        assert _correspondence(F.payload_metadata(**dict(own, **change))) == (L.REFUSE_PAYLOAD_MISMATCH, fact)
    # the order is the contract: of two disagreements the earlier fact is named
    both = dict(own, toolchain="tiler.hip.other-clang", entries=own["entries"][:-1])
    assert _correspondence(F.payload_metadata(**both)) == (L.REFUSE_PAYLOAD_MISMATCH, "toolchain")
    # facts outside the correspondence (family, language, obligations) do not move it
    assert _correspondence(F.payload_metadata(**dict(own, obligations=()))) == (L.OK, "")
    # a record that does not decode is malformed, with decode.rs's refusal
    st, why = _correspondence(_metadata()[:-3])
    assert st == L.REFUSE_MALFORMED_PAYLOAD and why
