"""Artifact envelopes: reading a TILERART envelope and routing the payload it
carries for this backend.

`read_envelope` calls `tiler_hip_read_envelope`. That reads the parts of an
encoded envelope a HIP loader needs (tiler-artifact/src/program/codec/
decode.rs:105-437, validate.rs:68-327):
- the 69-byte framing header;
- the manifest through its payload table;
- the section descriptors and the section stream;
- each carried payload's identity.
A refusal raises `Refusal(REFUSE_MALFORMED_PAYLOAD)`. Its diagnostic names the
ArtifactCodecError that decode.rs reports for the same bytes.

`select_payload` picks the carried payload this backend executes. Its
PayloadEntryMappings (payload.rs:589-640) name the kernel symbols a route may
dispatch. `tiler_amd.realize.route(..., payload=...)` prepares those symbols
from the payload's own code bytes rather than from the library's built-in code
object.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

from . import _lib as L
from .runtime import Refusal, _raise


def _bytes(p, n) -> bytes:
    return ctypes.string_at(p, n) if n else b""


def _text(p, n) -> str:
    return _bytes(p, n).decode()


@dataclass
class PayloadEntryMapping:
    key: bytes
    symbol: str
    transports: list


@dataclass
class PayloadSubject:
    """One payload's compilation subject (PayloadMetadata, payload.rs:228-424)."""
    source_representation: str
    source: bytes
    toolchain: str
    target: str
    family: str
    language: str
    deployment: tuple
    unversioned: bool
    component_count: int
    compile_flag_count: int
    link_flag_count: int
    obligation_count: int
    entries: list = field(default_factory=list)

    @property
    def symbols(self) -> list:
        return [e.symbol for e in self.entries]


@dataclass
class CarriedPayload:
    index: int
    backend: str
    representation: str
    schema: tuple
    digest: bytes
    profile_key: str
    carried: bool
    metadata: bytes = b""
    code: bytes = b""
    subject: PayloadSubject | None = None


@dataclass
class Envelope:
    total_bytes: int
    manifest_schema: tuple
    section_purposes: list
    feature_count: int
    input_count: int
    output_count: int
    provider_count: int
    payloads: list
    identity_digest: bytes
    _raw: L.Envelope = field(repr=False, default=None)
    _buf: object = field(repr=False, default=None)


def read_payload_metadata(data: bytes) -> PayloadSubject:
    """decode_metadata (payload.rs:589-660) through the C ABI."""
    buf = ctypes.create_string_buffer(bytes(data), max(1, len(data)))
    subject = L.PayloadSubject()
    diag = ctypes.create_string_buffer(256)
    lib = L.lib()
    _raise(lib.tiler_hip_read_payload_metadata(buf, len(data), ctypes.byref(subject), None, 0, diag, 256),
           "read_payload_metadata", diag.value.decode())
    n = subject.entry_count
    maps = (L.PayloadMapping * max(1, n))()
    _raise(lib.tiler_hip_read_payload_metadata(buf, len(data), ctypes.byref(subject), maps, n, diag, 256),
           "read_payload_metadata", diag.value.decode())
    entries = []
    for i in range(n):
        m = maps[i]
        raw = _bytes(m.transports, 4 * m.transport_count)
        entries.append(PayloadEntryMapping(
            _bytes(m.key, m.key_bytes), _text(m.symbol, m.symbol_bytes),
            [int.from_bytes(raw[4 * t:4 * t + 4], "big") for t in range(m.transport_count)]))
    return PayloadSubject(
        _text(subject.source_representation, subject.source_representation_bytes),
        _bytes(subject.source, subject.source_bytes),
        _text(subject.toolchain, subject.toolchain_bytes), _text(subject.target, subject.target_bytes),
        _text(subject.family, subject.family_bytes), _text(subject.language, subject.language_bytes),
        (subject.deployment_major, subject.deployment_minor), bool(subject.unversioned),
        subject.component_count, subject.compile_flag_count, subject.link_flag_count,
        subject.obligation_count, entries)


def read_envelope(data: bytes) -> Envelope:
    """Reads and checks one encoded envelope; raises Refusal on malformed bytes."""
    buf = ctypes.create_string_buffer(bytes(data), max(1, len(data)))
    raw = L.Envelope()
    diag = ctypes.create_string_buffer(512)
    _raise(L.lib().tiler_hip_read_envelope(buf, len(data), ctypes.byref(raw), diag, 512), "read_envelope",
           diag.value.decode())
    payloads = []
    for i in range(raw.payload_count):
        p = raw.payloads[i]
        payloads.append(CarriedPayload(
            i, _text(p.backend, p.backend_bytes), _text(p.representation, p.representation_bytes),
            (p.payload_schema_major, p.payload_schema_minor), _bytes(p.digest, p.digest_bytes),
            _text(p.profile_key, p.profile_key_bytes), bool(p.carried),
            _bytes(p.metadata, p.metadata_bytes), _bytes(p.code, p.code_bytes)))
    return Envelope(raw.total_bytes, (raw.manifest_schema_major, raw.manifest_schema_minor),
                    list(raw.section_purpose[:raw.section_count]), raw.feature_count, raw.input_count,
                    raw.output_count, raw.provider_count, payloads, bytes(raw.identity_digest), raw, buf)


def select_payload(envelope: Envelope) -> CarriedPayload:
    """The carried gfx950 code object of this backend, with its entry
    mappings; raises Refusal(REFUSE_FOREIGN_TARGET) when there is none."""
    index = ctypes.c_uint32()
    diag = ctypes.create_string_buffer(512)
    _raise(L.lib().tiler_hip_select_payload(ctypes.byref(envelope._raw), ctypes.byref(index), diag, 512),
           "select_payload", diag.value.decode())
    chosen = envelope.payloads[index.value]
    chosen.subject = read_payload_metadata(chosen.metadata)
    return chosen


__all__ = ["Envelope", "CarriedPayload", "PayloadSubject", "PayloadEntryMapping", "read_envelope",
           "read_payload_metadata", "select_payload", "Refusal"]
