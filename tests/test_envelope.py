"""The artifact envelope reader (`tiler_hip_read_envelope`,
`tiler_hip_read_payload_metadata`, `tiler_hip_select_payload`), device-free.

The cases follow the reference's own codec tests:
- tiler-artifact/src/program/codec/tests/byte_corruption.rs: every
  single-byte corruption and every truncation is refused; trailing bytes;
  manifest and section digests; tags refused by name; length prefixes;
  format, algorithm and schema versions; required features;
- carried_payloads.rs and payload_sections.rs: payload identity, section
  purposes, references and order.
Each refusal is checked by the ArtifactCodecError name decode.rs reports.

The envelopes come from `tests/envelope_fixture.py`, which restates the
reference encoder. hashlib computes its digests, independently of the
library's SHA-256. The reference ships no encoded envelope, and its encoder
needs a Rust toolchain this image does not have. So the reader is pinned by:
- the reference's constants, restated with citations in the fixture;
- SHA-256 (pinned by its own golden vectors);
- these refusal cases.
Byte-level agreement with the reference encoder is otherwise parity unpinned.
"""
from __future__ import annotations

import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(__file__))
import envelope_fixture as F  # noqa: E402

from tiler_amd import _lib as L  # noqa: E402
from tiler_amd import envelope as E  # noqa: E402
from tiler_amd.runtime import Refusal  # noqa: E402

ENTRIES = [(b"tiler_map_f32", "tiler_map_f32", [0, 1, 2]),
           (b"tiler_rms_norm_bf16_ch8_full", "tiler_rms_norm_bf16_ch8_full", [0, 1, 2])]


def artifact(**kw) -> F.Artifact:
    payloads = kw.pop("payloads", None)
    if payloads is None:
        payloads = [F.Payload(metadata=F.payload_metadata(entries=ENTRIES), code=b"\x7fELF code object")]
    return F.Artifact(payloads=payloads, **kw)


def refusal(data) -> str | None:
    """The diagnostic of a refused read, or None if the bytes were accepted."""
    try:
        E.read_envelope(bytes(data))
    except Refusal as r:
        assert r.status == L.REFUSE_MALFORMED_PAYLOAD
        return r.diagnostic
    return None


def test_an_encoded_envelope_reads_back():
    a = artifact()
    data = a.encode()
    env = E.read_envelope(data)
    assert env.total_bytes == len(data)
    assert env.manifest_schema == (22, 0)
    assert env.section_purposes == [F.KERNEL_PROGRAM, F.PAYLOAD_METADATA, F.PAYLOAD_CODE]
    assert (env.feature_count, env.input_count, env.output_count, env.provider_count) == (1, 1, 1, 1)
    assert env.identity_digest == a.identity_digest
    [p] = env.payloads
    assert (p.backend, p.representation, p.schema) == ("tiler.hip", "tiler.hip.gfx950.code-object-v1", (1, 0))
    assert p.carried and p.code == b"\x7fELF code object"
    assert p.metadata == a.payloads[0].metadata
    assert p.digest == F.payload_identity(p.metadata)
    assert p.profile_key == "tiler.hip.gfx950.profile-v1"


def test_the_unparsed_manifest_interior_is_covered_by_the_manifest_digest():
    # Whatever the arena, variants and realization record hold, the reader
    # frames around them; a flip inside them fails the manifest digest.
    data = bytearray(artifact(interior=F.u64(3) + bytes(range(200)) + F.framed(b"realization")).encode())
    assert refusal(data) is None
    at = data.index(bytes(range(200))) + 17
    data[at] ^= 0xFF
    assert refusal(data) == "ManifestDigestMismatch"


def test_single_byte_corruptions_are_rejected():
    data = artifact().encode()
    forged = bytearray(data)
    for i in range(len(data)):
        forged[i] ^= 0xFF
        assert refusal(forged) is not None, f"flipping byte {i} produced an accepted envelope"
        forged[i] = data[i]
    # The sweep can say no: the unflipped bytes are accepted.
    assert refusal(forged) is None


def test_every_truncation_is_rejected():
    data = artifact().encode()
    for n in range(len(data)):
        assert refusal(data[:n]) is not None, f"a {n}-byte prefix was accepted"
    assert refusal(data[:4]).startswith("Truncated")
    assert refusal(data[:-1]).startswith("TotalLengthMismatch")


def test_trailing_bytes_are_rejected():
    data = bytearray(artifact().encode()) + b"\x00"
    assert refusal(data).startswith("TotalLengthMismatch")
    F.reseal(data)
    assert refusal(data) == "TrailingBytes { count: 1 }"


def test_a_corrupted_manifest_is_rejected_before_it_is_parsed():
    data = bytearray(artifact().encode())
    data[F.HEADER_BYTES + len(F.MANIFEST_DOMAIN)] ^= 0xFF
    assert refusal(data) == "ManifestDigestMismatch"


def test_a_corrupted_section_is_rejected_by_its_own_digest():
    data = bytearray(artifact().encode())
    data[-1] ^= 0xFF
    F.reseal(data)
    assert refusal(data) == "SectionDigestMismatch { section: 2 }"


def test_a_flipped_tag_byte_is_rejected_by_name():
    data = bytearray(artifact().encode())
    routing_at = F.HEADER_BYTES + len(F.MANIFEST_DOMAIN) + 4 + 16
    assert data[routing_at] == 0x01
    data[routing_at] = 0x7F
    F.reseal(data)
    assert refusal(data) == "UnknownTag { subject: RoutingPolicy, tag: 127 }"


def test_the_retired_execution_policy_tag_is_refused_by_name():
    md = F.payload_metadata(entries=ENTRIES)
    data = artifact(payloads=[F.Payload(metadata=md, code=b"c", policy=0x02)]).encode()
    assert refusal(data) == "UnknownTag { subject: ExecutionPolicy, tag: 2 }"


def test_a_length_prefix_that_disagrees_with_its_payload_is_rejected():
    data = bytearray(artifact().encode())
    feature = F.text(F.FEATURE_EMBEDDED_PAYLOAD_CODE)
    length_at = F.HEADER_BYTES + len(F.MANIFEST_DOMAIN) + 4 + 16 + 1 + 8 + len(feature)
    assert int.from_bytes(data[length_at:length_at + 8], "big") == len(b"graph")
    data[length_at:length_at + 8] = F.u64(len(data))
    F.reseal(data)
    assert refusal(data).startswith("Truncated")


def test_an_unknown_envelope_format_version_is_rejected():
    data = bytearray(artifact().encode())
    data[8:10] = F.u16(2)
    F.reseal(data)
    assert refusal(data) == "UnsupportedEnvelopeFormat { major: 2, minor: 0 }"
    data = bytearray(artifact().encode())
    data[10:12] = F.u16(9)
    F.reseal(data)
    assert refusal(data) == "UnsupportedEnvelopeFormat { major: 1, minor: 9 }"
    data = bytearray(artifact().encode())
    data[14:16] = F.u16(1)
    F.reseal(data)
    assert refusal(data) == "UnsupportedCanonicalEncoding { major: 1, minor: 1 }"


def test_an_unknown_digest_algorithm_is_rejected_rather_than_inferred():
    data = bytearray(artifact().encode())
    data[16] = 0x02
    F.reseal(data)
    assert refusal(data) == "UnsupportedDigestAlgorithm { tag: 2 }"


def test_an_unknown_manifest_or_component_schema_is_rejected():
    schema_at = F.HEADER_BYTES + len(F.MANIFEST_DOMAIN)
    cases = [(0, 7, "UnsupportedManifestSchema { major: 7, minor: 0 }"),
             (2, 5, "UnsupportedManifestSchema { major: 22, minor: 5 }"),
             (4, 3, "UnsupportedComponentSchema { component: Program, major: 3, minor: 0 }"),
             (12, 1, "UnsupportedComponentSchema { component: GuardAndRouting, major: 1, minor: 0 }"),
             (18, 1, "UnsupportedComponentSchema { component: TargetRequirement, major: 3, minor: 1 }")]
    for offset, value, expected in cases:
        data = bytearray(artifact().encode())
        data[schema_at + offset:schema_at + offset + 2] = F.u16(value)
        F.reseal(data)
        assert refusal(data) == expected


def test_an_unsupported_required_feature_is_rejected():
    future = "tiler.artifact.feature.from-a-later-producer"
    data = artifact(features=[F.FEATURE_EMBEDDED_PAYLOAD_CODE, future]).encode()
    assert refusal(data) == f"UnsupportedRequiredFeature {{ feature: {future} }}"


def test_features_are_sorted_and_distinct():
    a = "tiler.artifact.feature.multi-stage-program"
    data = artifact(features=[a, F.FEATURE_EMBEDDED_PAYLOAD_CODE]).encode()
    assert refusal(data) == "NonCanonicalOrder { subject: Feature }"
    data = artifact(features=[F.FEATURE_EMBEDDED_PAYLOAD_CODE, F.FEATURE_EMBEDDED_PAYLOAD_CODE]).encode()
    assert refusal(data) == "DuplicateItem { subject: Feature }"


def test_the_embedded_code_feature_must_match_the_carried_payloads():
    assert refusal(artifact(features=[]).encode()) == "DeclaredFeatureMismatch"
    uncarried = [F.Payload(metadata=b"", code=b"", carried=False, digest=b"\x01" * 32)]
    assert refusal(artifact(payloads=uncarried).encode()) is None
    assert refusal(artifact(payloads=uncarried, features=[F.FEATURE_EMBEDDED_PAYLOAD_CODE]).encode()) == \
        "DeclaredFeatureMismatch"


def test_a_provider_is_required_and_providers_are_ordered():
    assert refusal(artifact(providers=[]).encode()) == "ModelObligation { MissingSelectedLoweringProvider }"
    a, b = F.provider_row(name="a-provider"), F.provider_row(name="b-provider")
    assert refusal(artifact(providers=[a, b]).encode()) is None
    assert refusal(artifact(providers=[b, a]).encode()) == "NonCanonicalOrder { subject: SelectedLoweringProvider }"
    assert refusal(artifact(providers=[a, a]).encode()) == "DuplicateItem { subject: SelectedLoweringProvider }"


def test_payloads_are_ordered_by_canonical_key():
    md1 = F.payload_metadata(entries=ENTRIES)
    md2 = F.payload_metadata(entries=ENTRIES[:1])
    p1 = F.Payload(metadata=md1, code=b"code one")
    p2 = F.Payload(metadata=md2, code=b"code two", backend="tiler.metal")
    assert refusal(artifact(payloads=[p1, p2]).encode()) is None
    keys = sorted([p1.head() + p1.tail(), p2.head() + p2.tail()])
    first = p1 if keys[0].startswith(p1.head()) else p2
    second = p2 if first is p1 else p1
    assert refusal(artifact(payloads=[second, first], sort_payloads=False).encode()) == \
        "NonCanonicalOrder { subject: Payload }"


def test_a_carried_payload_identity_is_rederived():
    md = F.payload_metadata(entries=ENTRIES)
    forged = F.Payload(metadata=md, code=b"c", digest=F.payload_identity(md + b"\x00"))
    assert refusal(artifact(payloads=[forged]).encode()) == "PayloadIdentityMismatch { payload: 0 }"


def test_a_carried_payload_must_name_sections_of_its_purposes():
    md = F.payload_metadata(entries=ENTRIES)
    # Sections: 0 kernel program, 1 metadata, 2 code.
    swapped = F.Payload(metadata=md, code=b"c", sections=(2, 1))
    assert refusal(artifact(payloads=[swapped]).encode()) == \
        "SectionPurposeMismatch { section: 2, expected: 2, actual: 3 }"
    missing = F.Payload(metadata=md, code=b"c", sections=(1, 9))
    assert refusal(artifact(payloads=[missing]).encode()) == "MissingReference { subject: Section, index: 9 }"


def test_an_unreferenced_payload_section_is_rejected(monkeypatch):
    # A second code section nothing names: the stream and the descriptors stay
    # framed and digested, so only the reference rule refuses it.
    a = artifact()
    derived = F.Artifact.sections
    monkeypatch.setattr(F.Artifact, "sections",
                        lambda self: (sorted(derived(self)[0] + [(F.PAYLOAD_CODE, b"zz orphan code")]),
                                      derived(self)[1]))
    assert refusal(a.encode()) == "UnreferencedSection { section: 3 }"


def test_sections_are_in_canonical_order(monkeypatch):
    a = artifact(kernel_programs=[b"program a", b"program b"])
    assert refusal(a.encode()) is None
    # The two kernel-program sections swapped in both the stream and the
    # descriptors: every digest still verifies, the order does not.
    derived = F.Artifact.sections

    def swapped(self):
        items, refs = derived(self)
        items[0], items[1] = items[1], items[0]
        return items, refs
    monkeypatch.setattr(F.Artifact, "sections", swapped)
    assert refusal(a.encode()) == "NonCanonicalOrder { subject: Section }"


def test_section_descriptors_are_checked_against_the_purpose():
    data = bytearray(artifact().encode())
    n = F.manifest_len(data)
    sections = 3
    desc0 = F.HEADER_BYTES + n - 32 - 50 * sections
    # Disposition, then schema, of section 0.
    for at, value, expected in [(desc0 + 5, 0x02, "SectionDispositionMismatch { section: 0, declared: 2, expected: 1 }"),
                                (desc0 + 5, 0x07, "UnknownTag { subject: SectionDisposition, tag: 7 }"),
                                (desc0 + 4, 0x09, "UnknownTag { subject: SectionKind, tag: 9 }")]:
        forged = bytearray(data)
        forged[at] = value
        F.reseal(forged)
        assert refusal(forged) == expected
    forged = bytearray(data)
    forged[desc0 + 6:desc0 + 8] = F.u16(2)
    F.reseal(forged)
    assert refusal(forged) == "UnsupportedSectionSchema { section: 0, major: 2, minor: 0 }"
    forged = bytearray(data)
    forged[F.SECTION_COUNT_AT:F.SECTION_COUNT_AT + 4] = F.u32(2)
    assert refusal(forged).startswith("SectionCountMismatch")


def test_section_framing_is_checked():
    data = bytearray(artifact().encode())
    stream = F.HEADER_BYTES + F.manifest_len(data)
    forged = bytearray(data)
    forged[stream:stream + 4] = F.u32(1)
    assert refusal(forged) == "NonCanonicalSectionId { position: 0, declared: 1 }"
    forged = bytearray(data)
    length = int.from_bytes(forged[stream + 4:stream + 12], "big")
    forged[stream + 4:stream + 12] = F.u64(length + 1)
    assert refusal(forged).startswith("SectionLengthMismatch { section: 0")


def test_budgets_are_enforced_before_use():
    data = bytearray(artifact().encode())
    forged = bytearray(data)
    forged[F.SECTION_COUNT_AT:F.SECTION_COUNT_AT + 4] = F.u32(65)
    assert refusal(forged) == "Limit { resource: Sections, actual: 65, limit: 64 }"
    forged = bytearray(data)
    forged[F.MANIFEST_LENGTH_AT:F.MANIFEST_LENGTH_AT + 8] = F.u64((64 << 20) + 1)
    assert refusal(forged) == f"Limit {{ resource: ManifestBytes, actual: {(64 << 20) + 1}, limit: {64 << 20} }}"
    assert refusal(artifact(features=["x" * 4097]).encode()).startswith("Limit { resource: TextBytes")


def test_governed_keys_and_interface_tags_are_checked():
    md = F.payload_metadata(entries=ENTRIES)
    bad = F.Payload(metadata=md, code=b"c", backend="Tiler.HIP")
    assert refusal(artifact(payloads=[bad]).encode()) == \
        "InvalidGovernedKey { cause: NoncanonicalKeyByte { kind: Backend, index: 0, value: 84 } }"
    entry = F.interface_entry(components=((None, (4,), None, 0x09, (0x01,), 0x06),))
    assert refusal(artifact(inputs=[entry]).encode()) == "UnknownTag { subject: StorageScalar, tag: 9 }"
    entry = F.interface_entry(components=((None, (4,), None, 0x03, (0x02, 3, 1, 1), 0x06),))
    assert refusal(artifact(inputs=[entry]).encode()) == "UnknownTag { subject: StorageEncoding, tag: 3 }"
    entry = F.interface_entry(components=((7, (4,), b"bf16", 0x03, (0x02, 4, 2, 1), 0x06),))
    assert refusal(artifact(inputs=[entry]).encode()) is None
    entry = F.interface_entry(extents=((3, 1),))
    assert refusal(artifact(inputs=[entry]).encode()) == "UnknownTag { subject: InterfaceExtentSource, tag: 3 }"


# --- payload metadata -------------------------------------------------------

def test_the_built_payload_metadata_reads_back():
    import ctypes
    lib = L.lib()
    need = ctypes.c_uint64()
    assert lib.tiler_hip_payload_metadata(None, 0, ctypes.byref(need)) == L.OK
    buf = ctypes.create_string_buffer(need.value)
    assert lib.tiler_hip_payload_metadata(buf, need.value, ctypes.byref(need)) == L.OK
    subject = E.read_payload_metadata(buf.raw)
    view = L.PayloadView()
    assert lib.tiler_hip_payload(ctypes.byref(view)) == L.OK
    assert subject.target == view.target.decode() == "amdgcn-amd-amdhsa--gfx950"
    assert subject.family == view.backend.decode() and subject.unversioned
    assert subject.source == ctypes.string_at(view.source, view.source_bytes)
    bindings = {}
    for i in range(view.entry_count):
        info = L.EntryInfo()
        assert lib.tiler_hip_payload_entry(i, ctypes.byref(info)) == L.OK
        bindings[info.symbol.decode()] = info.buffer_bindings
    assert subject.symbols == sorted(bindings)
    for e in subject.entries:
        assert e.key == e.symbol.encode()
        assert e.transports == list(range(bindings[e.symbol]))


def test_payload_metadata_refusals():
    def why(md):
        try:
            E.read_payload_metadata(md)
        except Refusal as r:
            return r.diagnostic
        return None
    assert why(F.payload_metadata(entries=ENTRIES)) is None
    assert why(b"tiler.artifact-envelope.payload-metadata.v2\0" + bytes(8)) == "BadPayloadMetadataDomain"
    assert why(F.payload_metadata(schema=(2, 0))) == "UnsupportedPayloadMetadataSchema { major: 2, minor: 0 }"
    assert why(F.payload_metadata(entries=ENTRIES[::-1])) == "NonCanonicalOrder { subject: PayloadEntryMapping }"
    assert why(F.payload_metadata(entries=ENTRIES[:1] * 2)) == "DuplicateItem { subject: PayloadEntryMapping }"
    assert why(F.payload_metadata(platform_tag=b"\x01")) == "UnknownTag { subject: PayloadPlatform, tag: 1 }"
    assert why(F.payload_metadata(sdk=("sdk", "", ""))) == "PlatformFieldWithoutPlatform { field: SdkName }"
    assert why(F.payload_metadata(deployment=(1, 0))) == "PlatformFieldWithoutPlatform { field: DeploymentMinimum }"
    assert why(F.payload_metadata(target="")) == "ModelRule { IncompletePayloadProvenance { field: Target } }"
    assert why(F.payload_metadata(components=(("compiler", ""),))) == \
        "ModelRule { IncompletePayloadProvenance { field: ToolComponentVersion } }"
    # The versioned-SDK shape (no platform tag) owes a deployment minimum and an SDK.
    assert why(F.payload_metadata(platform_tag=b"")) == \
        "ModelRule { IncompletePayloadProvenance { field: DeploymentMinimum } }"
    assert why(F.payload_metadata(platform_tag=b"", deployment=(14, 0), sdk=("rocm", "7.2", "1"))) is None
    assert why(F.payload_metadata(obligations=(("b", "1"), ("a", "1")))) == \
        "NonCanonicalOrder { subject: TargetObligation }"
    assert why(F.payload_metadata(entries=ENTRIES) + b"\x00") == "TrailingManifestBytes { count: 1 }"


# --- selection ---------------------------------------------------------------

def test_select_payload_picks_the_gfx950_code_object():
    ours = F.Payload(metadata=F.payload_metadata(entries=ENTRIES), code=b"gfx950 code")
    foreign = F.Payload(metadata=F.payload_metadata(target="air64-apple-macos", family="tiler.metal",
                                                    entries=ENTRIES[:1]),
                        code=b"metallib", backend="tiler.metal", representation="tiler.metal.metallib-v1")
    env = E.read_envelope(artifact(payloads=[foreign, ours]).encode())
    chosen = E.select_payload(env)
    assert chosen.code == b"gfx950 code" and chosen.backend == "tiler.hip"
    assert chosen.subject.symbols == [s for _, s, _ in ENTRIES]


def test_select_payload_refuses_a_foreign_only_envelope():
    other_target = F.Payload(metadata=F.payload_metadata(target="amdgcn-amd-amdhsa--gfx942", entries=ENTRIES),
                             code=b"gfx942 code")
    env = E.read_envelope(artifact(payloads=[other_target]).encode())
    with pytest.raises(Refusal) as r:
        E.select_payload(env)
    assert r.value.status == L.REFUSE_FOREIGN_TARGET
    uncarried = F.Payload(metadata=b"", code=b"", carried=False, digest=b"\x01" * 32)
    with pytest.raises(Refusal) as r:
        E.select_payload(E.read_envelope(artifact(payloads=[uncarried]).encode()))
    assert r.value.status == L.REFUSE_FOREIGN_TARGET


def test_the_reader_refuses_null_arguments():
    import ctypes
    assert L.lib().tiler_hip_read_envelope(None, 1, None, None, 0) == L.REFUSE_INVALID_ARGUMENT
    out = L.Envelope()
    assert L.lib().tiler_hip_read_envelope(None, 0, ctypes.byref(out), None, 0) == L.REFUSE_MALFORMED_PAYLOAD
