"""Test-side producer of TILERART artifact envelopes and PayloadMetadata
records, for the envelope reader's tests.

Test infrastructure, not part of the product. It restates the reference
encoders byte for byte:
- tiler-artifact/src/program/codec/encode.rs:336-590 (header, manifest,
  section framing) and 690-968 (section digest, provenance tables, section
  descriptors);
- codec/payload.rs:477-580 (payload metadata).
Digests use Python's hashlib SHA-256, which is independent of the library's
own SHA-256.

Two things are not produced as the reference would produce them:
- The manifest interior between the payload table and the section
  descriptors: the expression arena, the variants and the delivered-realization
  record. The reader under test does not parse it, so `interior` is
  caller-chosen bytes. The default is an empty arena, an empty variant table
  and an empty realization run, which the reference's full decoder would
  refuse as EmptyPortfolio.
- The identity digest: the reference derives it from the program's canonical
  identity, which needs the compiler. Here it is caller-chosen.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

MAGIC = b"TILERART"                     # encode.rs:29
HEADER_BYTES = 69                       # encode.rs:31
TOTAL_LENGTH_AT = 17
MANIFEST_LENGTH_AT = 25
SECTION_COUNT_AT = 33
MANIFEST_DIGEST_AT = 37
ENVELOPE_FORMAT = (1, 0)                # encode.rs:33
CANONICAL_ENCODING = (1, 0)             # encode.rs:35
MANIFEST_SCHEMA = (22, 0)               # encode.rs:288
COMPONENT_SCHEMAS = ((1, 0), (1, 0), (2, 0), (3, 0))  # program/model.rs:523-540
MANIFEST_DOMAIN = b"tiler.artifact-envelope.manifest.v1\0"                 # encode.rs:296
MANIFEST_DIGEST_DOMAIN = b"tiler.artifact-envelope.manifest-digest.v1\0"   # encode.rs:298
SECTION_DIGEST_DOMAIN = b"tiler.artifact-envelope.section-digest.v1\0"     # encode.rs:305
PAYLOAD_METADATA_DOMAIN = b"tiler.artifact-envelope.payload-metadata.v1\0"  # payload.rs:150-155
PAYLOAD_IDENTITY_DOMAIN = b"tiler.artifact-envelope.payload-identity.v1\0"  # payload.rs:160
FEATURE_EMBEDDED_PAYLOAD_CODE = "tiler.artifact.feature.embedded-payload-code"  # codec/model.rs:104
KERNEL_PROGRAM, PAYLOAD_METADATA, PAYLOAD_CODE = 0x01, 0x02, 0x03       # codec/model.rs:352-358


def u16(v):
    return int(v).to_bytes(2, "big")


def u32(v):
    return int(v).to_bytes(4, "big")


def u64(v):
    return int(v).to_bytes(8, "big")


def framed(b: bytes) -> bytes:
    return u64(len(b)) + b


def text(s: str) -> bytes:
    return framed(s.encode())


def governed(domain: bytes, data: bytes, qualifiers=()) -> bytes:
    return hashlib.sha256(domain + b"".join(qualifiers) + data).digest()


def payload_identity(metadata: bytes) -> bytes:
    return governed(PAYLOAD_IDENTITY_DOMAIN, metadata)


def section_digest(purpose: int, content: bytes) -> bytes:
    return governed(SECTION_DIGEST_DOMAIN, content, (bytes([purpose]), u16(1), u16(0)))


def payload_metadata(*, target="amdgcn-amd-amdhsa--gfx950", family="tiler.hip", language="hip-c++17",
                     toolchain="tiler.hip.rocm-clang", source=b"kernels", source_representation="tiler.hip.source-bundle.v1",
                     components=(("compiler", "clang 20"),), flags=("-O3",), link_flags=(),
                     entries=(), obligations=(("tiler.hip.target-arch", "gfx950"),), deployment=(0, 0),
                     sdk=("", "", ""), platform_tag=b"\x00", schema=(1, 0)) -> bytes:
    """One PayloadMetadata record in its canonical encoding (payload.rs:477-580).
    `entries` holds (key bytes, symbol, transports); `platform_tag` is the
    appended PayloadPlatform tag (b"" for the versioned-SDK shape)."""
    b = bytearray(PAYLOAD_METADATA_DOMAIN + u16(schema[0]) + u16(schema[1]))
    b += text(source_representation) + framed(source)
    b += text(toolchain) + text(target) + text(family) + text(language)
    b += u16(deployment[0]) + u16(deployment[1])
    b += u64(len(components)) + b"".join(text(r) + text(v) for r, v in components)
    b += b"".join(text(s) for s in sdk)
    b += u64(len(flags)) + b"".join(text(f) for f in flags)
    b += u64(len(link_flags)) + b"".join(text(f) for f in link_flags)
    b += u64(len(entries))
    for key, symbol, transports in entries:
        b += framed(key) + text(symbol) + u64(len(transports)) + b"".join(u32(t) for t in transports)
    b += u64(len(obligations)) + b"".join(text(k) + text(v) for k, v in obligations)
    b += platform_tag
    return bytes(b)


@dataclass
class Payload:
    """One backend payload descriptor (program/model.rs BackendPayloadDescriptor)."""
    metadata: bytes = b""
    code: bytes = b""
    backend: str = "tiler.hip"
    representation: str = "tiler.hip.gfx950.code-object-v1"
    schema: tuple = (1, 0)
    digest: bytes | None = None          # default: payload_identity(metadata)
    profile_key: str = "tiler.hip.gfx950.profile-v1"
    profile_descriptor: bytes = b"gfx950 wave64 lds163840 cu256"
    policy: int = 0x01                   # ArtifactExecutionPolicy::NativeImage
    carried: bool = True
    environment: bytes | None = None     # the encoded declaration after its 0x01 presence byte
    sections: tuple | None = None        # (metadata, code) section ids, overriding the derived ones

    def head(self) -> bytes:
        digest = self.digest if self.digest is not None else payload_identity(self.metadata)
        return (text(self.backend) + text(self.representation) + u16(self.schema[0]) + u16(self.schema[1])
                + framed(digest) + text(self.profile_key) + framed(self.profile_descriptor) + bytes([self.policy]))

    def tail(self) -> bytes:
        return b"\x00" if self.environment is None else b"\x01" + self.environment


def provider_row(namespace="tiler", name="tiler-hip", revision=1, family="tiler.realization",
                 op_namespace="tiler", op_name="realize", semantic_version=1, capability_revision=1) -> bytes:
    """One selected lowering provider row (encode.rs:705-721)."""
    return (text(namespace) + text(name) + u32(revision) + text(family) + text(op_namespace) + text(op_name)
            + u32(semantic_version) + u32(capability_revision))


def interface_entry(key="x", extents=((1, 8192), (2, b"scope", "n")), logical_type=b"tensor<bf16>",
                    components=((None, (8192, 4096), None, 0x03, (0x01,), 0x06),)) -> bytes:
    """One named input or output (encode.rs:624-636, 661-681).  An extent is
    (1, literal) or (2, scope bytes, symbol name); a component is (role or
    None, shape, resolved type or None, storage scalar tag, encoding,
    access type tag) with encoding (0x01,) or (0x02, bits, order, tail)."""
    b = bytearray(text(key) + u64(len(extents)))
    for ext in extents:
        b += bytes([ext[0]])
        b += framed(ext[1]) + text(ext[2]) if ext[0] == 2 else u64(ext[1])
    b += framed(logical_type) + u64(len(components))
    for role, shape, resolved, scalar, encoding, access in components:
        b += b"\x00" if role is None else b"\x01" + u32(role)
        b += u64(len(shape)) + b"".join(u64(d) for d in shape)
        b += b"\x00" if resolved is None else b"\x01" + framed(resolved)
        b += bytes([scalar]) + bytes(encoding) + bytes([access])
    return bytes(b)


DEFAULT_INTERIOR = u64(0) + u64(0) + framed(b"")


@dataclass
class Artifact:
    payloads: list = field(default_factory=list)
    kernel_programs: list = field(default_factory=lambda: [b"kernel program subject"])
    features: list | None = None         # default: derived (the embedded-code key iff a payload is carried)
    semantic: tuple = (b"graph", b"reached", b"admission", b"retained")
    inputs: list = field(default_factory=lambda: [interface_entry("x")])
    outputs: list = field(default_factory=lambda: [interface_entry("y", extents=((1, 8192), (1, 4096)))])
    providers: list = field(default_factory=lambda: [provider_row()])
    routing: int = 0x01
    manifest_schema: tuple = MANIFEST_SCHEMA
    components: tuple = COMPONENT_SCHEMAS
    interior: bytes = DEFAULT_INTERIOR
    identity_digest: bytes = b"\x5a" * 32
    sort_payloads: bool = True

    def sections(self):
        """(purpose, content) in canonical order (validate.rs:249-268), and the
        section ids of each carried payload's (metadata, code)."""
        items = [(KERNEL_PROGRAM, k) for k in self.kernel_programs]
        for p in self.payloads:
            if p.carried:
                items += [(PAYLOAD_METADATA, p.metadata), (PAYLOAD_CODE, p.code)]
        items = sorted(set(items))
        ids = {item: i for i, item in enumerate(items)}
        refs = [(ids[(PAYLOAD_METADATA, p.metadata)], ids[(PAYLOAD_CODE, p.code)]) if p.carried else None
                for p in self.payloads]
        return items, refs

    def manifest(self):
        items, refs = self.sections()
        features = self.features
        if features is None:
            features = [FEATURE_EMBEDDED_PAYLOAD_CODE] if any(p.carried for p in self.payloads) else []
        b = bytearray(MANIFEST_DOMAIN + u16(self.manifest_schema[0]) + u16(self.manifest_schema[1]))
        for major, minor in self.components:
            b += u16(major) + u16(minor)
        b += bytes([self.routing])
        b += u64(len(features)) + b"".join(text(f) for f in features)
        b += b"".join(framed(s) for s in self.semantic)
        b += u64(len(self.inputs)) + b"".join(self.inputs)
        b += u64(len(self.outputs)) + b"".join(self.outputs)
        b += u64(len(self.providers)) + b"".join(self.providers)
        rows = []
        for p, ref in zip(self.payloads, refs):
            if p.sections is not None:
                ref = p.sections
            content = b"\x01" + u32(ref[0]) + u32(ref[1]) if p.carried else b"\x00"
            rows.append((p.head() + p.tail(), p.head() + content + p.tail()))
        if self.sort_payloads:
            rows.sort(key=lambda r: r[0])
        b += u64(len(rows)) + b"".join(r[1] for r in rows)
        b += self.interior
        b += u64(len(items))
        for i, (purpose, content) in enumerate(items):
            b += u32(i) + bytes([purpose, 0x01]) + u16(1) + u16(0) + u64(len(content))
            b += section_digest(purpose, content)
        b += self.identity_digest
        return bytes(b), items

    def encode(self) -> bytes:
        manifest, items = self.manifest()
        stream = b"".join(u32(i) + framed(content) for i, (_, content) in enumerate(items))
        total = HEADER_BYTES + len(manifest) + len(stream)
        header = (MAGIC + u16(ENVELOPE_FORMAT[0]) + u16(ENVELOPE_FORMAT[1]) + u16(CANONICAL_ENCODING[0])
                  + u16(CANONICAL_ENCODING[1]) + b"\x01" + u64(total) + u64(len(manifest)) + u32(len(items))
                  + governed(MANIFEST_DIGEST_DOMAIN, manifest))
        assert len(header) == HEADER_BYTES
        return header + manifest + stream


def manifest_len(data: bytes) -> int:
    return int.from_bytes(data[MANIFEST_LENGTH_AT:MANIFEST_LENGTH_AT + 8], "big")


def reseal(data: bytearray) -> None:
    """Restores the declared total length and the manifest digest after an
    edit, so the check under test is not the digest (tests/support.rs:66-78)."""
    data[TOTAL_LENGTH_AT:TOTAL_LENGTH_AT + 8] = u64(len(data))
    n = manifest_len(data)
    data[MANIFEST_DIGEST_AT:MANIFEST_DIGEST_AT + 32] = governed(
        MANIFEST_DIGEST_DOMAIN, bytes(data[HEADER_BYTES:HEADER_BYTES + n]))
