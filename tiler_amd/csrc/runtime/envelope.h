// Reader of the target-neutral artifact envelope ("TILERART", envelope format
// 1.0, canonical encoding 1.0, manifest schema 22.0) as far as a HIP loader
// needs it, and of the PayloadMetadata record a carried payload names.
//
// The envelope (tiler-artifact/src/program/codec/encode.rs:336-590) is:
//   header    69 bytes: magic, format, encoding, digest algorithm, total
//             length, manifest length, section count, manifest digest;
//   manifest  domain, schema, component schemas, routing policy, features,
//             semantic subjects, interface, providers, payload descriptors,
//             expression arena, variants, delivered realization, section
//             descriptors, identity digest;
//   sections  (u32 ordinal, u64 length, bytes) each.
// Every check here is one decode.rs makes, with the same refusal name:
//   * framing, integrity (manifest and section digests), budgets, tags;
//   * the canonical order of features, providers, payloads and sections;
//   * section references and purposes;
//   * each carried payload's identity (validate.rs:299-327).
// The expression arena, the variants and the delivered-realization record are
// not parsed: the section descriptors are found from the manifest's end (their
// count is the header's), and the manifest digest covers the rest.  So the
// identity digest is carried, not re-derived, and what only a full decode
// proves (variant rules, every kernel-program section referenced, canonical
// re-encoding) is not claimed.
//
// Every Span in a result points into the caller's bytes.
#pragma once

#include <cstdint>
#include <string>

namespace tiler_rt {

struct Span {
  const uint8_t* p = nullptr;
  uint64_t n = 0;
};

constexpr uint32_t kMaxEnvelopeSections = 64;  // MAX_SECTIONS = MAX_ARTIFACT_VARIANTS (program/mod.rs:749)
constexpr uint32_t kMaxEnvelopePayloads = 16;  // MAX_ARTIFACT_PAYLOADS (program/mod.rs:770)

// Section purposes (codec/model.rs:352-358).
constexpr uint8_t kSectionKernelProgram = 0x01;
constexpr uint8_t kSectionPayloadMetadata = 0x02;
constexpr uint8_t kSectionPayloadCode = 0x03;

struct EnvelopePayload {
  Span backend, representation;
  uint16_t schema_major = 0, schema_minor = 0;
  Span digest;  // the descriptor's PayloadDigest
  Span profile_key, profile_descriptor;
  bool has_environment = false;
  bool carried = false;
  uint32_t metadata_section = 0, code_section = 0;
  Span metadata, code;  // the two sections' contents when carried
};

struct Envelope {
  uint64_t total_bytes = 0, manifest_bytes = 0;
  uint16_t manifest_major = 0, manifest_minor = 0;
  uint32_t section_count = 0;
  uint8_t section_kind[kMaxEnvelopeSections] = {};
  Span section[kMaxEnvelopeSections];
  uint64_t feature_count = 0, input_count = 0, output_count = 0, provider_count = 0;
  uint32_t payload_count = 0;
  EnvelopePayload payloads[kMaxEnvelopePayloads];
  uint8_t identity_digest[32] = {};  // as carried
};

// "" when the bytes pass; otherwise the decode.rs refusal that rejects them
// first (its ArtifactCodecError variant name), with detail.
std::string read_envelope(const uint8_t* bytes, uint64_t n, Envelope& out);

struct PayloadMapping {
  Span key, symbol;
  uint64_t transport_count = 0;
  Span transports;  // transport_count u32, big-endian
};

struct PayloadSubject {
  Span source_representation, source;
  Span toolchain, target, family, language;
  uint16_t deployment_major = 0, deployment_minor = 0;
  Span sdk_name, sdk_version, sdk_build;
  uint64_t component_count = 0, compile_flag_count = 0, link_flag_count = 0;
  uint64_t entry_count = 0, obligation_count = 0;
  bool unversioned = false;
  // The encoded lists as they lie in the record (counts included): the
  // ordered tool components, the compile and link flags, the entry mappings.
  Span components, flags, entries;
};

// decode_metadata (codec/payload.rs:589-660) with check_provenance
// (payload.rs:291-343).  The first `capacity` entry mappings are written to
// `mappings` (which may be null when capacity is 0).
std::string read_payload_metadata(const uint8_t* bytes, uint64_t n, PayloadSubject& out,
                                  PayloadMapping* mappings, uint64_t capacity);

// The first fact on which two decoded PayloadMetadata records disagree, in
// the order a payload's correspondence check reads them
// (tiler-build/tests/custom_backend/backend.rs:545-574,
// tiler-build/examples/identity_join_producer.rs:978-1003):
// "source-representation", "source", "toolchain", "target", "components",
// "flags", "entries"; "" when every one agrees.
const char* first_disagreeing_fact(const PayloadSubject& expected, const PayloadSubject& actual);

}  // namespace tiler_rt
