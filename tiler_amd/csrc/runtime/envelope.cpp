// Artifact envelope and payload-metadata reader; the header states what is
// read and what is not.
#include "envelope.h"

#include <cstring>
#include <vector>

#include "digest.h"

namespace tiler_rt {

namespace {

// Framing constants (codec/encode.rs:29-35, 320-326; model.rs:60-76;
// program/mod.rs:749-782; keys.rs:136-163).
constexpr char kMagic[] = "TILERART";
constexpr uint64_t kHeaderBytes = 69;
constexpr uint16_t kEnvelopeFormat[2] = {1, 0};
constexpr uint16_t kCanonicalEncoding[2] = {1, 0};
constexpr uint16_t kManifestSchema[2] = {22, 0};
// Governed component schemas: program, ABI expression, guard and routing,
// target requirement (program/model.rs:523-540).
constexpr uint16_t kComponentSchema[4][2] = {{1, 0}, {1, 0}, {2, 0}, {3, 0}};
constexpr uint8_t kDigestSha256 = 0x01;  // tiler-digest/src/lib.rs:134-141
constexpr uint64_t kMaxEnvelopeBytes = 256ull << 20;
constexpr uint64_t kMaxManifestBytes = 64ull << 20;
constexpr uint64_t kMaxSectionBytes = 64ull << 20;
constexpr uint64_t kMaxTextBytes = 4096;
constexpr uint64_t kMaxFeatures = 64;
constexpr uint64_t kMaxInterfaceEntries = 4096;
constexpr uint64_t kMaxShapeRank = 4096;
constexpr uint64_t kMaxEntryBindings = 64;
constexpr uint64_t kMaxProviders = 256;
constexpr uint64_t kMaxGovernedKeyBytes = 256;
constexpr uint64_t kMaxOpaqueIdentityBytes = 1024;
constexpr uint64_t kMaxProfileDescriptorBytes = 64 * 1024;
// Section descriptor: u32 id, u8 purpose, u8 disposition, u16 + u16 schema,
// u64 length, 32-byte digest (encode.rs:942-968).
constexpr uint64_t kDescriptorBytes = 4 + 1 + 1 + 2 + 2 + 8 + 32;

// Payload metadata (codec/payload.rs:155-184).
constexpr uint16_t kPayloadMetadataSchema[2] = {1, 0};
constexpr uint64_t kMaxPayloadSourceBytes = 16ull << 20;
constexpr uint64_t kMaxPayloadEntryMappings = 4096;
constexpr uint64_t kMaxEntryTransports = 64 + 16;  // MAX_ENTRY_BINDINGS + MAX_ENTRY_EXTENTS
constexpr uint64_t kMaxTargetObligations = 64;
constexpr uint64_t kMaxProvenanceComponents = 16;
constexpr uint64_t kMaxProvenanceFlags = 256;
constexpr uint64_t kMaxKernelIdentityBytes = 16ull << 20;
constexpr uint8_t kPlatformUnversioned = 0x00;

// Required-feature keys a reader of this schema understands (codec/model.rs:95-148).
constexpr const char* kSupportedFeatures[] = {
    "tiler.artifact.feature.deferred-predicates",   "tiler.artifact.feature.embedded-payload-code",
    "tiler.artifact.feature.launch-preconditions",  "tiler.artifact.feature.multi-payload-delivery",
    "tiler.artifact.feature.multi-stage-program",   "tiler.artifact.feature.multi-variant-routing",
    "tiler.artifact.feature.route-requirements"};
constexpr char kEmbeddedPayloadCode[] = "tiler.artifact.feature.embedded-payload-code";

// Domain separators, each with its terminating NUL (encode.rs:289-306,
// payload.rs:150-160).
constexpr char kManifestDomain[] = "tiler.artifact-envelope.manifest.v1";
constexpr char kManifestDigestDomain[] = "tiler.artifact-envelope.manifest-digest.v1";
constexpr char kSectionDigestDomain[] = "tiler.artifact-envelope.section-digest.v1";
constexpr char kPayloadMetadataDomain[] = "tiler.artifact-envelope.payload-metadata.v1";
constexpr char kPayloadIdentityDomain[] = "tiler.artifact-envelope.payload-identity.v1";

struct Reject {
  std::string why;
};

[[noreturn]] void reject(std::string why) { throw Reject{std::move(why)}; }

std::string num(uint64_t v) { return std::to_string(v); }

std::string limit(const char* resource, uint64_t actual, uint64_t bound) {
  return std::string("Limit { resource: ") + resource + ", actual: " + num(actual) + ", limit: " + num(bound) +
         " }";
}

// Rust's str::from_utf8 acceptance: shortest forms only, no surrogates,
// nothing above U+10FFFF.
bool utf8_valid(const uint8_t* p, uint64_t n) {
  uint64_t i = 0;
  while (i < n) {
    const uint8_t c = p[i];
    if (c < 0x80) {
      ++i;
      continue;
    }
    uint32_t extra;
    uint8_t lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) {
      extra = 1;
    } else if (c >= 0xE0 && c <= 0xEF) {
      extra = 2;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      extra = 3;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    } else {
      return false;
    }
    if (n - i <= extra) return false;
    if (p[i + 1] < lo || p[i + 1] > hi) return false;
    for (uint32_t k = 2; k <= extra; ++k)
      if ((p[i + k] & 0xC0) != 0x80) return false;
    i += extra + 1;
  }
  return true;
}

// Lexicographic byte order, the order of Rust's [u8] and str.
int compare(Span a, Span b) {
  const uint64_t m = a.n < b.n ? a.n : b.n;
  const int c = m ? std::memcmp(a.p, b.p, m) : 0;
  if (c) return c;
  return a.n < b.n ? -1 : (a.n > b.n ? 1 : 0);
}

bool equals(Span a, const char* s) {
  const uint64_t n = std::strlen(s);
  return a.n == n && (n == 0 || std::memcmp(a.p, s, n) == 0);
}

// require_sorted_and_distinct / require_canonical (decode.rs:1372-1393,
// payload.rs:853-869): strictly increasing.
void require_ordered(int cmp, const char* subject) {
  if (cmp == 0) reject(std::string("DuplicateItem { subject: ") + subject + " }");
  if (cmp > 0) reject(std::string("NonCanonicalOrder { subject: ") + subject + " }");
}

class Cursor {
 public:
  Cursor(const uint8_t* b, uint64_t n) : b_(b), n_(n) {}
  uint64_t remaining() const { return n_ - pos_; }
  uint64_t position() const { return pos_; }
  const uint8_t* at(uint64_t pos) const { return b_ + pos; }

  Span take(uint64_t len) {
    if (len > remaining())
      reject("Truncated { needed: " + num(len) + ", available: " + num(remaining()) + " }");
    Span s{b_ + pos_, len};
    pos_ += len;
    return s;
  }
  uint8_t u8() { return take(1).p[0]; }
  uint16_t u16() {
    const Span s = take(2);
    return (uint16_t)((uint16_t)s.p[0] << 8 | s.p[1]);
  }
  uint32_t u32() {
    const Span s = take(4);
    return (uint32_t)s.p[0] << 24 | (uint32_t)s.p[1] << 16 | (uint32_t)s.p[2] << 8 | s.p[3];
  }
  uint64_t u64() {
    const Span s = take(8);
    uint64_t v = 0;
    for (int i = 0; i < 8; ++i) v = v << 8 | s.p[i];
    return v;
  }
  // A governed count, refused beyond its budget before use.
  uint64_t count(uint64_t bound, const char* resource) {
    const uint64_t v = u64();
    if (v > bound) reject(limit(resource, v, bound));
    return v;
  }
  Span slice() { return take(u64()); }
  Span text() {
    const Span s = take(count(kMaxTextBytes, "TextBytes"));
    if (!utf8_valid(s.p, s.n)) reject("InvalidText");
    return s;
  }

 private:
  const uint8_t* b_;
  uint64_t n_;
  uint64_t pos_ = 0;
};

// BackendKey, RepresentationKey, TargetProfileKey (keys.rs:185-208).
Span governed_key(Cursor& c, const char* kind) {
  const Span s = c.text();
  if (s.n == 0) reject(std::string("InvalidGovernedKey { cause: EmptyKey { kind: ") + kind + " } }");
  if (s.n > kMaxGovernedKeyBytes)
    reject(std::string("InvalidGovernedKey { cause: KeyTooLong { kind: ") + kind + ", bytes: " + num(s.n) +
           ", limit: " + num(kMaxGovernedKeyBytes) + " } }");
  for (uint64_t i = 0; i < s.n; ++i) {
    const uint8_t b = s.p[i];
    const bool ok = (b >= 'a' && b <= 'z') || (b >= '0' && b <= '9') || b == '.' || b == '-' || b == '_';
    if (!ok)
      reject(std::string("InvalidGovernedKey { cause: NoncanonicalKeyByte { kind: ") + kind + ", index: " +
             num(i) + ", value: " + num(b) + " } }");
  }
  return s;
}

// PayloadDigest, TargetProfileDescriptorDigest, BackendEntryKey (keys.rs:210-226).
Span opaque(Cursor& c, const char* kind, uint64_t bound) {
  const Span s = c.slice();
  if (s.n == 0) reject(std::string("InvalidGovernedKey { cause: EmptyKey { kind: ") + kind + " } }");
  if (s.n > bound)
    reject(std::string("InvalidGovernedKey { cause: KeyTooLong { kind: ") + kind + ", bytes: " + num(s.n) +
           ", limit: " + num(bound) + " } }");
  return s;
}

void unknown_tag(const char* subject, uint8_t tag) {
  reject(std::string("UnknownTag { subject: ") + subject + ", tag: " + num(tag) + " }");
}

// ProviderIdentity: namespace, name, revision (decode.rs:1704-1710).
void provider_identity(Cursor& c) {
  c.text();
  c.text();
  c.u32();
}

// One interface entry's published boundary and components (decode.rs:439-475,
// 1502-1610).
void interface_entry(Cursor& c) {
  c.text();  // the input or output key
  const uint64_t rank = c.count(kMaxShapeRank, "ShapeRank");
  for (uint64_t a = 0; a < rank; ++a) {
    const uint8_t tag = c.u8();
    if (tag == 0x01) {  // SOURCED_EXTENT_LITERAL (model.rs:3414)
      c.u64();
    } else if (tag == 0x02) {  // SOURCED_EXTENT_SYMBOL: scope, name
      c.slice();
      c.text();
    } else {
      unknown_tag("InterfaceExtentSource", tag);
    }
  }
  c.slice();  // logical type
  const uint64_t components = c.count(kMaxEntryBindings, "EntryBindings");
  for (uint64_t k = 0; k < components; ++k) {
    const uint8_t role = c.u8();
    if (role == 1)
      c.u32();
    else if (role != 0)
      unknown_tag("ComponentPresence", role);
    const uint64_t shape_rank = c.count(kMaxShapeRank, "ShapeRank");
    c.take(8 * shape_rank);
    const uint8_t resolved = c.u8();
    if (resolved == 1)
      c.slice();
    else if (resolved != 0)
      unknown_tag("ComponentPresence", resolved);
    const uint8_t scalar = c.u8();  // StorageScalar (model.rs:2646-2654)
    if (scalar < 0x01 || scalar > 0x04) unknown_tag("StorageScalar", scalar);
    const uint8_t encoding = c.u8();  // StorageEncoding
    if (encoding == 0x02) {
      const uint8_t bits = c.u8();
      const uint8_t order = c.u8();
      if (order != 0x01 && order != 0x02) unknown_tag("PackedBitOrder", order);
      const uint8_t tail = c.u8();
      if (tail != 0x01) unknown_tag("PackedTailRule", tail);
      if (bits != 1 && bits != 2 && bits != 4) unknown_tag("StorageEncoding", bits);
    } else if (encoding != 0x01) {
      unknown_tag("StorageEncoding", encoding);
    }
    const uint8_t access = c.u8();  // KernelType (model.rs:2623-2634)
    if (access < 0x01 || access > 0x07) unknown_tag("ElementType", access);
  }
}

Span provider_row(Cursor& c) {
  const uint64_t start = c.position();
  provider_identity(c);
  c.text();  // capability family
  c.text();  // operation namespace
  c.text();  // operation name
  c.u32();   // operation semantic version
  c.u32();   // capability revision
  return Span{c.at(start), c.position() - start};
}

// One payload descriptor row (decode.rs:576-658).  `key` receives the row
// without its content reference: with the domain prefix every key shares, it
// is the payload's canonical key (program/model.rs:1055-1110).
void payload_row(Cursor& c, EnvelopePayload& p, Span& head, Span& tail) {
  const uint64_t start = c.position();
  p.backend = governed_key(c, "Backend");
  p.representation = governed_key(c, "Representation");
  p.schema_major = c.u16();
  p.schema_minor = c.u16();
  p.digest = opaque(c, "PayloadDigest", kMaxOpaqueIdentityBytes);
  p.profile_key = governed_key(c, "TargetProfile");
  p.profile_descriptor = opaque(c, "TargetProfileDescriptor", kMaxProfileDescriptorBytes);
  const uint8_t policy = c.u8();  // ArtifactExecutionPolicy: 0x01 NativeImage only
  if (policy != 0x01) unknown_tag("ExecutionPolicy", policy);
  head = Span{c.at(start), c.position() - start};
  const uint8_t content = c.u8();
  if (content == 0x01) {
    p.carried = true;
    p.metadata_section = c.u32();
    p.code_section = c.u32();
  } else if (content != 0x00) {
    unknown_tag("PayloadContent", content);
  }
  const uint64_t env_start = c.position();
  const uint8_t env = c.u8();
  if (env == 0x01) {
    p.has_environment = true;
    provider_identity(c);
    c.u16();
    c.u16();
    const Span d = c.slice();
    if (d.n > kMaxProfileDescriptorBytes)
      reject(limit("TargetEnvironmentDescriptorBytes", d.n, kMaxProfileDescriptorBytes));
  } else if (env != 0x00) {
    unknown_tag("TargetEnvironmentPresence", env);
  }
  tail = Span{c.at(env_start), c.position() - env_start};
}

void governed_digest_of(const char* domain, const void* const* q, const uint64_t* qn, uint32_t nq,
                        Span bytes, uint8_t out[32]) {
  governed_digest(domain, std::strlen(domain) + 1, q, qn, nq, bytes.p, bytes.n, out);
}

void section_digest(uint8_t kind, Span bytes, uint8_t out[32]) {
  // Qualifiers: purpose tag, content schema major and minor (encode.rs:690-701);
  // every purpose's schema is 1.0 (model.rs:375-381).
  const uint8_t tag[1] = {kind};
  const uint8_t major[2] = {0, 1};
  const uint8_t minor[2] = {0, 0};
  const void* q[3] = {tag, major, minor};
  const uint64_t qn[3] = {1, 2, 2};
  governed_digest_of(kSectionDigestDomain, q, qn, 3, bytes, out);
}

struct Descriptor {
  uint32_t id;
  uint8_t kind;
  uint64_t len;
  const uint8_t* digest;
};

// What parse_manifest (decode.rs:331-437) reads, in its order, up to the
// payload table; then the section descriptors and the identity digest from
// the manifest's end.
void parse_manifest(Span manifest, uint32_t header_sections, Envelope& e, Descriptor* desc,
                    bool& embedded_feature) {
  Cursor c(manifest.p, manifest.n);
  const Span domain = c.take(sizeof(kManifestDomain));
  if (std::memcmp(domain.p, kManifestDomain, sizeof(kManifestDomain)) != 0) reject("BadManifestDomain");
  e.manifest_major = c.u16();
  e.manifest_minor = c.u16();
  if (e.manifest_major != kManifestSchema[0] || e.manifest_minor > kManifestSchema[1])
    reject("UnsupportedManifestSchema { major: " + num(e.manifest_major) + ", minor: " + num(e.manifest_minor) +
           " }");
  static const char* const kComponents[4] = {"Program", "AbiExpression", "GuardAndRouting",
                                             "TargetRequirement"};
  uint16_t read[4][2];
  for (auto& v : read) {
    v[0] = c.u16();
    v[1] = c.u16();
  }
  for (int k = 0; k < 4; ++k)
    if (read[k][0] != kComponentSchema[k][0] || read[k][1] > kComponentSchema[k][1])
      reject(std::string("UnsupportedComponentSchema { component: ") + kComponents[k] +
             ", major: " + num(read[k][0]) + ", minor: " + num(read[k][1]) + " }");
  const uint8_t routing = c.u8();  // RoutingPolicy: 0x01 StablePriority only
  if (routing != 0x01) unknown_tag("RoutingPolicy", routing);

  e.feature_count = c.count(kMaxFeatures, "Features");
  Span features[kMaxFeatures];
  for (uint64_t i = 0; i < e.feature_count; ++i) features[i] = c.text();
  for (uint64_t i = 1; i < e.feature_count; ++i) require_ordered(compare(features[i - 1], features[i]), "Feature");
  embedded_feature = false;
  for (uint64_t i = 0; i < e.feature_count; ++i) {
    bool known = false;
    for (const char* k : kSupportedFeatures) known = known || equals(features[i], k);
    if (!known)
      reject("UnsupportedRequiredFeature { feature: " +
             std::string((const char*)features[i].p, features[i].n) + " }");
    embedded_feature = embedded_feature || equals(features[i], kEmbeddedPayloadCode);
  }

  // Semantic subjects: graph, reached definitions, admission provenance,
  // retained shape.  Framed runs whose contents their own decoders own.
  for (int k = 0; k < 4; ++k) c.slice();
  e.input_count = c.count(kMaxInterfaceEntries, "InterfaceEntries");
  for (uint64_t i = 0; i < e.input_count; ++i) interface_entry(c);
  e.output_count = c.count(kMaxInterfaceEntries, "InterfaceEntries");
  for (uint64_t i = 0; i < e.output_count; ++i) interface_entry(c);

  e.provider_count = c.count(kMaxProviders, "SelectedLoweringProviders");
  std::vector<Span> providers(e.provider_count);
  for (uint64_t i = 0; i < e.provider_count; ++i) providers[i] = provider_row(c);
  for (uint64_t i = 1; i < e.provider_count; ++i)
    require_ordered(compare(providers[i - 1], providers[i]), "SelectedLoweringProvider");

  e.payload_count = (uint32_t)c.count(kMaxEnvelopePayloads, "Payloads");
  std::string keys[kMaxEnvelopePayloads];
  for (uint32_t i = 0; i < e.payload_count; ++i) {
    Span head, tail;
    payload_row(c, e.payloads[i], head, tail);
    keys[i].assign((const char*)head.p, head.n);
    keys[i].append((const char*)tail.p, tail.n);
  }
  for (uint32_t i = 1; i < e.payload_count; ++i)
    require_ordered(keys[i - 1].compare(keys[i]) < 0 ? -1 : (keys[i - 1] == keys[i] ? 0 : 1), "Payload");

  // The section descriptors and the identity digest end the manifest, and
  // their count is the header's.  What lies between the payload table and
  // them (the expression arena, the variants, the delivered-realization
  // record) is covered by the manifest digest and not parsed here.
  const uint64_t tail_bytes = 8 + kDescriptorBytes * header_sections + 32;
  if (c.remaining() < tail_bytes)
    reject("Truncated { needed: " + num(tail_bytes) + ", available: " + num(c.remaining()) + " }");
  Cursor t(manifest.p, manifest.n);
  t.take(manifest.n - tail_bytes);
  const uint64_t declared = t.u64();
  if (declared != header_sections)
    reject("SectionCountMismatch { header: " + num(header_sections) + ", manifest: " + num(declared) + " }");
  for (uint32_t s = 0; s < header_sections; ++s) {
    Descriptor& d = desc[s];
    d.id = t.u32();
    const uint8_t kind = t.u8();
    if (kind < kSectionKernelProgram || kind > kSectionPayloadCode) unknown_tag("SectionKind", kind);
    const uint8_t disposition = t.u8();
    if (disposition != 0x01 && disposition != 0x02) unknown_tag("SectionDisposition", disposition);
    if (disposition != 0x01)  // every purpose is Required (model.rs:391-398)
      reject("SectionDispositionMismatch { section: " + num(d.id) + ", declared: " + num(disposition) +
             ", expected: 1 }");
    const uint16_t major = t.u16(), minor = t.u16();
    if (major != 1 || minor != 0)  // every purpose's content schema is 1.0 (model.rs:375-381)
      reject("UnsupportedSectionSchema { section: " + num(d.id) + ", major: " + num(major) + ", minor: " +
             num(minor) + " }");
    d.kind = kind;
    d.len = t.u64();
    d.digest = t.take(32).p;
    e.section_kind[s] = kind;
  }
  std::memcpy(e.identity_digest, t.take(32).p, 32);

  // A carried payload names its two sections, which must exist and carry the
  // purposes it claims (decode.rs:398-412).
  for (uint32_t i = 0; i < e.payload_count; ++i) {
    const EnvelopePayload& p = e.payloads[i];
    if (!p.carried) continue;
    const uint32_t refs[2] = {p.metadata_section, p.code_section};
    const uint8_t kinds[2] = {kSectionPayloadMetadata, kSectionPayloadCode};
    for (int r = 0; r < 2; ++r) {
      if (refs[r] >= header_sections)
        reject("MissingReference { subject: Section, index: " + num(refs[r]) + " }");
      if (desc[refs[r]].kind != kinds[r])
        reject("SectionPurposeMismatch { section: " + num(refs[r]) + ", expected: " + num(kinds[r]) +
               ", actual: " + num(desc[refs[r]].kind) + " }");
    }
  }
}

std::string read_envelope_or_throw(const uint8_t* bytes, uint64_t n, Envelope& e) {
  // decode (decode.rs:105-190) and read_header (decode.rs:195-252).
  if (n > kMaxEnvelopeBytes) reject(limit("EnvelopeBytes", n, kMaxEnvelopeBytes));
  Cursor c(bytes, n);
  const Span magic = c.take(8);
  if (std::memcmp(magic.p, kMagic, 8) != 0) reject("BadMagic");
  const uint16_t fmaj = c.u16(), fmin = c.u16();
  if (fmaj != kEnvelopeFormat[0] || fmin > kEnvelopeFormat[1])
    reject("UnsupportedEnvelopeFormat { major: " + num(fmaj) + ", minor: " + num(fmin) + " }");
  const uint16_t emaj = c.u16(), emin = c.u16();
  if (emaj != kCanonicalEncoding[0] || emin > kCanonicalEncoding[1])
    reject("UnsupportedCanonicalEncoding { major: " + num(emaj) + ", minor: " + num(emin) + " }");
  const uint8_t algorithm = c.u8();
  if (algorithm != kDigestSha256) reject("UnsupportedDigestAlgorithm { tag: " + num(algorithm) + " }");
  const uint64_t total = c.u64();
  if (total != n) reject("TotalLengthMismatch { declared: " + num(total) + ", actual: " + num(n) + " }");
  const uint64_t manifest_bytes = c.count(kMaxManifestBytes, "ManifestBytes");
  const uint32_t sections = c.u32();
  if (sections > kMaxEnvelopeSections) reject(limit("Sections", sections, kMaxEnvelopeSections));
  const Span manifest_digest = c.take(32);
  if (c.position() != kHeaderBytes) reject("the framing header is fixed width");
  e.total_bytes = n;
  e.manifest_bytes = manifest_bytes;
  e.section_count = sections;

  const Span manifest = c.take(manifest_bytes);
  uint8_t d[32];
  governed_digest_of(kManifestDigestDomain, nullptr, nullptr, 0, manifest, d);
  if (std::memcmp(d, manifest_digest.p, 32) != 0) reject("ManifestDigestMismatch");
  Descriptor desc[kMaxEnvelopeSections];
  bool embedded_feature = false;
  parse_manifest(manifest, sections, e, desc, embedded_feature);

  // The framed section stream (decode.rs:254-313).
  for (uint32_t s = 0; s < sections; ++s) {
    const uint32_t declared = c.u32();
    if (declared != s || desc[s].id != declared)
      reject("NonCanonicalSectionId { position: " + num(s) + ", declared: " + num(declared) + " }");
    const uint64_t framed = c.count(kMaxSectionBytes, "SectionBytes");
    if (framed != desc[s].len)
      reject("SectionLengthMismatch { section: " + num(declared) + ", declared: " + num(desc[s].len) +
             ", framed: " + num(framed) + " }");
    const Span content = c.take(framed);
    section_digest(desc[s].kind, content, d);
    if (std::memcmp(d, desc[s].digest, 32) != 0) reject("SectionDigestMismatch { section: " + num(declared) + " }");
    e.section[s] = content;
  }
  if (c.remaining() != 0) reject("TrailingBytes { count: " + num(c.remaining()) + " }");

  // validate (validate.rs:68-82), the parts this reader can decide.
  if (e.provider_count == 0) reject("ModelObligation { MissingSelectedLoweringProvider }");
  bool carried_any = false;
  for (uint32_t i = 0; i < e.payload_count; ++i) carried_any = carried_any || e.payloads[i].carried;
  if (carried_any != embedded_feature) reject("DeclaredFeatureMismatch");

  // check_sections (validate.rs:249-290): purpose, then content, strictly
  // increasing; every payload section referenced by a carried payload.  A
  // kernel-program section is referenced by a variant, which is not parsed.
  for (uint32_t s = 1; s < sections; ++s) {
    int cmp = (int)e.section_kind[s - 1] - (int)e.section_kind[s];
    if (cmp == 0) cmp = compare(e.section[s - 1], e.section[s]);
    require_ordered(cmp, "Section");
  }
  for (uint32_t s = 0; s < sections; ++s) {
    if (e.section_kind[s] == kSectionKernelProgram) continue;
    bool referenced = false;
    for (uint32_t i = 0; i < e.payload_count; ++i)
      referenced = referenced || (e.payloads[i].carried &&
                                  (e.payloads[i].metadata_section == s || e.payloads[i].code_section == s));
    if (!referenced) reject("UnreferencedSection { section: " + num(s) + " }");
  }

  // check_payload_identity (validate.rs:299-327).
  for (uint32_t i = 0; i < e.payload_count; ++i) {
    EnvelopePayload& p = e.payloads[i];
    if (!p.carried) continue;
    p.metadata = e.section[p.metadata_section];
    p.code = e.section[p.code_section];
    PayloadSubject subject;
    const std::string why = read_payload_metadata(p.metadata.p, p.metadata.n, subject, nullptr, 0);
    if (!why.empty()) reject(why);
    governed_digest_of(kPayloadIdentityDomain, nullptr, nullptr, 0, p.metadata, d);
    if (p.digest.n != 32 || std::memcmp(d, p.digest.p, 32) != 0)
      reject("PayloadIdentityMismatch { payload: " + num(i) + " }");
  }
  return "";
}

void metadata_or_throw(const uint8_t* bytes, uint64_t n, PayloadSubject& m, PayloadMapping* out,
                       uint64_t capacity) {
  Cursor c(bytes, n);
  const Span domain = c.take(sizeof(kPayloadMetadataDomain));
  if (std::memcmp(domain.p, kPayloadMetadataDomain, sizeof(kPayloadMetadataDomain)) != 0)
    reject("BadPayloadMetadataDomain");
  const uint16_t major = c.u16(), minor = c.u16();
  if (major != kPayloadMetadataSchema[0] || minor > kPayloadMetadataSchema[1])
    reject("UnsupportedPayloadMetadataSchema { major: " + num(major) + ", minor: " + num(minor) + " }");
  m.source_representation = governed_key(c, "Representation");
  m.source = c.slice();
  if (m.source.n > kMaxPayloadSourceBytes) reject(limit("PayloadSourceBytes", m.source.n, kMaxPayloadSourceBytes));

  // Provenance (payload.rs:805-851).
  m.toolchain = c.text();
  m.target = c.text();
  m.family = c.text();
  m.language = c.text();
  m.deployment_major = c.u16();
  m.deployment_minor = c.u16();
  const uint64_t components_at = c.position();
  m.component_count = c.count(kMaxProvenanceComponents, "ProvenanceComponents");
  // Each collection is read whole before its order is checked, as
  // Cursor::vec then require_canonical do.
  Span prev_role{}, prev_version{};
  std::string missing;
  int order = -1;
  for (uint64_t i = 0; i < m.component_count; ++i) {
    const Span role = c.text(), version = c.text();
    if (i && order < 0) {
      order = compare(prev_role, role);
      if (order == 0) order = compare(prev_version, version);
    }
    if (missing.empty() && role.n == 0) missing = "ToolComponentRole";
    if (missing.empty() && version.n == 0) missing = "ToolComponentVersion";
    prev_role = role;
    prev_version = version;
  }
  if (order >= 0) require_ordered(order, "ProvenanceComponent");
  m.components = Span{c.at(components_at), c.position() - components_at};
  m.sdk_name = c.text();
  m.sdk_version = c.text();
  m.sdk_build = c.text();
  const uint64_t flags_at = c.position();
  m.compile_flag_count = c.count(kMaxProvenanceFlags, "ProvenanceFlags");
  for (uint64_t i = 0; i < m.compile_flag_count; ++i) c.text();
  m.link_flag_count = c.count(kMaxProvenanceFlags, "ProvenanceFlags");
  for (uint64_t i = 0; i < m.link_flag_count; ++i) c.text();
  m.flags = Span{c.at(flags_at), c.position() - flags_at};

  const uint64_t entries_at = c.position();
  m.entry_count = c.count(kMaxPayloadEntryMappings, "PayloadEntryMappings");
  Span prev_key{};
  order = -1;
  for (uint64_t i = 0; i < m.entry_count; ++i) {
    PayloadMapping e;
    e.key = opaque(c, "BackendEntry", kMaxKernelIdentityBytes);
    e.symbol = c.text();
    e.transport_count = c.count(kMaxEntryTransports, "EntryTransports");
    e.transports = c.take(4 * e.transport_count);
    if (i && order < 0) order = compare(prev_key, e.key);
    prev_key = e.key;
    if (i < capacity && out) out[i] = e;
  }
  if (order >= 0) require_ordered(order, "PayloadEntryMapping");
  m.entries = Span{c.at(entries_at), c.position() - entries_at};

  m.obligation_count = c.count(kMaxTargetObligations, "TargetObligations");
  Span prev_ok{}, prev_ov{};
  order = -1;
  for (uint64_t i = 0; i < m.obligation_count; ++i) {
    const Span k = c.text(), v = c.text();
    if (i && order < 0) {
      order = compare(prev_ok, k);
      if (order == 0) order = compare(prev_ov, v);
    }
    prev_ok = k;
    prev_ov = v;
  }
  if (order >= 0) require_ordered(order, "TargetObligation");

  // The platform tag ends the record; its absence is the versioned-SDK shape
  // (payload.rs:731-774).
  if (c.remaining() != 0) {
    const uint8_t tag = c.u8();
    if (tag != kPlatformUnversioned) unknown_tag("PayloadPlatform", tag);
    m.unversioned = true;
  }
  if (m.unversioned) {
    const char* stated = nullptr;
    if (m.deployment_major != 0 || m.deployment_minor != 0) stated = "DeploymentMinimum";
    else if (m.sdk_name.n) stated = "SdkName";
    else if (m.sdk_version.n) stated = "SdkVersion";
    else if (m.sdk_build.n) stated = "SdkBuild";
    if (stated) reject(std::string("PlatformFieldWithoutPlatform { field: ") + stated + " }");
  }
  if (c.remaining() != 0) reject("TrailingManifestBytes { count: " + num(c.remaining()) + " }");

  // check_provenance (payload.rs:291-343).
  const char* field = nullptr;
  if (m.toolchain.n == 0) field = "Toolchain";
  else if (m.target.n == 0) field = "Target";
  else if (m.family.n == 0) field = "Family";
  else if (m.language.n == 0) field = "Language";
  else if (!missing.empty()) field = missing == "ToolComponentRole" ? "ToolComponentRole" : "ToolComponentVersion";
  else if (!m.unversioned) {
    if (m.deployment_major == 0) field = "DeploymentMinimum";
    else if (m.sdk_name.n == 0) field = "SdkName";
    else if (m.sdk_version.n == 0) field = "SdkVersion";
    else if (m.sdk_build.n == 0) field = "SdkBuild";
  }
  if (field)
    reject(std::string("ModelRule { IncompletePayloadProvenance { field: ") + field + " } }");
}

}  // namespace

std::string read_envelope(const uint8_t* bytes, uint64_t n, Envelope& out) {
  out = Envelope();
  if (!bytes && n) return "Truncated { needed: 8, available: 0 }";
  try {
    return read_envelope_or_throw(bytes, n, out);
  } catch (const Reject& r) {
    return r.why;
  } catch (...) {  // allocation failure: nothing crosses the C ABI
    return "AllocationFailure";
  }
}

const char* first_disagreeing_fact(const PayloadSubject& expected, const PayloadSubject& actual) {
  auto same = [](Span a, Span b) { return a.n == b.n && (a.n == 0 || std::memcmp(a.p, b.p, a.n) == 0); };
  if (!same(expected.source_representation, actual.source_representation)) return "source-representation";
  if (!same(expected.source, actual.source)) return "source";
  if (!same(expected.toolchain, actual.toolchain)) return "toolchain";
  if (!same(expected.target, actual.target)) return "target";
  if (!same(expected.components, actual.components)) return "components";
  if (!same(expected.flags, actual.flags)) return "flags";
  if (!same(expected.entries, actual.entries)) return "entries";
  return "";
}

std::string read_payload_metadata(const uint8_t* bytes, uint64_t n, PayloadSubject& out,
                                  PayloadMapping* mappings, uint64_t capacity) {
  out = PayloadSubject();
  if (!bytes && n) return "Truncated { needed: 1, available: 0 }";
  try {
    metadata_or_throw(bytes, n, out, mappings, capacity);
    return "";
  } catch (const Reject& r) {
    return r.why;
  } catch (...) {
    return "AllocationFailure";
  }
}

}  // namespace tiler_rt
