// The governed content digest: FIPS 180-4 SHA-256 over a domain separator,
// fixed-width qualifiers and one trailing byte run (tiler-digest/src/lib.rs:
// 168-240; algorithm tag 0x01, "tiler.digest.sha-256.v1"), and the
// canonical length framing identity encodings use (u64 big-endian length
// before every variable-length run; tiler-ir/src/identity.rs:84-111).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace tiler_rt {

class Sha256 {
 public:
  Sha256();
  void update(const void* data, uint64_t n);
  void finish(uint8_t out[32]);

 private:
  void compress(const uint8_t* block);
  uint32_t h_[8];
  uint8_t buf_[64];
  uint64_t total_;
  uint32_t fill_;
};

void governed_digest(const void* domain, uint64_t domain_bytes, const void* const* qualifiers,
                     const uint64_t* qualifier_bytes, uint32_t qualifier_count, const void* bytes,
                     uint64_t byte_count, uint8_t out[32]);

// Canonical framing primitives.
void push_len(std::vector<uint8_t>& out, uint64_t n);
void push_slice(std::vector<uint8_t>& out, const void* p, uint64_t n);
void push_str(std::vector<uint8_t>& out, const std::string& s);
void push_u16(std::vector<uint8_t>& out, uint16_t v);
void push_u32(std::vector<uint8_t>& out, uint32_t v);

}  // namespace tiler_rt
