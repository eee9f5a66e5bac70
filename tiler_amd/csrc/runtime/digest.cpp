// SHA-256 as FIPS 180-4 specifies it (sections 4.1.2, 4.2.2, 5.1.1, 5.3.3,
// 6.2.2), and the governed digest and framing built on it.
#include "digest.h"

#include <cstring>

namespace tiler_rt {

namespace {

// FIPS 180-4 section 4.2.2: the first 32 bits of the fractional parts of the
// cube roots of the first 64 primes.
constexpr uint32_t kRound[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

// Section 5.3.3: the first 32 bits of the fractional parts of the square
// roots of the first 8 primes.
constexpr uint32_t kInitial[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                  0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

}  // namespace

Sha256::Sha256() : total_(0), fill_(0) { std::memcpy(h_, kInitial, sizeof(h_)); }

void Sha256::compress(const uint8_t* p) {
  uint32_t w[64];
  for (int t = 0; t < 16; ++t)
    w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
  for (int t = 16; t < 64; ++t) {
    const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
    const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
    w[t] = w[t - 16] + s0 + w[t - 7] + s1;
  }
  uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
  for (int t = 0; t < 64; ++t) {
    const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = h + S1 + ch + kRound[t] + w[t];
    const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
    const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
    const uint32_t t2 = S0 + maj;
    h = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = b;
    b = a;
    a = t1 + t2;
  }
  h_[0] += a; h_[1] += b; h_[2] += c; h_[3] += d;
  h_[4] += e; h_[5] += f; h_[6] += g; h_[7] += h;
}

void Sha256::update(const void* data, uint64_t n) {
  if (n == 0) return;  // an empty run may come with a null pointer
  const uint8_t* p = static_cast<const uint8_t*>(data);
  total_ += n;
  if (fill_) {
    const uint64_t take = n < 64u - fill_ ? n : 64u - fill_;
    std::memcpy(buf_ + fill_, p, take);
    fill_ += (uint32_t)take;
    p += take;
    n -= take;
    if (fill_ < 64) return;
    compress(buf_);
    fill_ = 0;
  }
  for (; n >= 64; n -= 64, p += 64) compress(p);
  if (n) {
    std::memcpy(buf_, p, n);
    fill_ = (uint32_t)n;
  }
}

void Sha256::finish(uint8_t out[32]) {
  // Section 5.1.1: a one bit, zeros to 56 mod 64 bytes, the bit length as a
  // 64-bit big-endian integer.
  const uint64_t bits = total_ * 8;
  const uint8_t one = 0x80;
  update(&one, 1);
  const uint8_t zero[64] = {0};
  update(zero, fill_ <= 56 ? 56 - fill_ : 120 - fill_);
  uint8_t len[8];
  for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
  update(len, 8);
  for (int i = 0; i < 8; ++i) {
    out[4 * i] = (uint8_t)(h_[i] >> 24);
    out[4 * i + 1] = (uint8_t)(h_[i] >> 16);
    out[4 * i + 2] = (uint8_t)(h_[i] >> 8);
    out[4 * i + 3] = (uint8_t)h_[i];
  }
}

void governed_digest(const void* domain, uint64_t domain_bytes, const void* const* qualifiers,
                     const uint64_t* qualifier_bytes, uint32_t qualifier_count, const void* bytes,
                     uint64_t byte_count, uint8_t out[32]) {
  Sha256 s;
  s.update(domain, domain_bytes);
  for (uint32_t i = 0; i < qualifier_count; ++i) s.update(qualifiers[i], qualifier_bytes[i]);
  s.update(bytes, byte_count);
  s.finish(out);
}

void push_len(std::vector<uint8_t>& out, uint64_t n) {
  for (int i = 7; i >= 0; --i) out.push_back((uint8_t)(n >> (8 * i)));
}
void push_slice(std::vector<uint8_t>& out, const void* p, uint64_t n) {
  push_len(out, n);
  const uint8_t* b = static_cast<const uint8_t*>(p);
  out.insert(out.end(), b, b + n);
}
void push_str(std::vector<uint8_t>& out, const std::string& s) { push_slice(out, s.data(), s.size()); }
void push_u16(std::vector<uint8_t>& out, uint16_t v) {
  out.push_back((uint8_t)(v >> 8));
  out.push_back((uint8_t)v);
}
void push_u32(std::vector<uint8_t>& out, uint32_t v) {
  for (int i = 3; i >= 0; --i) out.push_back((uint8_t)(v >> (8 * i)));
}

}  // namespace tiler_rt
