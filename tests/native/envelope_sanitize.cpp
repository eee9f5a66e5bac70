// Host-only driver for the sanitizer test of the envelope reader: mutates
// one valid envelope and one valid payload-metadata record (files written
// by the Python test) and reads every mutant under AddressSanitizer and
// UndefinedBehaviorSanitizer.  After a manifest mutation the header is
// resealed (total length and manifest digest recomputed), so the mutant
// reaches the manifest parser rather than stopping at the digest.
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <random>
#include <vector>

#include "digest.h"
#include "envelope.h"

using namespace tiler_rt;

static std::vector<uint8_t> slurp(const char* path) {
  std::ifstream f(path, std::ios::binary);
  return std::vector<uint8_t>(std::istreambuf_iterator<char>(f), {});
}

static uint64_t be64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v = v << 8 | p[i];
  return v;
}

static void put64(uint8_t* p, uint64_t v) {
  for (int i = 7; i >= 0; --i, v >>= 8) p[i] = (uint8_t)v;
}

// Header fields: total length at 17, manifest length at 25, digest at 37.
static void reseal(std::vector<uint8_t>& b) {
  if (b.size() < 69) return;
  put64(&b[17], b.size());
  const uint64_t m = be64(&b[25]);
  if (m > b.size() - 69) return;
  static const char domain[] = "tiler.artifact-envelope.manifest-digest.v1";
  governed_digest(domain, sizeof(domain), nullptr, nullptr, 0, b.data() + 69, m, &b[37]);
}

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  const std::vector<uint8_t> env = slurp(argv[1]), md = slurp(argv[2]);
  Envelope e;
  PayloadSubject s;
  PayloadMapping maps[8];
  if (!read_envelope(env.data(), env.size(), e).empty() || e.payload_count == 0) {
    std::printf("the seed envelope was refused\n");
    return 1;
  }
  if (!read_payload_metadata(md.data(), md.size(), s, maps, 8).empty()) {
    std::printf("the seed metadata was refused\n");
    return 1;
  }
  std::mt19937_64 r(20261201);
  const uint64_t manifest_end = 69 + be64(&env[25]);
  uint64_t accepted = 0, reads = 0;
  for (int it = 0; it < 60000; ++it) {
    std::vector<uint8_t> b = env;
    const int kind = (int)(r() % 5);
    const uint64_t at = 69 + r() % (manifest_end - 69);
    if (kind == 0) {
      b[r() % b.size()] ^= (uint8_t)(1 + r() % 255);
    } else if (kind == 1 && at + 8 <= b.size()) {  // a length or count overwritten
      static const uint64_t big[] = {0, 1, 0xff, 0x1000, 0x10000, 1ull << 32, UINT64_MAX, UINT64_MAX - 7};
      put64(&b[at], big[r() % 8]);
      reseal(b);
    } else if (kind == 2) {
      b[at] ^= (uint8_t)(1 + r() % 255);
      reseal(b);
    } else if (kind == 3) {
      b.resize(r() % b.size());
      reseal(b);
    } else {
      // Bytes inserted with the manifest length unchanged: the framing after
      // them no longer agrees with the declared runs.
      b.insert(b.begin() + (long)at, (size_t)(1 + r() % 9), (uint8_t)r());
      reseal(b);
    }
    ++reads;
    Envelope m;
    if (read_envelope(b.data(), b.size(), m).empty()) ++accepted;
  }
  for (int it = 0; it < 60000; ++it) {
    std::vector<uint8_t> b = md;
    const uint64_t at = r() % b.size();
    if (r() % 2 && at + 8 <= b.size())
      put64(&b[at], r() % 2 ? UINT64_MAX : r() % 70000);
    else
      b[at] ^= (uint8_t)(1 + r() % 255);
    if (r() % 4 == 0) b.resize(r() % b.size());
    PayloadSubject ms;
    PayloadMapping mm[8];
    read_payload_metadata(b.data(), b.size(), ms, mm, 8);
    ++reads;
  }
  std::printf("envelope-sanitize ok: %llu reads, %llu envelope mutants accepted\n", (unsigned long long)reads,
              (unsigned long long)accepted);
  return 0;
}
