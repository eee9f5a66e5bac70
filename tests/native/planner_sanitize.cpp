// Host-only driver for the sanitizer test: runs every planner over many
// random and edge-case requests, plus the governed digest over random
// splits, under AddressSanitizer and UndefinedBehaviorSanitizer.  No device
// code and no HIP runtime: the planners and the digest are plain C++.
#include <cstdio>
#include <cstring>
#include <random>

#include "digest.h"
#include "program.h"

using namespace tiler_rt;

static uint64_t pick(std::mt19937_64& r) {
  static const uint64_t edges[] = {0, 1, 2, 7, 8, 15, 16, 63, 64, 255, 256, 257, 4095, 4096, 8191, 8192,
                                   8193, 65535, 1ull << 20, (1ull << 31) - 1, 1ull << 31, 0xffffffffull,
                                   1ull << 32, UINT64_MAX / 3, UINT64_MAX};
  if (r() % 3 == 0) return edges[r() % (sizeof(edges) / sizeof(edges[0]))];
  return r() % (r() % 2 ? 100000 : 5000000);
}

static void check(const Program& p) {
  for (uint32_t i = 0; i < p.nlaunches; ++i) {
    const Launch& l = p.launches[i];
    if (l.overflow || l.kernarg_bytes > kMaxKernargBytes || l.nargs > kMaxArgs) {
      std::printf("segment overflow in %s\n", l.symbol);
      std::exit(1);
    }
    for (uint32_t b = 0; b < l.nbindings; ++b)
      if (l.bindings[b].slot >= p.nslots || l.bindings[b].offset + 8 > l.kernarg_bytes) {
        std::printf("bad binding in %s\n", l.symbol);
        std::exit(1);
      }
  }
}

int main() {
  std::mt19937_64 r(20261201);
  uint64_t planned = 0;
  for (int it = 0; it < 20000; ++it) {
    const Target t{(uint32_t)(1 + r() % 512), 20000};
    const uintptr_t addr[kMaxSlots] = {r() % 2 ? 0u : 1u, r() % 2 ? 0u : 4u, 0, 16, 2, 0};
    const Mode mode = r() % 2 ? Mode::Direct : Mode::Realized;
    uint64_t dims[8], strides[8];
    for (int d = 0; d < 8; ++d) {
      dims[d] = pick(r) % 300;
      strides[d] = pick(r) % 1000;
    }
    tiler_hip_sum_plan sp{};
    sp.topology = (uint32_t)(r() % 5);
    sp.partitions = pick(r);
    sp.participants = pick(r);
    sp.per_partition = pick(r);
    sp.rounds = pick(r);
    Program p[10];
    plan_sum_f32(t, pick(r), pick(r), sp, addr, p[0]);
    plan_rms_norm((uint32_t)(r() % 3), (int32_t)(r() % 2), pick(r), pick(r), r() % 2 ? 0x3727C5ACu : (uint32_t)r(),
                  addr, p[1]);
    plan_softmax_f32(r() % 2 ? Mode::Direct : Mode::Realized, t, pick(r), pick(r), addr, p[2]);
    plan_map(mode, (uint32_t)(r() % 5), (uint32_t)(r() % 3), (int32_t)(r() % 2), pick(r), 1.0f, 2.0f, addr, p[3]);
    plan_broadcast(pick(r), (uint32_t)(r() % 10) % 9, dims, strides, (uint32_t)(r() % 6), p[4]);
    plan_gather(mode, pick(r), pick(r), pick(r), (uint32_t)(r() % 17), pick(r), (int32_t)(r() % 2), addr, p[5]);
    plan_convert(mode, (uint32_t)(r() % 3), pick(r), addr, p[6]);
    plan_contract_strict_f32(pick(r), pick(r), pick(r), p[7]);
    plan_contract_bf16(t, pick(r), pick(r), pick(r), (uint32_t)(r() % 3), addr, p[8]);
    for (int i = 0; i < 9; ++i) {
      check(p[i]);
      planned += p[i].nlaunches;
    }
  }
  // The governed digest over random lengths and qualifier splits: one run
  // split at random points must digest like the whole run.
  for (int it = 0; it < 2000; ++it) {
    std::vector<uint8_t> m(r() % 3000);
    for (auto& b : m) b = (uint8_t)r();
    uint8_t whole[32], split[32];
    governed_digest("d\0", 2, nullptr, nullptr, 0, m.data(), m.size(), whole);
    const size_t a = m.empty() ? 0 : r() % m.size(), b = m.empty() ? 0 : a + r() % (m.size() - a + 1);
    const void* qs[2] = {m.data(), m.data() + a};
    const uint64_t ql[2] = {a, b - a};
    governed_digest("d\0", 2, qs, ql, 2, m.data() + b, m.size() - b, split);
    if (std::memcmp(whole, split, 32) != 0) {
      std::printf("split digest differs at length %zu\n", m.size());
      return 1;
    }
  }
  std::printf("planner-sanitize ok: %llu launches planned\n", (unsigned long long)planned);
  return 0;
}
