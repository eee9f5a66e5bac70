// Host-only driver for the sanitizer test: runs every planner (and the
// expression compiler) over many random and edge-case requests, plus the
// governed digest over random splits, under AddressSanitizer and
// UndefinedBehaviorSanitizer.  No device
// code and no HIP runtime: the planners and the digest are plain C++.
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

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

// A random node array: mostly well formed (operands name earlier nodes,
// inputs dense), with every kind of defect mixed in (operands ahead of their
// node or past the array, unknown ops, repeated or sparse input ordinals).
// A well-formed DAG: a random tree in post-order (every node reachable),
// inputs shared where a leaf reuses an earlier ordinal; at most
// `max_inputs` inputs.
static uint32_t grow(std::mt19937_64& r, std::vector<tiler_hip_expression_node>& v, std::vector<uint32_t>& input_node,
                     uint32_t max_inputs, int depth) {
  const uint32_t kind = depth > 6 || v.size() > 3000 ? 0 : (uint32_t)(r() % 4);
  if (kind == 0) {  // a leaf
    if (r() % 4 == 0 && !input_node.empty()) {
      v.push_back({TILER_HIP_NODE_CONSTANT, r() % 2 ? 0x3f000000u : (uint32_t)(r() & 0xffffu), 0});
      return (uint32_t)v.size() - 1;
    }
    const uint32_t k = (uint32_t)(r() % (input_node.size() + 1));
    if (k < input_node.size() || input_node.size() >= max_inputs) return input_node[k % input_node.size()];
    v.push_back({TILER_HIP_NODE_INPUT, (uint32_t)input_node.size(), 0});
    input_node.push_back((uint32_t)v.size() - 1);
    return input_node.back();
  }
  if (kind == 1) {  // EXP or RSQRT
    const uint32_t a = grow(r, v, input_node, max_inputs, depth + 1);
    v.push_back({r() % 2 ? TILER_HIP_NODE_EXP : TILER_HIP_NODE_RSQRT, a, 0});
    return (uint32_t)v.size() - 1;
  }
  const uint32_t a = grow(r, v, input_node, max_inputs, depth + 1);
  const uint32_t b = grow(r, v, input_node, max_inputs, depth + 1);
  v.push_back({TILER_HIP_NODE_ADD + (uint32_t)(r() % 3), a, b});
  return (uint32_t)v.size() - 1;
}

static std::vector<tiler_hip_expression_node> random_nodes(std::mt19937_64& r, uint32_t& root, bool epilogue) {
  if (r() % 2) {
    std::vector<tiler_hip_expression_node> v;
    std::vector<uint32_t> input_node;
    root = grow(r, v, input_node, epilogue ? 1 : 1 + (uint32_t)(r() % 20), 0);
    return v;
  }
  const uint32_t count = r() % 5 == 0 ? (uint32_t)(r() % 5000) : 1 + (uint32_t)(r() % 40);
  std::vector<tiler_hip_expression_node> v(count);
  uint32_t inputs = 0;
  const bool sloppy = r() % 4 == 0;
  for (uint32_t i = 0; i < count; ++i) {
    tiler_hip_expression_node& n = v[i];
    n.op = sloppy && r() % 10 == 0 ? (uint32_t)r() : (uint32_t)(i == 0 ? 0 : r() % 7);
    if (n.op == TILER_HIP_NODE_INPUT) {
      n.a = sloppy && r() % 5 == 0 ? (uint32_t)(r() % 20) : inputs++;
      n.b = 0;
    } else if (n.op == TILER_HIP_NODE_CONSTANT) {
      n.a = (uint32_t)r();
      n.b = 0;
    } else {
      n.a = sloppy && r() % 8 == 0 ? (uint32_t)r() : (uint32_t)(i ? r() % i : 0);
      n.b = sloppy && r() % 8 == 0 ? (uint32_t)r() : (uint32_t)(i ? r() % i : 0);
    }
  }
  root = sloppy && r() % 4 == 0 ? (uint32_t)r() : (count ? count - 1 : 0);
  return v;
}

// A random contraction structure: labels from a small alphabet (so indices
// meet across operands), ranks up to one past the limit, extents from the
// edge list.
static tiler_hip_contraction_structure random_structure(std::mt19937_64& r) {
  tiler_hip_contraction_structure s{};
  for (int side = 0; side < 2; ++side) {
    s.operand_rank[side] = (uint32_t)(r() % 10);
    for (int d = 0; d < 8; ++d) {
      s.operand_indices[side][d] = 'a' + (uint32_t)(r() % 6);
      s.operand_dims[side][d] = r() % 3 == 0 ? pick(r) : 1 + r() % 70;
    }
  }
  s.output_rank = (uint32_t)(r() % 10);
  for (int d = 0; d < 8; ++d) s.output_indices[d] = 'a' + (uint32_t)(r() % 6);
  s.reserved = r() % 20 == 0 ? 1u : 0u;
  if (r() % 2) {  // a well-formed batched attention-like structure
    const uint64_t b = 1 + r() % 4, h = 1 + r() % 4, q = pick(r) % 600 + 1, k = pick(r) % 600 + 1,
                   d = pick(r) % 300 + 1;
    s = tiler_hip_contraction_structure{};
    s.operand_rank[0] = 4;
    s.operand_rank[1] = 3;
    s.output_rank = 4;
    const char* li = r() % 2 ? "bhqd" : "bhqk";
    const char* ri = li[3] == 'd' ? "bkd" : (r() % 2 ? "bkd" : "bdk");
    const char* oi = li[3] == 'd' ? "bhqk" : "bhqd";
    auto ext = [&](char c) { return c == 'b' ? b : c == 'h' ? h : c == 'q' ? q : c == 'k' ? k : d; };
    for (int i = 0; i < 4; ++i) {
      s.operand_indices[0][i] = (uint32_t)li[i];
      s.operand_dims[0][i] = ext(li[i]);
      s.output_indices[i] = (uint32_t)oi[i];
    }
    for (int i = 0; i < 3; ++i) {
      s.operand_indices[1][i] = (uint32_t)ri[i];
      s.operand_dims[1][i] = ext(ri[i]);
    }
  }
  return s;
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
    for (uint32_t x = 0; x < l.nextents; ++x)
      if (l.extents[x].id >= p.nlive || l.extents[x].offset + 4 > l.kernarg_bytes || l.extents[x].offset % 4) {
        std::printf("bad live extent in %s\n", l.symbol);
        std::exit(1);
      }
  }
  for (uint32_t x = 0; x < p.nlive; ++x)
    if (p.live[x].minimum < 1 || p.live[x].minimum > p.live[x].bound) {
      std::printf("empty live extent range\n");
      std::exit(1);
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
    plan_rms_norm(t, (uint32_t)(r() % 3), (int32_t)(r() % 2), pick(r), pick(r), r() % 2 ? 0x3727C5ACu : (uint32_t)r(),
                  addr, p[1], r() % 3 == 0);
    plan_softmax_f32(r() % 2 ? Mode::Direct : Mode::Realized, t, pick(r), pick(r), addr, p[2], r() % 4 == 0,
                     (uint32_t)(r() % 8));
    plan_map(mode, (uint32_t)(r() % 5), (uint32_t)(r() % 3), (int32_t)(r() % 2), pick(r), 1.0f, 2.0f, addr, p[3]);
    plan_broadcast(pick(r), (uint32_t)(r() % 10) % 9, dims, strides, (uint32_t)(r() % 6), p[4]);
    plan_gather(mode, pick(r), pick(r), pick(r), (uint32_t)(r() % 17), pick(r), (int32_t)(r() % 2), addr, p[5]);
    plan_convert(mode, (uint32_t)(r() % 3), pick(r), addr, p[6]);
    plan_contract_strict_f32(t, pick(r), pick(r), pick(r), addr, p[7], r() % 2 == 0);
    plan_contract_bf16(t, pick(r), pick(r), pick(r), (uint32_t)(r() % 3), addr, p[8], r() % 4 == 0,
                       (uint32_t)(r() % 6), r() % 3 == 0);
    for (int i = 0; i < 9; ++i) {
      check(p[i]);
      planned += p[i].nlaunches;
    }
    // Expressions: the compiler over random DAGs, then the planner over
    // what compiles (under each contract), alone and as a fold epilogue.
    Program q[6];
    uint64_t fdims[8];
    for (int d = 0; d < 8; ++d) fdims[d] = r() % 4 == 0 ? pick(r) : 1 + r() % 40;
    const uint32_t frank = (uint32_t)(r() % 10);
    const uint64_t fmask = r() % 3 == 0 ? r() : r() % (1u << (frank < 8 ? frank : 8));
    uint32_t root = 0;
    const bool epilogue = r() % 4 == 0;
    const std::vector<tiler_hip_expression_node> nodes = random_nodes(r, root, epilogue);
    const uint32_t edtype = (uint32_t)(r() % 3);
    ExpressionProgram prog;
    std::string diag;
    const uint32_t count = r() % 50 == 0 ? (uint32_t)r() % 8000 : (uint32_t)nodes.size();
    if (compile_expression(edtype, nodes.data(), count < nodes.size() ? count : (uint32_t)nodes.size(), root,
                           epilogue, prog, diag) == TILER_HIP_OK) {
      Contract c;
      c.reassociate = r() % 2;
      c.input_mode = 1 + (uint32_t)(r() % 3);
      c.result_mode = 1 + (uint32_t)(r() % 3);
      const uintptr_t eaddr[kMaxSlots] = {r() % 2 ? 0u : 4u, 0, 16, 0, 32, 0};
      plan_expression(t, edtype, pick(r), prog, c, eaddr, q[0]);
      if (epilogue)
        plan_fold((uint32_t)(r() % 5), frank, fdims, fmask, (uint32_t)r(), (uint32_t)r(), &prog, q[1]);
    }
    // Folds over random axis sets (ranks past the limit, empty and huge extents).
    plan_fold((uint32_t)(r() % 5), frank, fdims, fmask, 0x3f800000u, 0u, nullptr, q[2]);
    // Reindex with signed strides and bases, in and out of the source.
    int64_t sstrides[8];
    for (int d = 0; d < 8; ++d) sstrides[d] = (int64_t)(pick(r) % 2000) - 1000;
    plan_reindex(pick(r), (uint32_t)(r() % 10), dims, sstrides, (int64_t)(pick(r) % 100000) - 50000,
                 1u << (r() % 5), q[3]);
    // General contractions, strict and MFMA, with and without the epilogue.
    const tiler_hip_contraction_structure cs = random_structure(r);
    const uintptr_t caddr[kMaxSlots] = {r() % 2 ? 0u : 16u, 0, 0, 0, 0, 0};
    plan_contract_general(t, r() % 2 ? TILER_HIP_F32 : TILER_HIP_BF16, cs, (uint32_t)(r() % 3), r() % 2 == 0, caddr,
                          q[4]);
    for (int i = 0; i < 5; ++i) {
      check(q[i]);
      planned += q[i].nlaunches;
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
