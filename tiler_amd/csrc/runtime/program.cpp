// Planners of the realization families: the kernel each request runs, its
// launch geometry and argument segment, with the refusals the family entry
// points of include/tiler_hip.h document.
#include "program.h"

#include "../kernels/contract_geometry.h"

#include <cmath>
#include <cstdio>

namespace tiler_rt {

namespace {

uint64_t mul_sat(uint64_t a, uint64_t b) {
  if (a && b > UINT64_MAX / a) return UINT64_MAX;
  return a * b;
}

bool aligned16(uintptr_t a) { return (a & 15u) == 0; }

uint32_t pow2_at_least(uint64_t v) {
  uint32_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Rows longer than one wave holds (8192 elements) run one 1024-thread
// workgroup per row: chunks per thread rounded up to a power of two while the
// row fits in registers (<= 8 chunks), else 0 (the row is streamed).
uint32_t long_row_chunks(uint64_t extent, uint32_t vec) {
  uint64_t per = (((extent + vec - 1) / vec) + 1023) / 1024;
  if (per > 8) return 0;
  uint32_t ch = 1;
  while (ch < per) ch <<= 1;
  return ch;
}

// The launch geometry every family uses for grid-stride kernels.
uint32_t blocks_capped(uint64_t work, uint64_t cap) {
  uint64_t b = (work + 255) / 256;
  return (uint32_t)(b < cap ? b : cap);
}

// Host mirror of the kernels' BroadcastGeometry argument.
struct BroadcastGeometryHost {
  uint64_t out_dims[8];
  uint64_t src_strides[8];
  uint32_t rank;
  uint64_t base;
};

// Host mirror of fold.hip's FoldGeometry.
struct FoldGeometryHost {
  uint64_t dims[8];
  uint64_t strides[8];
  uint32_t kept_rank, red_rank;
};

}  // namespace

// ---------------------------------------------------------------------------
Launch& Launch::blob(const void* p, uint32_t bytes, uint32_t align) {
  uint32_t off = (kernarg_bytes + align - 1) / align * align;
  if (off + bytes > kMaxKernargBytes || nargs >= kMaxArgs) {
    overflow = true;
    return *this;
  }
  std::memset(kernargs + kernarg_bytes, 0, off - kernarg_bytes);
  if (p) std::memcpy(kernargs + off, p, bytes);
  else std::memset(kernargs + off, 0, bytes);
  arg_offsets[nargs++] = off;
  kernarg_bytes = off + bytes;
  return *this;
}
Launch& Launch::ptr(uint32_t slot, uint64_t addend) {
  if (nbindings >= kMaxBindings) {
    overflow = true;
    return *this;
  }
  blob(nullptr, 8, 8);
  if (!overflow) bindings[nbindings++] = {arg_offsets[nargs - 1], slot, addend};
  return *this;
}
Launch& Launch::null_ptr() { return blob(nullptr, 8, 8); }
Launch& Launch::ptr_table(const uint32_t* slots, uint32_t count, uint32_t capacity) {
  if (count > capacity || nbindings + count > kMaxBindings) {
    overflow = true;
    return *this;
  }
  blob(nullptr, 8 * capacity, 8);
  if (overflow) return *this;
  const uint32_t base = arg_offsets[nargs - 1];
  for (uint32_t i = 0; i < count; ++i) bindings[nbindings++] = {base + 8 * i, slots[i], 0};
  return *this;
}
Launch& Launch::u32(uint32_t v) { return blob(&v, 4, 4); }
Launch& Launch::live_u32(uint32_t id) {
  if (nextents >= kMaxLiveExtents) {
    overflow = true;
    return *this;
  }
  blob(nullptr, 4, 4);
  if (!overflow) extents[nextents++] = {arg_offsets[nargs - 1], id};
  return *this;
}
Launch& Launch::u64(uint64_t v) { return blob(&v, 8, 8); }
Launch& Launch::f32(float v) { return blob(&v, 4, 4); }

Program::Program() : nslots(0), nlaunches(0) {}

uint32_t Program::slot(uint64_t bytes, uint32_t role) {
  slot_bytes[nslots] = bytes;
  slot_roles[nslots] = role;
  return nslots++;
}

Launch& Program::add(const char* symbol, uint32_t gx, uint32_t gy, uint32_t block) {
  Launch& l = launches[nlaunches++];
  std::snprintf(l.symbol, sizeof(l.symbol), "%s", symbol);
  l.grid[0] = gx;
  l.grid[1] = gy;
  l.block = block;
  l.kernarg_bytes = 0;
  l.nargs = 0;
  l.nbindings = 0;
  l.nextents = 0;
  l.overflow = false;
  return l;
}

uint32_t tree_workgroups(const Target& t, uint64_t n) {
  uint64_t tiles = (n + 1023) / 1024;
  uint64_t cap = 2ull * t.compute_units;
  if (cap > kMaxSumWorkgroups) cap = kMaxSumWorkgroups;
  uint64_t g = tiles < cap ? tiles : cap;
  return g ? (uint32_t)g : 1u;
}

// ---------------------------------------------------------------------------
// Sum over the last axis of [rows, extent] f32.  Slots: 0 x, 1 out,
// 2 partials (multi-pass and the single-output tree).
// The strict serial fold of `nrows` contiguous rows of `length` elements
// (slot `src`, row v at v * length) into `dst`.  Rows of 64 or more elements
// are staged through LDS, R rows per workgroup with R the smallest of
// 1, 4, 16, 64 that keeps to one workgroup per CU (64 beyond), so that the
// folding chains of few long rows get a SIMD each; rows of 16..63 in stages
// of 16, 256 rows per workgroup; shorter rows take one lane per row, whose
// loads are already near one another.
// The rule-driven forms (a flushing contract, a fused prologue): the same
// stages with the rule's contributor and combine, seeded at the first
// contributor; rows under 16 take one lane per row (the general fold over the
// trailing axis of [nrows, length]).
static void add_rule_fold(const Target& t, uint32_t src, bool src_aligned, uint64_t nrows, uint64_t length,
                          uint32_t dst, const FoldRuleHost& rule, Program& p) {
  const bool vec = src_aligned && length % 4 == 0;
  char name[48];
  if (length >= 16) {
    const uint64_t cus = t.compute_units;
    const uint32_t R = length < 64 ? 256 : nrows <= cus ? 1 : nrows <= 4 * cus ? 4 : nrows <= 16 * cus ? 16 : 64;
    std::snprintf(name, sizeof(name), "tiler_sum_f32_staged_r%u%s_m", R, vec ? "" : "_u");
    p.add(name, (uint32_t)((nrows + R - 1) / R), 1, 256)
        .ptr(src).u64(nrows).u64(length).ptr(dst).blob(&rule, sizeof(rule), 4);
    return;
  }
  FoldGeometryHost g;
  std::memset(&g, 0, sizeof(g));
  g.dims[0] = nrows;
  g.strides[0] = length;
  g.dims[1] = length;
  g.strides[1] = 1;
  g.kept_rank = 1;
  g.red_rank = 1;
  p.add("tiler_fold_f32_m", blocks_capped(nrows, 65536), 1, 256)
      .ptr(src).ptr(dst).u64(nrows).u64(length).blob(&g, sizeof(g), 8).blob(&rule, sizeof(rule), 4).u32(0);
}

static void add_serial_fold(const Target& t, uint32_t src, bool src_aligned, uint64_t nrows, uint64_t length,
                            uint32_t dst, Program& p, const FoldRuleHost* rule = nullptr) {
  if (rule) {
    add_rule_fold(t, src, src_aligned, nrows, length, dst, *rule, p);
    return;
  }
  if (length >= 64) {
    const uint64_t cus = t.compute_units;
    const uint32_t R = nrows <= cus ? 1 : nrows <= 4 * cus ? 4 : nrows <= 16 * cus ? 16 : 64;
    const bool vec = src_aligned && length % 4 == 0;
    char name[40];
    std::snprintf(name, sizeof(name), "tiler_sum_f32_staged_r%u%s", R, vec ? "" : "_u");
    p.add(name, (uint32_t)((nrows + R - 1) / R), 1, 256).ptr(src).u64(nrows).u64(length).ptr(dst);
    return;
  }
  if (length >= 16) {  // stages of 16 elements, 256 rows per workgroup, every lane folding
    const bool vec = src_aligned && length % 4 == 0;
    p.add(vec ? "tiler_sum_f32_staged_r256" : "tiler_sum_f32_staged_r256_u", (uint32_t)((nrows + 255) / 256), 1, 256)
        .ptr(src).u64(nrows).u64(length).ptr(dst);
    return;
  }
  p.add("tiler_sum_f32_serial", (uint32_t)((nrows + 255) / 256), 1, 256)
      .ptr(src).u64(nrows).u64(length).u64(1).ptr(dst);
}

tiler_hip_status plan_sum_f32(const Target& t, uint64_t rows, uint64_t extent,
                              const tiler_hip_sum_plan& sp, const uintptr_t* addr, Program& p,
                              const FoldRuleHost* rule) {
  const uint32_t x = p.slot(mul_sat(mul_sat(rows, extent), 4), kSlotInput);
  const uint32_t out = p.slot(mul_sat(rows, 4), kSlotOutput);
  // The partials' fold takes the modes but not the prologue: it sums values
  // the first pass already produced (evaluate.rs:788-832).
  FoldRuleHost second;
  if (rule) {
    second = *rule;
    second.prologue = 0;
  }
  switch (sp.topology) {
    case TILER_HIP_SUM_SERIAL:
      if (rows == 0) return TILER_HIP_OK;
      if ((rows + 255) / 256 > 0x7fffffffull || (extent >= 16 && rows > 0x7fffffffull))
        return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
      add_serial_fold(t, x, aligned16(addr[x]), rows, extent, out, p, rule);
      return TILER_HIP_OK;
    case TILER_HIP_SUM_MULTIPASS: {
      const uint64_t P = sp.partitions, c = sp.per_partition;
      if (rows == 0) return TILER_HIP_OK;
      if (P == 0 || (c != 0 && P > UINT64_MAX / c) || P * c != extent)
        return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "partitions do not cover the axis exactly");
      if (mul_sat(rows, P) / 256 >= 0x7fffffffull || (c >= 16 && mul_sat(rows, P) > 0x7fffffffull))
        return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more partitions than the launch grid holds");
      const uint32_t part = p.slot(mul_sat(mul_sat(rows, P), 4), kSlotScratch);
      // With exact coverage partition p of row r is the contiguous run
      // (r*P + p) * c: pass 1 is the serial fold of rows*P rows of c.
      if (c >= 16)
        add_serial_fold(t, x, aligned16(addr[x]), rows * P, c, part, p, rule);
      else if (rule)
        p.add("tiler_sum_f32_partials_m", (uint32_t)((rows * P + 255) / 256), 1, 256)
            .ptr(x).u64(rows).u64(extent).u64(P).u64(c).ptr(part).blob(rule, sizeof(*rule), 4);
      else
        p.add("tiler_sum_f32_partials", (uint32_t)((rows * P + 255) / 256), 1, 256)
            .ptr(x).u64(rows).u64(extent).u64(P).u64(c).ptr(part);
      // the partials are the planner's own scratch, 16-byte aligned
      add_serial_fold(t, part, true, rows, P, out, p, rule ? &second : nullptr);
      return TILER_HIP_OK;
    }
    case TILER_HIP_SUM_COOPERATIVE: {
      const uint64_t P = sp.participants, c = sp.per_partition, R = sp.rounds;
      if (rows == 0) return TILER_HIP_OK;
      if (P == 0 || P > 1024 || c == 0 || R == 0 || P * c * R != extent)
        return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "grouping does not cover the axis exactly");
      if (rows > 0x7fffffffull) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
      Launch& l = p.add(rule ? "tiler_sum_f32_cooperative_m" : "tiler_sum_f32_cooperative", (uint32_t)rows, 1, (uint32_t)P)
                      .ptr(x).u64(extent).u32((uint32_t)P).u64(c).u64(R).u32(sp.participant_major ? 1u : 0u).ptr(out);
      if (rule) l.blob(rule, sizeof(*rule), 4);
      return TILER_HIP_OK;
    }
    case TILER_HIP_SUM_TREE: {
      // The tree's lanes start from the additive identity, which a flushing
      // result mode would make observable (a lone subnormal partial flushed
      // by an add the reference never performs), and its kernels take no
      // prologue: the reference's own groupings (the split, the cooperative
      // workgroup) realize those.
      if (rule)
        return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                        "the two-level tree realizes neither a flushing contract nor a fused prologue; the multi-pass "
                        "split and the cooperative workgroup do");
      if (rows == 0) return TILER_HIP_OK;
      if (rows == 1) {
        const uint32_t G = tree_workgroups(t, extent);
        const uint32_t part = p.slot((uint64_t)G * 4, kSlotScratch);
        p.add(aligned16(addr[x]) ? "tiler_sum_f32_grid" : "tiler_sum_f32_grid_unaligned", G, 1, 256)
            .ptr(x).u64(extent).ptr(part);
        p.add("tiler_sum_f32_grid_final", 1, 1, 256).ptr(part).u32(G).u64(extent).ptr(out);
        return TILER_HIP_OK;
      }
      if (rows > 0x7fffffffull) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
      if (extent >= 1 && extent <= 256) {  // the same grouping, one wave per row
        p.add(aligned16(addr[x]) && extent % 4 == 0 ? "tiler_sum_f32_rows_w" : "tiler_sum_f32_rows_w_u",
              (uint32_t)((rows + 3) / 4), 1, 256)
            .ptr(x).u64(rows).u32((uint32_t)extent).ptr(out);
        return TILER_HIP_OK;
      }
      p.add("tiler_sum_f32_rows", (uint32_t)rows, 1, 256).ptr(x).u64(extent).ptr(out);
      return TILER_HIP_OK;
    }
    default:
      return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "unknown reduction topology");
  }
}

// ---------------------------------------------------------------------------
// RMS normalization.  Slots: 0 x, 1 w, 2 y.
tiler_hip_status plan_rms_norm(const Target& t, uint32_t dtype, int32_t weight_broadcast, uint64_t rows,
                               uint64_t extent, uint32_t eps_bits, const uintptr_t* addr,
                               Program& p, bool strict, uint32_t in_mode, uint32_t out_mode) {
  // A flushing contract: the serial fold with the modes at every site (the
  // _m forms of the strict kernels, or the one-wave-per-row kernel, which
  // take them), whatever the topology.
  const bool modes = in_mode > 1 || out_mode > 1;
  if (modes) strict = true;
  float eps;
  std::memcpy(&eps, &eps_bits, 4);
  // rms_norm.rs:462-466: a non-positive or non-finite eps refuses.
  if (!(eps > 0.0f) || !std::isfinite(eps))
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "eps must be positive and finite");
  if (dtype != TILER_HIP_F32 && dtype != TILER_HIP_BF16)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "rms_norm dtype");
  const uint64_t elem = dtype == TILER_HIP_BF16 ? 2 : 4;
  const uint32_t x = p.slot(mul_sat(mul_sat(rows, extent), elem), kSlotInput);
  const uint32_t w = p.slot(mul_sat(weight_broadcast ? extent : mul_sat(rows, extent), elem), kSlotInput);
  const uint32_t y = p.slot(mul_sat(mul_sat(rows, extent), elem), kSlotOutput);
  if (rows == 0 || extent == 0) return TILER_HIP_OK;
  const uint32_t vec = dtype == TILER_HIP_BF16 ? 8 : 4;
  const uint32_t max_ch = dtype == TILER_HIP_BF16 ? 16 : 32;
  if (extent > 0xffffffffull)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "row longer than 2^32 - 1 elements");
  const char* ty = dtype == TILER_HIP_BF16 ? "bf16" : "f32";
  const bool al = aligned16(addr[x]) && aligned16(addr[w]) && aligned16(addr[y]) && (extent * elem) % 16 == 0;
  const uint64_t wstride = weight_broadcast ? 0 : extent;
  char name[64];
  const uint64_t cus = t.compute_units;
  const uint64_t per16 = 16 / elem;  // elements per 16-byte piece
  if (strict && al && extent % per16 == 0 && extent >= 16 * per16 && extent <= 512 * per16 && rows >= 8 * cus) {
    // Rows of at most 512 pieces held in registers, 8 per workgroup: x read
    // once, y written once, the fold of the squares 8 rows per wave
    // instruction (under a flushing contract the _m form, with the modes).
    if ((rows + 7) / 8 > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
    std::snprintf(name, sizeof(name), "tiler_rms_norm_%s_strict_rr8_p%u%s", ty, extent <= 256 * per16 ? 8u : 16u,
                  modes ? "_m" : "");
    Launch& l = p.add(name, (uint32_t)((rows + 7) / 8), 1, 256)
                    .ptr(x).ptr(w).u64(wstride).ptr(y).u64(rows).u32((uint32_t)extent).f32(eps);
    if (modes) l.u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  if (strict && extent >= 64) {
    // Otherwise the reference's serial fold of the squares, staged: R rows
    // per workgroup, the largest of 64, 16, 4 that still gives every CU a
    // workgroup (else 1), a folding lane per row (the _m forms with the
    // modes).
    const uint32_t R = rows >= 64 * cus ? 64 : rows >= 16 * cus ? 16 : rows >= 4 * cus ? 4 : 1;
    if ((rows + R - 1) / R > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
    std::snprintf(name, sizeof(name), "tiler_rms_norm_%s_strict_r%u%s%s", ty, R, al ? "" : "_u", modes ? "_m" : "");
    Launch& l = p.add(name, (uint32_t)((rows + R - 1) / R), 1, 256)
                    .ptr(x).ptr(w).u64(wstride).ptr(y).u64(rows).u32((uint32_t)extent).f32(eps);
    if (modes) l.u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  if (strict) {  // short rows: the reference's serial fold of the squares, one wave per row
    if ((rows + 3) / 4 > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
    std::snprintf(name, sizeof(name), "tiler_rms_norm_%s_strict", ty);
    p.add(name, (uint32_t)((rows + 3) / 4), 1, 256)
        .ptr(x).ptr(w).u64(wstride).ptr(y).u64(rows).u32((uint32_t)extent).f32(eps).u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  if (extent > kWaveRowMax) {  // one workgroup per row
    if (rows > 0x7fffffffull) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
    std::snprintf(name, sizeof(name), "tiler_rms_norm_%s_long%u%s", ty, long_row_chunks(extent, vec), al ? "_a" : "_u");
    p.add(name, (uint32_t)rows, 1, 1024).ptr(x).ptr(w).u64(wstride).ptr(y).u32((uint32_t)extent).f32(eps);
    return TILER_HIP_OK;
  }
  const uint32_t ch = pow2_at_least((extent + 64ull * vec - 1) / (64ull * vec));
  if (ch > max_ch) return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "row realization");
  const bool full = al && extent == (uint64_t)ch * 64 * vec;
  std::snprintf(name, sizeof(name), "tiler_rms_norm_%s_ch%u%s", ty, ch, full ? "_full" : al ? "" : "_u");
  // one row per wave, four waves per workgroup
  if ((rows + 3) / 4 > 0x7fffffffull)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
  p.add(name, (uint32_t)((rows + 3) / 4), 1, 256)
      .ptr(x).ptr(w).u64(wstride).ptr(y).u64(rows).u32((uint32_t)extent).f32(eps);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Softmax over the last axis.  Slots: 0 x, 1 y; the split form adds 2 the
// segment maxima and 3 the segment sums (scratch, rows * segments f32 each).
// Rows longer than 8192 elements fold by 8192-element segments; the planner
// picks how that fold runs, never what it computes:
// * a row of at most 4 segments: one 1024-thread workgroup per row, the row
//   in registers (read once);
// * longer rows: one 256-thread workgroup per segment in three launches
//   (maxima, sums, output; x read three times), the partials in scratch.
//   Measured faster than streaming each row through one workgroup at every
//   row count tried (1 to 512 rows), up to 68x for a single row;
// * longer rows, at most two workgroups per CU: the same workgroups in one
//   row-synchronized launch (x read once), its epoch and tagged words in
//   slot 2 -- for direct calls the context workspace's area, which stays
//   valid between calls; a realized plan's scratch is fresh, so its program
//   zeroes the area with a fill kernel first.
tiler_hip_status plan_softmax_f32(Mode mode, const Target& t, uint64_t rows, uint64_t extent,
                                  const uintptr_t* addr, Program& p, bool strict, uint32_t form,
                                  uint32_t in_mode, uint32_t out_mode) {
  const uint32_t x = p.slot(mul_sat(mul_sat(rows, extent), 4), kSlotInput);
  const uint32_t y = p.slot(mul_sat(mul_sat(rows, extent), 4), kSlotOutput);
  // A flushing contract: the serial exponent sum with the modes at every site
  // (the _m forms of the strict kernels, or the one-wave-per-row kernel,
  // which take them).
  const bool modes = in_mode > 1 || out_mode > 1;
  if (modes && form != TILER_HIP_FORM_AUTO)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "form: a flushing contract has the serial form only");
  if (modes) strict = true;
  if (form != TILER_HIP_FORM_AUTO) {
    if (strict || (form != TILER_HIP_FORM_SOFTMAX_SPLIT && form != TILER_HIP_FORM_SOFTMAX_ROW_SYNC))
      return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "form: not a form of this softmax");
    if ((extent + kSoftmaxSegment - 1) / kSoftmaxSegment <= 4)
      return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                      "segmented-rows: the split and row-synchronized forms take rows of more than four segments");
  }
  if (rows == 0 || extent == 0) return TILER_HIP_OK;
  if (extent > 0xffffffffull)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "row longer than 2^32 - 1 elements");
  const uint64_t cus = t.compute_units;
  const bool vec = aligned16(addr[x]) && aligned16(addr[y]) && extent % 4 == 0;
  char sname[48];
  if (strict && vec && extent >= 128 && extent <= 4096 && rows >= 8 * cus) {
    // Rows of at most 4096 held in registers, 8 per workgroup: x read once
    // and y written once, the fold 8 rows per wave instruction (the
    // 65536 x 2048 case: 0.50 ms staged, ~0.22 ms resident; 8192 x 4096:
    // 125 us staged, 86 us resident); under a flushing contract the _m
    // form, with the modes.
    if ((rows + 7) / 8 > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
    std::snprintf(sname, sizeof(sname), "tiler_softmax_f32_strict_rr8_p%u%s",
                  extent <= 1024 ? 8u : extent <= 2048 ? 16u : 32u, modes ? "_m" : "");
    Launch& l = p.add(sname, (uint32_t)((rows + 7) / 8), 1, 256).ptr(x).ptr(y).u64(rows).u32((uint32_t)extent);
    if (modes) l.u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  if (strict && extent >= 64) {
    // The reference's serial exponent sum (the _m forms with the modes).
    // Otherwise staged: R rows per workgroup as for the strict RMSNorm but
    // at most 16 (stages of at least 256 elements, so a stage's fold covers
    // the next stage's loads; 64 rows of 64-element stages ran the
    // 65536 x 2048 case in 611 us, 16 in 524 on the same build), three
    // streamed passes (maximum, exponents folded in order, output).
    const uint32_t R = rows >= 16 * cus ? 16 : rows >= 4 * cus ? 4 : 1;
    if ((rows + R - 1) / R > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
    std::snprintf(sname, sizeof(sname), "tiler_softmax_f32_strict_r%u%s%s", R, vec ? "" : "_u", modes ? "_m" : "");
    Launch& l = p.add(sname, (uint32_t)((rows + R - 1) / R), 1, 256).ptr(x).ptr(y).u64(rows).u32((uint32_t)extent);
    if (modes) l.u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  if (strict) {  // short rows: the reference's serial exponent sum, one wave per row
    if ((rows + 3) / 4 > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
    p.add("tiler_softmax_f32_strict", (uint32_t)((rows + 3) / 4), 1, 256)
        .ptr(x).ptr(y).u64(rows).u32((uint32_t)extent).u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  const bool al = aligned16(addr[x]) && aligned16(addr[y]) && extent % 4 == 0;
  const char* sfx = al ? "_a" : "_u";
  char name[64];
  if (extent > kWaveRowMax) {
    const uint64_t nseg = (extent + kSoftmaxSegment - 1) / kSoftmaxSegment;
    if (nseg <= 4) {
      if (rows > 0x7fffffffull) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
      std::snprintf(name, sizeof(name), "tiler_softmax_f32_long_r%s", sfx);
      p.add(name, (uint32_t)rows, 1, 1024).ptr(x).ptr(y).u32((uint32_t)extent);
      return TILER_HIP_OK;
    }
    const uint64_t wgs = mul_sat(rows, nseg);
    if (wgs > 0x7fffffffull) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more segments than the launch grid holds");
    const bool sync_fits = wgs <= 2ull * t.compute_units && wgs <= kRowSyncMaxWorkgroups;
    if (form == TILER_HIP_FORM_SOFTMAX_ROW_SYNC && !sync_fits)
      return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                      "row-sync-residency: the row-synchronized form needs every segment's workgroup resident "
                      "(at most two per CU)");
    if (sync_fits && form != TILER_HIP_FORM_SOFTMAX_SPLIT) {
      const uint64_t sync_bytes = 256 + 16 * wgs;
      const uint32_t sync = p.slot(sync_bytes, kSlotScratch);
      if (mode == Mode::Realized)
        p.add("tiler_fill_u32", blocks_capped(sync_bytes / 4, 64), 1, 256).ptr(sync).u32(0).u64(sync_bytes / 4);
      std::snprintf(name, sizeof(name), "tiler_softmax_f32_rowsync%s", sfx);
      p.add(name, (uint32_t)wgs, 1, 256)
          .ptr(x).ptr(y).u32((uint32_t)extent).u64(nseg).ptr(sync).u64(t.row_sync_wait_ticks);
      return TILER_HIP_OK;
    }
    const uint32_t pmax = p.slot(wgs * 4, kSlotScratch);
    const uint32_t psum = p.slot(wgs * 4, kSlotScratch);
    std::snprintf(name, sizeof(name), "tiler_softmax_f32_split_max%s", sfx);
    p.add(name, (uint32_t)wgs, 1, 256).ptr(x).u32((uint32_t)extent).u64(nseg).ptr(pmax);
    std::snprintf(name, sizeof(name), "tiler_softmax_f32_split_sum%s", sfx);
    p.add(name, (uint32_t)wgs, 1, 256).ptr(x).u32((uint32_t)extent).u64(nseg).ptr(pmax).ptr(psum);
    std::snprintf(name, sizeof(name), "tiler_softmax_f32_split_out%s", sfx);
    p.add(name, (uint32_t)wgs, 1, 256).ptr(x).ptr(y).u32((uint32_t)extent).u64(nseg).ptr(pmax).ptr(psum);
    return TILER_HIP_OK;
  }
  const uint32_t ch = pow2_at_least((extent + 255) / 256);
  if (ch > 32) return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "row realization");
  const bool full = al && extent == (uint64_t)ch * 256;
  std::snprintf(name, sizeof(name), "tiler_softmax_f32_ch%u%s", ch, full ? "_full" : al ? "" : "_u");
  if ((rows + 3) / 4 > 0x7fffffffull)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more rows than the launch grid holds");
  p.add(name, (uint32_t)((rows + 3) / 4), 1, 256).ptr(x).ptr(y).u64(rows).u32((uint32_t)extent);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Elementwise maps.  Slots: unary 0 x, 1 y; binary 0 x, 1 x2, 2 y.
// Direct: 16-byte vector kernel over the aligned head, scalar kernel over the
// rest.  Realized (no slot offsets): the vector kernel when it covers all n,
// the scalar kernel otherwise; both compute each element identically.
tiler_hip_status plan_map(Mode mode, uint32_t op, uint32_t dtype, int32_t x2_broadcast,
                          uint64_t n, float a, float b, const uintptr_t* addr, Program& p,
                          uint32_t in_mode, uint32_t out_mode) {
  if (op > TILER_HIP_MAP_MULTIPLY) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "map op");
  if (dtype != TILER_HIP_F32 && dtype != TILER_HIP_BF16)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "map dtype");
  if (dtype == TILER_HIP_BF16 && op == TILER_HIP_MAP_SILU)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "silu is an f32 family");
  const bool binary = op == TILER_HIP_MAP_ADD || op == TILER_HIP_MAP_MULTIPLY;
  const uint64_t eb = dtype == TILER_HIP_BF16 ? 2 : 4;
  const uint32_t x = p.slot(mul_sat(n, eb), kSlotInput);
  const uint32_t x2 = binary ? p.slot(x2_broadcast ? eb : mul_sat(n, eb), kSlotInput) : UINT32_MAX;
  const uint32_t y = p.slot(mul_sat(n, eb), kSlotOutput);
  if (n == 0) return TILER_HIP_OK;
  if (in_mode > 1 || out_mode > 1) {  // a flushing contract: the scalar form with the modes
    Launch& l = p.add(dtype == TILER_HIP_BF16 ? "tiler_map_bf16_m" : "tiler_map_f32_m", blocks_capped(n, 8192), 1, 256)
                    .ptr(x);
    if (binary) l.ptr(x2);
    else l.null_ptr();
    l.u64(x2_broadcast ? 0 : 1).u64(n).u32(op).f32(a).f32(b).ptr(y).u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  const uint64_t per = dtype == TILER_HIP_BF16 ? 8 : 4;  // elements per 16-byte chunk
  const bool vec_ok = aligned16(addr[x]) && aligned16(addr[y]) && (!binary || x2_broadcast || aligned16(addr[x2]));
  uint64_t head = vec_ok ? n / per * per : 0;  // elements the vector kernel covers
  if (mode == Mode::Realized && head != n) head = 0;
  if (head) {
    const uint64_t chunks = head / per;
    char name[48];
    std::snprintf(name, sizeof(name), "tiler_map_%s_op%u%s", dtype == TILER_HIP_BF16 ? "bf16_v8" : "f32_v4", op,
                  binary && x2_broadcast ? "_b" : "");
    Launch& l = p.add(name, blocks_capped(chunks, 8192), 1, 256).ptr(x);
    if (binary) l.ptr(x2);
    else l.null_ptr();
    l.u64(chunks).f32(a).f32(b).ptr(y);
    if (head == n) return TILER_HIP_OK;
  }
  // scalar kernel for unaligned operands or the tail after the 16-byte chunks
  const uint64_t rest = n - head;
  Launch& l = p.add(dtype == TILER_HIP_BF16 ? "tiler_map_bf16" : "tiler_map_f32", blocks_capped(rest, 8192), 1, 256)
                  .ptr(x, head * eb);
  if (binary) l.ptr(x2, x2_broadcast ? 0 : head * eb);
  else l.null_ptr();
  l.u64(x2_broadcast ? 0 : 1).u64(rest).u32(op).f32(a).f32(b).ptr(y, head * eb);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Broadcast (byte moves by axis mapping).  Slots: 0 src, 1 out.
tiler_hip_status plan_broadcast(uint64_t src_elements, uint32_t rank, const uint64_t* out_dims,
                                const uint64_t* src_strides, uint32_t element_bytes,
                                Program& p) {
  if (rank > 8 || (rank && (!out_dims || !src_strides)))
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "broadcast rank");
  if (element_bytes != 2 && element_bytes != 4)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "broadcast element width");
  BroadcastGeometryHost g;
  std::memset(&g, 0, sizeof(g));
  g.rank = rank;
  uint64_t n = 1, last = 0;  // output elements; largest source offset read
  bool overflow = false;
  for (uint32_t d = 0; d < rank; ++d) {
    g.out_dims[d] = out_dims[d];
    g.src_strides[d] = src_strides[d];
    if (out_dims[d] && n > UINT64_MAX / out_dims[d]) overflow = true;
    n *= out_dims[d];
  }
  const uint32_t src = p.slot(mul_sat(src_elements, element_bytes), kSlotInput);
  const uint32_t out = p.slot(mul_sat(n, element_bytes), kSlotOutput);
  if (n == 0) return TILER_HIP_OK;
  for (uint32_t d = 0; d < rank && !overflow; ++d) {
    const uint64_t span = out_dims[d] - 1;
    if (span && src_strides[d] > (UINT64_MAX - last) / span) overflow = true;
    else last += span * src_strides[d];
  }
  if (overflow || last >= src_elements)
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "broadcast geometry reads outside the source");
  const uint64_t inner = rank ? out_dims[rank - 1] : 1;
  if (rank && inner >= 256) {  // row mode: one source row offset per workgroup step
    const uint64_t rows = n / inner;
    p.add(element_bytes == 4 ? "tiler_broadcast_rows_u32" : "tiler_broadcast_rows_u16",
          (uint32_t)(rows < 8192 ? rows : 8192), 1, 256)
        .ptr(src).ptr(out).u64(rows).blob(&g, sizeof(g), 8);
    return TILER_HIP_OK;
  }
  p.add(element_bytes == 4 ? "tiler_broadcast_u32" : "tiler_broadcast_u16", blocks_capped(n, 8192), 1, 256)
      .ptr(src).ptr(out).u64(n).blob(&g, sizeof(g), 8);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Gather.  Slots: 0 source, 1 index, 2 out, 3 record (u64: lowest
// out-of-range position, all ones when none).  Realized programs arm the
// record first; direct calls use the context's record, armed at bind.
tiler_hip_status plan_gather(Mode mode, uint64_t outer, uint64_t gathered, uint64_t inner,
                             uint32_t element_bytes, uint64_t count, int32_t index_signed,
                             const uintptr_t* addr, Program& p) {
  if (element_bytes == 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "gather element width");
  const uint64_t run_bytes = mul_sat(inner, element_bytes);
  const uint32_t src = p.slot(mul_sat(mul_sat(outer, gathered), run_bytes), kSlotInput);
  const uint32_t idx = p.slot(mul_sat(count, 4), kSlotInput);
  const uint32_t out = p.slot(mul_sat(mul_sat(outer, count), run_bytes), kSlotOutput);
  const uint32_t rec = p.slot(8, kSlotScratch);
  const uint64_t runs = mul_sat(outer, count);
  if (runs == 0 || run_bytes == 0) return TILER_HIP_OK;
  const uintptr_t both = addr[src] | addr[out];
  uint32_t unit = 16;
  while (unit > 1 && (run_bytes % unit != 0 || (both & (unit - 1)) != 0)) unit >>= 1;
  const char* name = unit == 16 ? "tiler_gather_u128" : unit == 8 ? "tiler_gather_u64"
                   : unit == 4 ? "tiler_gather_u32" : unit == 2 ? "tiler_gather_u16"
                               : "tiler_gather_u8";
  if (mode == Mode::Realized) p.add("tiler_fill_u32", 1, 1, 256).ptr(rec).u32(0xffffffffu).u64(2);
  p.add(name, (uint32_t)(runs < (1ull << 20) ? runs : (1ull << 20)), 1, 256)
      .ptr(src).u64(outer).u64(gathered).u64(run_bytes / unit).ptr(idx).u64(count)
      .u32(index_signed ? 1u : 0u).ptr(out).ptr(rec);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// bf16 <-> binary32 conversion families.  Slots: 0 src, 1 dst.  Like the maps:
// the 16-byte vector kernel over the aligned head of whole 8-element groups,
// the scalar kernel for the rest (realized: one kernel over all n).
tiler_hip_status plan_convert(Mode mode, uint32_t direction, uint64_t n, const uintptr_t* addr,
                              Program& p) {
  if (direction != TILER_HIP_CONVERT_NARROW_F32_BF16 && direction != TILER_HIP_CONVERT_WIDEN_BF16_F32)
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "conversion direction");
  const bool narrow = direction == TILER_HIP_CONVERT_NARROW_F32_BF16;
  const uint64_t in_b = narrow ? 4 : 2, out_b = narrow ? 2 : 4;
  const uint32_t src = p.slot(mul_sat(n, in_b), kSlotInput);
  const uint32_t dst = p.slot(mul_sat(n, out_b), kSlotOutput);
  if (n == 0) return TILER_HIP_OK;
  uint64_t head = aligned16(addr[src]) && aligned16(addr[dst]) ? n / 8 * 8 : 0;
  if (mode == Mode::Realized && head != n) head = 0;
  if (head) {
    p.add(narrow ? "tiler_narrow_f32_bf16_v8" : "tiler_widen_bf16_f32_v8", blocks_capped(head / 8, 8192), 1, 256)
        .ptr(src).u64(head / 8).ptr(dst);
    if (head == n) return TILER_HIP_OK;
  }
  p.add(narrow ? "tiler_narrow_f32_bf16" : "tiler_widen_bf16_f32", blocks_capped(n - head, 8192), 1, 256)
      .ptr(src, head * in_b).u64(n - head).ptr(dst, head * out_b);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Strict-affine U4 dequantization (quantization.rs:218-246, :409-419).
// Direct: slots 0 codes (packed U4, (n + 1) / 2 carriers), 1 y f32 [n]; the
// host checked the scale and zero point, which travel as launch values.
// Realized: slots 0 codes, 1 scale (f32 scalar), 2 zero point (U8 scalar),
// 3 y, 4 the domain verdict the kernel records (scratch, 4 bytes).
tiler_hip_status plan_dequantize_u4(Mode mode, uint64_t n, uint32_t scale_bits, uint32_t zero_point,
                                    const uintptr_t* addr, Program& p) {
  const bool realized = mode == Mode::Realized;
  const uint32_t codes = p.slot(n / 2 + (n & 1), kSlotInput);
  uint32_t scale = 0, zero = 0;
  if (realized) {
    scale = p.slot(4, kSlotInput);
    zero = p.slot(1, kSlotInput);
  }
  const uint32_t y = p.slot(mul_sat(n, 4), kSlotOutput);
  const uint32_t record = realized ? p.slot(4, kSlotScratch) : 0;
  if (!realized) {
    const float sc = __builtin_bit_cast(float, scale_bits);
    if (!std::isnormal(sc) || sc < 0.0f)
      return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT,
                      "scale outside positive-normal-f32 (the strict-affine value contract)");
    if (zero_point > 15) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "zero point outside the U4 code domain 0..=15");
  }
  if (n == 0) return TILER_HIP_OK;
  const bool al = aligned16(addr[codes]) && aligned16(addr[y]);
  // Whole 2048-element wave blocks first (16-byte code loads), four per workgroup.
  const uint64_t blocks = al ? n / 2048 : 0;
  if (blocks && (!realized || blocks * 2048 == n)) {
    if ((blocks + 3) / 4 > 0xffffffffull) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more blocks than the launch grid holds");
    Launch& l = p.add(realized ? "tiler_dequantize_u4_f32_w_slots" : "tiler_dequantize_u4_f32_w",
                      (uint32_t)((blocks + 3) / 4), 1, 256)
                    .ptr(codes)
                    .u64(blocks);
    if (realized) l.ptr(scale).ptr(zero).ptr(y).ptr(record);
    else l.u32(scale_bits).u32(zero_point).ptr(y);
    if (blocks * 2048 == n) return TILER_HIP_OK;
  }
  const uint64_t done = realized ? 0 : blocks * 2048;  // elements the block kernel wrote
  uint64_t head = al ? n / 4 * 4 : 0;
  if (realized && head != n) head = 0;  // a plan binds slot bases: one kernel over all of it
  if (head > done) {
    const uint64_t n4 = (head - done) / 4;
    Launch& l = p.add(realized ? "tiler_dequantize_u4_f32_v4_slots" : "tiler_dequantize_u4_f32_v4",
                      blocks_capped((n4 + 1) / 2, 1u << 30), 1, 256)
                    .ptr(codes, done / 2)
                    .u64(n4);
    if (realized) l.ptr(scale).ptr(zero).ptr(y).ptr(record);
    else l.u32(scale_bits).u32(zero_point).ptr(y, done * 4);
    if (head == n) return TILER_HIP_OK;
  }
  if (head < done) head = done;
  if (realized) {
    p.add("tiler_dequantize_u4_f32_slots", blocks_capped(n, 8192), 1, 256)
        .ptr(codes).u64(n).ptr(scale).ptr(zero).ptr(y).ptr(record);
  } else {
    p.add("tiler_dequantize_u4_f32", blocks_capped(n - head, 8192), 1, 256)
        .ptr(codes).u64(head).u64(n - head).u32(scale_bits).u32(zero_point).ptr(y);
  }
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Contractions.  Slots: 0 a [m, k], 1 b [n, k], 2 c [m, n].
// The live contracted extent: read at dispatch from input 0 (A[m][k]), axis 1,
// at least 1 (an empty contracted domain has no unseeded result) and at most
// the bound the slots were sized for.
static void declare_live_k(Program& p, uint64_t bound) {
  p.live[0] = LiveExtent{0, 1, 1, bound};
  p.nlive = 1;
}

// Register-blocked strict tiles of 16·T x 16·T, T x T outputs per thread,
// T in {1, 2, 4}: the one with the least work on the busiest CU -- rounds of
// tiles over the CUs x outputs per tile x the time per output step, relative
// weights 31 : 20 : 18 (T = 1 measured 1.4-1.7 x T = 2 per output step on the
// 128 x 1024 x 3072 and 128 x 3072 x 1024 cells; T = 4 taken a tenth below
// T = 2).  Returns T.
static uint32_t strict_tile(const Target& t, uint64_t m, uint64_t n) {
  const uint64_t cus = t.compute_units;
  uint32_t best = 1;
  uint64_t best_cost = UINT64_MAX;
  for (uint32_t T : {1u, 2u, 4u}) {
    const uint64_t edge = 16ull * T;
    const uint64_t tiles = ((m + edge - 1) / edge) * ((n + edge - 1) / edge);
    const uint64_t weight = T == 1 ? 31 : T == 2 ? 20 : 18;
    const uint64_t cost = mul_sat(mul_sat((tiles + cus - 1) / cus, edge * edge), weight);
    if (cost < best_cost) best_cost = cost, best = T;
  }
  return best;
}

tiler_hip_status plan_contract_strict_f32(const Target& t, uint64_t m, uint64_t n, uint64_t k, const uintptr_t* addr,
                                          Program& p, bool live_k) {
  const uint32_t a = p.slot(mul_sat(mul_sat(m, k), 4), kSlotInput);
  const uint32_t b = p.slot(mul_sat(mul_sat(n, k), 4), kSlotInput);
  const uint32_t c = p.slot(mul_sat(mul_sat(m, n), 4), kSlotOutput);
  // contraction.rs:420-428: an empty contracted domain has no unseeded result.
  if (k == 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "empty contracted extent");
  if (live_k) declare_live_k(p, k);
  if (m == 0 || n == 0) return TILER_HIP_OK;
  if (m > 0xffffffffull || n > 0xffffffffull || k > 0xffffffffull || (m + 15) / 16 > 65535)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "contraction extents beyond the launch profile");
  if (m <= 16 && k >= 64) {
    // Few output rows (decode shapes): each output is the staged fold of the
    // products along one row of B (contiguous in k), one workgroup row per
    // output row, R output columns per workgroup chosen by the output count.
    // R <= 16 relay-fold; up to 32 outputs per CU the relay's R = 16 still
    // beat R = 64 on the device (1 x 8192 x 1024: 14.0 against 16.6 us; from
    // 128 per CU R = 64 won, 1 x 32768 x 1024: 21.4 against 30.8 us).  With
    // k live the 4-byte-load form takes any k.
    const uint64_t outputs = m * n, cus = t.compute_units;
    const uint32_t R = outputs <= cus ? 1 : outputs <= 4 * cus ? 4 : outputs <= 32 * cus ? 16 : 64;
    const bool vec = !live_k && k % 4 == 0 && aligned16(addr[a]) && aligned16(addr[b]);
    char name[40];
    std::snprintf(name, sizeof(name), "tiler_contract_strict_f32_s%u%s", R, vec ? "" : "_u");
    Launch& l = p.add(name, (uint32_t)((n + R - 1) / R), (uint32_t)m, 256)
                    .ptr(a).ptr(b).u32((uint32_t)m).u32((uint32_t)n);
    (live_k ? l.live_u32(0) : l.u32((uint32_t)k)).ptr(c);
    return TILER_HIP_OK;
  }
  if (k >= 64) {
    const uint32_t best = strict_tile(t, m, n);
    const uint32_t tile = 16 * best;
    static const char* const names[] = {nullptr, "tiler_contract_strict_f32_b16", "tiler_contract_strict_f32_b32",
                                        nullptr, "tiler_contract_strict_f32_b64"};
    Launch& l = p.add(names[best], (uint32_t)((n + tile - 1) / tile), (uint32_t)((m + tile - 1) / tile), 256)
                    .ptr(a).ptr(b).u32((uint32_t)m).u32((uint32_t)n);
    (live_k ? l.live_u32(0) : l.u32((uint32_t)k)).ptr(c);
    return TILER_HIP_OK;
  }
  // Short k: 16 x 16 tiles, one output per thread (the shape of the
  // reference's contraction_tiled_cooperative golden).
  Launch& l = p.add("tiler_contract_strict_f32", (uint32_t)((n + 15) / 16), (uint32_t)((m + 15) / 16), 256)
                  .ptr(a).ptr(b).u32((uint32_t)m).u32((uint32_t)n);
  (live_k ? l.live_u32(0) : l.u32((uint32_t)k)).ptr(c);
  return TILER_HIP_OK;
}

tiler_hip_status plan_contract_bf16(const Target& t, uint64_t m, uint64_t n, uint64_t k,
                                    uint32_t epilogue, const uintptr_t* addr, Program& p, bool strict,
                                    uint32_t form, bool live_k) {
  if (epilogue > TILER_HIP_EPILOGUE_SILU) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "epilogue");
  if (form != TILER_HIP_FORM_AUTO &&
      (strict || form < TILER_HIP_FORM_CONTRACT_SKINNY || form > TILER_HIP_FORM_CONTRACT_GENERAL_128))
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "form: not a form of this contraction");
  if (live_k && form != TILER_HIP_FORM_AUTO && form != TILER_HIP_FORM_CONTRACT_GENERAL_128)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                    "live-extent: with a live k only the general form (any k) runs");
  const uint32_t a = p.slot(mul_sat(mul_sat(m, k), 2), kSlotInput);
  const uint32_t b = p.slot(mul_sat(mul_sat(n, k), 2), kSlotInput);
  const uint32_t c = p.slot(mul_sat(mul_sat(m, n), 2), kSlotOutput);
  if (k == 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "empty contracted extent");
  if (live_k) declare_live_k(p, k);
  if (m == 0 || n == 0) return TILER_HIP_OK;
  if (strict) {  // the strict fold on exactly widened operands (MFMA regroups the k sum)
    if (m > 0xffffffffull || n > 0xffffffffull || k > 0xffffffffull || (m + 15) / 16 > 65535 ||
        (n + 15) / 16 > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "contraction extents beyond the launch profile");
    const bool silu = epilogue == TILER_HIP_EPILOGUE_SILU;
    if (k >= 64) {  // register-blocked tiles, chosen as for the f32 form
      const uint32_t T = strict_tile(t, m, n), tile = 16 * T;
      char name[48];
      std::snprintf(name, sizeof(name), "tiler_contract_strict_bf16_%sb%u", silu ? "silu_" : "", tile);
      Launch& l = p.add(name, (uint32_t)((n + tile - 1) / tile), (uint32_t)((m + tile - 1) / tile), 256)
                      .ptr(a).ptr(b).u32((uint32_t)m).u32((uint32_t)n);
      (live_k ? l.live_u32(0) : l.u32((uint32_t)k)).ptr(c);
      return TILER_HIP_OK;
    }
    Launch& l = p.add(silu ? "tiler_contract_strict_bf16_silu" : "tiler_contract_strict_bf16",
                      (uint32_t)((n + 15) / 16), (uint32_t)((m + 15) / 16), 256)
                    .ptr(a).ptr(b).u32((uint32_t)m).u32((uint32_t)n);
    (live_k ? l.live_u32(0) : l.u32((uint32_t)k)).ptr(c);
    return TILER_HIP_OK;
  }
  if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull || (m + 127) / 128 > 65535)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "contraction extents beyond the launch profile");
  const bool silu = epilogue == TILER_HIP_EPILOGUE_SILU;
  const uint32_t m32 = (uint32_t)m, n32 = (uint32_t)n, k32 = (uint32_t)k;
  if (live_k) {  // any k up to the bound: the general form, which takes k not a multiple of 8
    Launch& l = p.add(silu ? "tiler_contract_bf16_silu_g128_k" : "tiler_contract_bf16_g128_k",
                      (uint32_t)((n + 127) / 128), (uint32_t)((m + 127) / 128), 256)
                    .ptr(a).ptr(b).u32(m32).u32(n32);
    l.live_u32(0).ptr(c);
    return TILER_HIP_OK;
  }
  const bool pick = form == TILER_HIP_FORM_AUTO;
  // m <= 64 (decode shapes): B streamed once, one workgroup per 16 columns.
  const bool skinny_ok = m <= 64 && k % 8 == 0 && aligned16(addr[a]) && aligned16(addr[b]) &&
                         (n + 15) / 16 <= 0x7fffffffull;
  if (form == TILER_HIP_FORM_CONTRACT_SKINNY && !skinny_ok)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                    "skinny-rows: the skinny form takes m <= 64 and k a multiple of 8, aligned operands");
  if (skinny_ok && (pick || form == TILER_HIP_FORM_CONTRACT_SKINNY)) {
    char name[48];
    std::snprintf(name, sizeof(name), "tiler_contract_bf16_%sskinny%u", silu ? "silu_" : "", (uint32_t)((m + 15) / 16));
    p.add(name, (uint32_t)((n + 15) / 16), 1, 1024).ptr(a).ptr(b).u32(m32).u32(n32).u32(k32).ptr(c);
    return TILER_HIP_OK;
  }
  // The staged path addresses each operand panel (up to 256 rows) through one
  // buffer resource with 32-bit offsets (256 * k * 2 bytes must stay below
  // 2^31) and moves 16-byte rows: n and k multiples of 8, aligned operands.
  // 256-tiles when they fill every CU, 128-tiles (four times as many) when not.
  const bool staged_ok = n % 8 == 0 && k % 8 == 0 && k * 512ull < (1ull << 31) && aligned16(addr[a]) &&
                         aligned16(addr[b]) && aligned16(addr[c]);
  if ((form == TILER_HIP_FORM_CONTRACT_STAGED_256 || form == TILER_HIP_FORM_CONTRACT_STAGED_128) && !staged_ok)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                    "staged-rows: the staged forms take n and k multiples of 8 (k below 2^22), aligned operands");
  if (staged_ok && form != TILER_HIP_FORM_CONTRACT_SKINNY && form != TILER_HIP_FORM_CONTRACT_GENERAL_128) {
    const uint64_t t256 = ((m + 255) / 256) * ((n + 255) / 256);
    const uint64_t t128 = ((m + 127) / 128) * ((n + 127) / 128);
    const bool big = pick ? t256 >= t.compute_units : form == TILER_HIP_FORM_CONTRACT_STAGED_256;
    const uint64_t tiles = big ? t256 : t128;
    if (!pick && tiles > 0x7fffffffull)
      return p.refuse(TILER_HIP_REFUSE_CAPACITY, "more tiles than the launch grid holds");
    if (tiles <= 0x7fffffffull) {
      // k a multiple of 64: the forms without last-tile masking (_kf)
      char name[48];
      std::snprintf(name, sizeof(name), "tiler_contract_bf16_%st%u%s", silu ? "silu_" : "", big ? 256u : 128u,
                    k % 64 == 0 ? "_kf" : "");
      p.add(name, (uint32_t)tiles, 1, big ? 1024 : 256).ptr(a).ptr(b).u32(m32).u32(n32).u32(k32).ptr(c);
      return TILER_HIP_OK;
    }
  }
  const bool full = k % 8 == 0 && aligned16(addr[a]) && aligned16(addr[b]);
  const char* name = silu ? (full ? "tiler_contract_bf16_silu_g128" : "tiler_contract_bf16_silu_g128_k")
                          : (full ? "tiler_contract_bf16_g128" : "tiler_contract_bf16_g128_k");
  p.add(name, (uint32_t)((n + 127) / 128), (uint32_t)((m + 127) / 128), 256)
      .ptr(a).ptr(b).u32(m32).u32(n32).u32(k32).ptr(c);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Contraction over a general binary index structure.  Slots: 0 left, 1 right,
// 2 out; then the strict form's geometry (CONSTANT) or the MFMA form's
// transposed right operand (scratch).
namespace {

struct Axis {
  uint32_t label;
  uint64_t extent;
};

// Row-major element stride of the axis labelled `label` in an operand, or 0
// (and false) when the operand has no such axis.
bool stride_of(const tiler_hip_contraction_structure& s, int side, uint32_t label, uint64_t& stride) {
  uint64_t st = 1;
  for (int32_t a = (int32_t)s.operand_rank[side] - 1; a >= 0; --a) {
    if (s.operand_indices[side][a] == label) {
      stride = st;
      return true;
    }
    st = mul_sat(st, s.operand_dims[side][a]);
  }
  stride = 0;
  return false;
}

}  // namespace

tiler_hip_status plan_contract_general(const Target& t, uint32_t dtype, const tiler_hip_contraction_structure& s,
                                       uint32_t epilogue, bool strict, const uintptr_t* addr, Program& p,
                                       uint32_t in_mode, uint32_t out_mode) {
  using tiler_geom::kAxes;
  // A flushing contract: the strict fold with the modes at every site (the
  // MFMA units round each block of products without a per-product flush).
  const bool modes = in_mode > 1 || out_mode > 1;
  if (modes) strict = true;
  if (dtype != TILER_HIP_F32 && dtype != TILER_HIP_BF16) return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "contraction dtype");
  if (epilogue > TILER_HIP_EPILOGUE_SILU) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "epilogue");
  if (dtype == TILER_HIP_F32 && epilogue != TILER_HIP_EPILOGUE_NONE)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "the strict f32 contraction has no epilogue");
  if (s.reserved != 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "reserved structure field");
  if (s.operand_rank[0] > kAxes || s.operand_rank[1] > kAxes || s.output_rank > kAxes)
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "more than 8 indices in one tuple");
  const uint64_t eb = dtype == TILER_HIP_BF16 ? 2 : 4;
  // The five structural rules (tiler-ir/src/semantic/contraction.rs:804-900)
  // and one extent per index (tiler-reference/src/contraction.rs:386-399).
  for (int side = 0; side < 2; ++side)
    for (uint32_t a = 0; a < s.operand_rank[side]; ++a)
      for (uint32_t b = a + 1; b < s.operand_rank[side]; ++b)
        if (s.operand_indices[side][a] == s.operand_indices[side][b])
          return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "an index repeated within an operand");
  for (uint32_t a = 0; a < s.output_rank; ++a)
    for (uint32_t b = a + 1; b < s.output_rank; ++b)
      if (s.output_indices[a] == s.output_indices[b])
        return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "a duplicate output index");
  Axis seen[2 * kAxes];
  uint32_t nseen = 0;
  for (int side = 0; side < 2; ++side)
    for (uint32_t a = 0; a < s.operand_rank[side]; ++a) {
      uint32_t i = 0;
      while (i < nseen && seen[i].label != s.operand_indices[side][a]) ++i;
      if (i == nseen) {
        seen[nseen++] = {s.operand_indices[side][a], s.operand_dims[side][a]};
      } else if (seen[i].extent != s.operand_dims[side][a]) {
        return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "one index with two extents");
      }
    }
  auto extent_of = [&](uint32_t label, uint64_t& e) {
    for (uint32_t i = 0; i < nseen; ++i)
      if (seen[i].label == label) {
        e = seen[i].extent;
        return true;
      }
    return false;
  };
  uint64_t out_dims[kAxes] = {};
  uint64_t outputs = 1;
  for (uint32_t d = 0; d < s.output_rank; ++d) {
    if (!extent_of(s.output_indices[d], out_dims[d]))
      return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "an output index in no operand");
    outputs = mul_sat(outputs, out_dims[d]);
  }
  uint32_t con[2 * kAxes];
  uint32_t ncon = 0;
  for (uint32_t i = 0; i < nseen; ++i) {
    bool in_out = false;
    for (uint32_t d = 0; d < s.output_rank; ++d) in_out |= s.output_indices[d] == seen[i].label;
    if (in_out) continue;
    uint64_t unused;
    if (!stride_of(s, 0, seen[i].label, unused) || !stride_of(s, 1, seen[i].label, unused))
      return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "a summed index in one operand");
    uint32_t at = ncon++;
    while (at > 0 && con[at - 1] > seen[i].label) {
      con[at] = con[at - 1];
      --at;
    }
    con[at] = seen[i].label;
  }
  if (ncon == 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "no summed index (an outer product)");
  uint64_t left_elems = 1, right_elems = 1;
  for (uint32_t a = 0; a < s.operand_rank[0]; ++a) left_elems = mul_sat(left_elems, s.operand_dims[0][a]);
  for (uint32_t a = 0; a < s.operand_rank[1]; ++a) right_elems = mul_sat(right_elems, s.operand_dims[1][a]);
  const uint32_t l = p.slot(mul_sat(left_elems, eb), kSlotInput);
  const uint32_t r = p.slot(mul_sat(right_elems, eb), kSlotInput);
  const uint32_t o = p.slot(mul_sat(outputs, eb), kSlotOutput);
  uint64_t con_dims[kAxes] = {};
  uint64_t contracted = 1;
  for (uint32_t c = 0; c < ncon; ++c) {
    extent_of(con[c], con_dims[c]);
    contracted = mul_sat(contracted, con_dims[c]);
  }
  // contraction.rs:420-428: an empty contracted domain has no unseeded result.
  if (contracted == 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "empty contracted domain");
  if (left_elems == UINT64_MAX || right_elems == UINT64_MAX || outputs == UINT64_MAX)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "operand or result extents overflow");
  if (outputs == 0) return TILER_HIP_OK;
  const bool silu = epilogue == TILER_HIP_EPILOGUE_SILU;

  // MFMA: one summed index k, out [batch.., m, n], left [.., m, k],
  // right [.., n, k] or [.., k, n].
  if (!strict && dtype == TILER_HIP_BF16 && ncon == 1 && s.output_rank >= 2) {
    const uint32_t ki = con[0], mi = s.output_indices[s.output_rank - 2], ni = s.output_indices[s.output_rank - 1];
    const uint32_t lr = s.operand_rank[0], rr = s.operand_rank[1];
    uint64_t st;
    const bool left_ok = lr >= 2 && s.operand_indices[0][lr - 1] == ki && s.operand_indices[0][lr - 2] == mi &&
                         !stride_of(s, 1, mi, st);
    const bool right_nk = rr >= 2 && s.operand_indices[1][rr - 1] == ki && s.operand_indices[1][rr - 2] == ni;
    const bool right_kn = rr >= 2 && s.operand_indices[1][rr - 1] == ni && s.operand_indices[1][rr - 2] == ki;
    const bool ni_ok = !stride_of(s, 0, ni, st);
    const uint32_t nbatch = s.output_rank - 2;
    uint64_t m = 0, n = 0, k = con_dims[0];
    extent_of(mi, m);
    extent_of(ni, n);
    uint64_t batches = 1;
    for (uint32_t d = 0; d < nbatch; ++d) batches = mul_sat(batches, out_dims[d]);
    if (left_ok && ni_ok && (right_nk || right_kn) && nbatch <= (uint32_t)tiler_geom::kBatchAxes &&
        batches <= 65535 && m <= 0x7fffffffull && n <= 0x7fffffffull && k <= 0x7fffffffull) {
      tiler_geom::BatchGeometry g{};
      g.rank = nbatch;
      // The right operand as the kernels read it: its own layout, or (stored
      // [.., k, n]) transposed into scratch as [.., n, k], dense.
      uint64_t rbatch = 1;
      for (uint32_t a = 0; a + 2 < rr; ++a) rbatch = mul_sat(rbatch, s.operand_dims[1][a]);
      bool strides8 = true;
      uint64_t ostride = mul_sat(m, n);
      for (int32_t d = (int32_t)nbatch - 1; d >= 0; --d) {
        g.dims[d] = out_dims[d];
        g.c_stride[d] = ostride;
        ostride = mul_sat(ostride, out_dims[d]);
        stride_of(s, 0, s.output_indices[d], g.a_stride[d]);
        stride_of(s, 1, s.output_indices[d], g.b_stride[d]);  // the transposed layout keeps batch strides
        strides8 = strides8 && g.a_stride[d] % 8 == 0 && g.b_stride[d] % 8 == 0 && g.c_stride[d] % 8 == 0;
      }
      uint32_t right_slot = r;
      if (right_kn) {
        if (k > 0xffffffffull || n > 0xffffffffull) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "transpose extents");
        right_slot = p.slot(mul_sat(right_elems, 2), kSlotScratch);
        const uint64_t row_tiles = (k + 63) / 64, work = mul_sat(rbatch, row_tiles);
        p.add("tiler_transpose_bf16", (uint32_t)((n + 63) / 64), (uint32_t)(work < 65535 ? work : 65535), 256)
            .ptr(r).ptr(right_slot).u64(rbatch).u32((uint32_t)k).u32((uint32_t)n);
      }
      const uint32_t m32 = (uint32_t)m, n32 = (uint32_t)n, k32 = (uint32_t)k;
      const bool ab_al = aligned16(addr[l]) && (right_kn || aligned16(addr[r])) && strides8;
      char name[48];
      if (m <= 64 && k % 8 == 0 && ab_al) {
        std::snprintf(name, sizeof(name), "tiler_contract_bf16_%sskinny%u_b", silu ? "silu_" : "", (uint32_t)((m + 15) / 16));
        p.add(name, (uint32_t)((n + 15) / 16), (uint32_t)batches, 1024)
            .ptr(l).ptr(right_slot).u32(m32).u32(n32).u32(k32).ptr(o).blob(&g, sizeof g, 8);
        return TILER_HIP_OK;
      }
      if (n % 8 == 0 && k % 8 == 0 && k * 512ull < (1ull << 31) && ab_al && aligned16(addr[o])) {
        const uint64_t t256 = ((m + 255) / 256) * ((n + 255) / 256);
        const uint64_t t128 = ((m + 127) / 128) * ((n + 127) / 128);
        // 256-tiles only where a problem spans them (a head dimension of 128
        // would leave half of each idle) and they fill every CU
        const bool big = m >= 256 && n >= 256 && mul_sat(t256, batches) >= t.compute_units;
        const uint64_t tiles = big ? t256 : t128;
        if (tiles <= 0x7fffffffull) {
          std::snprintf(name, sizeof(name), "tiler_contract_bf16_%st%u_b", silu ? "silu_" : "", big ? 256u : 128u);
          p.add(name, (uint32_t)tiles, (uint32_t)batches, big ? 1024 : 256)
              .ptr(l).ptr(right_slot).u32(m32).u32(n32).u32(k32).ptr(o).blob(&g, sizeof g, 8);
          return TILER_HIP_OK;
        }
      }
      const uint64_t m_tiles = (m + 127) / 128;
      if (mul_sat(m_tiles, batches) <= 65535) {
        const bool full = k % 8 == 0 && ab_al;
        std::snprintf(name, sizeof(name), "tiler_contract_bf16_%sg128%s_b", silu ? "silu_" : "", full ? "" : "_k");
        p.add(name, (uint32_t)((n + 127) / 128), (uint32_t)(m_tiles * batches), 256)
            .ptr(l).ptr(right_slot).u32(m32).u32(n32).u32(k32).ptr(o).u32((uint32_t)m_tiles).blob(&g, sizeof g, 8);
        return TILER_HIP_OK;
      }
      // no MFMA launch fits: the strict fold below (drop the scratch slot)
      if (right_kn) {
        p.nslots = 3;
        p.nlaunches = 0;
      }
    }
  }

  // The strict fold, the geometry in a constant slot.
  tiler_geom::GeneralGeometry g{};
  g.out_rank = s.output_rank;
  g.con_rank = ncon;
  g.outputs = outputs;
  for (uint32_t d = 0; d < s.output_rank; ++d) {
    g.out_dims[d] = out_dims[d];
    stride_of(s, 0, s.output_indices[d], g.l_out[d]);
    stride_of(s, 1, s.output_indices[d], g.r_out[d]);
  }
  for (uint32_t c = 0; c < ncon; ++c) {
    g.con_dims[c] = con_dims[c];
    stride_of(s, 0, con[c], g.l_con[c]);
    stride_of(s, 1, con[c], g.r_con[c]);
  }
  const uint32_t geo = p.slot(sizeof g, TILER_HIP_SLOT_CONSTANT);
  p.constant_slot = geo;
  p.constant.assign(reinterpret_cast<const uint8_t*>(&g), reinterpret_cast<const uint8_t*>(&g) + sizeof g);
  const char* name = dtype == TILER_HIP_F32 ? (modes ? "tiler_contract_general_f32_m" : "tiler_contract_general_f32")
                     : silu ? (modes ? "tiler_contract_general_bf16_silu_m" : "tiler_contract_general_bf16_silu")
                            : (modes ? "tiler_contract_general_bf16_m" : "tiler_contract_general_bf16");
  Launch& launch = p.add(name, blocks_capped(outputs, 65536), 1, 256).ptr(l).ptr(r).ptr(o).ptr(geo);
  if (modes) launch.u32(in_mode).u32(out_mode);
  return TILER_HIP_OK;
}

}  // namespace tiler_rt

// ---------------------------------------------------------------------------
// Pointwise expressions.
namespace tiler_rt {

namespace {

void put16(std::vector<uint8_t>& v, uint32_t x) {
  v.push_back((uint8_t)x);
  v.push_back((uint8_t)(x >> 8));
}
void put32(std::vector<uint8_t>& v, uint32_t x) {
  put16(v, x & 0xffffu);
  put16(v, x >> 16);
}

}  // namespace

tiler_hip_status compile_expression(uint32_t dtype, const tiler_hip_expression_node* nodes, uint32_t count,
                                    uint32_t root, bool epilogue, ExpressionProgram& out, std::string& diag) {
  auto refuse = [&](tiler_hip_status st, const std::string& what) {
    diag = what;
    return st;
  };
  if (dtype != TILER_HIP_F32 && dtype != TILER_HIP_BF16) return refuse(TILER_HIP_REFUSE_UNSUPPORTED, "expression dtype");
  if (count == 0 || !nodes) return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "empty expression");
  if (count > TILER_HIP_MAX_EXPRESSION_NODES)
    return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "expression beyond the 4096-node limit");
  if (root >= count) return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "root is not a node");
  std::vector<int64_t> input_of(count, -1);  // node -> ordinal
  std::vector<uint32_t> ordinals;
  for (uint32_t i = 0; i < count; ++i) {
    const tiler_hip_expression_node& nd = nodes[i];
    const bool bf16_op = nd.op <= TILER_HIP_NODE_MULTIPLY;
    if (nd.op > TILER_HIP_NODE_RSQRT || (dtype == TILER_HIP_BF16 && !bf16_op))
      return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "node " + std::to_string(i) + ": operation outside the vocabulary");
    switch (nd.op) {
      case TILER_HIP_NODE_INPUT:
        input_of[i] = nd.a;
        ordinals.push_back(nd.a);
        break;
      case TILER_HIP_NODE_CONSTANT:
        if (dtype == TILER_HIP_BF16 && nd.a > 0xffffu)
          return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "node " + std::to_string(i) + ": a bf16 constant is 16 bits");
        break;
      case TILER_HIP_NODE_ADD:
      case TILER_HIP_NODE_MULTIPLY:
      case TILER_HIP_NODE_DIVIDE:
        if (nd.a >= i || nd.b >= i)
          return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "node " + std::to_string(i) + ": operand not defined before use");
        break;
      default:  // EXP, RSQRT
        if (nd.a >= i)
          return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "node " + std::to_string(i) + ": operand not defined before use");
    }
  }
  // Dense ordinals 0..n-1, each named once (pointwise.rs:222-235).
  std::vector<uint8_t> seen(ordinals.size(), 0);
  for (uint32_t o : ordinals) {
    if (o >= ordinals.size() || seen[o]) return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "input ordinals are not dense");
    seen[o] = 1;
  }
  if (ordinals.empty()) return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "expression reads no input");
  // Every node reachable from the root (pointwise.rs:420-428).
  std::vector<uint8_t> live(count, 0);
  live[root] = 1;
  for (int64_t i = root; i >= 0; --i) {
    if (!live[i]) continue;
    const tiler_hip_expression_node& nd = nodes[i];
    if (nd.op >= TILER_HIP_NODE_ADD) live[nd.a] = 1;
    if (nd.op >= TILER_HIP_NODE_ADD && nd.op <= TILER_HIP_NODE_DIVIDE) live[nd.b] = 1;
  }
  for (uint32_t i = 0; i < count; ++i)
    if (!live[i]) return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "node " + std::to_string(i) + " is unreachable from the root");
  const uint32_t nin = (uint32_t)ordinals.size();
  if (epilogue && (nin != 1 || nodes[root].op == TILER_HIP_NODE_INPUT))
    return refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "an epilogue reads exactly the folded value and transforms it");
  if (nin > kMaxExpressionInputs)
    return refuse(TILER_HIP_REFUSE_CAPACITY, "more than 16 expression inputs");

  // Execution order: the inputs by ordinal, then every other node in order.
  std::vector<uint32_t> order;
  order.reserve(count);
  std::vector<uint32_t> node_of_ordinal(nin);
  for (uint32_t i = 0; i < count; ++i)
    if (input_of[i] >= 0) node_of_ordinal[input_of[i]] = i;
  for (uint32_t k = 0; k < nin; ++k) order.push_back(node_of_ordinal[k]);
  for (uint32_t i = 0; i < count; ++i)
    if (input_of[i] < 0) order.push_back(i);
  std::vector<uint32_t> last(count, 0);  // execution step of the last read
  for (uint32_t s = 0; s < count; ++s) {
    const tiler_hip_expression_node& nd = nodes[order[s]];
    if (nd.op >= TILER_HIP_NODE_ADD) last[nd.a] = s;
    if (nd.op >= TILER_HIP_NODE_ADD && nd.op <= TILER_HIP_NODE_DIVIDE) last[nd.b] = s;
  }
  last[root] = count;  // the result stays live to the end
  // Linear scan: the lowest free register at each definition; an operand's
  // register is released at its last read, before the result is placed (the
  // kernel reads both operands before it writes).
  std::vector<uint32_t> reg(count, 0);
  std::vector<uint8_t> used;
  uint32_t high = 0;
  out.code.clear();
  out.code.reserve((size_t)count * kExpressionInstrBytes);
  for (uint32_t s = 0; s < count; ++s) {
    const uint32_t i = order[s];
    const tiler_hip_expression_node& nd = nodes[i];
    uint32_t ra = 0, rb = 0;
    if (nd.op >= TILER_HIP_NODE_ADD) {
      ra = reg[nd.a];
      rb = nd.op <= TILER_HIP_NODE_DIVIDE ? reg[nd.b] : ra;
      if (last[nd.a] == s) used[ra] = 0;
      if (nd.op <= TILER_HIP_NODE_DIVIDE && last[nd.b] == s) used[rb] = 0;
    }
    uint32_t d = 0;
    while (d < used.size() && used[d]) ++d;
    if (d == used.size()) used.push_back(0);
    used[d] = 1;
    reg[i] = d;
    if (d + 1 > high) high = d + 1;
    put16(out.code, nd.op);
    put16(out.code, d);
    put16(out.code, ra);
    put16(out.code, rb);
    put32(out.code, nd.op == TILER_HIP_NODE_INPUT ? nd.a : nd.op == TILER_HIP_NODE_CONSTANT ? nd.a : 0);
  }
  out.count = count;
  out.inputs = nin;
  out.registers = high;
  out.result = reg[root];
  return TILER_HIP_OK;
}

tiler_hip_status plan_expression(const Target& t, uint32_t dtype, uint64_t n, const ExpressionProgram& prog,
                                 const Contract& c, const uintptr_t* addr, Program& p) {
  (void)t;
  if (dtype != TILER_HIP_F32 && dtype != TILER_HIP_BF16) return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "expression dtype");
  const uint64_t eb = dtype == TILER_HIP_BF16 ? 2 : 4;
  uint32_t in_slots[kMaxExpressionInputs];
  for (uint32_t k = 0; k < prog.inputs; ++k) in_slots[k] = p.slot(mul_sat(n, eb), kSlotInput);
  const uint32_t y = p.slot(mul_sat(n, eb), kSlotOutput);
  const uint32_t code = p.slot(prog.code.size(), TILER_HIP_SLOT_CONSTANT);
  p.constant_slot = code;
  p.constant = prog.code;
  if (n == 0) return TILER_HIP_OK;
  const uint32_t in_mode = c.input_mode < 1 ? 1 : c.input_mode, out_mode = c.result_mode < 1 ? 1 : c.result_mode;
  const char* ty = dtype == TILER_HIP_BF16 ? "bf16" : "f32";
  char name[48];
  if (prog.registers <= kExpressionRegisters) {
    const uint64_t per = dtype == TILER_HIP_BF16 ? 8 : 4;
    bool vec = n % per == 0 && aligned16(addr[prog.inputs]);
    for (uint32_t k = 0; k < prog.inputs; ++k) vec = vec && aligned16(addr[k]);
    const uint32_t nin = prog.inputs <= 4 ? prog.inputs : 0;
    // the vector f32 form has a copy with the mode code compiled out; bf16
    // under a flushing contract takes the one-element form, which applies
    // the modes
    if (dtype == TILER_HIP_BF16 && c.flushes()) vec = false;
    const char* form = !vec ? "s" : (dtype == TILER_HIP_F32 && c.flushes()) ? "f" : "";
    const uint64_t work = vec ? n / per : n;
    std::snprintf(name, sizeof(name), "tiler_expr_%s_r16%s_i%u", ty, form, nin);
    p.add(name, blocks_capped(work, 8192), 1, 256)
        .ptr_table(in_slots, prog.inputs, kMaxExpressionInputs)
        .ptr(y).ptr(code).u32(prog.count).u32(prog.result).u64(work).u32(in_mode).u32(out_mode);
    return TILER_HIP_OK;
  }
  // Value store in scratch, [register][lane]: as many lanes as keep it within
  // 256 MiB (at least one workgroup, at most 65536 lanes).
  uint64_t lanes = (256ull << 20) / (4ull * prog.registers);
  if (lanes > 65536) lanes = 65536;
  lanes = lanes / 256 * 256;
  if (lanes == 0) lanes = 256;
  const uint64_t needed = (n + 255) / 256 * 256;
  if (lanes > needed) lanes = needed;
  const uint32_t store = p.slot(4ull * prog.registers * lanes, kSlotScratch);
  std::snprintf(name, sizeof(name), "tiler_expr_%s_mem", ty);
  p.add(name, (uint32_t)(lanes / 256), 1, 256)
      .ptr_table(in_slots, prog.inputs, kMaxExpressionInputs)
      .ptr(y).ptr(code).u32(prog.count).u32(prog.result).u64(n).u32(in_mode).u32(out_mode).ptr(store);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Serial folds over any reduced-axis set.  Slots: x, out, [epilogue program].
tiler_hip_status plan_fold(uint32_t op, uint32_t rank, const uint64_t* dims, uint64_t reduced_mask,
                           uint32_t scale_bits, uint32_t bias_bits, const ExpressionProgram* epilogue,
                           Program& p, const Contract& c, const Target* t, const tiler_hip_sum_plan* sp,
                           const uintptr_t* addr) {
  if (op > TILER_HIP_FOLD_MAXIMUM) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "fold variant");
  if (rank > 8 || (rank && !dims)) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "fold rank");
  if (reduced_mask >> rank) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "reduced axis beyond the rank");
  if (epilogue && op == TILER_HIP_FOLD_MAXIMUM)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "the maximum fold carries no epilogue");
  const uint32_t topology = sp ? sp->topology : TILER_HIP_SUM_SERIAL;
  // The maximum compares and is under no subnormal mode (softmax.rs:168-186);
  // its one realization is the serial fold.
  if (op == TILER_HIP_FOLD_MAXIMUM && topology != TILER_HIP_SUM_SERIAL)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "the maximum fold has one realization, the serial fold");
  const bool sums = op != TILER_HIP_FOLD_MAXIMUM;
  if (epilogue && (c.flushes() || topology != TILER_HIP_SUM_SERIAL))
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                    "a fold's epilogue is realized serially and under the preserving modes only");
  // A sum over the trailing axis under a flushing contract, or split by a
  // reassociating topology: the rule-driven sums (the prologue and the modes
  // in every combine), over the [rows, extent] view of the dense input.
  const bool trailing = rank >= 1 && reduced_mask == (1ull << (rank - 1));
  if (sums && !epilogue && (c.flushes() || topology != TILER_HIP_SUM_SERIAL)) {
    FoldRuleHost rule;
    rule.prologue = op == TILER_HIP_FOLD_SQUARED ? 1u : op == TILER_HIP_FOLD_FMA ? 2u : 0u;
    std::memcpy(&rule.scale, &scale_bits, 4);
    std::memcpy(&rule.bias, &bias_bits, 4);
    rule.in_mode = c.input_mode;
    rule.out_mode = c.result_mode;
    if (trailing && t && sp && addr) {
      uint64_t rows = 1;
      for (uint32_t d = 0; d + 1 < rank; ++d) rows = mul_sat(rows, dims[d]);
      return plan_sum_f32(*t, rows, dims[rank - 1], *sp, addr, p, &rule);
    }
    if (topology != TILER_HIP_SUM_SERIAL)
      return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "a split or workgroup fold reduces the trailing axis only");
    FoldGeometryHost g;
    std::memset(&g, 0, sizeof(g));
    uint64_t stride[8], total = 1, outputs = 1, contributors = 1;
    for (int d = (int)rank - 1; d >= 0; --d) {
      stride[d] = total;
      total = mul_sat(total, dims[d]);
    }
    for (uint32_t d = 0; d < rank; ++d)
      if (!(reduced_mask >> d & 1)) {
        g.dims[g.kept_rank] = dims[d];
        g.strides[g.kept_rank++] = stride[d];
        outputs = mul_sat(outputs, dims[d]);
      }
    for (uint32_t d = 0; d < rank; ++d)
      if (reduced_mask >> d & 1) {
        g.dims[g.kept_rank + g.red_rank] = dims[d];
        g.strides[g.kept_rank + g.red_rank++] = stride[d];
        contributors = mul_sat(contributors, dims[d]);
      }
    const uint32_t x = p.slot(mul_sat(total, 4), kSlotInput);
    const uint32_t out = p.slot(mul_sat(outputs, 4), kSlotOutput);
    if (outputs == 0) return TILER_HIP_OK;
    if (total == UINT64_MAX) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "fold extents overflow");
    p.add("tiler_fold_f32_m", blocks_capped(outputs, 65536), 1, 256)
        .ptr(x).ptr(out).u64(outputs).u64(contributors).blob(&g, sizeof(g), 8).blob(&rule, sizeof(rule), 4).u32(0);
    return TILER_HIP_OK;
  }
  // The fold kernel evaluates its epilogue in a 16-register file.
  if (epilogue && epilogue->registers > kExpressionRegisters)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "epilogue needs more than 16 live values");
  FoldGeometryHost g;
  std::memset(&g, 0, sizeof(g));
  uint64_t stride[8], total = 1, outputs = 1, contributors = 1;
  for (int d = (int)rank - 1; d >= 0; --d) {
    stride[d] = total;
    total = mul_sat(total, dims[d]);
  }
  for (uint32_t d = 0; d < rank; ++d) {
    if (reduced_mask >> d & 1) continue;
    g.dims[g.kept_rank] = dims[d];
    g.strides[g.kept_rank++] = stride[d];
    outputs = mul_sat(outputs, dims[d]);
  }
  for (uint32_t d = 0; d < rank; ++d) {
    if (!(reduced_mask >> d & 1)) continue;
    g.dims[g.kept_rank + g.red_rank] = dims[d];
    g.strides[g.kept_rank + g.red_rank++] = stride[d];
    contributors = mul_sat(contributors, dims[d]);
  }
  const uint32_t x = p.slot(mul_sat(total, 4), kSlotInput);
  const uint32_t out = p.slot(mul_sat(outputs, 4), kSlotOutput);
  uint32_t code = kMaxSlots;
  if (epilogue) {
    code = p.slot(epilogue->code.size(), TILER_HIP_SLOT_CONSTANT);
    p.constant_slot = code;
    p.constant = epilogue->code;
  }
  if (outputs == 0) return TILER_HIP_OK;
  if (total == UINT64_MAX) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "fold extents overflow");
  // model.rs:880-906: a maximum over no contributors has no value to commit.
  if (contributors == 0 && op == TILER_HIP_FOLD_MAXIMUM)
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "an empty maximum has no identity");
  static const char* const kNames[] = {"tiler_fold_sum_f32", "tiler_fold_squared_f32", "tiler_fold_fma_f32",
                                       "tiler_fold_maximum_f32"};
  float scale, bias;
  std::memcpy(&scale, &scale_bits, 4);
  std::memcpy(&bias, &bias_bits, 4);
  Launch& l = p.add(kNames[op], blocks_capped(outputs, 65536), 1, 256)
                  .ptr(x).ptr(out).u64(outputs).u64(contributors).blob(&g, sizeof(g), 8)
                  .f32(scale).f32(bias).u32(0);
  if (epilogue) l.ptr(code).u32(epilogue->count).u32(epilogue->result);
  else l.null_ptr().u32(0).u32(0);
  return TILER_HIP_OK;
}

// ---------------------------------------------------------------------------
// Reindex with signed strides.  Slots: src, out.
tiler_hip_status plan_reindex(uint64_t src_elements, uint32_t rank, const uint64_t* out_dims,
                              const int64_t* strides, int64_t base, uint32_t element_bytes, Program& p) {
  if (rank > 8 || (rank && (!out_dims || !strides))) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "reindex rank");
  if (element_bytes != 2 && element_bytes != 4)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "reindex element width");
  BroadcastGeometryHost g;
  std::memset(&g, 0, sizeof(g));
  g.rank = rank;
  g.base = (uint64_t)base;
  uint64_t n = 1;
  __int128 lo = base, hi = base;
  bool overflow = false;
  for (uint32_t d = 0; d < rank; ++d) {
    g.out_dims[d] = out_dims[d];
    g.src_strides[d] = (uint64_t)strides[d];
    n = mul_sat(n, out_dims[d]);
    if (out_dims[d] == 0) continue;
    const __int128 span = (__int128)strides[d] * (__int128)(out_dims[d] - 1);
    if (span < 0) lo += span;
    else hi += span;
    if (lo < -((__int128)1 << 100) || hi > ((__int128)1 << 100)) overflow = true;
  }
  const uint32_t src = p.slot(mul_sat(src_elements, element_bytes), kSlotInput);
  const uint32_t out = p.slot(mul_sat(n, element_bytes), kSlotOutput);
  if (n == 0) return TILER_HIP_OK;
  if (overflow || n == UINT64_MAX || lo < 0 || hi >= (__int128)src_elements)
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "reindex geometry reads outside the source");
  const uint64_t inner = rank ? out_dims[rank - 1] : 1;
  if (rank && inner >= 256) {
    const uint64_t rows = n / inner;
    p.add(element_bytes == 4 ? "tiler_broadcast_rows_u32" : "tiler_broadcast_rows_u16",
          (uint32_t)(rows < 8192 ? rows : 8192), 1, 256)
        .ptr(src).ptr(out).u64(rows).blob(&g, sizeof(g), 8);
    return TILER_HIP_OK;
  }
  p.add(element_bytes == 4 ? "tiler_broadcast_u32" : "tiler_broadcast_u16", blocks_capped(n, 8192), 1, 256)
      .ptr(src).ptr(out).u64(n).blob(&g, sizeof(g), 8);
  return TILER_HIP_OK;
}

}  // namespace tiler_rt
