// Planners of the realization families: the kernel each request runs, its
// launch geometry and argument segment, with the refusals the family entry
// points of include/tiler_hip.h document.
#include "program.h"

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
Launch& Launch::u32(uint32_t v) { return blob(&v, 4, 4); }
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
tiler_hip_status plan_sum_f32(const Target& t, uint64_t rows, uint64_t extent,
                              const tiler_hip_sum_plan& sp, const uintptr_t* addr, Program& p) {
  const uint32_t x = p.slot(mul_sat(mul_sat(rows, extent), 4), kSlotInput);
  const uint32_t out = p.slot(mul_sat(rows, 4), kSlotOutput);
  switch (sp.topology) {
    case TILER_HIP_SUM_SERIAL:
      if (rows == 0) return TILER_HIP_OK;
      p.add("tiler_sum_f32_serial", (uint32_t)((rows + 255) / 256), 1, 256)
          .ptr(x).u64(rows).u64(extent).u64(1).ptr(out);
      return TILER_HIP_OK;
    case TILER_HIP_SUM_MULTIPASS: {
      const uint64_t P = sp.partitions, c = sp.per_partition;
      if (rows == 0) return TILER_HIP_OK;
      if (P == 0 || (c != 0 && P > UINT64_MAX / c) || P * c != extent)
        return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "partitions do not cover the axis exactly");
      const uint32_t part = p.slot(mul_sat(mul_sat(rows, P), 4), kSlotScratch);
      p.add("tiler_sum_f32_partials", (uint32_t)((rows * P + 255) / 256), 1, 256)
          .ptr(x).u64(rows).u64(extent).u64(P).u64(c).ptr(part);
      p.add("tiler_sum_f32_serial", (uint32_t)((rows + 255) / 256), 1, 256)
          .ptr(part).u64(rows).u64(P).u64(1).ptr(out);
      return TILER_HIP_OK;
    }
    case TILER_HIP_SUM_COOPERATIVE: {
      const uint64_t P = sp.participants, c = sp.per_partition, R = sp.rounds;
      if (rows == 0) return TILER_HIP_OK;
      if (P == 0 || P > 1024 || c == 0 || R == 0 || P * c * R != extent)
        return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "grouping does not cover the axis exactly");
      p.add("tiler_sum_f32_cooperative", (uint32_t)rows, 1, (uint32_t)P)
          .ptr(x).u64(extent).u32((uint32_t)P).u64(c).u64(R).u32(sp.participant_major ? 1u : 0u).ptr(out);
      return TILER_HIP_OK;
    }
    case TILER_HIP_SUM_TREE: {
      if (rows == 0) return TILER_HIP_OK;
      if (rows == 1) {
        const uint32_t G = tree_workgroups(t, extent);
        const uint32_t part = p.slot((uint64_t)G * 4, kSlotScratch);
        p.add(aligned16(addr[x]) ? "tiler_sum_f32_grid" : "tiler_sum_f32_grid_unaligned", G, 1, 256)
            .ptr(x).u64(extent).ptr(part);
        p.add("tiler_sum_f32_grid_final", 1, 1, 256).ptr(part).u32(G).u64(extent).ptr(out);
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
tiler_hip_status plan_rms_norm(uint32_t dtype, int32_t weight_broadcast, uint64_t rows,
                               uint64_t extent, uint32_t eps_bits, const uintptr_t* addr,
                               Program& p) {
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
                                  const uintptr_t* addr, Program& p) {
  const uint32_t x = p.slot(mul_sat(mul_sat(rows, extent), 4), kSlotInput);
  const uint32_t y = p.slot(mul_sat(mul_sat(rows, extent), 4), kSlotOutput);
  if (rows == 0 || extent == 0) return TILER_HIP_OK;
  if (extent > 0xffffffffull)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "row longer than 2^32 - 1 elements");
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
    if (wgs <= 2ull * t.compute_units && wgs <= kRowSyncMaxWorkgroups) {
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
                          uint64_t n, float a, float b, const uintptr_t* addr, Program& p) {
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
// Contractions.  Slots: 0 a [m, k], 1 b [n, k], 2 c [m, n].
tiler_hip_status plan_contract_strict_f32(uint64_t m, uint64_t n, uint64_t k, Program& p) {
  const uint32_t a = p.slot(mul_sat(mul_sat(m, k), 4), kSlotInput);
  const uint32_t b = p.slot(mul_sat(mul_sat(n, k), 4), kSlotInput);
  const uint32_t c = p.slot(mul_sat(mul_sat(m, n), 4), kSlotOutput);
  // contraction.rs:420-428: an empty contracted domain has no unseeded result.
  if (k == 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "empty contracted extent");
  if (m == 0 || n == 0) return TILER_HIP_OK;
  if (m > 0xffffffffull || n > 0xffffffffull || k > 0xffffffffull || (m + 15) / 16 > 65535)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "contraction extents beyond the launch profile");
  p.add("tiler_contract_strict_f32", (uint32_t)((n + 15) / 16), (uint32_t)((m + 15) / 16), 256)
      .ptr(a).ptr(b).u32((uint32_t)m).u32((uint32_t)n).u32((uint32_t)k).ptr(c);
  return TILER_HIP_OK;
}

tiler_hip_status plan_contract_bf16(const Target& t, uint64_t m, uint64_t n, uint64_t k,
                                    uint32_t epilogue, const uintptr_t* addr, Program& p) {
  if (epilogue > TILER_HIP_EPILOGUE_SILU) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "epilogue");
  const uint32_t a = p.slot(mul_sat(mul_sat(m, k), 2), kSlotInput);
  const uint32_t b = p.slot(mul_sat(mul_sat(n, k), 2), kSlotInput);
  const uint32_t c = p.slot(mul_sat(mul_sat(m, n), 2), kSlotOutput);
  if (k == 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "empty contracted extent");
  if (m == 0 || n == 0) return TILER_HIP_OK;
  if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull || (m + 127) / 128 > 65535)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "contraction extents beyond the launch profile");
  const bool silu = epilogue == TILER_HIP_EPILOGUE_SILU;
  const uint32_t m32 = (uint32_t)m, n32 = (uint32_t)n, k32 = (uint32_t)k;
  // m <= 64 (decode shapes): B streamed once, one workgroup per 16 columns.
  if (m <= 64 && k % 8 == 0 && aligned16(addr[a]) && aligned16(addr[b]) && (n + 15) / 16 <= 0x7fffffffull) {
    char name[48];
    std::snprintf(name, sizeof(name), "tiler_contract_bf16_%sskinny%u", silu ? "silu_" : "", (uint32_t)((m + 15) / 16));
    p.add(name, (uint32_t)((n + 15) / 16), 1, 1024).ptr(a).ptr(b).u32(m32).u32(n32).u32(k32).ptr(c);
    return TILER_HIP_OK;
  }
  // The staged path addresses each operand panel (up to 256 rows) through one
  // buffer resource with 32-bit offsets (256 * k * 2 bytes must stay below
  // 2^31) and moves 16-byte rows: n and k multiples of 8, aligned operands.
  // 256-tiles when they fill every CU, 128-tiles (four times as many) when not.
  if (n % 8 == 0 && k % 8 == 0 && k * 512ull < (1ull << 31) && aligned16(addr[a]) && aligned16(addr[b]) &&
      aligned16(addr[c])) {
    const uint64_t t256 = ((m + 255) / 256) * ((n + 255) / 256);
    const uint64_t t128 = ((m + 127) / 128) * ((n + 127) / 128);
    const bool big = t256 >= t.compute_units;
    const uint64_t tiles = big ? t256 : t128;
    if (tiles <= 0x7fffffffull) {
      const char* name = big ? (silu ? "tiler_contract_bf16_silu_t256" : "tiler_contract_bf16_t256")
                             : (silu ? "tiler_contract_bf16_silu_t128" : "tiler_contract_bf16_t128");
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

}  // namespace tiler_rt
