// Sum-reduction realizations (the strict-serial-sum-f32 family) for gfx950.
//
// Four topologies, one per ReductionTopology the planner can select
// (tiler-ir/src/schedule/model.rs:1327-1555):
//   * tiler_sum_f32_serial       Serial: one invocation per output, the strict
//                                left fold of tiler-reference/src/evaluate.rs:498-589.
//   * tiler_sum_f32_partials     MultiPass pass 1: one invocation per
//                                (output, partition), evaluate.rs:612-776; pass 2
//                                is tiler_sum_f32_serial over the partials.
//   * tiler_sum_f32_cooperative  CooperativeWorkgroup: one workgroup per output
//                                with a declared (participants, contributors,
//                                rounds, layout) grouping, evaluate.rs:845-1158.
//   * tiler_sum_f32_grid(+final)/ The reassociating two-level tree (a
//     tiler_sum_f32_rows         REASSOCIATE-class contract): wave64 xor
//                                butterflies, an ascending cross-wave fold in LDS
//                                and, for one output, a second one-workgroup
//                                launch combining the workgroup partials.
// The first three are bit-exact with the reference; the tree's exact order is
// its declared grouping, restated by the oracle's grid/row grouped sums.
#include <type_traits>

#include "common.h"

using tiler::canon;

// ---------------------------------------------------------------------------
// Serial: out[o*inner+i] = strict fold over p of x[(o*extent+p)*inner+i].
// Seeding at -0.0 and adding every contributor equals seeding at the first
// contributor bit for bit (-0.0 is the exact additive identity under
// round-to-nearest), NaN payloads aside, which the commit canonicalizes.
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_serial(const float* __restrict__ x, uint64_t outer, uint64_t extent,
                     uint64_t inner, float* __restrict__ out) {
  uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= outer * inner) return;
  uint64_t o = id / inner, i = id - o * inner;
  const float* base = x + o * extent * inner + i;
  float acc = -0.0f;
  for (uint64_t p = 0; p < extent; ++p) acc = acc + base[p * inner];
  out[id] = extent == 0 ? 0.0f : canon(acc);
}

// Serial over contiguous rows, staged through LDS: out[v] = the same strict
// fold of x[v*length .. +length), ascending from a -0.0 seed, as
// tiler_sum_f32_serial computes.  A lane that folds its own row straight from
// global memory waits a memory latency per load (each load of a wave touches
// 64 rows); here a 256-thread workgroup serves R rows.  Stage s holds
// C = 4096/R elements of each row.  All four waves load stage s+1 into
// registers (coalesced: consecutive lanes read consecutive elements of one
// row), the folding lanes fold stage s from LDS, and then stage s+1 is stored
// to the other buffer.  Row r is folded by lane r/4 of wave r%4 (R = 1: lane 0
// of wave 0), so a workgroup's chains sit on its four waves' SIMDs rather
// than sharing one.  The chain of adds bounds a long row, and the loads hide
// behind it.  kVec: 16-byte loads (aligned x, length a multiple of 4).
//
// kDot: the fold of products instead, out[v] = fold over e of fl(a[e] *
// x[v*length + e]) -- one output row of the strict contraction, with x the
// right operand's rows and `a` the left operand's row, staged beside them.
template <int R, bool kVec, bool kDot>
__device__ __forceinline__ void staged_fold_body(const float* __restrict__ x, uint64_t nrows, uint64_t length,
                                                 const float* __restrict__ a, float* __restrict__ out) {
  constexpr uint32_t C = 4096 / R;               // elements of a row per stage
  constexpr uint32_t kStride = C + 4;            // LDS row stride in floats (16-byte aligned, staggered banks)
  constexpr uint32_t W = kVec ? 4 : 1;           // elements per load
  constexpr uint32_t kRowPieces = C / W;         // loads per row per stage
  constexpr uint32_t kPer = 4096 / W / 256;      // loads per thread per stage
  constexpr uint32_t kAPer = kDot ? (kRowPieces + 255) / 256 : 0;  // loads of the left row per thread
  __shared__ __align__(16) float stage[2][R * kStride];
  __shared__ __align__(16) float astage[kDot ? 2 : 1][kDot ? C : 4];
  const uint32_t t = threadIdx.x;
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const uint64_t stages = (length + C - 1) / C;
  typedef typename std::conditional<kVec, f32x4, float>::type piece;
  piece reg[kPer];
  piece areg[kAPer > 0 ? kAPer : 1];
  auto load = [&](uint64_t s) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const uint64_t e = s * C + (uint64_t)(q % kRowPieces) * W;
      if (row0 + r < nrows && e < length) {
        const float* src = x + (row0 + r) * length + e;
        if constexpr (kVec) reg[i] = *reinterpret_cast<const f32x4*>(src);
        else reg[i] = *src;
      } else {
        reg[i] = piece{};  // never folded: past the row or past the last row
      }
    }
#pragma unroll
    for (uint32_t i = 0; i < kAPer; ++i) {
      const uint32_t q = t + 256u * i;
      const uint64_t e = s * C + (uint64_t)q * W;
      if (q < kRowPieces && e < length) {
        if constexpr (kVec) areg[i] = *reinterpret_cast<const f32x4*>(a + e);
        else areg[i] = a[e];
      } else {
        areg[i] = piece{};
      }
    }
  };
  auto store = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      *reinterpret_cast<piece*>(&stage[buf][r * kStride + (q % kRowPieces) * W]) = reg[i];
    }
#pragma unroll
    for (uint32_t i = 0; i < kAPer; ++i) {
      const uint32_t q = t + 256u * i;
      if (q < kRowPieces) *reinterpret_cast<piece*>(&astage[buf][q * W]) = areg[i];
    }
  };
  const uint32_t fr = R == 1 ? 0u : (t & 63u) * 4u + (t >> 6);  // the row this lane folds
  const bool folds = (R == 1 ? t == 0 : (t & 63u) < (uint32_t)R / 4u) && row0 + fr < nrows;
  float acc = -0.0f;
  if (stages > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (uint64_t s = 0; s < stages; ++s) {
    const bool more = s + 1 < stages;
    if (more) load(s + 1);
    if (folds) {
      const float* row = &stage[s & 1][fr * kStride];
      const float* arow = &astage[kDot ? (s & 1) : 0][0];
      const uint32_t count = (uint32_t)(length - s * C < C ? length - s * C : C);
      // one fold step: the element, or under kDot its product with the left
      // row's element (two roundings: no FMA)
      // The left row's elements are the same for every folding lane: they
      // are read from global memory at a wave-uniform address (the scalar
      // cache serves them), not from LDS.
      const float* aglob = a + s * C;
      auto step4 = [&](const f32x4 v, uint32_t c) {
        if constexpr (kDot) {
          f32x4 w;
          if constexpr (kVec) {
            w = *reinterpret_cast<const f32x4*>(aglob + c);
          } else {
            w.x = aglob[c];
            w.y = aglob[c + 1];
            w.z = aglob[c + 2];
            w.w = aglob[c + 3];
          }
          acc = acc + w.x * v.x;
          acc = acc + w.y * v.y;
          acc = acc + w.z * v.z;
          acc = acc + w.w * v.w;
        } else {
          acc = acc + v.x;
          acc = acc + v.y;
          acc = acc + v.z;
          acc = acc + v.w;
        }
      };
      if (count == C) {
        // A whole stage: ping-pong batches of 16-byte reads, the next batch's
        // reads in flight while the current one is added, so the chain of
        // adds does not wait out an LDS latency per read; long rows run one
        // workgroup per CU, with registers for batches of 16 reads.
        constexpr uint32_t kBatch = C / 4 < (R <= 4 ? 16u : 8u) ? C / 4 : (R <= 4 ? 16u : 8u);
        constexpr uint32_t kBatches = C / 4 / kBatch;
        const f32x4* rv = reinterpret_cast<const f32x4*>(row);
        f32x4 ba[kBatch], bb[kBatch];
        auto add_batch = [&](const f32x4* v, uint32_t first) {
#pragma unroll
          for (uint32_t j = 0; j < kBatch; ++j) step4(v[j], (first + j) * 4u);
        };
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) ba[j] = rv[j];
        for (uint32_t b = 0; b < kBatches; b += 2) {
          if (b + 1 < kBatches) {
#pragma unroll
            for (uint32_t j = 0; j < kBatch; ++j) bb[j] = rv[(b + 1) * kBatch + j];
          }
          add_batch(ba, b * kBatch);
          if (b + 1 < kBatches) {
            if (b + 2 < kBatches) {
#pragma unroll
              for (uint32_t j = 0; j < kBatch; ++j) ba[j] = rv[(b + 2) * kBatch + j];
            }
            add_batch(bb, (b + 1) * kBatch);
          }
        }
      } else {
        // The last stage: only elements below `length` are folded (a padded
        // +0.0 would turn a -0.0 total into +0.0).
        uint32_t c = 0;
        for (; c + 4 <= count; c += 4) step4(*reinterpret_cast<const f32x4*>(row + c), c);
        for (; c < count; ++c) {
          if constexpr (kDot) acc = acc + arow[c] * row[c];
          else acc = acc + row[c];
        }
      }
    }
    if (more) store((uint32_t)((s + 1) & 1));
    __syncthreads();
  }
  if (folds) out[row0 + fr] = length == 0 ? 0.0f : canon(acc);
}

// The same stages and the same fold, for R in {1, 4, 16} (rows of at least
// 256 elements per stage), with the chain kept in registers: the folding
// waves relay-fold (tiler::relay_fold_chunk) each row's stage in passes of
// 256 elements, lane 8 g + s of a folding wave holding elements
// 32 s .. 32 s + 31 of the pass, read from the stage with 16-byte reads; the
// next pass's segment is read while the current one is folded.  R = 1: wave
// 0 folds the row; R = 4: wave w folds row w; R = 16: wave w folds rows
// 4 w .. 4 w + 3 in its groups 0..3 (groups 4..7 repeat groups 0..3's reads
// and their sums are not used).  Elements past the row's end are staged as
// -0.0, which leaves every sum unchanged (s + -0.0 == s for every s, the
// zeros and NaN included), so whole passes are folded.  Same order, same
// -0.0 seed, same commit as staged_fold_body.
//
// kDot: the fold of products fl(a[e] * x[v*length + e]) (staged_fold_body's
// kDot): the threads that stage x also load the matching elements of the
// left row `a` (the same for every row, so the caches serve them) and stage
// the rounded products, each rounded once as the fold would round it; the
// relay then folds them as it folds a row of the sum.
template <int R, bool kVec, bool kDot = false>
__device__ __forceinline__ void staged_relay_body(const float* __restrict__ x, uint64_t nrows, uint64_t length,
                                                  const float* __restrict__ a, float* __restrict__ out) {
  static_assert(R == 1 || R == 4 || R == 16, "rows of at least 256 elements per stage");
  constexpr uint32_t C = 4096 / R;               // elements of a row per stage
  constexpr uint32_t kStride = C + 4;            // LDS row stride in floats (16-byte aligned)
  constexpr uint32_t W = kVec ? 4 : 1;           // elements per load
  constexpr uint32_t kRowPieces = C / W;         // loads per row per stage
  constexpr uint32_t kPer = 4096 / W / 256;      // loads per thread per stage
  constexpr uint32_t S4 = 8;                     // 16-byte slots per lane per pass
  constexpr uint32_t kPass = 32 * S4;            // elements of a row per pass
  constexpr uint32_t kPasses = C / kPass;        // passes per whole stage
  constexpr uint32_t kRowsPerWave = R == 16 ? 4u : 1u;
  __shared__ __align__(16) float stage[2][R * kStride];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, g = lane >> 3, s = lane & 7u;
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const uint64_t stages = (length + C - 1) / C;
  typedef typename std::conditional<kVec, f32x4, float>::type piece;
  const float nz = -0.0f;
  piece reg[kPer];
  auto load = [&](uint64_t st) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const uint64_t e = st * C + (uint64_t)(q % kRowPieces) * W;
      if (row0 + r < nrows && e < length) {
        const float* src = x + (row0 + r) * length + e;
        if constexpr (kVec) {
          reg[i] = *reinterpret_cast<const f32x4*>(src);
          if constexpr (kDot) reg[i] = *reinterpret_cast<const f32x4*>(a + e) * reg[i];  // two roundings: no FMA
        } else {
          reg[i] = *src;
          if constexpr (kDot) reg[i] = a[e] * reg[i];
        }
      } else {
        if constexpr (kVec) reg[i] = f32x4{nz, nz, nz, nz};
        else reg[i] = nz;
      }
    }
  };
  auto store = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      *reinterpret_cast<piece*>(&stage[buf][r * kStride + (q % kRowPieces) * W]) = reg[i];
    }
  };
  const bool folding_wave = R == 1 ? wave == 0 : true;
  const uint32_t fr = R == 1 ? 0u : wave * kRowsPerWave + g % kRowsPerWave;  // the row this group folds
  float acc = -0.0f;
  if (stages > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (uint64_t st = 0; st < stages; ++st) {
    const bool more = st + 1 < stages;
    if (more) load(st + 1);
    if (folding_wave) {
      const uint32_t count = (uint32_t)(length - st * C < C ? length - st * C : C);
      const uint32_t passes = (count + kPass - 1) / kPass;
      acc = tiler::relay_fold_row<kPasses>(reinterpret_cast<const f32x4*>(&stage[st & 1][fr * kStride]), s, passes,
                                           acc);
    }
    if (more) store((uint32_t)((st + 1) & 1));
    __syncthreads();
  }
  // A group's row sum is in its lane 8 g after the last pass's final hop.
  if (folding_wave && s == 0 && g < kRowsPerWave && row0 + fr < nrows)
    out[row0 + fr] = length == 0 ? 0.0f : canon(acc);
}

// The same stages under a FoldRule (a flushing contract, a fused prologue),
// rows of at least 16.  Every thread turns the values it stages into
// apply_to_operand(contributor(x)) as it stores them to LDS (the prologue and
// the input mode are elementwise, so they run on all 256 lanes); the folding
// lane's chain is then only acc = R(O(acc) + t) per element, seeded at the
// first contributor (peeled: an identity seed would meet the result mode).
// kIn / kOut: whether the input / result mode flushes; with kOut the sum
// that leaves R is never subnormal, so O(acc) is acc itself.  A subnormal is
// found by v_cmp_class (the subnormal classes of both signs), which leaves
// zeros alone, and replaced by its own sign bit (mode 2) or +0 (mode 3).
template <int R>
constexpr uint32_t kRuleStageFloats = 2u * R * (4096u / R + 4u);  // both buffers of R rows

template <int R, bool kVec, bool kIn, bool kOut>
__device__ __forceinline__ void staged_rule_body(const float* __restrict__ x, uint64_t nrows, uint64_t length,
                                                 float* __restrict__ out, const tiler::FoldRule& rule,
                                                 float* __restrict__ lds) {
  constexpr uint32_t C = 4096 / R;
  constexpr uint32_t kStride = C + 4;
  constexpr uint32_t W = kVec ? 4 : 1;
  constexpr uint32_t kRowPieces = C / W;
  constexpr uint32_t kPer = 4096 / W / 256;
  float(*stage)[R * kStride] = reinterpret_cast<float(*)[R * kStride]>(lds);
  const uint32_t t = threadIdx.x;
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const uint64_t stages = (length + C - 1) / C;
  typedef typename std::conditional<kVec, f32x4, float>::type piece;
  piece reg[kPer];
  const uint32_t imask = rule.in_mode == 2u ? 0x80000000u : 0u;
  const uint32_t rmask = rule.out_mode == 2u ? 0x80000000u : 0u;
  auto flush = [](float v, uint32_t mask) {
    return __builtin_amdgcn_classf(v, 0x90) ? __uint_as_float(__float_as_uint(v) & mask) : v;
  };
  auto operand = [&](float v) {  // apply_to_operand(contributor(v))
    const float c = tiler::fold_contributor(rule, v);
    return kIn ? flush(c, imask) : c;
  };
  auto load = [&](uint64_t s) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const uint64_t e = s * C + (uint64_t)(q % kRowPieces) * W;
      if (row0 + r < nrows && e < length) {
        const float* src = x + (row0 + r) * length + e;
        if constexpr (kVec) reg[i] = *reinterpret_cast<const f32x4*>(src);
        else reg[i] = *src;
      } else {
        reg[i] = piece{};  // never folded: past the row or past the last row
      }
    }
  };
  auto store = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      piece v = reg[i];
      if constexpr (kVec) {
        v = f32x4{operand(v.x), operand(v.y), operand(v.z), operand(v.w)};
      } else {
        v = operand(v);
      }
      *reinterpret_cast<piece*>(&stage[buf][r * kStride + (q % kRowPieces) * W]) = v;
    }
  };
  const uint32_t fr = R == 1 ? 0u : (t & 63u) * 4u + (t >> 6);
  const bool folds = (R == 1 ? t == 0 : (t & 63u) < (uint32_t)R / 4u) && row0 + fr < nrows;
  float acc = 0.0f, acc_o = 0.0f;  // R's last result, and O of it
  auto step = [&](float to) {
    const float sum = acc_o + to;
    acc = kOut ? flush(sum, rmask) : sum;
    acc_o = (kIn && !kOut) ? flush(acc, imask) : acc;
  };
  if (stages > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (uint64_t s = 0; s < stages; ++s) {
    const bool more = s + 1 < stages;
    if (more) load(s + 1);
    if (folds) {
      const float* row = &stage[s & 1][fr * kStride];
      const uint32_t count = (uint32_t)(length - s * C < C ? length - s * C : C);
      uint32_t c = 0;
      if (s == 0) {  // the seed: the first contributor (as an operand of the first combine)
        acc = acc_o = row[0];
        c = 1;
        for (; c < 4 && c < count; ++c) step(row[c]);
      }
      for (; c + 4 <= count; c += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(row + c);
        step(v.x);
        step(v.y);
        step(v.z);
        step(v.w);
      }
      for (; c < count; ++c) step(row[c]);
    }
    if (more) store((uint32_t)((s + 1) & 1));
    __syncthreads();
  }
  if (folds) out[row0 + fr] = tiler::canon(acc);
}

// R in {1, 4, 16}: the relay fold; R = 64 and 256 (rows of 16..255): the
// lane-per-row fold of staged_fold_body, whose chains per stage are short.
#define TILER_SUM_STAGED(R, BODY)                                                                      \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_sum_f32_staged_r##R(const float* __restrict__ x, uint64_t nrows, uint64_t length,          \
                                float* __restrict__ out) {                                             \
    BODY<R, true>(x, nrows, length, nullptr, out);                                                     \
  }                                                                                                    \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_sum_f32_staged_r##R##_u(const float* __restrict__ x, uint64_t nrows, uint64_t length,      \
                                    float* __restrict__ out) {                                         \
    BODY<R, false>(x, nrows, length, nullptr, out);                                                    \
  }
template <int R, bool kVec, bool kDot = false>
__device__ __forceinline__ void staged_lane_body(const float* __restrict__ x, uint64_t nrows, uint64_t length,
                                                 const float* __restrict__ a, float* __restrict__ out) {
  staged_fold_body<R, kVec, kDot>(x, nrows, length, a, out);
}
TILER_SUM_STAGED(1, staged_relay_body)
TILER_SUM_STAGED(4, staged_relay_body)
TILER_SUM_STAGED(16, staged_relay_body)
TILER_SUM_STAGED(64, staged_lane_body)
TILER_SUM_STAGED(256, staged_lane_body)  // rows of 16..63: stages of 16 elements, every lane folding a row

// staged_rule_body's fold with the relay of staged_relay_body, for R in
// {1, 4, 16}: the staged contributors are apply_to_operand(contributor(x)),
// and the relay's step is the rule's combine acc = R(O(acc) + t), the row
// opening with its first contributor as the seed (relay_fold<.., true> on
// the first pass of the first stage).  Positions past the row's end are
// staged as -0.0 after the prologue and the input mode (which could turn it
// into +0.0): with a flushing result mode, or with no mode, a -0.0 step
// leaves the value unchanged (R(acc + -0.0) = R(acc) = acc for a value that
// came out of R); with only the input mode flushing it would leave O(acc),
// so there the row's last pass takes a step only below the row's end.
template <int R, bool kVec, bool kIn, bool kOut>
__device__ __forceinline__ void staged_rule_relay_body(const float* __restrict__ x, uint64_t nrows, uint64_t length,
                                                       float* __restrict__ out, const tiler::FoldRule& rule,
                                                       float* __restrict__ lds) {
  static_assert(R == 1 || R == 4 || R == 16, "rows of at least 256 elements per stage");
  constexpr uint32_t C = 4096 / R;
  constexpr uint32_t kStride = C + 4;
  constexpr uint32_t W = kVec ? 4 : 1;
  constexpr uint32_t kRowPieces = C / W;
  constexpr uint32_t kPer = 4096 / W / 256;
  constexpr uint32_t S4 = 8;
  constexpr uint32_t kPass = 32 * S4;
  constexpr uint32_t kRowsPerWave = R == 16 ? 4u : 1u;
  float(*stage)[R * kStride] = reinterpret_cast<float(*)[R * kStride]>(lds);
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, g = lane >> 3, s = lane & 7u;
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const uint64_t stages = (length + C - 1) / C;
  typedef typename std::conditional<kVec, f32x4, float>::type piece;
  piece reg[kPer];
  const uint32_t imask = rule.in_mode == 2u ? 0x80000000u : 0u;
  const uint32_t rmask = rule.out_mode == 2u ? 0x80000000u : 0u;
  auto flush = [](float v, uint32_t mask) {
    return __builtin_amdgcn_classf(v, 0x90) ? __uint_as_float(__float_as_uint(v) & mask) : v;
  };
  auto operand = [&](float v) {  // apply_to_operand(contributor(v))
    const float c = tiler::fold_contributor(rule, v);
    return kIn ? flush(c, imask) : c;
  };
  auto load = [&](uint64_t st) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const uint64_t e = st * C + (uint64_t)(q % kRowPieces) * W;
      if (row0 + r < nrows && e < length) {
        const float* src = x + (row0 + r) * length + e;
        if constexpr (kVec) reg[i] = *reinterpret_cast<const f32x4*>(src);
        else reg[i] = *src;
      } else {
        reg[i] = piece{};
      }
    }
  };
  auto store = [&](uint32_t buf, uint64_t st) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const uint64_t e = st * C + (uint64_t)(q % kRowPieces) * W;
      const bool in = row0 + r < nrows && e < length;  // kVec: length is a multiple of 4
      piece v = reg[i];
      if constexpr (kVec) {
        v = in ? f32x4{operand(v.x), operand(v.y), operand(v.z), operand(v.w)} : f32x4{-0.0f, -0.0f, -0.0f, -0.0f};
      } else {
        v = in ? operand(v) : -0.0f;
      }
      *reinterpret_cast<piece*>(&stage[buf][r * kStride + (q % kRowPieces) * W]) = v;
    }
  };
  // acc is R's last result; O(acc) is taken at the next step.
  auto step = [&](float acc, float to) {
    const float acc_o = (kIn && !kOut) ? flush(acc, imask) : acc;
    const float sum = acc_o + to;
    return kOut ? flush(sum, rmask) : sum;
  };
  const bool folding_wave = R == 1 ? wave == 0 : true;
  const uint32_t fr = R == 1 ? 0u : wave * kRowsPerWave + g % kRowsPerWave;
  float acc = 0.0f;
  if (stages > 0) {
    load(0);
    store(0, 0);
  }
  __syncthreads();
  for (uint64_t st = 0; st < stages; ++st) {
    const bool more = st + 1 < stages;
    if (more) load(st + 1);
    if (folding_wave) {
      const uint32_t count = (uint32_t)(length - st * C < C ? length - st * C : C);
      const uint32_t passes = (count + kPass - 1) / kPass;
      const f32x4* src = reinterpret_cast<const f32x4*>(&stage[st & 1][fr * kStride]) + s * S4;
      // The row's last pass, when it runs past the row's end: a step only
      // at positions below the end (this lane's segment holds `valid` of
      // them).  A -0.0 step is exact only after a step has gone through R,
      // and a row's only contributor is its seed, so every mode guards it.
      const bool ragged = !more && passes * kPass != count;
      const uint32_t seg0 = (passes - 1) * kPass + 32u * s;
      const uint32_t valid = count > seg0 ? (count - seg0 < 32u ? count - seg0 : 32u) : 0u;
      // A loop over the passes (not unrolled: each relay variant appears
      // once); the next pass's segment is read into nxt while cur is folded.
      f32x4 cur[S4], nxt[S4];
#pragma unroll
      for (uint32_t k = 0; k < S4; ++k) cur[k] = src[k];
      for (uint32_t p = 0; p < passes; ++p) {
        const f32x4* next = src + (p + 1 < passes ? p + 1 : p) * (kPass / 4);
#pragma unroll
        for (uint32_t k = 0; k < S4; ++k) nxt[k] = next[k];
        const bool seed = p == 0 && st == 0;
        auto run = [&](auto seeded, auto f) { acc = tiler::relay_fold<S4, decltype(seeded)::value>(cur, acc, f); };
        if (ragged && p + 1 == passes) {
          // i counts the contributors taken in step order, the seed included
          // (it takes no step), so i & 31 is a contributor's position in the
          // hot lane's segment.
          uint32_t i = seed ? 1u : 0u;
          auto guarded = [&](float a0, float c) { return (i++ & 31u) < valid ? step(a0, c) : a0; };
          if (seed) run(tiler::Step<1>{}, guarded);
          else run(tiler::Step<0>{}, guarded);
        } else if (seed) {
          run(tiler::Step<1>{}, step);
        } else {
          run(tiler::Step<0>{}, step);
        }
#pragma unroll
        for (uint32_t k = 0; k < S4; ++k) cur[k] = nxt[k];
      }
    }
    if (more) store((uint32_t)((st + 1) & 1), st + 1);
    __syncthreads();
  }
  if (folding_wave && s == 0 && g < kRowsPerWave && row0 + fr < nrows) out[row0 + fr] = tiler::canon(acc);
}

// The same stages under a FoldRule: a flushing contract's serial fold, and the
// fused prologues (squared, scale-bias) over a trailing axis; one body per
// pair of flushing dimensions, chosen by a uniform branch.
template <int R, bool kVec>
__device__ __forceinline__ void staged_rule_dispatch(const float* __restrict__ x, uint64_t nrows, uint64_t length,
                                                     float* __restrict__ out, const tiler::FoldRule& rule) {
  __shared__ __align__(16) float lds[kRuleStageFloats<R>];
  const bool in = rule.in_mode > 1u, res = rule.out_mode > 1u;
  if constexpr (R <= 16) {  // the relay fold (rows of at least 256 elements per stage)
    if (in && res) staged_rule_relay_body<R, kVec, true, true>(x, nrows, length, out, rule, lds);
    else if (in) staged_rule_relay_body<R, kVec, true, false>(x, nrows, length, out, rule, lds);
    else if (res) staged_rule_relay_body<R, kVec, false, true>(x, nrows, length, out, rule, lds);
    else staged_rule_relay_body<R, kVec, false, false>(x, nrows, length, out, rule, lds);
  } else {
    if (in && res) staged_rule_body<R, kVec, true, true>(x, nrows, length, out, rule, lds);
    else if (in) staged_rule_body<R, kVec, true, false>(x, nrows, length, out, rule, lds);
    else if (res) staged_rule_body<R, kVec, false, true>(x, nrows, length, out, rule, lds);
    else staged_rule_body<R, kVec, false, false>(x, nrows, length, out, rule, lds);
  }
}
#define TILER_SUM_STAGED_RULE(R)                                                                       \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_sum_f32_staged_r##R##_m(const float* __restrict__ x, uint64_t nrows, uint64_t length,      \
                                    float* __restrict__ out, tiler::FoldRule rule) {                   \
    staged_rule_dispatch<R, true>(x, nrows, length, out, rule);                                        \
  }                                                                                                    \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_sum_f32_staged_r##R##_u_m(const float* __restrict__ x, uint64_t nrows, uint64_t length,    \
                                      float* __restrict__ out, tiler::FoldRule rule) {                 \
    staged_rule_dispatch<R, false>(x, nrows, length, out, rule);                                       \
  }
TILER_SUM_STAGED_RULE(1)
TILER_SUM_STAGED_RULE(4)
TILER_SUM_STAGED_RULE(16)
TILER_SUM_STAGED_RULE(64)
TILER_SUM_STAGED_RULE(256)

// MultiPass pass 1: partials[r*P + p] = strict fold of
// x[r*extent + p*chunk .. +chunk]; an empty partition commits +0.0.
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_partials(const float* __restrict__ x, uint64_t rows, uint64_t extent,
                       uint64_t partitions, uint64_t chunk, float* __restrict__ partials) {
  uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * partitions) return;
  uint64_t r = id / partitions, p = id - r * partitions;
  const float* base = x + r * extent + p * chunk;
  float acc = -0.0f;
  for (uint64_t w = 0; w < chunk; ++w) acc = acc + base[w];
  partials[id] = chunk == 0 ? 0.0f : canon(acc);
}

// The same under a FoldRule (evaluate.rs:612-776 strict_partial_sums_under):
// each partition seeded at its first contributor, so a one-contributor
// partition transports its value unchanged under every mode.
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_partials_m(const float* __restrict__ x, uint64_t rows, uint64_t extent, uint64_t partitions,
                         uint64_t chunk, float* __restrict__ partials, tiler::FoldRule rule) {
  uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * partitions) return;
  uint64_t r = id / partitions, p = id - r * partitions;
  const float* base = x + r * extent + p * chunk;
  float acc = 0.0f;
  for (uint64_t w = 0; w < chunk; ++w) {
    const float t = tiler::fold_contributor(rule, base[w]);
    acc = w == 0 ? t : tiler::fold_combine(rule, acc, t);
  }
  partials[id] = chunk == 0 ? 0.0f : canon(acc);
}

// CooperativeWorkgroup: one workgroup per row; blockDim.x == participants.
// Round r: participant p folds cell (RoundMajor r*P+p | ParticipantMajor p*R+r)
// of `chunk` contributors; staged partials go to LDS; participant 0 folds them
// in ascending p and accumulates round totals in ascending r -- the single
// workgroup tree of tiler-metal's cooperative_workgroup_reduction golden.
extern "C" __global__ void __launch_bounds__(1024)
tiler_sum_f32_cooperative(const float* __restrict__ x, uint64_t extent, uint32_t participants,
                          uint64_t chunk, uint64_t rounds, uint32_t participant_major,
                          float* __restrict__ out) {
  __shared__ float staged[1024];
  const uint32_t p = threadIdx.x;
  const float* row = x + (uint64_t)blockIdx.x * extent;
  float total = -0.0f;
  for (uint64_t r = 0; r < rounds; ++r) {
    uint64_t cell = participant_major ? (uint64_t)p * rounds + r : r * participants + p;
    const float* range = row + cell * chunk;
    float partial = -0.0f;
    for (uint64_t w = 0; w < chunk; ++w) partial = partial + range[w];
    staged[p] = partial;
    __syncthreads();
    if (p == 0) {
      float s = -0.0f;
      for (uint32_t q = 0; q < participants; ++q) s = s + staged[q];
      total = total + s;
    }
    __syncthreads();
  }
  if (p == 0) out[blockIdx.x] = canon(total);
}

// The same under a FoldRule (evaluate.rs:845-1158 cooperative_grouped_sum_under):
// every cell, the staged partials and the round totals seeded at their first
// value.
extern "C" __global__ void __launch_bounds__(1024)
tiler_sum_f32_cooperative_m(const float* __restrict__ x, uint64_t extent, uint32_t participants,
                            uint64_t chunk, uint64_t rounds, uint32_t participant_major,
                            float* __restrict__ out, tiler::FoldRule rule) {
  __shared__ float staged[1024];
  const uint32_t p = threadIdx.x;
  const float* row = x + (uint64_t)blockIdx.x * extent;
  float total = 0.0f;
  for (uint64_t r = 0; r < rounds; ++r) {
    uint64_t cell = participant_major ? (uint64_t)p * rounds + r : r * participants + p;
    const float* range = row + cell * chunk;
    float partial = tiler::fold_contributor(rule, range[0]);
    for (uint64_t w = 1; w < chunk; ++w) partial = tiler::fold_combine(rule, partial, tiler::fold_contributor(rule, range[w]));
    staged[p] = partial;
    __syncthreads();
    if (p == 0) {
      float s = staged[0];
      for (uint32_t q = 1; q < participants; ++q) s = tiler::fold_combine(rule, s, staged[q]);
      total = r == 0 ? s : tiler::fold_combine(rule, total, s);
    }
    __syncthreads();
  }
  if (p == 0) out[blockIdx.x] = canon(total);
}

// ---------------------------------------------------------------------------
// Reassociating tree.
//
// In-workgroup combine of 256 thread partials: per-wave xor butterfly, then the
// four wave sums in ascending wave order.
__device__ __forceinline__ float block_sum256(float v, float* lds4) {
  v = tiler::wave_sum_butterfly(v);
  const uint32_t t = threadIdx.x;
  if ((t & 63u) == 0) lds4[t >> 6] = v;
  __syncthreads();
  float s = lds4[0];
  s = s + lds4[1];
  s = s + lds4[2];
  s = s + lds4[3];
  return s;
}

// One output over n contributors, two launches.  Tile = 1024 elements
// (256 threads x 4); stage 1: workgroup b folds tiles b, b+G, ... in
// ascending (tile, component) order per thread and writes its partial;
// stage 2 (one workgroup): thread t folds partials t, t+256, ..., then the
// same in-workgroup combine.  The kernel boundary orders the partials: no
// device-scope fence is taken per workgroup (each costs an L2 write-back).
template <bool kAligned>
__device__ __forceinline__ void sum_stage1_body(const float* __restrict__ x, uint64_t n,
                                                float* __restrict__ partials) {
  __shared__ float lds4[4];
  const uint32_t t = threadIdx.x, b = blockIdx.x, G = gridDim.x;
  const uint64_t tiles = (n + 1023) >> 10;
  const uint64_t full = n >> 10;
  float acc = -0.0f;
  uint64_t tile = b;
  if (kAligned) {
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
    for (; tile + 3ull * G < full; tile += 4ull * G) {
      f32x4 v0 = __builtin_nontemporal_load(&x4[(tile) * 256 + t]);
      f32x4 v1 = __builtin_nontemporal_load(&x4[(tile + G) * 256 + t]);
      f32x4 v2 = __builtin_nontemporal_load(&x4[(tile + 2ull * G) * 256 + t]);
      f32x4 v3 = __builtin_nontemporal_load(&x4[(tile + 3ull * G) * 256 + t]);
      acc = acc + v0.x; acc = acc + v0.y; acc = acc + v0.z; acc = acc + v0.w;
      acc = acc + v1.x; acc = acc + v1.y; acc = acc + v1.z; acc = acc + v1.w;
      acc = acc + v2.x; acc = acc + v2.y; acc = acc + v2.z; acc = acc + v2.w;
      acc = acc + v3.x; acc = acc + v3.y; acc = acc + v3.z; acc = acc + v3.w;
    }
    for (; tile < full; tile += G) {
      f32x4 v0 = __builtin_nontemporal_load(&x4[tile * 256 + t]);
      acc = acc + v0.x; acc = acc + v0.y; acc = acc + v0.z; acc = acc + v0.w;
    }
  }
  for (; tile < tiles; tile += G) {
    uint64_t base = (tile << 10) + 4ull * t;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (base + e < n) acc = acc + x[base + e];
  }
  float s = block_sum256(acc, lds4);
  if (t == 0) partials[b] = s;
}

extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_grid(const float* __restrict__ x, uint64_t n, float* __restrict__ partials) {
  sum_stage1_body<true>(x, n, partials);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_grid_unaligned(const float* __restrict__ x, uint64_t n,
                             float* __restrict__ partials) {
  sum_stage1_body<false>(x, n, partials);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_grid_final(const float* __restrict__ partials, uint32_t G, uint64_t n,
                         float* __restrict__ out) {
  __shared__ float lds4[4];
  float acc = -0.0f;
  for (uint32_t i = threadIdx.x; i < G; i += 256) acc = acc + partials[i];
  float total = block_sum256(acc, lds4);
  if (threadIdx.x == 0) out[0] = n == 0 ? 0.0f : canon(total);
}

// Rows of at most 256: the same grouping, one wave per row.  Thread t of the
// 256-thread form folds elements 4t..4t+3, so for extent <= 256 only wave 0
// holds contributors; waves 1-3 fold nothing and their butterflies give
// -0.0, which the ascending fold of the four wave sums adds exactly
// (w + -0.0 == w for every w).  The row's value is therefore wave 0's
// butterfly alone, computed here by each wave for its own row (4 rows per
// workgroup).  kVec: 16-byte loads (aligned x, extent a multiple of 4).
template <bool kVec>
__device__ __forceinline__ void sum_rows_wave_body(const float* __restrict__ x, uint64_t rows, uint32_t extent,
                                                   float* __restrict__ out) {
  const uint32_t l = threadIdx.x & 63u;
  const uint64_t row = (uint64_t)blockIdx.x * 4u + (threadIdx.x >> 6);
  if (row >= rows) return;  // a whole wave: no barrier below
  const float* r = x + row * extent;
  float acc = -0.0f;
  const uint32_t p = 4u * l;
  if (kVec) {
    if (p < extent) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(r + p);
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
  } else {
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e)
      if (p + e < extent) acc = acc + r[p + e];
  }
  const float s = tiler::wave_sum_butterfly(acc);
  if (l == 0) out[row] = canon(s);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_rows_w(const float* __restrict__ x, uint64_t rows, uint32_t extent, float* __restrict__ out) {
  sum_rows_wave_body<true>(x, rows, extent, out);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_rows_w_u(const float* __restrict__ x, uint64_t rows, uint32_t extent, float* __restrict__ out) {
  sum_rows_wave_body<false>(x, rows, extent, out);
}

// Many outputs: one 256-thread workgroup per row of `extent` contributors,
// grouping (vec 4, waves 4): thread t folds elements p with (p/4)%256 == t in
// ascending p, then block_sum256.  On a 16-byte-aligned row the whole
// 1024-element tiles go four at a time, their loads issued before their adds
// (a workgroup per row is otherwise latency-bound: one load in flight per
// thread); the adds keep the order.
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_rows(const float* __restrict__ x, uint64_t extent, float* __restrict__ out) {
  __shared__ float lds4[4];
  const uint32_t t = threadIdx.x;
  const float* row = x + (uint64_t)blockIdx.x * extent;
  float acc = -0.0f;
  uint64_t base = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15u) == 0) {  // uniform across the workgroup
    const f32x4* r4 = reinterpret_cast<const f32x4*>(row);
    for (; base + 4096 <= extent; base += 4096) {
      f32x4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = __builtin_nontemporal_load(&r4[(base >> 2) + 256u * j + t]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc = acc + v[j].x;
        acc = acc + v[j].y;
        acc = acc + v[j].z;
        acc = acc + v[j].w;
      }
    }
  }
  for (; base < extent; base += 1024) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint64_t p = base + 4ull * t + e;
      if (p < extent) acc = acc + row[p];
    }
  }
  float s = block_sum256(acc, lds4);
  if (t == 0) out[blockIdx.x] = extent == 0 ? 0.0f : canon(s);
}
