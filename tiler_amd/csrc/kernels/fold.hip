// Serial folds over any reduced-axis set, one invocation per output -- the
// emitted form of tiler-ir's emit_reduction / emit_maximum_reduction
// (tiler-ir/src/kernel/lower.rs:1236-1305, 2485-2500; tiler-metal goldens
// reduction_single_axis, reduction_multi_axis, reduction_fused_multiply_add):
//   StrictSerialSum               acc = canon(acc + x)
//   SquaredSerialSum              acc = canon(acc + canon(x * x))
//   FusedMultiplyAddSerialSum     acc = canon(acc + canon(canon(x * scale) + bias))
//                                 (contraction is permitted, never required:
//                                 the unfused form is what every contract admits)
//   StrictSerialMaximum           acc = maximum(acc, x), NaN-propagating,
//                                 -0 < +0 (tiler-reference/src/softmax.rs:168-186)
// over the contributors in lexicographic order of the reduced coordinates
// (tiler-reference/src/evaluate.rs:548-585), seeded at the first contributor.
// Seeding a sum at -0.0 and adding every (canonical) contributor value is the
// same bits: -0.0 is the exact additive identity, and each combine is
// canonicalized; a maximum seeded at -inf likewise (-inf is its two-sided
// identity, model.rs:889-900).  The sums' result is canonicalized; an empty
// sum commits the identity bits.  An optional one-input epilogue program
// (SquaredSerialSumThenEpilogue, model.rs:815-830) transforms the folded value.
#include "common.h"

namespace {

// Kept axes first (output order), then reduced axes (contributor order); each
// with its dense input stride in elements.
struct FoldGeometry {
  uint64_t dims[8];
  uint64_t strides[8];
  uint32_t kept_rank, red_rank;
};

enum : uint32_t { kFoldSum = 0, kFoldSquared = 1, kFoldFma = 2, kFoldMaximum = 3 };

template <uint32_t OP>
__device__ __forceinline__ void fold_body(const float* __restrict__ x, float* __restrict__ out,
                                          uint64_t outputs, uint64_t contributors, const FoldGeometry& g,
                                          float scale, float bias, uint32_t empty_bits,
                                          const ExprInstr* __restrict__ epi, uint32_t epi_count,
                                          uint32_t epi_result) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < outputs; id += stride) {
    uint64_t rem = id, base = 0;
    for (int d = (int)g.kept_rank - 1; d >= 0; --d) {
      const uint64_t c = rem % g.dims[d];
      rem /= g.dims[d];
      base += c * g.strides[d];
    }
    float acc = OP == kFoldMaximum ? -__builtin_huge_valf() : -0.0f;
    uint64_t coord[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint64_t off = base;
    const uint32_t r0 = g.kept_rank, rn = g.kept_rank + g.red_rank;
    for (uint64_t p = 0; p < contributors; ++p) {
      const float v = x[off];
      if (OP == kFoldMaximum) {
        acc = tiler::maximum_f32(acc, v);
      } else {
        float t = v;
        if (OP == kFoldSquared) t = tiler::canon(v * v);
        if (OP == kFoldFma) t = tiler::canon(tiler::canon(v * scale) + bias);
        acc = tiler::canon(acc + t);
      }
      // odometer over the reduced axes, last axis fastest
      for (int d = (int)rn - 1; d >= (int)r0; --d) {
        off += g.strides[d];
        if (++coord[d] < g.dims[d]) break;
        off -= g.strides[d] * g.dims[d];
        coord[d] = 0;
      }
    }
    float total = contributors == 0 ? __uint_as_float(empty_bits) : tiler::canon(acc);
    if (epi) total = expr_epilogue_f32(epi, epi_count, epi_result, total);
    out[id] = total;
  }
}

// The sums under a FoldRule: its prologue and the declared subnormal modes at
// every arithmetic site, seeded at the first contributor (the form a flushing
// contract realizes as; the maximum compares and takes no mode).
__device__ __forceinline__ void fold_rule_body(const float* __restrict__ x, float* __restrict__ out,
                                               uint64_t outputs, uint64_t contributors, const FoldGeometry& g,
                                               const tiler::FoldRule& rule, uint32_t empty_bits) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < outputs; id += stride) {
    uint64_t rem = id, base = 0;
    for (int d = (int)g.kept_rank - 1; d >= 0; --d) {
      const uint64_t c = rem % g.dims[d];
      rem /= g.dims[d];
      base += c * g.strides[d];
    }
    float acc = 0.0f;
    uint64_t coord[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint64_t off = base;
    const uint32_t r0 = g.kept_rank, rn = g.kept_rank + g.red_rank;
    for (uint64_t p = 0; p < contributors; ++p) {
      const float t = tiler::fold_contributor(rule, x[off]);
      acc = p == 0 ? t : tiler::fold_combine(rule, acc, t);
      for (int d = (int)rn - 1; d >= (int)r0; --d) {
        off += g.strides[d];
        if (++coord[d] < g.dims[d]) break;
        off -= g.strides[d] * g.dims[d];
        coord[d] = 0;
      }
    }
    out[id] = contributors == 0 ? __uint_as_float(empty_bits) : tiler::canon(acc);
  }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
tiler_fold_f32_m(const float* __restrict__ x, float* __restrict__ out, uint64_t outputs, uint64_t contributors,
                 FoldGeometry g, tiler::FoldRule rule, uint32_t empty_bits) {
  fold_rule_body(x, out, outputs, contributors, g, rule, empty_bits);
}

#define TILER_FOLD(NAME, OP)                                                                         \
  extern "C" __global__ void __launch_bounds__(256) NAME(                                            \
      const float* __restrict__ x, float* __restrict__ out, uint64_t outputs, uint64_t contributors, \
      FoldGeometry g, float scale, float bias, uint32_t empty_bits, const ExprInstr* __restrict__ epi, \
      uint32_t epi_count, uint32_t epi_result) {                                                     \
    fold_body<OP>(x, out, outputs, contributors, g, scale, bias, empty_bits, epi, epi_count, epi_result); \
  }
TILER_FOLD(tiler_fold_sum_f32, kFoldSum)
TILER_FOLD(tiler_fold_squared_f32, kFoldSquared)
TILER_FOLD(tiler_fold_fma_f32, kFoldFma)
TILER_FOLD(tiler_fold_maximum_f32, kFoldMaximum)
