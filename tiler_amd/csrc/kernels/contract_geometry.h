// Geometry records the contraction planner writes and the contraction kernels
// read; one definition for both sides (plain integers, natural alignment).
#pragma once

#include <stdint.h>

namespace tiler_geom {

constexpr int kAxes = 8;
constexpr int kBatchAxes = 6;

// The strict general contraction (contract_general.hip), in a CONSTANT slot:
// per output / contracted axis, its extent and the element stride it moves in
// each operand.  Contracted axes in ascending label order; the last one is
// the innermost of the fold.
struct GeneralGeometry {
  uint32_t out_rank, con_rank;
  uint64_t outputs;
  uint64_t out_dims[kAxes], con_dims[kAxes];
  uint64_t l_out[kAxes], r_out[kAxes], l_con[kAxes], r_con[kAxes];
};

// Batched MFMA contractions (contract.hip *_b kernels), by value: batch b of
// the launch's batch dimension decodes row-major over dims[0..rank) and moves
// each operand by the element strides of its coordinates.
struct BatchGeometry {
  uint32_t rank, reserved;
  uint64_t dims[kBatchAxes];
  uint64_t a_stride[kBatchAxes], b_stride[kBatchAxes], c_stride[kBatchAxes];
};

}  // namespace tiler_geom
