// Elementwise (pointwise) maps for gfx950, f32 and bf16 storage.
//
// Reference arithmetic: tiler-reference/src/evaluate.rs:448-485 `binary`
// (operand/result conformance around canon(op(l, r)), rank-0 operands
// broadcast); the emitted forms are tiler-metal's goldens
// pointwise_scale_bias{,_bf16}.metal:41-58 (one statement per operation, NaN
// canonicalized per result) and elementary_silu_activation.metal:41-62.
//
// bf16 storage computes each operation in binary32 on exactly widened operands
// and narrows the one result (ADR 0091 decision 2).  For a single add or
// multiply that equals the exact-rational bf16 result of
// tiler-reference/src/bf16.rs: binary32 carries 24 >= 2*8+2 bits, so the
// double rounding is innocuous; scale-bias is two operations and narrows after
// each, as the bf16 golden does.
//
// Ops: 0 scale-bias y = x*a + b (two roundings), 1 SiLU, 2 add, 3 multiply.
// `x2` is the second operand of add/multiply; x2_stride 0 broadcasts a rank-0
// operand, 1 reads it elementwise.
#include "common.h"

using tiler::canon;

namespace {

__device__ __forceinline__ float map_op(uint32_t op, float x, float x2, float a, float b) {
  switch (op) {
    case 0: {
      float t = canon(x * a);
      return canon(t + b);
    }
    case 1:
      return canon(tiler::silu_f32(x));
    case 2:
      return canon(x + x2);
    default:
      return canon(x * x2);
  }
}

__device__ __forceinline__ float map_op_bf16(uint32_t op, float x, float x2, float a, float b) {
  switch (op) {
    case 0: {
      float t = tiler::bf16_widen(tiler::bf16_narrow(x * a));
      return t + b;
    }
    case 1:
      return tiler::silu_f32(x);
    case 2:
      return x + x2;
    default:
      return x * x2;
  }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
tiler_map_f32(const float* __restrict__ x, const float* __restrict__ x2, uint64_t x2_stride,
              uint64_t n, uint32_t op, float a, float b, float* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float s2 = x2 ? x2[i * x2_stride] : 0.0f;
    y[i] = map_op(op, x[i], s2, a, b);
  }
}

extern "C" __global__ void __launch_bounds__(256)
tiler_map_bf16(const uint16_t* __restrict__ x, const uint16_t* __restrict__ x2,
               uint64_t x2_stride, uint64_t n, uint32_t op, float a, float b,
               uint16_t* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float s2 = x2 ? tiler::bf16_widen(x2[i * x2_stride]) : 0.0f;
    y[i] = (uint16_t)tiler::bf16_narrow(map_op_bf16(op, tiler::bf16_widen(x[i]), s2, a, b));
  }
}

// Broadcast / reindex (tiler-reference/src/structural.rs:75-108): a pure move.
// out element o (row-major over out_dims) reads source offset
// sum_d coord_d(o) * src_stride_d; a broadcast axis has stride 0.  Rank <= 8.
struct BroadcastGeometry {
  uint64_t out_dims[8];
  uint64_t src_strides[8];
  uint32_t rank;
};

template <typename T>
__device__ __forceinline__ void broadcast_body(const T* __restrict__ src, T* __restrict__ out,
                                               uint64_t n, const BroadcastGeometry& g) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint64_t rem = i, off = 0;
    for (int d = (int)g.rank - 1; d >= 0; --d) {
      uint64_t c = rem % g.out_dims[d];
      rem /= g.out_dims[d];
      off += c * g.src_strides[d];
    }
    out[i] = src[off];
  }
}

extern "C" __global__ void __launch_bounds__(256)
tiler_broadcast_u32(const uint32_t* __restrict__ src, uint32_t* __restrict__ out, uint64_t n,
                    BroadcastGeometry g) {
  broadcast_body<uint32_t>(src, out, n, g);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_broadcast_u16(const uint16_t* __restrict__ src, uint16_t* __restrict__ out, uint64_t n,
                    BroadcastGeometry g) {
  broadcast_body<uint16_t>(src, out, n, g);
}

// Fill: dst[i] = value for i < words.  A kernel rather than a memset so that a
// captured graph holds kernel nodes only.
extern "C" __global__ void __launch_bounds__(256)
tiler_fill_u32(uint32_t* __restrict__ dst, uint32_t value, uint64_t words) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride)
    dst[i] = value;
}
