// Exhaustive device audit of the contraction epilogue's SiLU
// (tiler::silu_for_bf16 in tiler_amd/csrc/kernels/common.h): for every
// binary32 input x in [first, first + count) (as bit patterns), compare
// bf16_narrow(silu_for_bf16(x)) with bf16_narrow(silu_f32(x)), the reference
// SiLU (tiler-reference/src/silu.rs:511-533) narrowed once.
//
// result[0] mismatching inputs          result[1] lowest mismatching pattern
// result[2] fast-domain inputs marked for silu_f32 (near a bf16 midpoint)
// result[3] largest distance, in binary32 steps, between silu_fast_f32(x)
//           and silu_f32(x) over the fast domain (-80 < x < 2^127)
// result[4] inputs in the fast domain
//
// Test infrastructure: compiled into its own code object by the test build
// and loaded through tiler_hip_prepare_entries; the product never loads it.
#include "../../tiler_amd/csrc/kernels/common.h"

namespace {

__device__ __forceinline__ int64_t ordered(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? -(int64_t)(b & 0x7fffffffu) : (int64_t)b;
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
tiler_audit_silu_for_bf16(uint64_t first, uint64_t count, unsigned long long* result) {
  __shared__ unsigned long long s_mis, s_low, s_fall, s_dist, s_fast;
  if (threadIdx.x == 0) {
    s_mis = 0;
    s_low = ~0ull;
    s_fall = 0;
    s_dist = 0;
    s_fast = 0;
  }
  __syncthreads();
  unsigned long long mis = 0, low = ~0ull, fall = 0, dist = 0, fast = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const uint32_t bits = (uint32_t)(first + i);
    const float x = __uint_as_float(bits);
    const float exact = tiler::silu_f32(x);
    const uint32_t want = tiler::bf16_narrow(exact);
    const uint32_t got = tiler::bf16_narrow(tiler::silu_for_bf16(x));
    if (got != want) {
      ++mis;
      if (bits < low) low = bits;
    }
    if (x > -80.0f && x < 0x1.0p127f) {
      ++fast;
      bool marked;
      const float s = tiler::silu_bf16_candidate(x, marked);
      const int64_t d = ordered(s) - ordered(exact);
      const unsigned long long ad = (unsigned long long)(d < 0 ? -d : d);
      if (ad > dist) dist = ad;
      if (marked) ++fall;
    }
  }
  atomicAdd(&s_mis, mis);
  atomicMin(&s_low, low);
  atomicAdd(&s_fall, fall);
  atomicMax(&s_dist, dist);
  atomicAdd(&s_fast, fast);
  __syncthreads();
  if (threadIdx.x == 0) {
    atomicAdd(&result[0], s_mis);
    atomicMin(&result[1], s_low);
    atomicAdd(&result[2], s_fall);
    atomicMax(&result[3], s_dist);
    atomicAdd(&result[4], s_fast);
  }
}
