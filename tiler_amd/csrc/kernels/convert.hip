// bf16 <-> binary32 conversion, two typed families, one per direction
// (docs/decisions/0091-...md decision 2):
//   * widening bf16 -> binary32 is exact and total: the 16 bits become the
//     high half of the binary32 pattern (a NaN keeps its payload);
//   * narrowing binary32 -> bf16 rounds to nearest, ties to even, overflows
//     to a signed infinity at the inclusive midpoint above the largest finite
//     bf16, maps every NaN to 0x7fc0, underflows gradually and keeps the sign
//     of zero.
// Both are pure HBM streams.  The vector forms move 16 bytes per lane per
// side with non-temporal accesses; the narrowing one canonicalizes NaNs and
// then uses v_cvt_pk_bf16_f32, which rounds exactly like the rule above on
// every non-NaN binary32 input (checked on the device over all of them).  The
// scalar forms serve unaligned storage and tails.
#include "common.h"

namespace {

typedef float f32x2c __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2c __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t narrow_pair(float lo, float hi) {
  const float qnan = __uint_as_float(0x7fc00000u);
  const f32x2c f = {lo != lo ? qnan : lo, hi != hi ? qnan : hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2c));
}

}  // namespace

// n8 groups of 8 elements: two f32x4 in, one 16-byte bf16 chunk out.
extern "C" __global__ void __launch_bounds__(256)
tiler_narrow_f32_bf16_v8(const f32x4* __restrict__ x, uint64_t n8, u32x4* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
    const f32x4 a = __builtin_nontemporal_load(&x[2 * i]);
    const f32x4 b = __builtin_nontemporal_load(&x[2 * i + 1]);
    const u32x4 o = {narrow_pair(a.x, a.y), narrow_pair(a.z, a.w), narrow_pair(b.x, b.y), narrow_pair(b.z, b.w)};
    __builtin_nontemporal_store(o, &y[i]);
  }
}

extern "C" __global__ void __launch_bounds__(256)
tiler_narrow_f32_bf16(const float* __restrict__ x, uint64_t n, uint16_t* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (uint16_t)tiler::bf16_narrow(x[i]);
}

// n8 groups of 8 elements: one 16-byte bf16 chunk in, two f32x4 out.
extern "C" __global__ void __launch_bounds__(256)
tiler_widen_bf16_f32_v8(const u32x4* __restrict__ x, uint64_t n8, f32x4* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(&x[i]);
    const f32x4 a = {__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                     __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
    const f32x4 b = {__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xffff0000u),
                     __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xffff0000u)};
    __builtin_nontemporal_store(a, &y[2 * i]);
    __builtin_nontemporal_store(b, &y[2 * i + 1]);
  }
}

extern "C" __global__ void __launch_bounds__(256)
tiler_widen_bf16_f32(const uint16_t* __restrict__ x, uint64_t n, float* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = __uint_as_float((uint32_t)x[i] << 16);
}
