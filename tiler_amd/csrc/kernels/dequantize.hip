// Strict per-tensor affine U4 -> binary32 dequantization
// (ScalarProgram::StrictAffineU4Dequantize, tiler-ir/src/schedule/model.rs:682-696;
// tiler-reference/src/quantization.rs:218-246, :409-419).
//
// Codes arrive packed U4, LSB-first, in U8 carriers with a zero tail: element
// i is nibble i % 2 of byte i / 2 (low nibble first).  The scale is one
// positive normal binary32 and the zero point one U8 carrier whose value lies
// in 0..=15.  Each element is fl((code - zero_point) * scale): the difference
// is an exact small integer, so the one multiply is the only rounding; the
// zero point's own code gives (+0) * scale = +0.0, which is the reference's
// +0.0 special case because the scale is positive.  Overflow to +-inf follows
// the IEEE product.  No subnormal can arise (|difference| >= 1 and the scale
// is normal), so the declared subnormal modes have nothing to act on.
//
// An HBM stream: 0.5 B read and 4 B written per element.  The wave-block
// form (_w) takes whole 2048-element blocks with 16-byte code loads; the
// vector form moves four elements per chunk (a 2-byte carrier load, one
// 16-byte store), two chunks in flight per lane, each wave's loads and
// stores contiguous; the scalar form serves unaligned storage and tails.
//
// The *_slots forms are the realized region's: the scale and the zero point
// are read from their own slots and checked against their domains there (the
// value contract, quantization.rs:318-370).  Workgroup 0's first lane writes
// the verdict to `record` on every launch (0 in domain, 1 scale, 2 zero
// point); out of domain, nothing is written to the output.
#include "common.h"

namespace {

// 0 when the scale is a positive normal binary32 and the zero point a U4 code.
__device__ __forceinline__ uint32_t strict_affine_domain(uint32_t scale_bits, uint32_t zero_point) {
  const uint32_t biased = (scale_bits >> 23) & 0xffu;
  if ((scale_bits >> 31) != 0u || biased == 0u || biased == 0xffu) return 1u;
  if (zero_point > 15u) return 2u;
  return 0u;
}

__device__ __forceinline__ float decode(uint32_t code, int32_t zero_point, float scale) {
  return (float)((int32_t)code - zero_point) * scale;
}

// Four elements from two carriers (one 16-bit load).
__device__ __forceinline__ f32x4 decode4(uint32_t w, int32_t zp, float scale) {
  return f32x4{decode(w & 15u, zp, scale), decode((w >> 4) & 15u, zp, scale), decode((w >> 8) & 15u, zp, scale),
               decode((w >> 12) & 15u, zp, scale)};
}

// n4 chunks of four elements: chunk g is carriers 2g, 2g+1 (one 16-bit load)
// and y's 16 bytes at 16g.  Lane t takes chunks t and t + S of each round (S
// the grid's lanes), so every load and every store of a wave is one
// contiguous run with two chunks in flight per lane; the host launches a
// grid that covers the tensor in one round.  Measured at 2^28 elements: two
// chunks per lane over the whole tensor 206 us, one 227 us, four (a capped
// grid) 247 us; plain stores ran at or above non-temporal ones here, and a
// pure 1 GiB write stream at 158 us is the floor.
__device__ __forceinline__ void dequantize_v4_body(const uint16_t* __restrict__ codes, uint64_t n4,
                                                   float scale, int32_t zp, f32x4* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; g < n4; g += 2 * stride) {
    uint32_t w[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint64_t c = g + (uint64_t)q * stride;
      w[q] = c < n4 ? (uint32_t)__builtin_nontemporal_load(&codes[c]) : 0u;
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint64_t c = g + (uint64_t)q * stride;
      if (c < n4) y[c] = decode4(w[q], zp, scale);
    }
  }
}

// Whole wave blocks of 2048 elements (1 KiB of codes, 8 KiB of y): each lane
// loads 16 bytes of codes, and the wave writes eight contiguous 1 KiB runs.
// Run j's lane t holds chunk 64 j + t, whose two carriers are code bytes
// 128 j + 2 t .. +1 of the block: bytes 2 (t % 8) .. +1 of lane 8 j + t / 8's
// load, taken with one cross-lane read per 32-bit word.  Measured at 2^28
// elements: 204-209 us against 231 us for the two-chunk form, whose 2-byte
// code loads take eight times the load instructions.
__device__ __forceinline__ void dequantize_block_body(const u32x4* __restrict__ codes, uint64_t blocks, float scale,
                                                      int32_t zp, f32x4* __restrict__ y) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t b = (uint64_t)blockIdx.x * (blockDim.x / 64u) + (threadIdx.x >> 6);
  if (b >= blocks) return;
  const u32x4 w = __builtin_nontemporal_load(&codes[b * 64u + lane]);
  f32x4* out = y + b * 512u;
  const uint32_t word = (lane & 7u) >> 1;
  const bool high = lane & 1u;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int src = 8 * j + (int)(lane >> 3);
    const uint32_t v0 = __shfl(w.x, src, 64), v1 = __shfl(w.y, src, 64);
    const uint32_t v2 = __shfl(w.z, src, 64), v3 = __shfl(w.w, src, 64);
    const uint32_t sel = word == 0 ? v0 : word == 1 ? v1 : word == 2 ? v2 : v3;
    out[64u * j + lane] = decode4(high ? sel >> 16 : sel & 0xffffu, zp, scale);
  }
}

// Elements [first, first + n) of the packed tensor, one per lane.
__device__ __forceinline__ void dequantize_scalar_body(const uint8_t* __restrict__ codes, uint64_t first,
                                                       uint64_t n, float scale, int32_t zp,
                                                       float* __restrict__ y) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride) {
    const uint64_t i = first + j;
    const uint32_t code = ((uint32_t)codes[i >> 1] >> ((uint32_t)(i & 1u) * 4u)) & 15u;
    y[i] = decode(code, zp, scale);
  }
}

// The realized forms' scalar operands: read, checked, the verdict recorded.
__device__ __forceinline__ bool read_operands(const uint32_t* __restrict__ scale_slot,
                                              const uint8_t* __restrict__ zero_slot,
                                              uint32_t* __restrict__ record, float& scale, int32_t& zp) {
  const uint32_t bits = *scale_slot, z = *zero_slot;
  const uint32_t verdict = strict_affine_domain(bits, z);
  if (blockIdx.x == 0 && threadIdx.x == 0) *record = verdict;
  scale = __uint_as_float(bits);
  zp = (int32_t)z;
  return verdict == 0u;
}

}  // namespace

// Direct forms: the host checked the scale and zero point before commit.
extern "C" __global__ void __launch_bounds__(256)
tiler_dequantize_u4_f32_v4(const uint16_t* __restrict__ codes, uint64_t n4, uint32_t scale_bits,
                           uint32_t zero_point, f32x4* __restrict__ y) {
  dequantize_v4_body(codes, n4, __uint_as_float(scale_bits), (int32_t)zero_point, y);
}

extern "C" __global__ void __launch_bounds__(256)
tiler_dequantize_u4_f32_w(const u32x4* __restrict__ codes, uint64_t blocks, uint32_t scale_bits, uint32_t zero_point,
                          f32x4* __restrict__ y) {
  dequantize_block_body(codes, blocks, __uint_as_float(scale_bits), (int32_t)zero_point, y);
}

extern "C" __global__ void __launch_bounds__(256)
tiler_dequantize_u4_f32(const uint8_t* __restrict__ codes, uint64_t first, uint64_t n, uint32_t scale_bits,
                        uint32_t zero_point, float* __restrict__ y) {
  dequantize_scalar_body(codes, first, n, __uint_as_float(scale_bits), (int32_t)zero_point, y);
}

// Realized forms: the scale and zero point from their slots.
extern "C" __global__ void __launch_bounds__(256)
tiler_dequantize_u4_f32_v4_slots(const uint16_t* __restrict__ codes, uint64_t n4,
                                 const uint32_t* __restrict__ scale_slot, const uint8_t* __restrict__ zero_slot,
                                 f32x4* __restrict__ y, uint32_t* __restrict__ record) {
  float scale;
  int32_t zp;
  if (read_operands(scale_slot, zero_slot, record, scale, zp)) dequantize_v4_body(codes, n4, scale, zp, y);
}

extern "C" __global__ void __launch_bounds__(256)
tiler_dequantize_u4_f32_w_slots(const u32x4* __restrict__ codes, uint64_t blocks,
                                const uint32_t* __restrict__ scale_slot, const uint8_t* __restrict__ zero_slot,
                                f32x4* __restrict__ y, uint32_t* __restrict__ record) {
  float scale;
  int32_t zp;
  if (read_operands(scale_slot, zero_slot, record, scale, zp)) dequantize_block_body(codes, blocks, scale, zp, y);
}

extern "C" __global__ void __launch_bounds__(256)
tiler_dequantize_u4_f32_slots(const uint8_t* __restrict__ codes, uint64_t n,
                              const uint32_t* __restrict__ scale_slot, const uint8_t* __restrict__ zero_slot,
                              float* __restrict__ y, uint32_t* __restrict__ record) {
  float scale;
  int32_t zp;
  if (read_operands(scale_slot, zero_slot, record, scale, zp)) dequantize_scalar_body(codes, 0, n, scale, zp, y);
}
