// Strict row folds: RMS normalization and softmax whose exponent sum (and
// RMSNorm's sum of squares) is the reference's serial left fold itself --
// the realization for a region whose contract grants no reassociation
// (ReductionTopology::Serial with permits_reassociation false,
// tiler-ir/src/schedule/model.rs:1330-1340; SquaredSerialSumThenEpilogue is
// serial-only, model.rs:780-800).  Bit-exact with
// tiler-reference/src/rms_norm.rs:134-195, 453-489 and softmax.rs:237-315.
//
// One wave64 per row.  The row is taken in segments of 1024 elements: every
// lane computes its elements' contributor values (fl(x^2), or
// certified exp(fl(x - m))) in parallel into the wave's LDS segment, then
// lane 0 folds the segment in ascending position (16-byte LDS reads, one
// dependent add per element).  The softmax maximum is order-insensitive
// (model.rs:906-912), so the wave computes it with a butterfly.  The
// epilogue (scale or reciprocal multiply, weight, narrowing) runs on every
// lane and re-reads the row.
#include "common.h"

namespace {

constexpr uint32_t kStrictSeg = 1024;
constexpr uint32_t kStrictWaves = 4;

template <bool kBf16>
__device__ __forceinline__ float load_elem(const void* __restrict__ p, uint64_t i) {
  return kBf16 ? tiler::bf16_widen(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

template <bool kBf16>
__device__ __forceinline__ void store_elem(void* __restrict__ p, uint64_t i, float v) {
  if (kBf16) static_cast<uint16_t*>(p)[i] = (uint16_t)tiler::bf16_narrow(v);
  else static_cast<float*>(p)[i] = v;
}

// Lane 0's strict fold of seg[0 .. len) onto acc (seeded: acc is the value
// so far, or the first contributor when `seeded` is false).
__device__ __forceinline__ float fold_segment(const float* seg, uint32_t len, float acc, bool& seeded) {
  uint32_t i = 0;
  if (!seeded && len) {
    acc = seg[0];
    seeded = true;
    i = 1;
  }
  for (; i < (len & ~3u) && (i & 3u); ++i) acc = acc + seg[i];
  for (; i + 4 <= len; i += 4) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(seg + i);
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
  }
  for (; i < len; ++i) acc = acc + seg[i];
  return acc;
}

template <bool kBf16>
__device__ __forceinline__ void rms_strict_body(const void* __restrict__ x, const void* __restrict__ w,
                                                uint64_t w_row_stride, void* __restrict__ y, uint64_t rows,
                                                uint32_t extent, float eps) {
  __shared__ __attribute__((aligned(16))) float seg[kStrictWaves][kStrictSeg];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint64_t row = (uint64_t)blockIdx.x * kStrictWaves + wave;
  if (row >= rows) return;
  const uint64_t base = row * extent;
  float acc = 0.0f;
  bool seeded = false;
  for (uint32_t s0 = 0; s0 < extent; s0 += kStrictSeg) {
    const uint32_t len = extent - s0 < kStrictSeg ? extent - s0 : kStrictSeg;
    for (uint32_t i = lane; i < len; i += 64) {
      const float v = load_elem<kBf16>(x, base + s0 + i);
      seg[wave][i] = v * v;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes landed
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) acc = fold_segment(seg[wave], len, acc, seeded);
    __builtin_amdgcn_wave_barrier();
  }
  // rms_norm.rs:177-187: a division by N, then + eps, then the certified rsqrt.
  float s = 0.0f;
  if (lane == 0) {
    const float mean = acc / (float)extent;
    s = tiler::rsqrt_f32_cr(mean + eps);
  }
  s = __shfl(s, 0, 64);
  const uint64_t wbase = row * w_row_stride;
  for (uint32_t i = lane; i < extent; i += 64) {
    const float normalized = load_elem<kBf16>(x, base + i) * s;
    store_elem<kBf16>(y, base + i, tiler::canon(load_elem<kBf16>(w, wbase + i) * normalized));
  }
}

__device__ __forceinline__ void softmax_strict_body(const float* __restrict__ x, float* __restrict__ y,
                                                    uint64_t rows, uint32_t extent) {
  __shared__ __attribute__((aligned(16))) float seg[kStrictWaves][kStrictSeg];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint64_t row = (uint64_t)blockIdx.x * kStrictWaves + wave;
  if (row >= rows) return;
  const float* xr = x + row * extent;
  float* yr = y + row * extent;
  float m = -__builtin_huge_valf();  // the maximum's two-sided identity
  for (uint32_t i = lane; i < extent; i += 64) m = tiler::maximum_f32(m, xr[i]);
  m = tiler::wave_max(m);
  float d = 0.0f;
  bool seeded = false;
  for (uint32_t s0 = 0; s0 < extent; s0 += kStrictSeg) {
    const uint32_t len = extent - s0 < kStrictSeg ? extent - s0 : kStrictSeg;
    for (uint32_t i = lane; i < len; i += 64) seg[wave][i] = tiler::exp_f32_cr(xr[s0 + i] - m);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) d = fold_segment(seg[wave], len, d, seeded);
    __builtin_amdgcn_wave_barrier();
  }
  float r = 0.0f;
  if (lane == 0) r = 1.0f / d;  // softmax.rs:302-313: the reciprocal, then a multiply
  r = __shfl(r, 0, 64);
  for (uint32_t i = lane; i < extent; i += 64) yr[i] = tiler::canon(tiler::exp_f32_cr(xr[i] - m) * r);
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
tiler_rms_norm_f32_strict(const float* __restrict__ x, const float* __restrict__ w, uint64_t w_row_stride,
                          float* __restrict__ y, uint64_t rows, uint32_t extent, float eps) {
  rms_strict_body<false>(x, w, w_row_stride, y, rows, extent, eps);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_rms_norm_bf16_strict(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                           uint64_t w_row_stride, uint16_t* __restrict__ y, uint64_t rows, uint32_t extent,
                           float eps) {
  rms_strict_body<true>(x, w, w_row_stride, y, rows, extent, eps);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_softmax_f32_strict(const float* __restrict__ x, float* __restrict__ y, uint64_t rows, uint32_t extent) {
  softmax_strict_body(x, y, rows, extent);
}
