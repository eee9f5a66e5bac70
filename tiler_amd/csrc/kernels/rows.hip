// Row-wise fold-with-epilogue realizations for gfx950: RMS normalization
// (tiler-reference/src/rms_norm.rs:134-195, 453-489; staged law
// tiler-ir/src/index/law.rs:200-236) and softmax with the governed-maximum
// shift (tiler-reference/src/softmax.rs:237-315; law.rs:238-289).
//
// One wave64 per row, rows resident in registers between the fold and the
// epilogue, so every element is read from HBM once and written once.  Lane l
// holds the 16-byte chunks c*64 + l of its row (c = 0..CH-1): each load
// instruction of the wave covers 1 KiB of contiguous row, fully coalesced.
// Per lane the contributors are folded in ascending position, then the wave
// combines lanes with an xor butterfly: the declared grouping (vec = elements
// per 16 bytes, waves = 1) the oracle restates.
#include "common.h"

using tiler::bf16_narrow;
using tiler::bf16_widen;
using tiler::canon;

namespace {

constexpr uint32_t kWavesPerBlock = 4;

// ---------------------------------------------------------------------------
// RMS normalization.  s = rsqrt(fl(fl(sum fl(x^2)) / N) + eps) with the sum in
// the declared grouping and a true division by N; y = fl(w * fl(x * s)),
// narrowed to bf16 for bf16 storage (ADR 0091 narrowing).  The weight is
// either one row broadcast over all rows (w_row_stride 0) or a full tensor.

template <int CH, bool AL>
__device__ __forceinline__ void rms_bf16_row(const uint16_t* __restrict__ x,
                                             const uint16_t* __restrict__ w,
                                             uint16_t* __restrict__ y, uint32_t extent,
                                             float eps, uint32_t lane) {
  // chunk c covers positions [c*512 + lane*8, +8)
  u32x4 xv[CH];
  const uint32_t nfull = AL ? extent >> 9 : 0;  // chunks loaded as whole 16 B
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 512u + lane * 8u;
    if ((uint32_t)c < nfull) {
      xv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + p0));
    } else {
      uint32_t tmp[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p0 + e < extent) tmp[e >> 1] |= (uint32_t)x[p0 + e] << (16 * (e & 1));
      xv[c] = u32x4{tmp[0], tmp[1], tmp[2], tmp[3]};
    }
  }
  float acc = -0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 512u + lane * 8u;
    uint32_t words[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if ((uint32_t)c < nfull || p0 + e < extent) {
        float v = bf16_widen((words[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        float sq = v * v;
        acc = acc + sq;
      }
    }
  }
  float total = tiler::wave_sum_butterfly(acc);
  float mean = total / (float)extent;
  float s = tiler::rsqrt_f32_cr(mean + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 512u + lane * 8u;
    uint32_t words[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
    u32x4 wv;
    if ((uint32_t)c < nfull) {
      wv = *reinterpret_cast<const u32x4*>(w + p0);
    } else {
      uint32_t tmp[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p0 + e < extent) tmp[e >> 1] |= (uint32_t)w[p0 + e] << (16 * (e & 1));
      wv = u32x4{tmp[0], tmp[1], tmp[2], tmp[3]};
    }
    uint32_t wwords[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t out[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float x0 = bf16_widen(words[h] & 0xffffu), x1 = bf16_widen(words[h] >> 16);
      float w0 = bf16_widen(wwords[h] & 0xffffu), w1 = bf16_widen(wwords[h] >> 16);
      float n0 = x0 * s, n1 = x1 * s;
      float y0 = w0 * n0, y1 = w1 * n1;
      out[h] = tiler::bf16_pack2(y0, y1);
    }
    if ((uint32_t)c < nfull) {
      __builtin_nontemporal_store(u32x4{out[0], out[1], out[2], out[3]},
                                  reinterpret_cast<u32x4*>(y + p0));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p0 + e < extent) y[p0 + e] = (uint16_t)(out[e >> 1] >> (16 * (e & 1)));
    }
  }
}

template <int CH, bool AL>
__device__ __forceinline__ void rms_f32_row(const float* __restrict__ x,
                                            const float* __restrict__ w, float* __restrict__ y,
                                            uint32_t extent, float eps, uint32_t lane) {
  // chunk c covers positions [c*256 + lane*4, +4)
  f32x4 xv[CH];
  const uint32_t nfull = AL ? extent >> 8 : 0;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 256u + lane * 4u;
    if ((uint32_t)c < nfull) {
      xv[c] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + p0));
    } else {
      float tmp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (p0 + e < extent) tmp[e] = x[p0 + e];
      xv[c] = f32x4{tmp[0], tmp[1], tmp[2], tmp[3]};
    }
  }
  float acc = -0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 256u + lane * 4u;
    float v4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if ((uint32_t)c < nfull || p0 + e < extent) {
        float sq = v4[e] * v4[e];
        acc = acc + sq;
      }
  }
  float total = tiler::wave_sum_butterfly(acc);
  float mean = total / (float)extent;
  float s = tiler::rsqrt_f32_cr(mean + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 256u + lane * 4u;
    float v4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
    float w4[4] = {0.f, 0.f, 0.f, 0.f};
    if ((uint32_t)c < nfull) {
      f32x4 wv = *reinterpret_cast<const f32x4*>(w + p0);
      w4[0] = wv.x; w4[1] = wv.y; w4[2] = wv.z; w4[3] = wv.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (p0 + e < extent) w4[e] = w[p0 + e];
    }
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float n = v4[e] * s;
      o[e] = canon(w4[e] * n);
    }
    if ((uint32_t)c < nfull) {
      __builtin_nontemporal_store(f32x4{o[0], o[1], o[2], o[3]},
                                  reinterpret_cast<f32x4*>(y + p0));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (p0 + e < extent) y[p0 + e] = o[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Softmax over f32 rows: m = maximum fold (order-free: the IEEE maximum with
// -0 < +0 is associative and commutative, softmax/tests.rs:112-147);
// e = exp(fl(x - m)) correctly rounded; d = sum of e in the declared grouping;
// y = canon(fl(e * fl(1/d))) -- the reciprocal multiply, not a division.
template <int CH, bool AL>
__device__ __forceinline__ void softmax_f32_row(const float* __restrict__ x,
                                                float* __restrict__ y, uint32_t extent,
                                                uint32_t lane) {
  f32x4 xv[CH];
  const uint32_t nfull = AL ? extent >> 8 : 0;
  const float ninf = -__builtin_huge_valf();
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 256u + lane * 4u;
    if ((uint32_t)c < nfull) {
      xv[c] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + p0));
    } else {
      float tmp[4] = {ninf, ninf, ninf, ninf};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (p0 + e < extent) tmp[e] = x[p0 + e];
      xv[c] = f32x4{tmp[0], tmp[1], tmp[2], tmp[3]};
    }
  }
  // -inf is the maximum's identity on every operand (including -inf itself).
  float m = ninf;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    m = tiler::maximum_f32(m, xv[c].x);
    m = tiler::maximum_f32(m, xv[c].y);
    m = tiler::maximum_f32(m, xv[c].z);
    m = tiler::maximum_f32(m, xv[c].w);
  }
  m = tiler::wave_max(m);
  float acc = -0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 256u + lane * 4u;
    float v4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bool live = (uint32_t)c < nfull || p0 + e < extent;
      float ex = tiler::exp_f32_cr(v4[e] - m);
      v4[e] = ex;
      if (live) acc = acc + ex;
    }
    xv[c] = f32x4{v4[0], v4[1], v4[2], v4[3]};
  }
  float d = tiler::wave_sum_butterfly(acc);
  float r = 1.0f / d;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 256u + lane * 4u;
    float o[4] = {canon(xv[c].x * r), canon(xv[c].y * r), canon(xv[c].z * r),
                  canon(xv[c].w * r)};
    if ((uint32_t)c < nfull) {
      __builtin_nontemporal_store(f32x4{o[0], o[1], o[2], o[3]},
                                  reinterpret_cast<f32x4*>(y + p0));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (p0 + e < extent) y[p0 + e] = o[e];
    }
  }
}

}  // namespace

// Entry points: one 256-thread workgroup = 4 rows (one per wave).  CH is the
// number of 16-byte chunks per lane, the smallest power of two covering the
// row; the host picks the instance.  The plain instances load whole 16-byte
// chunks and need every row 16-byte aligned (aligned base, extent*elem % 16 ==
// 0); the _u instances load element by element in the same order.
#define TILER_RMS_BF16(CH, AL, SFX)                                                         \
  extern "C" __global__ void __launch_bounds__(256) tiler_rms_norm_bf16_ch##CH##SFX(             \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint64_t w_row_stride, \
      uint16_t* __restrict__ y, uint64_t rows, uint32_t extent, float eps) {                 \
    uint64_t row = (uint64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);             \
    if (row >= rows) return;                                                                \
    rms_bf16_row<CH, AL>(x + row * extent, w + row * w_row_stride, y + row * extent, extent,     \
                     eps, threadIdx.x & 63u);                                               \
  }
TILER_RMS_BF16(1, true, )
TILER_RMS_BF16(1, false, _u)
TILER_RMS_BF16(2, true, )
TILER_RMS_BF16(2, false, _u)
TILER_RMS_BF16(4, true, )
TILER_RMS_BF16(4, false, _u)
TILER_RMS_BF16(8, true, )
TILER_RMS_BF16(8, false, _u)
TILER_RMS_BF16(16, true, )
TILER_RMS_BF16(16, false, _u)

#define TILER_RMS_F32(CH, AL, SFX)                                                          \
  extern "C" __global__ void __launch_bounds__(256) tiler_rms_norm_f32_ch##CH##SFX(              \
      const float* __restrict__ x, const float* __restrict__ w, uint64_t w_row_stride,       \
      float* __restrict__ y, uint64_t rows, uint32_t extent, float eps) {                    \
    uint64_t row = (uint64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);             \
    if (row >= rows) return;                                                                \
    rms_f32_row<CH, AL>(x + row * extent, w + row * w_row_stride, y + row * extent, extent, eps, \
                    threadIdx.x & 63u);                                                     \
  }
TILER_RMS_F32(1, true, )
TILER_RMS_F32(1, false, _u)
TILER_RMS_F32(2, true, )
TILER_RMS_F32(2, false, _u)
TILER_RMS_F32(4, true, )
TILER_RMS_F32(4, false, _u)
TILER_RMS_F32(8, true, )
TILER_RMS_F32(8, false, _u)
TILER_RMS_F32(16, true, )
TILER_RMS_F32(16, false, _u)
TILER_RMS_F32(32, true, )
TILER_RMS_F32(32, false, _u)

#define TILER_SOFTMAX_F32(CH, AL, SFX)                                                      \
  extern "C" __global__ void __launch_bounds__(256) tiler_softmax_f32_ch##CH##SFX(               \
      const float* __restrict__ x, float* __restrict__ y, uint64_t rows, uint32_t extent) {  \
    uint64_t row = (uint64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);             \
    if (row >= rows) return;                                                                \
    softmax_f32_row<CH, AL>(x + row * extent, y + row * extent, extent, threadIdx.x & 63u);     \
  }
TILER_SOFTMAX_F32(1, true, )
TILER_SOFTMAX_F32(1, false, _u)
TILER_SOFTMAX_F32(2, true, )
TILER_SOFTMAX_F32(2, false, _u)
TILER_SOFTMAX_F32(4, true, )
TILER_SOFTMAX_F32(4, false, _u)
TILER_SOFTMAX_F32(8, true, )
TILER_SOFTMAX_F32(8, false, _u)
TILER_SOFTMAX_F32(16, true, )
TILER_SOFTMAX_F32(16, false, _u)
TILER_SOFTMAX_F32(32, true, )
TILER_SOFTMAX_F32(32, false, _u)
