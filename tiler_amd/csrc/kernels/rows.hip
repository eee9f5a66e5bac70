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

// The bf16 row runs in three phases so a workgroup can issue its rows' HBM
// loads before anything else (staging the weight, the barrier) and fold them
// while the weight arrives.  Chunk c of lane l covers positions
// [c*512 + l*8, +8); x stays packed (4 VGPRs per chunk) from load to epilogue.
// AL: 2 every chunk whole (extent == CH*512, no guards), 1 aligned rows,
// 0 unaligned (element loads, same order).
template <int CH, int AL>
__device__ __forceinline__ void rms_bf16_load(u32x4 (&xv)[CH], const uint16_t* __restrict__ x,
                                              uint32_t extent, uint32_t lane) {
  const uint32_t nfull = AL == 2 ? CH : AL ? extent >> 9 : 0;  // chunks loaded as whole 16 B
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
}

// This lane's strict fold of fl(x^2) in ascending position.
template <int CH, int AL>
__device__ __forceinline__ float rms_bf16_fold(u32x4 (&xv)[CH], uint32_t extent, uint32_t lane) {
  const uint32_t nfull = AL == 2 ? CH : AL ? extent >> 9 : 0;
  float acc = -0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 512u + lane * 8u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if ((uint32_t)c < nfull || p0 + e < extent) {
        float v = bf16_widen((xv[c][e >> 1] >> (16 * (e & 1))) & 0xffffu);
        float sq = v * v;
        acc = acc + sq;
      }
    }
  }
  // Opaque to the optimizer: the epilogue re-widens from the packed words
  // instead of keeping 8*CH widened floats live across the butterfly.
#pragma unroll
  for (int c = 0; c < CH; ++c) asm volatile("" : "+v"(xv[c]));
  return acc;
}

// Wave combine, scale, and y = fl(w * fl(x * s)) narrowed to bf16.
template <int CH, int AL>
__device__ __forceinline__ void rms_bf16_epilogue(const u32x4 (&xv)[CH], float acc,
                                                  const uint16_t* __restrict__ w,
                                                  uint16_t* __restrict__ y, uint32_t extent,
                                                  float eps, uint32_t lane) {
  const uint32_t nfull = AL == 2 ? CH : AL ? extent >> 9 : 0;
  float total = tiler::wave_sum_butterfly(acc);
  float mean = total / (float)extent;
  float s = tiler::rsqrt_f32_cr(mean + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 512u + lane * 8u;
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
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float x0 = bf16_widen(xv[c][h] & 0xffffu), x1 = bf16_widen(xv[c][h] >> 16);
      float w0 = bf16_widen(wv[h] & 0xffffu), w1 = bf16_widen(wv[h] >> 16);
      float n0 = x0 * s, n1 = x1 * s;
      float y0 = w0 * n0, y1 = w1 * n1;
      o[h] = tiler::bf16_pack2(y0, y1);
    }
    if ((uint32_t)c < nfull) {
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(y + p0));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p0 + e < extent) y[p0 + e] = (uint16_t)(o[e >> 1] >> (16 * (e & 1)));
    }
  }
}

template <int CH, int AL>
__device__ __forceinline__ void rms_f32_row(const float* __restrict__ x,
                                            const float* __restrict__ w, float* __restrict__ y,
                                            uint32_t extent, float eps, uint32_t lane) {
  // chunk c covers positions [c*256 + lane*4, +4)
  f32x4 xv[CH];
  const uint32_t nfull = AL == 2 ? CH : AL ? extent >> 8 : 0;
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
template <int CH, int AL>
__device__ __forceinline__ void softmax_f32_load(f32x4 (&xv)[CH], const float* __restrict__ x,
                                                 uint32_t extent, uint32_t lane) {
  const uint32_t nfull = AL == 2 ? CH : AL ? extent >> 8 : 0;
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
}

// The row maximum.  -inf is the maximum's identity on every operand (including
// -inf itself), so the padding the load put past the row's end is inert.
template <int CH>
__device__ __forceinline__ float softmax_f32_max(const f32x4 (&xv)[CH]) {
  float m = -__builtin_huge_valf();
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    m = tiler::maximum_f32(m, xv[c].x);
    m = tiler::maximum_f32(m, xv[c].y);
    m = tiler::maximum_f32(m, xv[c].z);
    m = tiler::maximum_f32(m, xv[c].w);
  }
  return tiler::wave_max(m);
}

template <int CH, int AL>
__device__ __forceinline__ void softmax_f32_finish(f32x4 (&xv)[CH], float m, float* __restrict__ y,
                                                   uint32_t extent, uint32_t lane,
                                                   const double* exp_table) {
  const uint32_t nfull = AL == 2 ? CH : AL ? extent >> 8 : 0;
  float acc = -0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t p0 = c * 256u + lane * 4u;
    float v4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bool live = (uint32_t)c < nfull || p0 + e < extent;
      float ex = tiler::exp_f32_cr_nonpositive(v4[e] - m, exp_table);  // m is the IEEE maximum: x - m <= 0 or NaN
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
// row; the host picks the instance.  The _full instances serve rows of exactly
// CH whole chunks with no guards; the plain instances load whole 16-byte chunks
// and need every row 16-byte aligned (aligned base, extent*elem % 16 == 0);
// the _u instances load element by element in the same order.
// bf16 RMSNorm workgroups are four waves (one row each).  Each wave issues its
// row's loads first; with a broadcast weight (w_row_stride 0) and aligned rows
// the weight row is then staged once per workgroup in LDS (up to 8192 bf16)
// while those loads are in flight, the row is folded, and the barrier before
// the epilogue publishes the staged weight.
#define TILER_RMS_BF16(CH, AL, SFX)                                                         \
  extern "C" __global__ void __launch_bounds__(256) tiler_rms_norm_bf16_ch##CH##SFX(            \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint64_t w_row_stride, \
      uint16_t* __restrict__ y, uint64_t rows, uint32_t extent, float eps) {                 \
    __shared__ __attribute__((aligned(16))) uint16_t wl[AL ? CH * 512 : 8];                \
    const uint64_t row = (uint64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);       \
    const uint32_t lane = threadIdx.x & 63u;                                                \
    const bool active = row < rows;                                                         \
    const bool stage = AL && w_row_stride == 0;                                             \
    u32x4 xv[CH];                                                                           \
    if (active) rms_bf16_load<CH, AL>(xv, x + row * extent, extent, lane);                 \
    if (stage) {                                                                            \
      for (uint32_t i = threadIdx.x; i * 8u < extent; i += blockDim.x)                    \
        *reinterpret_cast<u32x4*>(wl + i * 8u) = *reinterpret_cast<const u32x4*>(w + i * 8u); \
    }                                                                                       \
    float acc = active ? rms_bf16_fold<CH, AL>(xv, extent, lane) : 0.0f;                   \
    if (stage) __syncthreads();                                                             \
    if (!active) return;                                                                    \
    rms_bf16_epilogue<CH, AL>(xv, acc, stage ? wl : w + row * w_row_stride, y + row * extent, \
                              extent, eps, lane);                                           \
  }
TILER_RMS_BF16(1, 2, _full)
TILER_RMS_BF16(1, 1, )
TILER_RMS_BF16(1, 0, _u)
TILER_RMS_BF16(2, 2, _full)
TILER_RMS_BF16(2, 1, )
TILER_RMS_BF16(2, 0, _u)
TILER_RMS_BF16(4, 2, _full)
TILER_RMS_BF16(4, 1, )
TILER_RMS_BF16(4, 0, _u)
TILER_RMS_BF16(8, 2, _full)
TILER_RMS_BF16(8, 1, )
TILER_RMS_BF16(8, 0, _u)
TILER_RMS_BF16(16, 2, _full)
TILER_RMS_BF16(16, 1, )
TILER_RMS_BF16(16, 0, _u)

#define TILER_RMS_F32(CH, AL, SFX)                                                          \
  extern "C" __global__ void __launch_bounds__(256) tiler_rms_norm_f32_ch##CH##SFX(              \
      const float* __restrict__ x, const float* __restrict__ w, uint64_t w_row_stride,       \
      float* __restrict__ y, uint64_t rows, uint32_t extent, float eps) {                    \
    uint64_t row = (uint64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);             \
    if (row >= rows) return;                                                                \
    rms_f32_row<CH, AL>(x + row * extent, w + row * w_row_stride, y + row * extent, extent, eps, \
                    threadIdx.x & 63u);                                                     \
  }
TILER_RMS_F32(1, 2, _full)
TILER_RMS_F32(1, 1, )
TILER_RMS_F32(1, 0, _u)
TILER_RMS_F32(2, 2, _full)
TILER_RMS_F32(2, 1, )
TILER_RMS_F32(2, 0, _u)
TILER_RMS_F32(4, 2, _full)
TILER_RMS_F32(4, 1, )
TILER_RMS_F32(4, 0, _u)
TILER_RMS_F32(8, 2, _full)
TILER_RMS_F32(8, 1, )
TILER_RMS_F32(8, 0, _u)
TILER_RMS_F32(16, 2, _full)
TILER_RMS_F32(16, 1, )
TILER_RMS_F32(16, 0, _u)
TILER_RMS_F32(32, 2, _full)
TILER_RMS_F32(32, 1, )
TILER_RMS_F32(32, 0, _u)

// Softmax workgroups also issue their rows' loads first and stage the 64-entry
// exp table in LDS while those loads are in flight.
#define TILER_SOFTMAX_F32(CH, AL, SFX)                                                      \
  extern "C" __global__ void __launch_bounds__(256) tiler_softmax_f32_ch##CH##SFX(               \
      const float* __restrict__ x, float* __restrict__ y, uint64_t rows, uint32_t extent) {  \
    __shared__ double tab[64];                                                              \
    const uint64_t row = (uint64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);       \
    const uint32_t lane = threadIdx.x & 63u;                                                \
    const bool active = row < rows;                                                         \
    f32x4 xv[CH];                                                                           \
    if (active) softmax_f32_load<CH, AL>(xv, x + row * extent, extent, lane);              \
    if (threadIdx.x < 64) tab[threadIdx.x] = kExp2Table64[threadIdx.x];                     \
    const float m = active ? softmax_f32_max<CH>(xv) : 0.0f;                               \
    __syncthreads();                                                                        \
    if (!active) return;                                                                    \
    softmax_f32_finish<CH, AL>(xv, m, y + row * extent, extent, lane, tab);                \
  }
TILER_SOFTMAX_F32(1, 2, _full)
TILER_SOFTMAX_F32(1, 1, )
TILER_SOFTMAX_F32(1, 0, _u)
TILER_SOFTMAX_F32(2, 2, _full)
TILER_SOFTMAX_F32(2, 1, )
TILER_SOFTMAX_F32(2, 0, _u)
TILER_SOFTMAX_F32(4, 2, _full)
TILER_SOFTMAX_F32(4, 1, )
TILER_SOFTMAX_F32(4, 0, _u)
TILER_SOFTMAX_F32(8, 2, _full)
TILER_SOFTMAX_F32(8, 1, )
TILER_SOFTMAX_F32(8, 0, _u)
TILER_SOFTMAX_F32(16, 2, _full)
TILER_SOFTMAX_F32(16, 1, )
TILER_SOFTMAX_F32(16, 0, _u)
TILER_SOFTMAX_F32(32, 2, _full)
TILER_SOFTMAX_F32(32, 1, )
TILER_SOFTMAX_F32(32, 0, _u)
