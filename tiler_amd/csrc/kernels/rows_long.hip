// Long-row realizations of RMS normalization and softmax
// (tiler-reference/src/rms_norm.rs:134-195, 453-489; softmax.rs:237-315), for
// rows longer than one wave holds in registers (8192 elements).
//
// RMSNorm: one 1024-thread workgroup (16 waves) per row.  Thread t owns the
// 16-byte chunks t, t + 1024, t + 2048, ... of the row and folds their
// elements in ascending position; each wave combines its lanes with the xor
// butterfly and the 16 wave results are added in ascending wave order -- the
// declared grouping (vec = elements per chunk, waves = 16) the oracle
// restates.  CH > 0: the row's chunks stay in registers between passes (CH
// per thread, rows up to 1024 * CH chunks), so HBM sees each byte once.
// CH == 0: rows of any length are streamed (read twice: fold, epilogue).
//
// Softmax: the exponent sum folds by 8192-element segments (described at
// softmax_f32_seg_row), so a row can also be split across workgroups: one
// workgroup per row up to 4 segments, one per segment beyond (one
// row-synchronized launch, or three launches).
//
// AL: 1 when the row base and extent keep every chunk 16-byte aligned; 0 loads
// and stores element by element in the same order.
#include "common.h"

namespace {

constexpr uint32_t kLongThreads = 1024;
constexpr uint32_t kLongWaves = kLongThreads / 64;

// Strict ascending sum of the 16 wave results (every thread gets the total).
__device__ __forceinline__ float long_block_sum(float v, float* lds) {
  v = tiler::wave_sum_butterfly(v);
  const uint32_t t = threadIdx.x;
  if ((t & 63u) == 0) lds[t >> 6] = v;
  __syncthreads();
  float total = lds[0];
#pragma unroll
  for (uint32_t w = 1; w < kLongWaves; ++w) total = total + lds[w];
  __syncthreads();  // lds may be reused by the caller's next combine
  return total;
}

__device__ __forceinline__ float long_block_max(float v, float* lds) {
  v = tiler::wave_max(v);
  const uint32_t t = threadIdx.x;
  if ((t & 63u) == 0) lds[t >> 6] = v;
  __syncthreads();
  float m = lds[0];
#pragma unroll
  for (uint32_t w = 1; w < kLongWaves; ++w) m = tiler::maximum_f32(m, lds[w]);
  __syncthreads();
  return m;
}

// ---- chunk access --------------------------------------------------------
// bf16 chunk q = elements [8q, 8q+8); absent elements read as 0 (never folded).
template <int AL>
__device__ __forceinline__ u32x4 load_bf16_chunk(const uint16_t* __restrict__ x, uint64_t q,
                                                 uint32_t extent) {
  const uint64_t p0 = q * 8u;
  if (AL && p0 + 8u <= extent) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + p0));
  uint32_t tmp[4] = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (p0 + e < extent) tmp[e >> 1] |= (uint32_t)x[p0 + e] << (16 * (e & 1));
  return u32x4{tmp[0], tmp[1], tmp[2], tmp[3]};
}

template <int AL>
__device__ __forceinline__ void store_bf16_chunk(uint16_t* __restrict__ y, uint64_t q, uint32_t extent,
                                                 u32x4 v) {
  const uint64_t p0 = q * 8u;
  if (AL && p0 + 8u <= extent) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(y + p0));
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (p0 + e < extent) y[p0 + e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
}

// f32 chunk q = elements [4q, 4q+4); absent elements read as `pad`.
template <int AL>
__device__ __forceinline__ f32x4 load_f32_chunk(const float* __restrict__ x, uint64_t q, uint32_t extent,
                                                float pad) {
  const uint64_t p0 = q * 4u;
  if (AL && p0 + 4u <= extent) return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + p0));
  float tmp[4] = {pad, pad, pad, pad};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (p0 + e < extent) tmp[e] = x[p0 + e];
  return f32x4{tmp[0], tmp[1], tmp[2], tmp[3]};
}

template <int AL>
__device__ __forceinline__ void store_f32_chunk(float* __restrict__ y, uint64_t q, uint32_t extent, f32x4 v) {
  const uint64_t p0 = q * 4u;
  if (AL && p0 + 4u <= extent) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(y + p0));
    return;
  }
  const float o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (p0 + e < extent) y[p0 + e] = o[e];
}

// ---- RMSNorm, bf16 -----------------------------------------------------------
__device__ __forceinline__ float fold_sq_bf16(float acc, u32x4 v, uint64_t q, uint32_t extent) {
  const uint64_t p0 = q * 8u;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (p0 + e < extent) {
      float x = tiler::bf16_widen((v[e >> 1] >> (16 * (e & 1))) & 0xffffu);
      float sq = x * x;
      acc = acc + sq;
    }
  return acc;
}

__device__ __forceinline__ u32x4 rms_out_bf16(u32x4 xv, u32x4 wv, float s) {
  u32x4 o;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    float x0 = tiler::bf16_widen(xv[h] & 0xffffu), x1 = tiler::bf16_widen(xv[h] >> 16);
    float w0 = tiler::bf16_widen(wv[h] & 0xffffu), w1 = tiler::bf16_widen(wv[h] >> 16);
    float n0 = x0 * s, n1 = x1 * s;
    o[h] = tiler::bf16_pack2(w0 * n0, w1 * n1);
  }
  return o;
}

template <int CH, int AL>
__device__ __forceinline__ void rms_bf16_long_row(const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w,
                                                  uint16_t* __restrict__ y, uint32_t extent,
                                                  float eps, float* lds) {
  const uint32_t t = threadIdx.x;
  const uint64_t chunks = (extent + 7u) / 8u;
  float acc = -0.0f;
  u32x4 xv[CH > 0 ? CH : 1];
  if (CH > 0) {
#pragma unroll
    for (int c = 0; c < (CH > 0 ? CH : 1); ++c) {
      const uint64_t q = t + (uint64_t)c * kLongThreads;
      xv[c] = q < chunks ? load_bf16_chunk<AL>(x, q, extent) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int c = 0; c < (CH > 0 ? CH : 1); ++c) {
      const uint64_t q = t + (uint64_t)c * kLongThreads;
      if (q < chunks) acc = fold_sq_bf16(acc, xv[c], q, extent);
    }
  } else {
    for (uint64_t q = t; q < chunks; q += kLongThreads) acc = fold_sq_bf16(acc, load_bf16_chunk<AL>(x, q, extent), q, extent);
  }
  const float total = long_block_sum(acc, lds);
  const float s = tiler::rsqrt_f32_cr(total / (float)extent + eps);
  if (CH > 0) {
#pragma unroll
    for (int c = 0; c < (CH > 0 ? CH : 1); ++c) {
      const uint64_t q = t + (uint64_t)c * kLongThreads;
      if (q < chunks) store_bf16_chunk<AL>(y, q, extent, rms_out_bf16(xv[c], load_bf16_chunk<AL>(w, q, extent), s));
    }
  } else {
    for (uint64_t q = t; q < chunks; q += kLongThreads)
      store_bf16_chunk<AL>(y, q, extent, rms_out_bf16(load_bf16_chunk<AL>(x, q, extent), load_bf16_chunk<AL>(w, q, extent), s));
  }
}

// ---- RMSNorm, f32 ------------------------------------------------------------
__device__ __forceinline__ float fold_sq_f32(float acc, f32x4 v, uint64_t q, uint32_t extent) {
  const uint64_t p0 = q * 4u;
  const float e4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (p0 + e < extent) {
      float sq = e4[e] * e4[e];
      acc = acc + sq;
    }
  return acc;
}

__device__ __forceinline__ f32x4 rms_out_f32(f32x4 xv, f32x4 wv, float s) {
  return f32x4{tiler::canon(wv.x * (xv.x * s)), tiler::canon(wv.y * (xv.y * s)),
               tiler::canon(wv.z * (xv.z * s)), tiler::canon(wv.w * (xv.w * s))};
}

template <int CH, int AL>
__device__ __forceinline__ void rms_f32_long_row(const float* __restrict__ x, const float* __restrict__ w,
                                                 float* __restrict__ y, uint32_t extent, float eps,
                                                 float* lds) {
  const uint32_t t = threadIdx.x;
  const uint64_t chunks = (extent + 3u) / 4u;
  float acc = -0.0f;
  f32x4 xv[CH > 0 ? CH : 1];
  if (CH > 0) {
#pragma unroll
    for (int c = 0; c < (CH > 0 ? CH : 1); ++c) {
      const uint64_t q = t + (uint64_t)c * kLongThreads;
      xv[c] = q < chunks ? load_f32_chunk<AL>(x, q, extent, 0.0f) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int c = 0; c < (CH > 0 ? CH : 1); ++c) {
      const uint64_t q = t + (uint64_t)c * kLongThreads;
      if (q < chunks) acc = fold_sq_f32(acc, xv[c], q, extent);
    }
  } else {
    for (uint64_t q = t; q < chunks; q += kLongThreads)
      acc = fold_sq_f32(acc, load_f32_chunk<AL>(x, q, extent, 0.0f), q, extent);
  }
  const float total = long_block_sum(acc, lds);
  const float s = tiler::rsqrt_f32_cr(total / (float)extent + eps);
  if (CH > 0) {
#pragma unroll
    for (int c = 0; c < (CH > 0 ? CH : 1); ++c) {
      const uint64_t q = t + (uint64_t)c * kLongThreads;
      if (q < chunks) store_f32_chunk<AL>(y, q, extent, rms_out_f32(xv[c], load_f32_chunk<AL>(w, q, extent, 0.0f), s));
    }
  } else {
    for (uint64_t q = t; q < chunks; q += kLongThreads)
      store_f32_chunk<AL>(y, q, extent,
                          rms_out_f32(load_f32_chunk<AL>(x, q, extent, 0.0f), load_f32_chunk<AL>(w, q, extent, 0.0f), s));
  }
}

// ---- softmax, f32 ------------------------------------------------------------
__device__ __forceinline__ float max_chunk(float m, f32x4 v) {
  m = tiler::maximum_f32(m, v.x);
  m = tiler::maximum_f32(m, v.y);
  m = tiler::maximum_f32(m, v.z);
  return tiler::maximum_f32(m, v.w);
}

// m is the row's IEEE maximum, so fl(x - m) <= 0 or NaN for every element of
// the row (a padding lane's value past the row's end is never used).
__device__ __forceinline__ f32x4 exp_chunk(f32x4 v, float m, const double* tab) {
  return f32x4{tiler::exp_f32_cr_nonpositive(v.x - m, tab), tiler::exp_f32_cr_nonpositive(v.y - m, tab),
               tiler::exp_f32_cr_nonpositive(v.z - m, tab), tiler::exp_f32_cr_nonpositive(v.w - m, tab)};
}

__device__ __forceinline__ float fold_chunk(float acc, f32x4 e, uint64_t q, uint32_t extent) {
  const uint64_t p0 = q * 4u;
  const float e4[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (p0 + i < extent) acc = acc + e4[i];
  return acc;
}

__device__ __forceinline__ f32x4 scale_chunk(f32x4 e, float r) {
  return f32x4{tiler::canon(e.x * r), tiler::canon(e.y * r), tiler::canon(e.z * r), tiler::canon(e.w * r)};
}

// Softmax rows longer than 8192 elements fold their exponent sum by segments
// of kSegElems elements: lane l of a 256-thread group folds the segment's
// 16-byte chunks l, l + 256, ..., l + 1792 in ascending position, each wave
// combines its lanes with the butterfly, the segment's partial is its 4 wave
// results added in ascending order, and the row total is the left fold of the
// partials in ascending segment order (the grouping vec 4, waves 4, segment
// 8192 that tiler_hip_row_grouping reports).  The same fold is computed by one
// 1024-thread workgroup per row (rows of at most 4 segments, group g of 256
// threads takes segment g) and by one 256-thread workgroup per segment (the
// row-synchronized launch, or the split form's three launches), so which one
// runs never changes a bit.
constexpr uint32_t kSegThreads = 256;
constexpr uint32_t kSegChunks = 8;                                 // per lane per segment
constexpr uint64_t kSegChunkSpan = (uint64_t)kSegThreads * kSegChunks;  // 2048 chunks
constexpr uint64_t kSegElems = kSegChunkSpan * 4;                  // 8192 elements

// Folds the four group partials into `total` (groups g < `active` hold a
// segment) and returns it; every thread of the 1024 gets it.
__device__ __forceinline__ float seg_round_fold(float acc, uint32_t active, float* lds, float total) {
  acc = tiler::wave_sum_butterfly(acc);
  const uint32_t t = threadIdx.x;
  if ((t & 63u) == 0) lds[t >> 6] = acc;
  __syncthreads();
  for (uint32_t g = 0; g < active; ++g) {
    float p = lds[4 * g];
    p = p + lds[4 * g + 1];
    p = p + lds[4 * g + 2];
    p = p + lds[4 * g + 3];
    total = total + p;  // total starts at -0.0: the first add is exact
  }
  __syncthreads();
  return total;
}

// Chunks q0, q0 + 256, ..., q0 + 1792 of a row into registers, -inf past the
// row.  The padding is written before the (masked) load, never after it, so
// the 8 loads stay in flight together: a select or a second path writing the
// load's registers would make the compiler wait for each load in turn.  AL:
// the planner's _a condition (extent % 4 == 0, aligned base) makes every
// chunk below `chunks` whole.
template <int AL>
__device__ __forceinline__ void load_chunks(const float* __restrict__ x, uint64_t q0, uint64_t chunks,
                                            uint32_t extent, f32x4 (&xv)[kSegChunks]) {
  const float ninf = -__builtin_huge_valf();
#pragma unroll
  for (uint32_t c = 0; c < kSegChunks; ++c) {
    const uint64_t q = q0 + c * kSegThreads;
    xv[c] = f32x4{ninf, ninf, ninf, ninf};
    if (q < chunks) {
      if (AL) {
        xv[c] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + q * 4u));
      } else {
        const uint64_t p0 = q * 4u;
        if (p0 < extent) xv[c].x = x[p0];
        if (p0 + 1 < extent) xv[c].y = x[p0 + 1];
        if (p0 + 2 < extent) xv[c].z = x[p0 + 2];
        if (p0 + 3 < extent) xv[c].w = x[p0 + 3];
      }
    }
  }
}

// One 1024-thread workgroup per row of at most 4 segments: group g keeps
// segment g in registers between the passes, so x is read once.
template <int AL>
__device__ __forceinline__ void softmax_f32_seg_row(const float* __restrict__ x, float* __restrict__ y,
                                                    uint32_t extent, float* lds, double* tab) {
  const uint32_t t = threadIdx.x, g = t >> 8, l = t & 255u;
  const uint64_t chunks = (extent + 3u) / 4u;
  const uint32_t nseg = (uint32_t)((extent + kSegElems - 1) / kSegElems);  // <= 4 (the planner's choice)
  const float ninf = -__builtin_huge_valf();
  f32x4 xv[kSegChunks];
  float m = ninf;
  load_chunks<AL>(x, g * kSegChunkSpan + l, chunks, extent, xv);
  const double tv = kExp2Table64[t & 63u];  // the exponent table, filled after the row's loads are issued
#pragma unroll
  for (uint32_t c = 0; c < kSegChunks; ++c) m = max_chunk(m, xv[c]);
  if (t < 64) tab[t] = tv;
  m = long_block_max(m, lds);  // its barrier also publishes tab
  float acc = -0.0f;
#pragma unroll
  for (uint32_t c = 0; c < kSegChunks; ++c) {
    const uint64_t q = g * kSegChunkSpan + l + c * kSegThreads;
    xv[c] = exp_chunk(xv[c], m, tab);
    if (q < chunks) acc = fold_chunk(acc, xv[c], q, extent);
  }
  const float total = seg_round_fold(acc, nseg < 4 ? nseg : 4u, lds, -0.0f);
  const float r = 1.0f / total;
#pragma unroll
  for (uint32_t c = 0; c < kSegChunks; ++c) {
    const uint64_t q = g * kSegChunkSpan + l + c * kSegThreads;
    if (q < chunks) store_f32_chunk<AL>(y, q, extent, scale_chunk(xv[c], r));
  }
}

// ---- split form: one 256-thread workgroup per segment -------------------------
// Workgroup b takes segment b % nseg of row b / nseg (a flat grid, so any
// row count launches).
__device__ __forceinline__ float seg_block_max(float v, float* lds) {
  v = tiler::wave_max(v);
  const uint32_t t = threadIdx.x;
  if ((t & 63u) == 0) lds[t >> 6] = v;
  __syncthreads();
  float m = lds[0];
  m = tiler::maximum_f32(m, lds[1]);
  m = tiler::maximum_f32(m, lds[2]);
  m = tiler::maximum_f32(m, lds[3]);
  __syncthreads();
  return m;
}

// The row maximum from its segment maxima (the maximum is order-free), per
// wave: no barrier, so the segment's loads issued before it stay in flight.
__device__ __forceinline__ float row_max_of(const float* __restrict__ pmax, uint64_t nseg) {
  float m = -__builtin_huge_valf();
  for (uint64_t j = threadIdx.x & 63u; j < nseg; j += 64) m = tiler::maximum_f32(m, pmax[j]);
  return tiler::wave_max(m);
}

// The row's exponent sum: the left fold of its segment partials in ascending
// order, seeded by the first.  Each wave loads 64 partials at a time (one per
// lane) and folds them in lane order.
__device__ __forceinline__ float row_sum_of(const float* __restrict__ psum, uint64_t nseg) {
  const uint32_t lane = threadIdx.x & 63u;
  float d = -0.0f;  // -0.0 + p == p: the fold is seeded by the first partial
  for (uint64_t j0 = 0; j0 < nseg; j0 += 64) {
    const float v = j0 + lane < nseg ? psum[j0 + lane] : 0.0f;
    const uint32_t n = nseg - j0 < 64 ? (uint32_t)(nseg - j0) : 64u;
    for (uint32_t k = 0; k < n; ++k)
      d = d + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
  }
  return d;
}

template <int AL>
__device__ __forceinline__ void load_segment(const float* __restrict__ x, uint64_t sg, uint64_t chunks,
                                             uint32_t extent, f32x4 (&xv)[kSegChunks]) {
  load_chunks<AL>(x, sg * kSegChunkSpan + threadIdx.x, chunks, extent, xv);
}

// Split pass 1: pmax[row * nseg + s] = the maximum of segment s.
template <int AL>
__device__ __forceinline__ void softmax_split_max(const float* __restrict__ x, uint32_t extent, uint64_t nseg,
                                                  float* __restrict__ pmax) {
  __shared__ float lds[4];
  const uint64_t row = blockIdx.x / nseg, sg = blockIdx.x % nseg;
  const uint64_t chunks = (extent + 3u) / 4u;
  f32x4 xv[kSegChunks];
  load_segment<AL>(x + row * extent, sg, chunks, extent, xv);
  float m = -__builtin_huge_valf();
#pragma unroll
  for (uint32_t c = 0; c < kSegChunks; ++c) m = max_chunk(m, xv[c]);
  m = seg_block_max(m, lds);
  if (threadIdx.x == 0) pmax[row * nseg + sg] = m;
}

// Split pass 2: psum[row * nseg + s] = segment s's partial of the exponent sum.
template <int AL>
__device__ __forceinline__ void softmax_split_sum(const float* __restrict__ x, uint32_t extent, uint64_t nseg,
                                                  const float* __restrict__ pmax, float* __restrict__ psum,
                                                  double* tab) {
  __shared__ float lds[4];
  const uint64_t row = blockIdx.x / nseg, sg = blockIdx.x % nseg;
  const uint64_t chunks = (extent + 3u) / 4u;
  f32x4 xv[kSegChunks];
  load_segment<AL>(x + row * extent, sg, chunks, extent, xv);
  const double tv = kExp2Table64[threadIdx.x & 63u];  // filled after the segment's loads are issued
  const float m = row_max_of(pmax + row * nseg, nseg);
  if (threadIdx.x < 64) tab[threadIdx.x] = tv;
  __syncthreads();
  float acc = -0.0f;
#pragma unroll
  for (uint32_t c = 0; c < kSegChunks; ++c) {
    const uint64_t q = sg * kSegChunkSpan + threadIdx.x + c * kSegThreads;
    if (q < chunks) acc = fold_chunk(acc, exp_chunk(xv[c], m, tab), q, extent);
  }
  acc = tiler::wave_sum_butterfly(acc);
  if ((threadIdx.x & 63u) == 0) lds[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float p = lds[0];
    p = p + lds[1];
    p = p + lds[2];
    p = p + lds[3];
    psum[row * nseg + sg] = p;
  }
}

// Split pass 3: y = canon(exp(x - m) * (1 / d)), d the left fold of the row's
// partials in ascending segment order.
template <int AL>
__device__ __forceinline__ void softmax_split_out(const float* __restrict__ x, float* __restrict__ y,
                                                  uint32_t extent, uint64_t nseg, const float* __restrict__ pmax,
                                                  const float* __restrict__ psum, double* tab) {
  const uint64_t row = blockIdx.x / nseg, sg = blockIdx.x % nseg;
  const uint64_t chunks = (extent + 3u) / 4u;
  f32x4 xv[kSegChunks];
  load_segment<AL>(x + row * extent, sg, chunks, extent, xv);
  const double tv = kExp2Table64[threadIdx.x & 63u];  // filled after the segment's loads are issued
  const float m = row_max_of(pmax + row * nseg, nseg);
  const float r = 1.0f / row_sum_of(psum + row * nseg, nseg);
  if (threadIdx.x < 64) tab[threadIdx.x] = tv;
  __syncthreads();
  float* yr = y + row * extent;
#pragma unroll
  for (uint32_t c = 0; c < kSegChunks; ++c) {
    const uint64_t q = sg * kSegChunkSpan + threadIdx.x + c * kSegThreads;
    if (q < chunks) store_f32_chunk<AL>(yr, q, extent, scale_chunk(exp_chunk(xv[c], m, tab), r));
  }
}

// ---- row-synchronized form: one launch -----------------------------------------
// The split form's three passes in one kernel: each 256-thread workgroup keeps
// its segment in registers, publishes its segment maximum, reads every
// maximum of its row, publishes its segment partial and reads every partial
// of its row.  A published value is one 64-bit word, (tag << 32) | bits,
// written and polled with relaxed agent-scope atomics: a word is valid when
// its tag is this call's, so no ordering between locations (and no cache
// write-back) is needed.
// The epoch is a 64-bit word; a workgroup reads it (e) first and takes the
// call number c = e + 1, or e + 2 when the low 32 bits of e + 1 are zero;
// the tag is the low 32 bits of c, never 0 (the workspace's initial words).
// At its end a workgroup raises the epoch to c by an atomic maximum that
// nobody waits on -- segment 0 of each row, and any workgroup whose wait ran
// out.  Every tag a call publishes under is then at most the next call's
// epoch: a row whose workgroups agree on the tag has its segment 0 raise the
// epoch to it, and in a row whose workgroups read different epochs (one
// started after another workgroup of the call ended) no wait can complete,
// so every one of them raises the epoch to its own.  Tags so only repeat
// after 2^32 - 1 calls.  (A counter of arrivals that picks the last
// workgroup would serialize every workgroup on one address and put that on
// the kernel's critical path: 3.5 us of 20.5 at 32 x 131072.)
// A wait is bounded (`wait_ticks` of the 100 MHz real-time clock); a
// workgroup whose wait runs out computes the row maximum, or the row sum with
// the same segment fold, from the row itself, so results never depend on the
// workgroups being resident together -- only the speed does.
//
// sync: u64 epoch, pad to 256 bytes, then u64 words for the maxima
// [rows * nseg] and the partials [rows * nseg].
constexpr uint32_t kRowSyncHeaderBytes = 256;

// Wave 0 only: the row's nseg words of this call's tag, 64 per lane group in
// ascending order, combined into the row maximum (sum == false; order-free)
// or the left fold of the partials in ascending segment order (sum == true).
// Returns false when the wait bound runs out first.
__device__ __forceinline__ bool collect_row(const uint64_t* words, uint64_t nseg, uint32_t tag,
                                            uint64_t wait_ticks, bool sum, float* out) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t t0 = wall_clock64();
  float acc = sum ? -0.0f : -__builtin_huge_valf();  // -0.0 + p == p: seeded by the first
  for (uint64_t j0 = 0; j0 < nseg; j0 += 64) {
    const uint64_t j = j0 + lane;
    uint64_t v = 0;
    bool have = j >= nseg;
    while (true) {
      if (!have) {
        v = __hip_atomic_load(&words[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        have = (uint32_t)(v >> 32) == tag;
      }
      if (__all(have)) break;
      if (wall_clock64() - t0 >= wait_ticks) return false;
      __builtin_amdgcn_s_sleep(1);
    }
    const float val = __uint_as_float((uint32_t)v);
    if (sum) {
      const uint32_t n = nseg - j0 < 64 ? (uint32_t)(nseg - j0) : 64u;
      for (uint32_t k = 0; k < n; ++k)
        acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, val), k));
    } else {
      acc = tiler::maximum_f32(acc, tiler::wave_max(j < nseg ? val : -__builtin_huge_valf()));
    }
  }
  *out = acc;
  return true;
}

// The row maximum from the row itself (order-free), all 256 threads.
template <int AL>
__device__ __forceinline__ float row_max_direct(const float* __restrict__ xr, uint64_t chunks, uint32_t extent,
                                                float* lds) {
  const float ninf = -__builtin_huge_valf();
  float m = ninf;
  for (uint64_t q = threadIdx.x; q < chunks; q += kSegThreads) m = max_chunk(m, load_f32_chunk<AL>(xr, q, extent, ninf));
  return seg_block_max(m, lds);
}

// The row's exponent sum from the row itself: every segment's partial by the
// segment fold, left-folded in ascending order (all 256 threads get it).
template <int AL>
__device__ __forceinline__ float row_sum_direct(const float* __restrict__ xr, uint64_t chunks, uint32_t extent,
                                                uint64_t nseg, float m, float* lds, const double* tab) {
  float d = -0.0f;
  for (uint64_t j = 0; j < nseg; ++j) {
    f32x4 xv[kSegChunks];
    load_segment<AL>(xr, j, chunks, extent, xv);
    float acc = -0.0f;
#pragma unroll
    for (uint32_t c = 0; c < kSegChunks; ++c) {
      const uint64_t q = j * kSegChunkSpan + threadIdx.x + c * kSegThreads;
      if (q < chunks) acc = fold_chunk(acc, exp_chunk(xv[c], m, tab), q, extent);
    }
    acc = tiler::wave_sum_butterfly(acc);
    if ((threadIdx.x & 63u) == 0) lds[threadIdx.x >> 6] = acc;
    __syncthreads();
    float p = lds[0];
    p = p + lds[1];
    p = p + lds[2];
    p = p + lds[3];
    d = d + p;
    __syncthreads();
  }
  return d;
}

__device__ __forceinline__ uint64_t tagged(uint32_t tag, float v) {
  return ((uint64_t)tag << 32) | __float_as_uint(v);
}

// `tab` is filled here, after the segment's loads are issued, so the
// workgroup's first memory round trips overlap instead of queueing.
template <int AL>
__device__ __forceinline__ void softmax_rowsync(const float* __restrict__ x, float* __restrict__ y, uint32_t extent,
                                                uint64_t nseg, uint8_t* __restrict__ sync, uint64_t wait_ticks,
                                                double* tab) {
  __shared__ float lds[4];
  __shared__ uint32_t sh_ok, sh_late;
  __shared__ float sh_val;
  const uint32_t t = threadIdx.x;
  const uint64_t wgs = gridDim.x;
  const uint64_t row = blockIdx.x / nseg, sg = blockIdx.x % nseg;
  const uint64_t chunks = (extent + 3u) / 4u;
  const float* xr = x + row * extent;
  uint64_t* epoch = reinterpret_cast<uint64_t*>(sync);
  uint64_t* wmax = reinterpret_cast<uint64_t*>(sync + kRowSyncHeaderBytes) + row * nseg;
  uint64_t* wsum = reinterpret_cast<uint64_t*>(sync + kRowSyncHeaderBytes) + wgs + row * nseg;
  f32x4 xv[kSegChunks];
  load_segment<AL>(xr, sg, chunks, extent, xv);
  // Only wave 0 publishes and polls, so only its lanes need the epoch.
  const uint64_t e = t < 64 ? __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
  const double tv = kExp2Table64[t & 63u];
  float m = -__builtin_huge_valf();
#pragma unroll
  for (uint32_t i = 0; i < kSegChunks; ++i) m = max_chunk(m, xv[i]);
  if (t < 64) tab[t] = tv;
  if (t == 0) sh_late = 0;
  m = seg_block_max(m, lds);  // its barrier also publishes tab and sh_late
  const uint64_t call = (uint32_t)(e + 1) == 0u ? e + 2 : e + 1;
  const uint32_t tag = (uint32_t)call;
  if (t < 64) {
    if (t == 0) __hip_atomic_store(&wmax[sg], tagged(tag, m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float v;
    const bool ok = collect_row(wmax, nseg, tag, wait_ticks, false, &v);
    if (t == 0) {
      sh_ok = ok ? 1u : 0u;
      sh_late |= ok ? 0u : 1u;
      sh_val = v;
    }
  }
  __syncthreads();
  m = sh_ok ? sh_val : row_max_direct<AL>(xr, chunks, extent, lds);
  float acc = -0.0f;
#pragma unroll
  for (uint32_t i = 0; i < kSegChunks; ++i) {
    const uint64_t q = sg * kSegChunkSpan + t + i * kSegThreads;
    xv[i] = exp_chunk(xv[i], m, tab);
    if (q < chunks) acc = fold_chunk(acc, xv[i], q, extent);
  }
  acc = tiler::wave_sum_butterfly(acc);
  __syncthreads();  // every wave is past its reads of sh_ok, sh_val and lds
  if ((t & 63u) == 0) lds[t >> 6] = acc;
  __syncthreads();
  if (t < 64) {
    if (t == 0) {
      float p = lds[0];
      p = p + lds[1];
      p = p + lds[2];
      p = p + lds[3];
      __hip_atomic_store(&wsum[sg], tagged(tag, p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float v;
    const bool ok = collect_row(wsum, nseg, tag, wait_ticks, true, &v);
    if (t == 0) {
      sh_ok = ok ? 1u : 0u;
      sh_late |= ok ? 0u : 1u;
      sh_val = v;
    }
  }
  __syncthreads();
  const float d = sh_ok ? sh_val : row_sum_direct<AL>(xr, chunks, extent, nseg, m, lds, tab);
  const float r = 1.0f / d;
  float* yr = y + row * extent;
#pragma unroll
  for (uint32_t i = 0; i < kSegChunks; ++i) {
    const uint64_t q = sg * kSegChunkSpan + t + i * kSegThreads;
    if (q < chunks) store_f32_chunk<AL>(yr, q, extent, scale_chunk(xv[i], r));
  }
  if (t == 0 && (sg == 0 || sh_late)) __hip_atomic_fetch_max(epoch, call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// Entry points: blockIdx.x is the row; 1024 threads.  Instances CH in
// {1, 2, 4, 8} (register-resident) and 0 (streamed), each aligned (_a) and
// element-wise (_u).  RMSNorm weights are one broadcast row (w_row_stride 0)
// or a full tensor.
#define TILER_RMS_BF16_LONG(CH, AL, SFX)                                                        \
  extern "C" __global__ void __launch_bounds__(1024) tiler_rms_norm_bf16_long##CH##SFX(         \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint64_t w_row_stride,     \
      uint16_t* __restrict__ y, uint32_t extent, float eps) {                                    \
    __shared__ float lds[kLongWaves];                                                            \
    const uint64_t row = blockIdx.x;                                                             \
    rms_bf16_long_row<CH, AL>(x + row * extent, w + row * w_row_stride, y + row * extent, extent, \
                              eps, lds);                                                          \
  }
#define TILER_RMS_F32_LONG(CH, AL, SFX)                                                         \
  extern "C" __global__ void __launch_bounds__(1024) tiler_rms_norm_f32_long##CH##SFX(          \
      const float* __restrict__ x, const float* __restrict__ w, uint64_t w_row_stride,           \
      float* __restrict__ y, uint32_t extent, float eps) {                                       \
    __shared__ float lds[kLongWaves];                                                            \
    const uint64_t row = blockIdx.x;                                                             \
    rms_f32_long_row<CH, AL>(x + row * extent, w + row * w_row_stride, y + row * extent, extent, \
                             eps, lds);                                                           \
  }
#define TILER_LONG_FAMILY(M) M(1, 1, _a) M(1, 0, _u) M(2, 1, _a) M(2, 0, _u) M(4, 1, _a) M(4, 0, _u) \
  M(8, 1, _a) M(8, 0, _u) M(0, 1, _a) M(0, 0, _u)
TILER_LONG_FAMILY(TILER_RMS_BF16_LONG)
TILER_LONG_FAMILY(TILER_RMS_F32_LONG)

// Softmax rows longer than 8192 elements (the segmented fold above).
// tiler_softmax_f32_long_r{_a,_u}: blockIdx.x is the row, 1024 threads, rows
// of at most 4 segments.  tiler_softmax_f32_split_{max,sum,out}{_a,_u} and
// tiler_softmax_f32_rowsync{_a,_u}: a flat grid of rows * nseg workgroups of
// 256 threads; pmax and psum hold rows * nseg partials; sync is the
// row-synchronized form's area (header and 2 * rows * nseg words).
#define TILER_SOFTMAX_F32_SEG(AL, SFX)                                                                     \
  extern "C" __global__ void __launch_bounds__(1024) tiler_softmax_f32_long_r##SFX(                       \
      const float* __restrict__ x, float* __restrict__ y, uint32_t extent) {                              \
    __shared__ float lds[kLongWaves];                                                                     \
    __shared__ double tab[64];                                                                            \
    const uint64_t row = blockIdx.x;                                                                      \
    softmax_f32_seg_row<AL>(x + row * extent, y + row * extent, extent, lds, tab);                     \
  }                                                                                                       \
  extern "C" __global__ void __launch_bounds__(256) tiler_softmax_f32_split_max##SFX(                     \
      const float* __restrict__ x, uint32_t extent, uint64_t nseg, float* __restrict__ pmax) {            \
    softmax_split_max<AL>(x, extent, nseg, pmax);                                                         \
  }                                                                                                       \
  extern "C" __global__ void __launch_bounds__(256) tiler_softmax_f32_split_sum##SFX(                     \
      const float* __restrict__ x, uint32_t extent, uint64_t nseg, const float* __restrict__ pmax,        \
      float* __restrict__ psum) {                                                                         \
    __shared__ double tab[64];                                                                            \
    softmax_split_sum<AL>(x, extent, nseg, pmax, psum, tab);                                              \
  }                                                                                                       \
  extern "C" __global__ void __launch_bounds__(256) tiler_softmax_f32_split_out##SFX(                     \
      const float* __restrict__ x, float* __restrict__ y, uint32_t extent, uint64_t nseg,                 \
      const float* __restrict__ pmax, const float* __restrict__ psum) {                                   \
    __shared__ double tab[64];                                                                            \
    softmax_split_out<AL>(x, y, extent, nseg, pmax, psum, tab);                                           \
  }                                                                                                       \
  extern "C" __global__ void __launch_bounds__(256) tiler_softmax_f32_rowsync##SFX(                       \
      const float* __restrict__ x, float* __restrict__ y, uint32_t extent, uint64_t nseg,                 \
      uint8_t* __restrict__ sync, uint64_t wait_ticks) {                                                  \
    __shared__ double tab[64];                                                                            \
    softmax_rowsync<AL>(x, y, extent, nseg, sync, wait_ticks, tab);                                       \
  }
TILER_SOFTMAX_F32_SEG(1, _a)
TILER_SOFTMAX_F32_SEG(0, _u)
