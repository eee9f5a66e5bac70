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
#include <type_traits>

#include "common.h"

namespace {

using tiler::relay_fold_chunk;
using tiler::unrolled_while;

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

// in_mode / out_mode: the declared subnormal modes (tiler::subnormal), applied
// at every arithmetic site as rms_norm.rs:405-489 and softmax.rs:200-315 apply
// them under a conformance (operands flushed before, results after); 1 and 1
// preserve, which is the strict reading.  Under flushing modes the segments
// hold the contributors as F(c) = O(R(c)) (tiler::result_as_operand) and
// fold_segment folds them plainly: the fold's sum is read only as an
// operand, and a sum of two non-negative values that are not subnormal is
// never subnormal, so the reference's acc = R(O(acc) + O(c)) read as O(acc)
// is that plain fold (rms_strict_resident_body states the argument).
template <bool kBf16>
__device__ __forceinline__ void rms_strict_body(const void* __restrict__ x, const void* __restrict__ w,
                                                uint64_t w_row_stride, void* __restrict__ y, uint64_t rows,
                                                uint32_t extent, float eps, uint32_t im, uint32_t rm) {
  using tiler::subnormal;
  const tiler::Flush F = tiler::result_as_operand(im, rm);
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
      const float v = subnormal(im, load_elem<kBf16>(x, base + s0 + i));
      seg[wave][i] = F(v * v);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes landed
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) acc = fold_segment(seg[wave], len, acc, seeded);
    __builtin_amdgcn_wave_barrier();
  }
  // rms_norm.rs:177-187: a division by N, then + eps, then the certified rsqrt.
  float s = 0.0f;
  if (lane == 0) {
    const float mean = subnormal(rm, subnormal(im, acc) / subnormal(im, (float)extent));
    s = subnormal(rm, tiler::rsqrt_f32_cr(subnormal(im, subnormal(rm, subnormal(im, mean) + subnormal(im, eps)))));
  }
  s = __shfl(s, 0, 64);
  const uint64_t wbase = row * w_row_stride;
  for (uint32_t i = lane; i < extent; i += 64) {
    const float normalized = subnormal(rm, subnormal(im, load_elem<kBf16>(x, base + i)) * subnormal(im, s));
    store_elem<kBf16>(y, base + i,
                      tiler::canon(subnormal(rm, subnormal(im, load_elem<kBf16>(w, wbase + i)) * subnormal(im, normalized))));
  }
}

__device__ __forceinline__ void softmax_strict_body(const float* __restrict__ x, float* __restrict__ y,
                                                    uint64_t rows, uint32_t extent, uint32_t im, uint32_t rm) {
  using tiler::subnormal;
  const tiler::Flush F = tiler::result_as_operand(im, rm);
  // O(e_i) = O(apply_to_result(exp(apply_to_operand(fl(x_i - m) under the modes))))
  auto expo = [&](float v, float m) { return F(tiler::exp_f32_cr(F(subnormal(im, v) - subnormal(im, m)))); };
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
    for (uint32_t i = lane; i < len; i += 64) seg[wave][i] = expo(xr[s0 + i], m);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) d = fold_segment(seg[wave], len, d, seeded);
    __builtin_amdgcn_wave_barrier();
  }
  float r = 0.0f;
  if (lane == 0) r = subnormal(rm, 1.0f / subnormal(im, d));  // softmax.rs:302-313: the reciprocal, then a multiply
  r = __shfl(r, 0, 64);
  for (uint32_t i = lane; i < extent; i += 64)
    yr[i] = tiler::canon(subnormal(rm, expo(xr[i], m) * subnormal(im, r)));
}

// Strict RMSNorm over many rows, staged like the strict serial sum
// (reduce.hip, tiler_sum_f32_staged_r*).
// * Each 256-thread workgroup serves R rows. Stage s holds C = 4096/R
//   elements of each row.
// * All threads load stage s+1, coalesced (16-byte loads: kVec), and store
//   the squares fl(x*x) of the exactly widened elements into the other LDS
//   buffer.
// * Lane r/4 of wave r%4 folds row r's squares in ascending order, with the
//   next batch of LDS reads in flight. One wave instruction advances R/4
//   rows' chains, where one wave per row spent a whole instruction slot on
//   one lane's add.
// * The fold starts from -0.0. A square is never -0.0, so -0.0 plus the
//   first square is the first square.
// * Then, per row, rms_norm.rs:177-187: the division by N, + eps, the
//   certified rsqrt. All threads write y = canon(w * fl(x * s)), re-reading x.
template <typename T, int R, bool kVec, bool kModes = false>
__device__ __forceinline__ void rms_strict_staged_body(const T* __restrict__ x, const T* __restrict__ w,
                                                       uint64_t w_row_stride, T* __restrict__ y, uint64_t rows,
                                                       uint32_t extent, float eps, uint32_t im = 1u,
                                                       uint32_t rm = 1u) {
  constexpr bool kBf16 = sizeof(T) == 2;
  constexpr uint32_t C = 4096 / R;
  constexpr uint32_t kStride = C + 4;
  constexpr uint32_t W = kVec ? 16 / sizeof(T) : 1;  // elements per load
  constexpr uint32_t kRowPieces = C / W;
  constexpr uint32_t kPer = 4096 / W / 256;
  typedef typename std::conditional<kVec, u32x4, T>::type raw;
  __shared__ __align__(16) float stage[2][R * kStride];
  __shared__ float scale[R];
  const uint32_t t = threadIdx.x;
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const uint32_t stages = (extent + C - 1) / C;
  auto widen = [](uint32_t bits) -> float {
    if constexpr (kBf16) return tiler::bf16_widen(bits);
    else return __uint_as_float(bits);
  };
  // Under the modes (the _m forms) the squares are staged as F(O(x) * O(x))
  // and the fold is the plain one, as in rms_strict_resident_body.
  const tiler::Flush O(im), Rz(rm), F = tiler::result_as_operand(im, rm);
  auto sq = [&](float v) {
    if constexpr (kModes) {
      const float o = O(v);
      return F(o * o);
    } else {
      return v * v;
    }
  };
  auto sq4 = [&](f32x4 a) -> f32x4 {
    if constexpr (kModes) return f32x4{sq(a.x), sq(a.y), sq(a.z), sq(a.w)};
    else return a * a;
  };
  raw reg[kPer];
  auto load = [&](uint32_t s) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const uint32_t e = s * C + (q % kRowPieces) * W;
      if (row0 + r < rows && e < extent) reg[i] = *reinterpret_cast<const raw*>(x + (row0 + r) * extent + e);
      else reg[i] = raw{};
    }
  };
  // Squares past the row's end (or of a row past the last) are staged as
  // -0.0 for the relay fold, which folds whole passes (s + -0.0 == s).
  const f32x4 nz = {-0.0f, -0.0f, -0.0f, -0.0f};
  auto store = [&](uint32_t buf, uint32_t s) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const bool in = row0 + r < rows && s * C + (q % kRowPieces) * W < extent;
      float* dst = &stage[buf][r * kStride + (q % kRowPieces) * W];
      if constexpr (!kVec) {
        const float v = kBf16 ? tiler::bf16_widen(reg[i]) : (float)reg[i];
        if constexpr (kModes) *dst = in ? sq(v) : -0.0f;
        else *dst = in ? v * v : -0.0f;
      } else if constexpr (kBf16) {  // 8 bf16 -> 8 squares
        const u32x4 u = reg[i];
        f32x4 lo, hi;
        lo.x = widen(u.x & 0xffffu); lo.y = widen(u.x >> 16); lo.z = widen(u.y & 0xffffu); lo.w = widen(u.y >> 16);
        hi.x = widen(u.z & 0xffffu); hi.y = widen(u.z >> 16); hi.z = widen(u.w & 0xffffu); hi.w = widen(u.w >> 16);
        if constexpr (kModes) {
          *reinterpret_cast<f32x4*>(dst) = in ? sq4(lo) : nz;
          *reinterpret_cast<f32x4*>(dst + 4) = in ? sq4(hi) : nz;
        } else {
          *reinterpret_cast<f32x4*>(dst) = in ? lo * lo : nz;
          *reinterpret_cast<f32x4*>(dst + 4) = in ? hi * hi : nz;
        }
      } else {
        const u32x4 u = reg[i];
        f32x4 v;
        v.x = widen(u.x); v.y = widen(u.y); v.z = widen(u.z); v.w = widen(u.w);
        if constexpr (kModes) *reinterpret_cast<f32x4*>(dst) = in ? sq4(v) : nz;
        else *reinterpret_cast<f32x4*>(dst) = in ? v * v : nz;
      }
    }
  };
  // R <= 16: the relay fold (tiler::relay_fold_row), the folding waves'
  // 8-lane groups each taking a row in 256-element passes (R = 1: wave 0;
  // R = 4: wave w row w; R = 16: wave w rows 4 w .. 4 w + 3), every dependent
  // add on registers.  R = 64: lane r / 4 of wave r % 4 folds row r.
  constexpr bool kRelay = R <= 16;
  constexpr uint32_t kRowsPerWave = R == 16 ? 4u : 1u;
  const uint32_t lane = t & 63u, wave = t >> 6, g = lane >> 3, sg = lane & 7u;
  const uint32_t fr = kRelay ? (R == 1 ? 0u : wave * kRowsPerWave + g % kRowsPerWave)
                             : (t & 63u) * 4u + (t >> 6);  // the row this lane folds
  const bool folds = kRelay ? (R == 1 ? wave == 0 : true)
                            : (t & 63u) < (uint32_t)R / 4u && row0 + fr < rows;
  float acc = -0.0f;
  if (stages > 0) {
    load(0);
    store(0, 0);
  }
  __syncthreads();
  for (uint32_t s = 0; s < stages; ++s) {
    const bool more = s + 1 < stages;
    if (more) load(s + 1);
    if (kRelay && folds) {
      const uint32_t count = extent - s * C < C ? extent - s * C : C;
      acc = tiler::relay_fold_row<(kRelay ? C / 256u : 1u)>(reinterpret_cast<const f32x4*>(&stage[s & 1][fr * kStride]),
                                                            sg, (count + 255u) / 256u, acc);
    } else if (folds) {
      const float* row = &stage[s & 1][fr * kStride];
      const uint32_t count = extent - s * C < C ? extent - s * C : C;
      if (count == C) {
        constexpr uint32_t kBatch = C / 4 < 8 ? C / 4 : 8;
        constexpr uint32_t kBatches = C / 4 / kBatch;
        const f32x4* rv = reinterpret_cast<const f32x4*>(row);
        f32x4 ba[kBatch], bb[kBatch];
        auto add_batch = [&](const f32x4* v) {
#pragma unroll
          for (uint32_t j = 0; j < kBatch; ++j) {
            acc = acc + v[j].x;
            acc = acc + v[j].y;
            acc = acc + v[j].z;
            acc = acc + v[j].w;
          }
        };
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) ba[j] = rv[j];
        for (uint32_t b = 0; b < kBatches; b += 2) {
          if (b + 1 < kBatches) {
#pragma unroll
            for (uint32_t j = 0; j < kBatch; ++j) bb[j] = rv[(b + 1) * kBatch + j];
          }
          add_batch(ba);
          if (b + 1 < kBatches) {
            if (b + 2 < kBatches) {
#pragma unroll
              for (uint32_t j = 0; j < kBatch; ++j) ba[j] = rv[(b + 2) * kBatch + j];
            }
            add_batch(bb);
          }
        }
      } else {
        for (uint32_t c = 0; c < count; ++c) acc = acc + row[c];
      }
    }
    if (more) store((s + 1) & 1u, s + 1);
    __syncthreads();
  }
  // A relay group's row sum is in its lane 8 g.
  if (kRelay ? folds && sg == 0 && g < kRowsPerWave && row0 + fr < rows : folds)
    scale[fr] = kModes ? F(tiler::rsqrt_f32_cr(F(F(acc / (float)extent) + O(eps))))
                       : tiler::rsqrt_f32_cr(acc / (float)extent + eps);
  __syncthreads();
  // w * fl(x * s), under the modes R(O(w) * F(O(x) * O(s))).
  auto scaled = [&](float xf, float wf, float sc) -> float {
    if constexpr (kModes) return Rz(O(wf) * F(O(xf) * sc));
    else return wf * (xf * sc);
  };
  for (uint32_t r = 0; r < (uint32_t)R; ++r) {
    if (row0 + r >= rows) break;
    const float sc = scale[r];
    const uint64_t base = (row0 + r) * extent, wbase = (row0 + r) * w_row_stride;
    if constexpr (kVec) {
      for (uint32_t e = t * W; e < extent; e += 256u * W) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(x + base + e);
        const u32x4 wv = *reinterpret_cast<const u32x4*>(w + wbase + e);
        u32x4 out;
        if constexpr (kBf16) {
          auto one = [&](uint32_t xb, uint32_t wb) -> uint32_t {
            if constexpr (kModes) return tiler::bf16_narrow(tiler::canon(scaled(widen(xb), widen(wb), sc)));
            else return tiler::bf16_narrow(tiler::canon(widen(wb) * (widen(xb) * sc)));
          };
          out.x = one(xv.x & 0xffffu, wv.x & 0xffffu) | (one(xv.x >> 16, wv.x >> 16) << 16);
          out.y = one(xv.y & 0xffffu, wv.y & 0xffffu) | (one(xv.y >> 16, wv.y >> 16) << 16);
          out.z = one(xv.z & 0xffffu, wv.z & 0xffffu) | (one(xv.z >> 16, wv.z >> 16) << 16);
          out.w = one(xv.w & 0xffffu, wv.w & 0xffffu) | (one(xv.w >> 16, wv.w >> 16) << 16);
        } else {
          auto one = [&](uint32_t xb, uint32_t wb) -> uint32_t {
            if constexpr (kModes) return __float_as_uint(tiler::canon(scaled(widen(xb), widen(wb), sc)));
            else return __float_as_uint(tiler::canon(widen(wb) * (widen(xb) * sc)));
          };
          out.x = one(xv.x, wv.x);
          out.y = one(xv.y, wv.y);
          out.z = one(xv.z, wv.z);
          out.w = one(xv.w, wv.w);
        }
        *reinterpret_cast<u32x4*>(y + base + e) = out;
      }
    } else {
      for (uint32_t e = t; e < extent; e += 256u) {
        if constexpr (kModes) {
          store_elem<kBf16>(y, base + e,
                            tiler::canon(scaled(load_elem<kBf16>(x, base + e), load_elem<kBf16>(w, wbase + e), sc)));
        } else {
          const float normalized = load_elem<kBf16>(x, base + e) * sc;
          store_elem<kBf16>(y, base + e, tiler::canon(load_elem<kBf16>(w, wbase + e) * normalized));
        }
      }
    }
  }
}

// Strict softmax over many rows, staged the same way (R rows per workgroup,
// stages of C = 4096/R elements of each row), in three streamed passes over
// each row (softmax.rs:237-315):
// * The maximum. It is order-insensitive (model.rs:906-912), so each thread
//   keeps the running maximum of its own pieces and the pieces of a row are
//   combined from LDS afterwards.
// * The exponents e = certified exp(fl(x - m)), stored into LDS stage by
//   stage. Lane r/4 of wave r%4 folds row r's exponents in ascending order
//   from -0.0 (an exponent is never -0.0, so -0.0 plus the first is the first).
// * y = canon(fl(exp(fl(x - m)) * fl(1 / d))): the reciprocal, then a
//   multiply, the exponent recomputed (the same correctly rounded value).
template <int R, bool kVec, bool kModes = false>
__device__ __forceinline__ void softmax_strict_staged_body(const float* __restrict__ x, float* __restrict__ y,
                                                           uint64_t rows, uint32_t extent, uint32_t im = 1u,
                                                           uint32_t rm = 1u) {
  constexpr uint32_t C = 4096 / R;
  constexpr uint32_t kStride = C + 4;
  constexpr uint32_t W = kVec ? 4 : 1;
  constexpr uint32_t kRowPieces = C / W;
  constexpr uint32_t kPer = 4096 / W / 256;
  typedef typename std::conditional<kVec, f32x4, float>::type piece;
  __shared__ __align__(16) float stage[2][R * kStride];
  __shared__ float rowmax[R];
  __shared__ float recip[R];
  __shared__ double tab[64];
  const uint32_t t = threadIdx.x;
  if (t < 64) tab[t] = kExp2Table64[t];
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const uint32_t stages = (extent + C - 1) / C;
  auto valid = [&](uint32_t i, uint32_t s, uint32_t& r, uint32_t& e) {
    const uint32_t q = t + 256u * i;
    r = q / kRowPieces;
    e = s * C + (q % kRowPieces) * W;
    return row0 + r < rows && e < extent;
  };
  // Pass 1: the maximum.  Piece i of this thread always belongs to the same
  // row and column of the stage, so its running maximum is one per piece.
  float pm[kPer];
#pragma unroll
  for (uint32_t i = 0; i < kPer; ++i) pm[i] = -__builtin_huge_valf();  // the maximum's two-sided identity
#pragma unroll 2
  for (uint32_t s = 0; s < stages; ++s) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      uint32_t r, e;
      if (!valid(i, s, r, e)) continue;
      const float* src = x + (row0 + r) * extent + e;
      if constexpr (kVec) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(src);
        pm[i] = tiler::maximum_f32(tiler::maximum_f32(tiler::maximum_f32(tiler::maximum_f32(pm[i], v.x), v.y), v.z),
                                   v.w);
      } else {
        pm[i] = tiler::maximum_f32(pm[i], *src);
      }
    }
  }
  // Combine: stage buffer 0 holds every piece's maximum at [row][column].
#pragma unroll
  for (uint32_t i = 0; i < kPer; ++i) {
    const uint32_t q = t + 256u * i;
    stage[0][(q / kRowPieces) * kStride + q % kRowPieces] = pm[i];
  }
  __syncthreads();
  // Each row's piece maxima are combined by the 256 / R threads of its
  // group: a strided pass, then a butterfly within the group (and, for
  // R = 1, across the four waves through LDS).
  {
    constexpr uint32_t kTPR = 256 / R;  // threads per row
    const uint32_t cr = t / kTPR, cl = t % kTPR;
    float m = -__builtin_huge_valf();
    for (uint32_t c = cl; c < kRowPieces; c += kTPR) m = tiler::maximum_f32(m, stage[0][cr * kStride + c]);
#pragma unroll
    for (uint32_t o = (kTPR < 64 ? kTPR : 64) / 2; o >= 1; o >>= 1) m = tiler::maximum_f32(m, __shfl_xor(m, o, 64));
    if constexpr (kTPR == 256) {
      __shared__ float wm[4];
      if ((t & 63u) == 0) wm[t >> 6] = m;
      __syncthreads();
      m = tiler::maximum_f32(tiler::maximum_f32(wm[0], wm[1]), tiler::maximum_f32(wm[2], wm[3]));
    }
    if (cl == 0) rowmax[cr] = m;
  }
  // The relay fold (tiler::relay_fold_row): the folding waves' 8-lane groups
  // each take a row in 256-element passes (R = 1: wave 0; R = 4: wave w row
  // w; R = 16: wave w rows 4 w .. 4 w + 3), every dependent add on
  // registers; a group's row sum ends in its lane 8 g.
  static_assert(R == 1 || R == 4 || R == 16, "stages of at least 256 elements per row");
  constexpr uint32_t kRowsPerWave = R == 16 ? 4u : 1u;
  const uint32_t lane = t & 63u, wave = t >> 6, g = lane >> 3, sg = lane & 7u;
  const uint32_t fr = R == 1 ? 0u : wave * kRowsPerWave + g % kRowsPerWave;  // the row this group folds
  const bool folds = R == 1 ? wave == 0 : true;
  __syncthreads();
  // Pass 2: the exponents, folded in order.  Under the modes (the _m forms)
  // they are F(exp(F(O(x) - O(m)))), staged and written to y as such, and
  // the fold is the plain one, as in rms_strict_resident_body.
  const tiler::Flush O(im), Rz(rm), F = tiler::result_as_operand(im, rm);
  auto expo = [&](float xv, float m) {
    if constexpr (kModes) return F(tiler::exp_f32_cr(F(O(xv) - O(m)), tab));
    else return tiler::exp_f32_cr(xv - m, tab);
  };
  piece reg[kPer];
  auto load = [&](uint32_t s) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      uint32_t r, e;
      if (valid(i, s, r, e)) reg[i] = *reinterpret_cast<const piece*>(x + (row0 + r) * extent + e);
      else reg[i] = piece{};
    }
  };
  auto store_some = [&](uint32_t buf, uint32_t sbuf, auto guard) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = t + 256u * i, r = q / kRowPieces;
      const float m = rowmax[r < R ? r : 0];
      float* dst = &stage[buf][r * kStride + (q % kRowPieces) * W];
      // The exponents also go to y, where the output pass scales them.
      const uint32_t e = sbuf * C + (q % kRowPieces) * W;
      // Slots past the row's end or the last row hold -0.0, which leaves the
      // relay's sums unchanged (s + -0.0 == s), and are not written to y.
      if (decltype(guard)::value && !(row0 + r < rows && e < extent)) {
        if constexpr (kVec) *reinterpret_cast<f32x4*>(dst) = f32x4{-0.0f, -0.0f, -0.0f, -0.0f};
        else *dst = -0.0f;
        continue;
      }
      if constexpr (kVec) {
        f32x4 ev;
        ev.x = expo(reg[i].x, m);
        ev.y = expo(reg[i].y, m);
        ev.z = expo(reg[i].z, m);
        ev.w = expo(reg[i].w, m);
        *reinterpret_cast<f32x4*>(dst) = ev;
        *reinterpret_cast<f32x4*>(y + (row0 + r) * extent + e) = ev;
      } else {
        const float ev = expo(reg[i], m);
        *dst = ev;
        y[(row0 + r) * extent + e] = ev;
      }
    }
  };
  // Whole stages (every slot a row's element) take the unguarded form, so the
  // pieces' exponents interleave; only a workgroup's edge stages test slots.
  auto store = [&](uint32_t buf, uint32_t sbuf) {
    if (row0 + R <= rows && (uint64_t)(sbuf + 1) * C <= extent) store_some(buf, sbuf, std::false_type{});
    else store_some(buf, sbuf, std::true_type{});
  };
  float acc = -0.0f;
  if (stages > 0) {
    load(0);
    store(0, 0);
  }
  __syncthreads();
  for (uint32_t s = 0; s < stages; ++s) {
    const bool more = s + 1 < stages;
    if (more) load(s + 1);
    if (folds) {
      const uint32_t count = extent - s * C < C ? extent - s * C : C;
      acc = tiler::relay_fold_row<C / 256u>(reinterpret_cast<const f32x4*>(&stage[s & 1][fr * kStride]), sg,
                                            (count + 255u) / 256u, acc);
    }
    if (more) store((s + 1) & 1u, s + 1);
    __syncthreads();
  }
  // softmax.rs:302-313: the reciprocal, then a multiply.
  if (folds && sg == 0 && g < kRowsPerWave && row0 + fr < rows) recip[fr] = kModes ? F(1.0f / acc) : 1.0f / acc;
  auto out = [&](float e, float rc) {  // canon(fl(e * r)), under the modes canon(R(O(e) * O(r)))
    if constexpr (kModes) return tiler::canon(Rz(e * rc));
    else return tiler::canon(e * rc);
  };
  __syncthreads();
  // Pass 3: y, over the workgroup's rows as one flat run of pieces (the
  // iterations are independent, so several loads are in flight per thread).
  const uint64_t nrows = rows - row0 < (uint64_t)R ? rows - row0 : (uint64_t)R;
  const uint64_t per_row = (extent + W - 1) / W, pieces = nrows * per_row;
#pragma unroll 4
  for (uint64_t idx = t; idx < pieces; idx += 256u) {
    const uint32_t r = (uint32_t)(idx / per_row);
    const uint32_t e = (uint32_t)(idx - (uint64_t)r * per_row) * W;
    const float rc = recip[r];
    const uint64_t at = (row0 + r) * extent + e;
    if constexpr (kVec) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(y + at);  // the exponents pass 2 wrote
      f32x4 o;
      o.x = out(v.x, rc);
      o.y = out(v.y, rc);
      o.z = out(v.z, rc);
      o.w = out(v.w, rc);
      *reinterpret_cast<f32x4*>(y + at) = o;
    } else {
      y[at] = out(y[at], rc);
    }
  }
}

// Strict RMSNorm with a workgroup's rows resident in registers, for rows of
// at most 32 P E elements (E = 8 bf16 or 4 f32 per 16-byte piece; extent a
// multiple of E, 16-byte aligned rows and weight): 8 rows per workgroup of
// 256 threads, half a wave per row; lane l of a row holds the row's
// elements E (l + 32 j) .. +E-1 for j < P.  x is read once and y written
// once (rms_norm.rs:134-195, 453-489):
// * the squares fl(x * x) of the exactly widened elements go through a
//   two-chunk LDS ring, chunk j (32 E columns) as soon as piece j of every
//   lane has landed, laid out so that lane 8 g + s of wave 0 reads segment s
//   (4 E consecutive columns) of row g's chunk with conflict-free 16-byte
//   reads; wave 0 relay-folds chunk j (relay_fold_chunk) while chunk j + 1
//   is written, from -0.0 (a square is never -0.0, so -0.0 plus the first
//   square is the first square).  Columns past the row's end hold -0.0,
//   which leaves every sum unchanged (s + -0.0 == s for every s, NaN and the
//   zeros included), so whole chunks are folded.  The serial fold runs while
//   the row is still arriving;
// * per row the division by N, + eps and the certified rsqrt
//   (rms_norm.rs:177-187);
// * y = canon(fl(w * fl(x * s))) from the registers, weight after the
//   normalization (rms_norm.rs:474-485), narrowed once for bf16.
// The _m forms (kModes, here and in the resident softmax) take a flushing
// contract's two subnormal modes (tiler::subnormal) at every arithmetic site
// as rms_norm.rs:405-489 and softmax.rs:200-315 apply them: O (the in mode)
// on each operand, R (the out mode) on each result.  Every computed value but
// the outputs is read only as an operand, so the kernels carry O(value): F,
// O after R, is one flush (tiler::result_as_operand).  The reference's fold
// acc = R(O(acc) + O(c)), seeded at the first contributor, then carries
// b = O(acc) as b = F(b + F(c)) from -0.0 (-0.0 + F(c) = F(c) = O(c), c being
// a result).  The contributors F(c) -- squares, exponents -- are +0, at least
// 2^-126, infinite or NaN, and so is b, so b + F(c) is never subnormal and F
// leaves it: under the modes the fold is the plain relay fold of the flushed
// contributors, the -0.0 padding included.
template <typename T, int R, int P, bool kModes = false>
__device__ __forceinline__ void rms_strict_resident_body(const T* __restrict__ x, const T* __restrict__ w,
                                                         uint64_t w_row_stride, T* __restrict__ y, uint64_t rows,
                                                         uint32_t extent, float eps, uint32_t im = 1u,
                                                         uint32_t rm = 1u) {
  static_assert(R == 8, "eight rows: one 8-lane relay group per row in wave 0");
  constexpr bool kBf16 = sizeof(T) == 2;
  constexpr uint32_t E = 16 / sizeof(T);  // elements per piece
  constexpr uint32_t F4 = E / 4;          // float4 slots of squares per piece
  constexpr uint32_t S4 = 4 * F4;         // float4 slots per relay segment (4 pieces)
  constexpr uint32_t kChunk = 64 * S4;    // float4 slots per chunk: slot k of lane L at k * 64 + L
  __shared__ f32x4 ring[2 * kChunk];
  __shared__ float scale[R];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t r = wave * 2u + (lane >> 5), l = lane & 31u;
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const bool row_ok = row0 + r < rows;
  auto widen = [](uint32_t bits) -> float {
    if constexpr (kBf16) return tiler::bf16_widen(bits);
    else return __uint_as_float(bits);
  };
  const tiler::Flush O(im), Rz(rm), F = tiler::result_as_operand(im, rm);
  auto square = [&](f32x4 a) -> f32x4 {
    if constexpr (kModes) {  // F(O(x) * O(x))
      auto one = [&](float e) {
        const float o = O(e);
        return F(o * o);
      };
      return f32x4{one(a.x), one(a.y), one(a.z), one(a.w)};
    } else {
      return a * a;
    }
  };
  // Piece j is loaded while chunk j - W is written (W ahead): with every
  // piece requested at once the memory system completes chunk 0 late, and
  // the fold, which needs chunk 0 first, starts late.  The loads are
  // branch-free (a piece past the row's end, or of a row past the last,
  // reads a valid element of the last row instead; its square goes to the
  // ring as -0.0 and it is never stored), so each wait counts exactly the
  // loads issued after the piece it waits for.
  constexpr int W = P < 4 ? P : 4;
  const T* xc = x + (row_ok ? row0 + r : rows - 1) * extent;
  u32x4 v[P];
  auto load = [&](int j) {
    const uint32_t e = E * (l + 32u * j);
    v[j] = *reinterpret_cast<const u32x4*>(xc + (e < extent ? e : extent - E));
  };
#pragma unroll
  for (int j = 0; j < W; ++j) load(j);
  float acc = -0.0f;
  constexpr uint32_t kChunkElems = 32 * E;
  const f32x4 nz = {-0.0f, -0.0f, -0.0f, -0.0f};
  // Piece j of lane l is pieces 4 (l / 4) + l % 4 of the chunk's segment
  // l / 4: its slots are k = F4 (l % 4) + f of relay lane 8 r + l / 4.
  f32x4* const mine = ring + (l & 3u) * F4 * 64u + 8u * r + (l >> 2);
  // Chunk j into ring half j & 1, one barrier per chunk: half j & 1 was last
  // read by the fold of chunk j - 2, whose reads wave 0 waited for before it
  // reached the barrier of chunk j - 1.
  auto chunk = [&](auto step) -> bool {
    constexpr int j = decltype(step)::value;
    if ((uint32_t)j * kChunkElems >= extent) return false;
    if constexpr (j + W < P) load(j + W);
    const u32x4 u = v[j];
    const bool in = E * (l + 32u * j) < extent;
    f32x4* dst = mine + (j & 1) * kChunk;
    if constexpr (kBf16) {
      f32x4 lo, hi;
      lo.x = widen(u.x & 0xffffu); lo.y = widen(u.x >> 16); lo.z = widen(u.y & 0xffffu); lo.w = widen(u.y >> 16);
      hi.x = widen(u.z & 0xffffu); hi.y = widen(u.z >> 16); hi.z = widen(u.w & 0xffffu); hi.w = widen(u.w >> 16);
      if constexpr (kModes) {
        dst[0] = in ? square(lo) : nz;
        dst[64] = in ? square(hi) : nz;
      } else {
        dst[0] = in ? lo * lo : nz;
        dst[64] = in ? hi * hi : nz;
      }
    } else {
      f32x4 a;
      a.x = widen(u.x); a.y = widen(u.y); a.z = widen(u.z); a.w = widen(u.w);
      dst[0] = in ? square(a) : nz;
    }
    __syncthreads();
    if (wave == 0) {
      const f32x4* src = ring + (j & 1) * kChunk + lane;
      f32x4 seg[S4];
#pragma unroll
      for (uint32_t k = 0; k < S4; ++k) seg[k] = src[k * 64u];
      acc = relay_fold_chunk<S4>(seg, acc);
    }
    return true;
  };
  unrolled_while<0, P>(chunk);
  // Row g's sum is in lane 8 g after the last chunk's final hop.
  if (wave == 0 && (lane & 7u) == 0) {
    if constexpr (kModes)  // O(s) = F(rsqrt(F(F(acc / N) + O(eps)))), N a normal number
      scale[lane >> 3] = F(tiler::rsqrt_f32_cr(F(F(acc / (float)extent) + O(eps))));
    else
      scale[lane >> 3] = tiler::rsqrt_f32_cr(acc / (float)extent + eps);
  }
  __syncthreads();
  if (!row_ok) return;
  const float sc = scale[r];
  auto scaled = [&](float xf, float wf) -> float {
    if constexpr (kModes)  // R(O(w) * F(O(x) * O(s)))
      return Rz(O(wf) * F(O(xf) * sc));
    else
      return wf * (xf * sc);
  };
  const T* wr = w + (row0 + r) * w_row_stride;
  T* yr = y + (row0 + r) * extent;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const uint32_t e = E * (l + 32u * j);
    if (e < extent) {
      const u32x4 xv = v[j];
      const u32x4 wv = *reinterpret_cast<const u32x4*>(wr + e);
      u32x4 out;
      if constexpr (kBf16) {
        // Every workgroup reaches this pass at once, so its VALU work is
        // issued four waves to a SIMD: the pair narrows in one instruction.
        auto one = [&](uint32_t xb, uint32_t wb) -> float { return scaled(widen(xb), widen(wb)); };
        auto two = [&](uint32_t xw, uint32_t ww) -> uint32_t {
          return tiler::bf16_pack2_rne(one(xw & 0xffffu, ww & 0xffffu), one(xw >> 16, ww >> 16));
        };
        out.x = two(xv.x, wv.x);
        out.y = two(xv.y, wv.y);
        out.z = two(xv.z, wv.z);
        out.w = two(xv.w, wv.w);
      } else {
        auto one = [&](uint32_t xb, uint32_t wb) -> uint32_t {
          return __float_as_uint(tiler::canon(scaled(widen(xb), widen(wb))));
        };
        out.x = one(xv.x, wv.x);
        out.y = one(xv.y, wv.y);
        out.z = one(xv.z, wv.z);
        out.w = one(xv.w, wv.w);
      }
      __builtin_nontemporal_store(out, reinterpret_cast<u32x4*>(yr + e));
    }
  }
}

// Strict softmax with a workgroup's rows resident in registers, for rows of
// at most 128 P elements (extent a multiple of 4, 16-byte aligned rows):
// R rows per workgroup of 32 R threads, half a wave per row; lane l of a
// row holds the row's elements 4 (l + 32 j) .. +3 for j < P as P float4
// pieces.  x is read once and y written once (softmax.rs:237-315):
// * the maximum: each lane's pieces, then a butterfly over the row's 32
//   lanes;
// * the exponents e = certified exp(fl(x - m)), in place in the registers;
// * the fold: the exponents pass through an LDS ring in 128-column chunks,
//   eight chunks a round, laid out so that lane 8 g + s of the folding wave reads
//   segment s (16 columns) of row g's chunk with conflict-free 16-byte
//   reads, and that wave relay-folds each chunk (relay_fold_chunk) from -0.0
//   (an exponent is never -0.0, so -0.0 plus the first is the first): one
//   wave instruction advances the eight rows' chains;
// * y = fl(e * fl(1 / d)) from the registers: the reciprocal, then a
//   multiply (softmax.rs:302-313), canonical NaN where the row's d is NaN.
// Three steps take the short form because the row's values cannot tell:
// * the maximum is the hardware one (v_max_f32) instead of the IEEE
//   maximum: on a row without NaN both are the largest element, up to the
//   sign of a zero maximum, and fl(x - (+0)) and fl(x - (-0)) differ only
//   for x = -0, as -0 and +0, whose exponents are both 1; a row with a NaN
//   gets e = NaN at that element whatever m is, so d = NaN and every output
//   is the canonical NaN, as under the reference's NaN maximum;
// * the exponent is exp_f32_cr_nonpositive, since s = fl(x - m) <= 0 or NaN;
// * the output's NaN test is the row's: an e is NaN only where d is, and
//   e <= 1 <= d, so a product e * fl(1 / d) is NaN exactly when d is.
template <int R, int P, bool kModes = false>
__device__ __forceinline__ void softmax_strict_resident_body(const float* __restrict__ x, float* __restrict__ y,
                                                             uint64_t rows, uint32_t extent, uint32_t im = 1u,
                                                             uint32_t rm = 1u) {
  static_assert(R == 8, "eight rows: one 8-lane relay group per row in wave 0");
  constexpr int Q = 8;               // ring chunks: the fold runs once per Q chunks
  constexpr uint32_t kChunk = 64 * 4;  // float4 slots per 128-column chunk: slot k of lane L at k * 64 + L
  __shared__ f32x4 ring[Q * kChunk];
  __shared__ float recip[R];
  __shared__ double tab[64];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t r = wave * 2u + (lane >> 5), l = lane & 31u;
  if (t < 64) tab[t] = kExp2Table64[t];
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const bool row_ok = row0 + r < rows;
  const float* xr = x + (row0 + r) * extent;
  const float ninf = -__builtin_huge_valf();
  f32x4 v[P];
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const uint32_t e = 4u * (l + 32u * j);
    v[j] = row_ok && e < extent ? *reinterpret_cast<const f32x4*>(xr + e) : f32x4{ninf, ninf, ninf, ninf};
  }
  float m = ninf;
#pragma unroll
  for (int j = 0; j < P; ++j)
    m = __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fmaxf(v[j].x, v[j].y)), __builtin_fmaxf(v[j].z, v[j].w));
#pragma unroll
  for (uint32_t o = 16; o >= 1; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o, 64));
  __syncthreads();  // the exponent table
  const tiler::Flush O(im), Rz(rm), F = tiler::result_as_operand(im, rm);
  const float om = O(m);
  auto expo = [&](float xv) {
    if constexpr (kModes)  // F(exp(F(O(x) - O(m)))): an argument <= 0 or NaN, O being monotone
      return F(tiler::exp_f32_cr_nonpositive(F(O(xv) - om), tab));
    else
      return tiler::exp_f32_cr_nonpositive(xv - m, tab);
  };
#pragma unroll
  for (int j = 0; j < P; ++j) {
    v[j].x = expo(v[j].x);
    v[j].y = expo(v[j].y);
    v[j].z = expo(v[j].z);
    v[j].w = expo(v[j].w);
  }
  // The folding wave relay-folds (relay_fold_chunk): lane 8 g + s holds segment s
  // (16 columns) of row g's chunk.  Columns past the row's end go to the
  // ring as -0.0, which leaves every sum unchanged, so whole chunks are
  // folded; the next chunk's segment is read while the current one is
  // folded (its address clamped to the current chunk at the round's end, so
  // the reads are unconditional and each LDS wait counts exactly).
  float acc = -0.0f;
  const f32x4 nz = {-0.0f, -0.0f, -0.0f, -0.0f};
  f32x4* const mine = ring + (l & 3u) * 64u + 8u * r + (l >> 2);
  // The folding wave: wave 0, or for P >= 16 wave blockIdx % 4, so that the
  // chains of the workgroups a CU holds at once are spread over its SIMDs
  // rather than all issued by one (65536 x 2048: 217-224 us with wave 0,
  // 200-204 rotated; 8192 x 4096: 85-86 against 79-80; the same rotation
  // measured no faster for P = 8 and for the resident RMSNorm).
  const uint32_t fw = P >= 16 ? (blockIdx.x & 3u) : 0u;
  auto round = [&](auto step) -> bool {
    constexpr int c0 = decltype(step)::value * Q;
    if ((uint32_t)c0 * 128u >= extent) return false;
#pragma unroll
    for (int q = 0; q < Q && c0 + q < P; ++q)
      mine[q * kChunk] = 4u * (l + 32u * (c0 + q)) < extent ? v[c0 + q] : nz;
    __syncthreads();
    if (wave == fw) {
      const uint32_t left = extent - (uint32_t)c0 * 128u;
      const uint32_t nq = left < Q * 128u ? (left + 127u) / 128u : (uint32_t)Q;
      const f32x4* src = ring + lane;
      f32x4 a[4], b[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] = src[k * 64];
      auto chunk = [&](auto qs) -> bool {
        constexpr int q = decltype(qs)::value;
        if ((uint32_t)q >= nq) return false;
        f32x4(&cur)[4] = (q & 1) ? b : a;
        f32x4(&nxt)[4] = (q & 1) ? a : b;
        const f32x4* next = src + ((uint32_t)q + 1 < nq ? q + 1 : q) * kChunk;
#pragma unroll
        for (int k = 0; k < 4; ++k) nxt[k] = next[k * 64];
        acc = relay_fold_chunk<4>(cur, acc);
        return true;
      };
      unrolled_while<0, Q>(chunk);
    }
    __syncthreads();  // the ring is refilled next
    return true;
  };
  unrolled_while<0, (P + Q - 1) / Q>(round);
  // Row g's sum is in lane 8 g after the last chunk's final hop.
  if (wave == fw && (lane & 7u) == 0) recip[lane >> 3] = kModes ? F(1.0f / acc) : 1.0f / acc;
  __syncthreads();
  if (!row_ok) return;
  const float rc = recip[r];
  const bool nan_row = rc != rc;
  const float qnan = __uint_as_float(TILER_CANONICAL_F32_NAN);
  float* yr = y + (row0 + r) * extent;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const uint32_t e = 4u * (l + 32u * j);
    if (e < extent) {
      f32x4 o;
      if constexpr (kModes) {  // canon(R(O(e) * O(r)))
        auto one = [&](float e) { return tiler::canon(Rz(e * rc)); };
        o = f32x4{one(v[j].x), one(v[j].y), one(v[j].z), one(v[j].w)};
      } else {
        o = f32x4{nan_row ? qnan : v[j].x * rc, nan_row ? qnan : v[j].y * rc, nan_row ? qnan : v[j].z * rc,
                  nan_row ? qnan : v[j].w * rc};
      }
      __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(yr + e));
    }
  }
}

}  // namespace

#define TILER_SOFTMAX_STRICT_RESIDENT(R, P)                                                           \
  extern "C" __global__ void __launch_bounds__(32 * R)                                                \
      tiler_softmax_f32_strict_rr##R##_p##P(const float* __restrict__ x, float* __restrict__ y,       \
                                            uint64_t rows, uint32_t extent) {                         \
    softmax_strict_resident_body<R, P>(x, y, rows, extent);                                           \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(32 * R)                                                \
      tiler_softmax_f32_strict_rr##R##_p##P##_m(const float* __restrict__ x, float* __restrict__ y,   \
                                                uint64_t rows, uint32_t extent, uint32_t in_mode,     \
                                                uint32_t out_mode) {                                  \
    softmax_strict_resident_body<R, P, true>(x, y, rows, extent, in_mode, out_mode);                 \
  }
TILER_SOFTMAX_STRICT_RESIDENT(8, 32)
TILER_SOFTMAX_STRICT_RESIDENT(8, 16)
TILER_SOFTMAX_STRICT_RESIDENT(8, 8)

#define TILER_RMS_STRICT_RESIDENT(TY, T, R, P)                                                        \
  extern "C" __global__ void __launch_bounds__(32 * R)                                                \
      tiler_rms_norm_##TY##_strict_rr##R##_p##P(const T* __restrict__ x, const T* __restrict__ w,     \
                                                uint64_t w_row_stride, T* __restrict__ y, uint64_t rows,\
                                                uint32_t extent, float eps) {                         \
    rms_strict_resident_body<T, R, P>(x, w, w_row_stride, y, rows, extent, eps);                      \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(32 * R)                                                \
      tiler_rms_norm_##TY##_strict_rr##R##_p##P##_m(const T* __restrict__ x, const T* __restrict__ w, \
                                                    uint64_t w_row_stride, T* __restrict__ y,         \
                                                    uint64_t rows, uint32_t extent, float eps,        \
                                                    uint32_t in_mode, uint32_t out_mode) {            \
    rms_strict_resident_body<T, R, P, true>(x, w, w_row_stride, y, rows, extent, eps, in_mode,        \
                                            out_mode);                                                \
  }
TILER_RMS_STRICT_RESIDENT(bf16, uint16_t, 8, 16)
TILER_RMS_STRICT_RESIDENT(bf16, uint16_t, 8, 8)
TILER_RMS_STRICT_RESIDENT(f32, float, 8, 16)
TILER_RMS_STRICT_RESIDENT(f32, float, 8, 8)

#define TILER_SOFTMAX_STRICT_STAGED(R)                                                                \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_softmax_f32_strict_r##R(const float* __restrict__ x, float* __restrict__ y, uint64_t rows, \
                                    uint32_t extent) {                                                \
    softmax_strict_staged_body<R, true>(x, y, rows, extent);                                          \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_softmax_f32_strict_r##R##_u(const float* __restrict__ x, float* __restrict__ y,           \
                                        uint64_t rows, uint32_t extent) {                             \
    softmax_strict_staged_body<R, false>(x, y, rows, extent);                                         \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_softmax_f32_strict_r##R##_m(const float* __restrict__ x, float* __restrict__ y,           \
                                        uint64_t rows, uint32_t extent, uint32_t in_mode,             \
                                        uint32_t out_mode) {                                          \
    softmax_strict_staged_body<R, true, true>(x, y, rows, extent, in_mode, out_mode);                 \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_softmax_f32_strict_r##R##_u_m(const float* __restrict__ x, float* __restrict__ y,         \
                                          uint64_t rows, uint32_t extent, uint32_t in_mode,           \
                                          uint32_t out_mode) {                                        \
    softmax_strict_staged_body<R, false, true>(x, y, rows, extent, in_mode, out_mode);                \
  }
TILER_SOFTMAX_STRICT_STAGED(1)
TILER_SOFTMAX_STRICT_STAGED(4)
TILER_SOFTMAX_STRICT_STAGED(16)

#define TILER_RMS_STRICT_STAGED(TY, T, R)                                                             \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_rms_norm_##TY##_strict_r##R(const T* __restrict__ x, const T* __restrict__ w,             \
                                        uint64_t w_row_stride, T* __restrict__ y, uint64_t rows,      \
                                        uint32_t extent, float eps) {                                 \
    rms_strict_staged_body<T, R, true>(x, w, w_row_stride, y, rows, extent, eps);                     \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_rms_norm_##TY##_strict_r##R##_u(const T* __restrict__ x, const T* __restrict__ w,         \
                                            uint64_t w_row_stride, T* __restrict__ y, uint64_t rows,  \
                                            uint32_t extent, float eps) {                             \
    rms_strict_staged_body<T, R, false>(x, w, w_row_stride, y, rows, extent, eps);                    \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_rms_norm_##TY##_strict_r##R##_m(const T* __restrict__ x, const T* __restrict__ w,         \
                                            uint64_t w_row_stride, T* __restrict__ y, uint64_t rows,  \
                                            uint32_t extent, float eps, uint32_t in_mode,             \
                                            uint32_t out_mode) {                                      \
    rms_strict_staged_body<T, R, true, true>(x, w, w_row_stride, y, rows, extent, eps, in_mode,       \
                                             out_mode);                                               \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(256)                                                   \
      tiler_rms_norm_##TY##_strict_r##R##_u_m(const T* __restrict__ x, const T* __restrict__ w,       \
                                              uint64_t w_row_stride, T* __restrict__ y,               \
                                              uint64_t rows, uint32_t extent, float eps,              \
                                              uint32_t in_mode, uint32_t out_mode) {                  \
    rms_strict_staged_body<T, R, false, true>(x, w, w_row_stride, y, rows, extent, eps, in_mode,      \
                                              out_mode);                                              \
  }
TILER_RMS_STRICT_STAGED(f32, float, 1)
TILER_RMS_STRICT_STAGED(f32, float, 4)
TILER_RMS_STRICT_STAGED(f32, float, 16)
TILER_RMS_STRICT_STAGED(f32, float, 64)
TILER_RMS_STRICT_STAGED(bf16, uint16_t, 1)
TILER_RMS_STRICT_STAGED(bf16, uint16_t, 4)
TILER_RMS_STRICT_STAGED(bf16, uint16_t, 16)
TILER_RMS_STRICT_STAGED(bf16, uint16_t, 64)

extern "C" __global__ void __launch_bounds__(256)
tiler_rms_norm_f32_strict(const float* __restrict__ x, const float* __restrict__ w, uint64_t w_row_stride,
                          float* __restrict__ y, uint64_t rows, uint32_t extent, float eps, uint32_t in_mode,
                          uint32_t out_mode) {
  rms_strict_body<false>(x, w, w_row_stride, y, rows, extent, eps, in_mode, out_mode);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_rms_norm_bf16_strict(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                           uint64_t w_row_stride, uint16_t* __restrict__ y, uint64_t rows, uint32_t extent,
                           float eps, uint32_t in_mode, uint32_t out_mode) {
  rms_strict_body<true>(x, w, w_row_stride, y, rows, extent, eps, in_mode, out_mode);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_softmax_f32_strict(const float* __restrict__ x, float* __restrict__ y, uint64_t rows, uint32_t extent,
                         uint32_t in_mode, uint32_t out_mode) {
  softmax_strict_body(x, y, rows, extent, in_mode, out_mode);
}
