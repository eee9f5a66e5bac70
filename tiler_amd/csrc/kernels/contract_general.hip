// Contraction over a general binary index structure (ADR 0087; the
// reference evaluates it in tiler-reference/src/contraction.rs:346-715).
//
// * tiler_contract_general_{f32,bf16,bf16_silu}: the strict fold, one
//   invocation per output element (grid-stride).  The output coordinate is
//   decoded row-major; the contracted coordinate walks its row-major odometer
//   over the contracted set in ascending label order (the host resolves the
//   order and every stride).  Seeded at the first product, p = fl(a*b),
//   acc = fl(acc + p), no FMA; canonical NaN at the commit (a NaN product or
//   sum stays NaN through every later addition, so per-step canonicalization
//   changes no committed bit).  bf16 operands are widened exactly; SiLU is
//   tiler::silu_f32 (the reference SiLU) on the canonical accumulator; one
//   bf16 narrowing.
// * tiler_transpose_bf16: [batch][rows][cols] -> [batch][cols][rows] through
//   64 x 64 LDS tiles, for a right operand stored [k, n] ahead of the MFMA
//   kernels, which take it [n, k].
#include "common.h"
#include "contract_geometry.h"

using tiler::canon;
using tiler_geom::GeneralGeometry;

namespace {

constexpr int kAxes = tiler_geom::kAxes;

template <typename T>
__device__ __forceinline__ float widen(T v) {
  if constexpr (sizeof(T) == 2) return tiler::bf16_widen(v);
  else return v;
}

// kModes: the declared subnormal modes at every site of the fold
// (contraction.rs:600-625): each factor as an operand, the product and every
// accumulation as results, the accumulator as an operand; seeded at the first
// product itself; the SiLU under the same modes (silu.rs:511-533).
template <typename T, bool kSilu, bool kModes = false>
__device__ __forceinline__ void general_body(const T* __restrict__ l, const T* __restrict__ r,
                                             T* __restrict__ out, const GeneralGeometry& g, uint32_t im = 1u,
                                             uint32_t rm = 1u) {
  using tiler::subnormal;
  // g lives in a constant slot: every read is a uniform (scalar) load.
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint32_t inner = g.con_rank - 1;
  uint64_t in_dim = 0, in_l = 0, in_r = 0;
#pragma unroll
  for (int d = 0; d < kAxes; ++d)
    if ((uint32_t)d == inner) {
      in_dim = g.con_dims[d];
      in_l = g.l_con[d];
      in_r = g.r_con[d];
    }
  for (uint64_t o = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; o < g.outputs; o += stride) {
    uint64_t lb = 0, rb = 0, rem = o;
#pragma unroll
    for (int d = kAxes - 1; d >= 0; --d)
      if ((uint32_t)d < g.out_rank) {
        const uint64_t c = rem % g.out_dims[d];
        rem /= g.out_dims[d];
        lb += c * g.l_out[d];
        rb += c * g.r_out[d];
      }
    uint64_t coord[kAxes];
#pragma unroll
    for (int d = 0; d < kAxes; ++d) coord[d] = 0;
    float acc = -0.0f;  // -0 + first product == first product, bit for bit
    bool seeded = false;
    for (;;) {
      const T* lp = l + lb;
      const T* rp = r + rb;
      for (uint64_t i = 0; i < in_dim; ++i) {
        if constexpr (kModes) {
          const float p = subnormal(rm, subnormal(im, widen(lp[i * in_l])) * subnormal(im, widen(rp[i * in_r])));
          acc = seeded ? subnormal(rm, subnormal(im, acc) + subnormal(im, p)) : p;
          seeded = true;
        } else {
          const float p = widen(lp[i * in_l]) * widen(rp[i * in_r]);
          acc = acc + p;
        }
      }
      // the next outer contracted coordinate (axes inner-1 .. 0)
      bool carry = true;
#pragma unroll
      for (int d = kAxes - 1; d >= 0; --d)
        if (carry && (uint32_t)d < inner) {
          lb += g.l_con[d];
          rb += g.r_con[d];
          if (++coord[d] < g.con_dims[d]) {
            carry = false;
          } else {
            lb -= coord[d] * g.l_con[d];
            rb -= coord[d] * g.r_con[d];
            coord[d] = 0;
          }
        }
      if (carry) break;
    }
    float v = canon(acc);
    if constexpr (sizeof(T) == 2) {
      if (kSilu) {
        if constexpr (kModes) {
          if (v == v && v != __builtin_huge_valf() && v != -__builtin_huge_valf()) {
            const float a = subnormal(im, v);
            const float e = subnormal(rm, tiler::exp_f32_cr(subnormal(im, -a)));
            const float divisor = subnormal(rm, 1.0f + subnormal(im, e));
            v = subnormal(rm, subnormal(im, a) / subnormal(im, divisor));
          } else {
            v = tiler::silu_f32(v);
          }
        } else {
          v = tiler::silu_f32(v);
        }
      }
      out[o] = (T)tiler::bf16_narrow(v);
    } else {
      out[o] = v;
    }
  }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
tiler_contract_general_f32(const float* __restrict__ l, const float* __restrict__ r, float* __restrict__ out,
                           const GeneralGeometry* __restrict__ g) {
  general_body<float, false>(l, r, out, *g);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_general_bf16(const uint16_t* __restrict__ l, const uint16_t* __restrict__ r,
                            uint16_t* __restrict__ out, const GeneralGeometry* __restrict__ g) {
  general_body<uint16_t, false>(l, r, out, *g);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_general_bf16_silu(const uint16_t* __restrict__ l, const uint16_t* __restrict__ r,
                                 uint16_t* __restrict__ out, const GeneralGeometry* __restrict__ g) {
  general_body<uint16_t, true>(l, r, out, *g);
}

// The strict folds under the declared subnormal modes (a flushing contract).
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_general_f32_m(const float* __restrict__ l, const float* __restrict__ r, float* __restrict__ out,
                             const GeneralGeometry* __restrict__ g, uint32_t in_mode, uint32_t out_mode) {
  general_body<float, false, true>(l, r, out, *g, in_mode, out_mode);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_general_bf16_m(const uint16_t* __restrict__ l, const uint16_t* __restrict__ r,
                              uint16_t* __restrict__ out, const GeneralGeometry* __restrict__ g, uint32_t in_mode,
                              uint32_t out_mode) {
  general_body<uint16_t, false, true>(l, r, out, *g, in_mode, out_mode);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_general_bf16_silu_m(const uint16_t* __restrict__ l, const uint16_t* __restrict__ r,
                                   uint16_t* __restrict__ out, const GeneralGeometry* __restrict__ g,
                                   uint32_t in_mode, uint32_t out_mode) {
  general_body<uint16_t, true, true>(l, r, out, *g, in_mode, out_mode);
}

// dst[b][c][r] = src[b][r][c]; grid (ceil(cols/64), min(batches * row tiles,
// 65535)) with 256 threads: y walks (batch, 64-row tile) pairs, grid-stride.
extern "C" __global__ void __launch_bounds__(256)
tiler_transpose_bf16(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, uint64_t batches,
                     uint32_t rows, uint32_t cols) {
  __shared__ uint16_t tile[64][66];
  const uint32_t tx = threadIdx.x & 63u, ty = threadIdx.x >> 6;  // 64 x 4
  const uint32_t c0 = blockIdx.x * 64u;
  const uint64_t plane = (uint64_t)rows * cols;
  const uint64_t row_tiles = ((uint64_t)rows + 63) / 64, work = batches * row_tiles;
  for (uint64_t w = blockIdx.y; w < work; w += gridDim.y) {
    const uint64_t b = w / row_tiles;
    const uint32_t r0 = (uint32_t)(w - b * row_tiles) * 64u;
    const uint16_t* s = src + b * plane;
    uint16_t* d = dst + b * plane;
#pragma unroll
    for (uint32_t i = 0; i < 64; i += 4) {
      const uint32_t rr = r0 + ty + i, cc = c0 + tx;
      if (rr < rows && cc < cols) tile[ty + i][tx] = s[(uint64_t)rr * cols + cc];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t i = 0; i < 64; i += 4) {
      const uint32_t cc = c0 + ty + i, rr = r0 + tx;
      if (rr < rows && cc < cols) d[(uint64_t)cc * rows + rr] = tile[tx][ty + i];
    }
    __syncthreads();
  }
}
