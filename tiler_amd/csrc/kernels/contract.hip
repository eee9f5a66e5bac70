// Tensor contraction C[m, n] = sum_k A[m, k] * B[n, k]  (td,od->to) for gfx950.
//
// * tiler_contract_strict_f32 -- the governed strict contraction
//   (tiler-reference/src/contraction.rs:558-630): per output, p = fl(a*b),
//   seeded at the first product, acc = fl(acc + p) over ascending k, no FMA.
//   16x16 LDS tiles with a serial in-tile fold, the shape of tiler-metal's
//   contraction_tiled_cooperative golden; bit-exact with the reference.
// * tiler_contract_bf16_* -- the cooperative bf16 contraction on MFMA
//   (v_mfma_f32_32x32x16_bf16): bf16 operands, f32 accumulation, an optional
//   fused SiLU epilogue on the f32 accumulator, one bf16 narrowing.  Guarded
//   tails: out-of-range operand elements are zero-filled, out-of-range outputs
//   are not stored.
#include "common.h"

using tiler::canon;

// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_strict_f32(const float* __restrict__ a, const float* __restrict__ b, uint32_t m,
                          uint32_t n, uint32_t k, float* __restrict__ c) {
  __shared__ float as[16][17];
  __shared__ float bs[16][17];
  const uint32_t tx = threadIdx.x & 15u, ty = threadIdx.x >> 4;
  const uint32_t i0 = blockIdx.y * 16u, j0 = blockIdx.x * 16u;
  float acc = -0.0f;  // -0 + first product == first product, bit for bit
  for (uint32_t k0 = 0; k0 < k; k0 += 16) {
    uint32_t kk = k0 + tx;
    as[ty][tx] = (i0 + ty < m && kk < k) ? a[(uint64_t)(i0 + ty) * k + kk] : 0.0f;
    bs[ty][tx] = (j0 + ty < n && kk < k) ? b[(uint64_t)(j0 + ty) * k + kk] : 0.0f;
    __syncthreads();
    const uint32_t steps = (k - k0) < 16u ? (k - k0) : 16u;
    for (uint32_t s = 0; s < steps; ++s) {
      float p = as[ty][s] * bs[tx][s];
      acc = acc + p;
    }
    __syncthreads();
  }
  if (i0 + ty < m && j0 + tx < n) c[(uint64_t)(i0 + ty) * n + j0 + tx] = canon(acc);
}

// ---------------------------------------------------------------------------
// bf16 MFMA contraction.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdsRow = kBK + 8;  // bf16 elements per LDS row: 16 B pad breaks bank aliasing

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// Loads one 128 x 64 operand tile (rows r0.., k0..) into registers: thread t
// owns 16-byte chunks t + 256*i (row = id/8, kchunk = id%8).
template <bool kFullK>
__device__ __forceinline__ void load_tile(const uint16_t* __restrict__ g, uint32_t rows,
                                          uint32_t k, uint32_t r0, uint32_t k0, u32x4 (&regs)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t id = threadIdx.x + 256u * i;
    uint32_t row = id >> 3, kc = id & 7u;
    uint32_t gr = r0 + row, gk = k0 + kc * 8u;
    if (kFullK && gr < rows && gk + 8u <= k) {
      regs[i] = *reinterpret_cast<const u32x4*>(g + (uint64_t)gr * k + gk);
    } else {
      uint32_t w[4] = {0, 0, 0, 0};
      if (gr < rows) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (gk + e < k) w[e >> 1] |= (uint32_t)g[(uint64_t)gr * k + gk + e] << (16 * (e & 1));
      }
      regs[i] = u32x4{w[0], w[1], w[2], w[3]};
    }
  }
}

__device__ __forceinline__ void store_tile(uint16_t* lds, const u32x4 (&regs)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t id = threadIdx.x + 256u * i;
    uint32_t row = id >> 3, kc = id & 7u;
    *reinterpret_cast<u32x4*>(lds + row * kLdsRow + kc * 8u) = regs[i];
  }
}

template <bool kFullK, bool kSilu>
__device__ __forceinline__ void contract_bf16_body(const uint16_t* __restrict__ a,
                                                   const uint16_t* __restrict__ b, uint32_t m,
                                                   uint32_t n, uint32_t k,
                                                   uint16_t* __restrict__ c) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][kBM * kLdsRow];  // [buf][A|B]
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t wm = (wave >> 1) * 64u, wn = (wave & 1u) * 64u;  // wave's 64x64 sub-tile
  const uint32_t m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  u32x4 ra[4], rb[4];
  load_tile<kFullK>(a, m, k, m0, 0, ra);
  load_tile<kFullK>(b, n, k, n0, 0, rb);
  store_tile(lds[0][0], ra);
  store_tile(lds[0][1], rb);
  __syncthreads();

  const uint32_t ktiles = (k + kBK - 1) / kBK;
  for (uint32_t kt = 0; kt < ktiles; ++kt) {
    const uint32_t cur = kt & 1u;
    const bool more = kt + 1 < ktiles;
    if (more) {
      load_tile<kFullK>(a, m, k, m0, (kt + 1) * kBK, ra);
      load_tile<kFullK>(b, n, k, n0, (kt + 1) * kBK, rb);
    }
    const uint16_t* la = lds[cur][0];
    const uint16_t* lb = lds[cur][1];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      // lane holds row (lane%32), k slice [(lane/32)*8, +8) of the 32x16 step
      const uint32_t kofs = ks * 16u + (lane >> 5) * 8u;
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(
            la + (wm + i * 32u + (lane & 31u)) * kLdsRow + kofs));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        fb[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(
            lb + (wn + j * 32u + (lane & 31u)) * kLdsRow + kofs));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      store_tile(lds[cur ^ 1u][0], ra);
      store_tile(lds[cur ^ 1u][1], rb);
    }
    __syncthreads();
  }

  // Epilogue: acc[i][j][r] is C[wm + 32i + (r/4)*8 + (lane/32)*4 + r%4][wn + 32j + lane%32].
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        uint32_t row = m0 + wm + i * 32u + (r >> 2) * 8u + (lane >> 5) * 4u + (r & 3);
        uint32_t col = n0 + wn + j * 32u + (lane & 31u);
        float v = acc[i][j][r];
        if (kSilu) v = tiler::silu_f32(v);
        if (row < m && col < n) c[(uint64_t)row * n + col] = (uint16_t)tiler::bf16_narrow(v);
      }
}

}  // namespace

#define TILER_CONTRACT_BF16(NAME, FULLK, SILU)                                                 \
  extern "C" __global__ void __launch_bounds__(256)                                            \
      NAME(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m,         \
           uint32_t n, uint32_t k, uint16_t* __restrict__ c) {                                  \
    contract_bf16_body<FULLK, SILU>(a, b, m, n, k, c);                                          \
  }
TILER_CONTRACT_BF16(tiler_contract_bf16_t128, true, false)
TILER_CONTRACT_BF16(tiler_contract_bf16_silu_t128, true, true)
TILER_CONTRACT_BF16(tiler_contract_bf16_t128_k, false, false)
TILER_CONTRACT_BF16(tiler_contract_bf16_silu_t128_k, false, true)
