// Tensor contraction C[m, n] = sum_k A[m, k] * B[n, k]  (td,od->to) for gfx950.
//
// * tiler_contract_strict_f32 -- the governed strict contraction
//   (tiler-reference/src/contraction.rs:558-630): per output, p = fl(a*b),
//   seeded at the first product, acc = fl(acc + p) over ascending k, no FMA.
//   16x16 LDS tiles with a serial in-tile fold, the shape of tiler-metal's
//   contraction_tiled_cooperative golden; bit-exact with the reference.
// * tiler_contract_bf16_{,silu_}t256 / t128 -- the cooperative bf16
//   contraction on MFMA (v_mfma_f32_16x16x32_bf16), LDS-staged by buffer
//   loads: bf16 operands, f32 accumulation, an optional fused SiLU epilogue on
//   the f32 accumulator (the reference SiLU: bf16(silu_f32(acc)) exactly, via
//   tiler::silu_for_bf16), one bf16 narrowing.  Any m; n and k multiples of 8.
// * tiler_contract_bf16_{,silu_}skinny{1..4} -- m <= 64 (decode shapes): B
//   streamed once into registers, k split over 16 waves, LDS reduction.
// * tiler_contract_bf16_{,silu_}g128[_k] -- the guarded general form
//   (v_mfma_f32_32x32x16_bf16, register-staged) for any n and k: out-of-range
//   operand elements are zero-filled, out-of-range outputs are not stored.
#include "common.h"
#include "contract_geometry.h"

using tiler::canon;

// ---------------------------------------------------------------------------
// Strict contraction.  T = float: the f32 family.  T = uint16_t: bf16
// operands widened exactly to binary32, the same fold, then (optionally) the
// reference SiLU and one bf16 narrowing -- the realization of a bf16
// contraction region whose contract grants no reassociation (the MFMA forms
// below regroup the k sum).
template <typename T, bool kSilu>
__device__ __forceinline__ void contract_strict_body(const T* __restrict__ a, const T* __restrict__ b,
                                                     uint32_t m, uint32_t n, uint32_t k, T* __restrict__ c) {
  constexpr bool kBf16 = sizeof(T) == 2;
  __shared__ float as[16][17];
  __shared__ float bs[16][17];
  const uint32_t tx = threadIdx.x & 15u, ty = threadIdx.x >> 4;
  const uint32_t i0 = blockIdx.y * 16u, j0 = blockIdx.x * 16u;
  auto widen = [](T v) -> float {
    if constexpr (kBf16) return tiler::bf16_widen(v);
    else return v;
  };
  float acc = -0.0f;  // -0 + first product == first product, bit for bit
  for (uint32_t k0 = 0; k0 < k; k0 += 16) {
    uint32_t kk = k0 + tx;
    as[ty][tx] = (i0 + ty < m && kk < k) ? widen(a[(uint64_t)(i0 + ty) * k + kk]) : 0.0f;
    bs[ty][tx] = (j0 + ty < n && kk < k) ? widen(b[(uint64_t)(j0 + ty) * k + kk]) : 0.0f;
    __syncthreads();
    const uint32_t steps = (k - k0) < 16u ? (k - k0) : 16u;
    for (uint32_t s = 0; s < steps; ++s) {
      float p = as[ty][s] * bs[tx][s];
      acc = acc + p;
    }
    __syncthreads();
  }
  if (i0 + ty < m && j0 + tx < n) {
    float v = canon(acc);
    if (kSilu) v = tiler::silu_f32(v);
    if constexpr (kBf16) c[(uint64_t)(i0 + ty) * n + j0 + tx] = (uint16_t)tiler::bf16_narrow(v);
    else c[(uint64_t)(i0 + ty) * n + j0 + tx] = v;
  }
}

extern "C" __global__ void __launch_bounds__(256)
tiler_contract_strict_f32(const float* __restrict__ a, const float* __restrict__ b, uint32_t m,
                          uint32_t n, uint32_t k, float* __restrict__ c) {
  contract_strict_body<float, false>(a, b, m, n, k, c);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_strict_bf16(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m,
                           uint32_t n, uint32_t k, uint16_t* __restrict__ c) {
  contract_strict_body<uint16_t, false>(a, b, m, n, k, c);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_strict_bf16_silu(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m,
                                uint32_t n, uint32_t k, uint16_t* __restrict__ c) {
  contract_strict_body<uint16_t, true>(a, b, m, n, k, c);
}

// Register-blocked: a workgroup of 16 x 16 threads owns a (16 TM) x (16 TN)
// output tile and each thread TM x TN outputs (rows ty*TM.., columns
// tx*TN..), every one of them the same ascending first-product fold; the
// TM*TN chains of a thread interleave, so the dependent adds do not wait on
// one another.  A and B k-tiles of 16 are loaded into registers one tile
// ahead (coalesced along k) and stored transposed (k-major) into the other
// LDS buffer, so each k step reads TM values of A and TN of B per thread for
// TM*TN products.  Only k steps below k are folded: the zeros loaded past k
// never enter a chain (a +0.0 product would turn a -0.0 total into +0.0).
//
// T = uint16_t: bf16 operands widened exactly on load, then (kSilu) the
// reference SiLU and one bf16 narrowing on commit -- the strict bf16 form.
template <int TM, int TN, typename T = float, bool kSilu = false>
__device__ __forceinline__ void contract_strict_blocked_body(const T* __restrict__ a, const T* __restrict__ b,
                                                             uint32_t m, uint32_t n, uint32_t k,
                                                             T* __restrict__ c) {
  constexpr bool kBf16 = sizeof(T) == 2;
  auto widen = [](T v) -> float {
    if constexpr (kBf16) return tiler::bf16_widen(v);
    else return v;
  };
  constexpr uint32_t BM = 16 * TM, BN = 16 * TN, BK = 16;
  __shared__ __align__(16) float as[2][BK][BM + 4];
  __shared__ __align__(16) float bs[2][BK][BN + 4];
  const uint32_t t = threadIdx.x, tx = t & 15u, ty = t >> 4;
  const uint32_t i0 = blockIdx.y * BM, j0 = blockIdx.x * BN;
  float ra[TM], rb[TN];  // this thread's share of the next k-tile: element t + 256 q
  auto load = [&](uint32_t k0) {
#pragma unroll
    for (uint32_t q = 0; q < TM; ++q) {
      const uint32_t e = t + 256u * q, r = e / BK, kk = k0 + e % BK;
      ra[q] = (i0 + r < m && kk < k) ? widen(a[(uint64_t)(i0 + r) * k + kk]) : 0.0f;
    }
#pragma unroll
    for (uint32_t q = 0; q < TN; ++q) {
      const uint32_t e = t + 256u * q, r = e / BK, kk = k0 + e % BK;
      rb[q] = (j0 + r < n && kk < k) ? widen(b[(uint64_t)(j0 + r) * k + kk]) : 0.0f;
    }
  };
  auto store = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t q = 0; q < TM; ++q) {
      const uint32_t e = t + 256u * q;
      as[buf][e % BK][e / BK] = ra[q];
    }
#pragma unroll
    for (uint32_t q = 0; q < TN; ++q) {
      const uint32_t e = t + 256u * q;
      bs[buf][e % BK][e / BK] = rb[q];
    }
  };
  float acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = -0.0f;  // -0 + first product == first product
  const uint32_t tiles = (k + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  for (uint32_t kt = 0; kt < tiles; ++kt) {
    const uint32_t buf = kt & 1u;
    if (kt + 1 < tiles) load((kt + 1) * BK);
    const uint32_t steps = k - kt * BK < BK ? k - kt * BK : BK;
    for (uint32_t s = 0; s < steps; ++s) {
      float fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = as[buf][s][ty * TM + i];
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = bs[buf][s][tx * TN + j];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc[i][j] + fa[i] * fb[j];
    }
    if (kt + 1 < tiles) store(buf ^ 1u);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const uint32_t row = i0 + ty * TM + i;
    if (row >= m) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint32_t col = j0 + tx * TN + j;
      if (col >= n) continue;
      float v = canon(acc[i][j]);
      if (kSilu) v = tiler::silu_f32(v);
      if constexpr (kBf16) c[(uint64_t)row * n + col] = (uint16_t)tiler::bf16_narrow(v);
      else c[(uint64_t)row * n + col] = v;
    }
  }
}

extern "C" __global__ void __launch_bounds__(256)
tiler_contract_strict_f32_b16(const float* __restrict__ a, const float* __restrict__ b, uint32_t m, uint32_t n,
                              uint32_t k, float* __restrict__ c) {
  contract_strict_blocked_body<1, 1>(a, b, m, n, k, c);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_contract_strict_f32_b32(const float* __restrict__ a, const float* __restrict__ b, uint32_t m, uint32_t n,
                              uint32_t k, float* __restrict__ c) {
  contract_strict_blocked_body<2, 2>(a, b, m, n, k, c);
}
#define TILER_CONTRACT_STRICT_BF16_BLOCKED(EDGE, T)                                                    \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_contract_strict_bf16_b##EDGE(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,\
                                         uint32_t m, uint32_t n, uint32_t k, uint16_t* __restrict__ c) {\
    contract_strict_blocked_body<T, T, uint16_t, false>(a, b, m, n, k, c);                            \
  }                                                                                                    \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_contract_strict_bf16_silu_b##EDGE(const uint16_t* __restrict__ a,                          \
                                              const uint16_t* __restrict__ b, uint32_t m, uint32_t n,  \
                                              uint32_t k, uint16_t* __restrict__ c) {                  \
    contract_strict_blocked_body<T, T, uint16_t, true>(a, b, m, n, k, c);                             \
  }
TILER_CONTRACT_STRICT_BF16_BLOCKED(16, 1)
TILER_CONTRACT_STRICT_BF16_BLOCKED(32, 2)
TILER_CONTRACT_STRICT_BF16_BLOCKED(64, 4)

extern "C" __global__ void __launch_bounds__(256)
tiler_contract_strict_f32_b64(const float* __restrict__ a, const float* __restrict__ b, uint32_t m, uint32_t n,
                              uint32_t k, float* __restrict__ c) {
  contract_strict_blocked_body<4, 4>(a, b, m, n, k, c);
}

// Few output rows: output row i = blockIdx.y is the staged strict fold
// (tiler_sum_f32_staged_r*, reduce.hip) of the products of A's row i with B's
// rows, which are contiguous in k -- the same first-product fold, ascending k,
// two roundings per step, bit for bit.  R output columns per workgroup; R in
// {1, 4, 16} relay-fold the staged products (staged_relay_body), R = 64 folds
// a row per lane (staged_fold_body).
#define TILER_CONTRACT_STRICT_ROWS(R, BODY)                                                            \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_contract_strict_f32_s##R(const float* __restrict__ a, const float* __restrict__ b,          \
                                     uint32_t m, uint32_t n, uint32_t k, float* __restrict__ c) {      \
    (void)m;                                                                                           \
    const uint64_t i = blockIdx.y;                                                                     \
    BODY<R, true, true>(b, n, k, a + i * k, c + i * n);                                                \
  }                                                                                                    \
  extern "C" __global__ void __launch_bounds__(256)                                                    \
      tiler_contract_strict_f32_s##R##_u(const float* __restrict__ a, const float* __restrict__ b,      \
                                         uint32_t m, uint32_t n, uint32_t k, float* __restrict__ c) {  \
    (void)m;                                                                                           \
    const uint64_t i = blockIdx.y;                                                                     \
    BODY<R, false, true>(b, n, k, a + i * k, c + i * n);                                               \
  }
TILER_CONTRACT_STRICT_ROWS(1, staged_relay_body)
TILER_CONTRACT_STRICT_ROWS(4, staged_relay_body)
TILER_CONTRACT_STRICT_ROWS(16, staged_relay_body)
TILER_CONTRACT_STRICT_ROWS(64, staged_lane_body)

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
                                                   uint16_t* __restrict__ c, uint32_t m_tile) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][kBM * kLdsRow];  // [buf][A|B]
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t wm = (wave >> 1) * 64u, wn = (wave & 1u) * 64u;  // wave's 64x64 sub-tile
  const uint32_t m0 = m_tile * kBM, n0 = blockIdx.x * kBN;

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

// ---------------------------------------------------------------------------
// Staged bf16 contraction: any m >= 1, n and k multiples of 8, 16-byte aligned
// operands, 256 * k * 2 < 2^31 (the host checks all of it).
//
// One workgroup per TILE x TILE output tile (TILE 256: 16 waves in a 4 x 4
// grid; TILE 128: 4 waves in 2 x 2), wave (wm, wn) owning a 64 x 64 sub-tile as
// 4 x 4 accumulator blocks of v_mfma_f32_16x16x32_bf16 (64 f32 per lane).
// The 16x16x32 form moves half the accumulator data per flop of the 32x32x16
// one; with Gaussian operands the chip is power-limited, and that runs it at a
// higher clock.  The host takes TILE 128 when 256-tiles would leave CUs idle.
//
// Operands: each workgroup's TILE-row A and B panels are addressed through one
// buffer resource apiece (32-bit offsets; the record count stops at the last
// real row, so rows past m or n load as zeros) and move global -> LDS with
// buffer_load_dwordx4 ... lds, in TILE x 64 tiles double-buffered.  LDS rows
// are 128 B; 16-byte chunk c of row r sits at chunk c ^ ((r >> 1) & 7), so the
// 16 rows one ds_read_b128 phase touches cover all 64 banks.  When k is not a
// multiple of 64, the last tile's fragments past k are zeroed in both operands
// (the bytes loaded there belong to the next row).
//
// Schedule per 64-deep k tile: two k steps of 32, each eight fragment reads
// and sixteen MFMAs (the compiler waits per fragment, so the MFMAs start as
// their operands land); the barrier that retires the stage follows, and the
// refill of that stage with tile kt+2 is issued right after it.
//
// Tile order is XCD-aware: the 8 XCDs receive workgroups round robin, and the
// 32 that one XCD runs together form a 4 x 8 block of tiles that share 4 A and
// 8 B panels in that XCD's L2.  The epilogue (optional SiLU on the f32
// accumulator, then one bf16 narrowing) transposes through LDS so C leaves in
// 16-byte row chunks; rows past m and chunks past n are not stored.
namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kK = 64;

// Epilogue store word for a pair of adjacent output rows.  Lanes 2c and 2c+1
// of a 16x16 MFMA block hold the same two rows (v0: row r, v1: row r+1) of
// columns 2c and 2c+1.  Each lane narrows its (v0, v1) with
// v_cvt_pk_bf16_f32, which rounds to nearest even exactly like the ADR 0091
// narrowing for every non-NaN input (NaNs are made canonical first, since
// the instruction keeps a NaN's sign and payload; kCanon = false skips that
// where every NaN lane is rewritten afterwards); a DPP quad_perm [1,0,3,2]
// swaps the packed words between the two lanes, and v_perm_b32 forms the
// 32-bit column pair: row r of columns 2c, 2c+1 on the even lane, row r+1 on
// the odd one.  sel is 0x05040100 on even lanes, 0x03020706 on odd lanes.
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
template <bool kCanon = true>
__device__ __forceinline__ uint32_t pack_row_pair(float v0, float v1, uint32_t sel) {
  const float qnan = __uint_as_float(0x7fc00000u);
  const f32x2v f = {kCanon && v0 != v0 ? qnan : v0, kCanon && v1 != v1 ? qnan : v1};
  const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2v));
  const uint32_t q = (uint32_t)__builtin_amdgcn_mov_dpp((int)p, 0xB1, 0xF, 0xF, true);
  return __builtin_amdgcn_perm(q, p, sel);
}

// One value's bf16 bits, narrowed as pack_row_pair narrows.
__device__ __forceinline__ uint16_t narrow_one(float v) {
  const float qnan = __uint_as_float(0x7fc00000u);
  const f32x2v f = {v != v ? qnan : v, 0.0f};
  return (uint16_t)__builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2v));
}

// Row pair p = 8i + 2j + r/2 of a wave's 4 x 4 MFMA blocks (accumulators
// r, r+1 of block (i, j)), p wave-uniform: a scalar branch per case, which
// needs neither indexed registers nor private memory.
__device__ __forceinline__ void accumulator_pair(const f32x4 (&acc)[4][4], uint32_t p, float& x0, float& x1) {
  switch (p) {
#define TILER_PAIR_CASE(t)                         \
  case t:                                          \
    x0 = acc[(t) >> 3][((t) >> 1) & 3][((t)&1) * 2]; \
    x1 = acc[(t) >> 3][((t) >> 1) & 3][((t)&1) * 2 + 1]; \
    return;
    TILER_PAIR_CASE(0) TILER_PAIR_CASE(1) TILER_PAIR_CASE(2) TILER_PAIR_CASE(3)
    TILER_PAIR_CASE(4) TILER_PAIR_CASE(5) TILER_PAIR_CASE(6) TILER_PAIR_CASE(7)
    TILER_PAIR_CASE(8) TILER_PAIR_CASE(9) TILER_PAIR_CASE(10) TILER_PAIR_CASE(11)
    TILER_PAIR_CASE(12) TILER_PAIR_CASE(13) TILER_PAIR_CASE(14) TILER_PAIR_CASE(15)
    TILER_PAIR_CASE(16) TILER_PAIR_CASE(17) TILER_PAIR_CASE(18) TILER_PAIR_CASE(19)
    TILER_PAIR_CASE(20) TILER_PAIR_CASE(21) TILER_PAIR_CASE(22) TILER_PAIR_CASE(23)
    TILER_PAIR_CASE(24) TILER_PAIR_CASE(25) TILER_PAIR_CASE(26) TILER_PAIR_CASE(27)
    TILER_PAIR_CASE(28) TILER_PAIR_CASE(29) TILER_PAIR_CASE(30)
#undef TILER_PAIR_CASE
    default:
      x0 = acc[3][3][2];
      x1 = acc[3][3][3];
  }
}

// s_waitcnt immediates (gfx9 layout: vmcnt [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8]); a field at its maximum does not wait.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int kWaitVmLgkm0 = 0x0070;  // vmcnt(0) lgkmcnt(0)
constexpr int kWaitLgkm0 = 0xC07F;    // lgkmcnt(0)

// Issues this wave's share of one TILE x 64 operand tile: load j fills rows
// R = (wave * LOADS + j) * 8 .. R + 7 of the LDS tile, lane i the physical
// chunk i % 8 of row R + i / 8.  voff[j] is that lane's byte offset in the
// panel at k = 0 (with the chunk swizzle applied); k0_bytes moves along k.
// The k offset is part of the per-lane offset, not the scalar one: the
// buffer range check counts the per-lane offset only, so this way the
// panel's record count bounds every byte read (a ragged last k-tile's
// chunks past the panel's last row load as zeros, never past the operand).
template <int LOADS>
__device__ __forceinline__ void issue_operand_tile(__amdgpu_buffer_rsrc_t panel, const uint32_t* voff,
                                                   uint32_t k0_bytes, uint16_t* lds_tile,
                                                   uint32_t wave_s) {
#pragma unroll
  for (int j = 0; j < LOADS; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        panel, (lds_void*)(lds_tile + (wave_s * LOADS + j) * 8u * kK), 16, voff[j] + k0_bytes, 0, 0, 0);
}

// kRaggedK = false: k is a multiple of 64 (the planner's guarantee), so the
// last tile needs no masking -- and without that code the SiLU form fits its
// registers without spilling in the last tile.
template <int TILE, bool kSilu, bool kRaggedK = true>
__device__ __forceinline__ void contract_bf16_staged_body(const uint16_t* __restrict__ a,
                                                          const uint16_t* __restrict__ b,
                                                          uint32_t m, uint32_t n, uint32_t k,
                                                          uint16_t* __restrict__ c) {
  constexpr int kGrid = TILE / 64;                    // waves per side
  constexpr int kWaves = kGrid * kGrid;
  constexpr int kLoads = TILE / 8 / kWaves;           // 8-row loads per wave per operand tile
  constexpr uint32_t kStageElems = 2u * TILE * kK;    // A tile then B tile, bf16 elements
  // The operand stages, then (SiLU) the exponent table of the epilogue's
  // exact path: a divergent lookup in LDS costs an LDS round trip, not a
  // global one, on the path every wave with a marked element waits for at
  // the end.  One array on purpose: with a second LDS object the compiler
  // can no longer tell the fragment reads from the in-flight LDS-DMA refill
  // and drains the refill (vmcnt(0)) before every tile.
  __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * kStageElems + (kSilu ? 256 : 0)];
  double* const silu_table = reinterpret_cast<double*>(smem + 2 * kStageElems);
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t wm = wave / kGrid, wn = wave % kGrid;
  // wave 0's table entry, loaded ahead of the operand tiles (loads retire in
  // order, so waiting for it later waits for nothing issued after it)
  double table_entry = 0.0;
  if (kSilu && wave_s == 0) table_entry = kExp2Table64[lane];

  // XCD-aware tile order: workgroup id -> (xcd, slot); xcd picks a 4x8 block
  // of the tile grid, slot a tile inside it.  Row-major when the grid is not a
  // whole number of 4x8 blocks per XCD.
  const uint32_t tiles_n = (n + TILE - 1) / TILE, tiles_m = (m + TILE - 1) / TILE;
  uint32_t tm, tn;
  {
    const uint32_t id = blockIdx.x;
    const uint32_t total = tiles_m * tiles_n;
    if (tiles_m % 4 == 0 && tiles_n % 8 == 0 && total % 256 == 0) {
      const uint32_t xcd = id & 7u, slot = id >> 3;          // slot: 0 .. total/8-1
      const uint32_t blocks_n = tiles_n / 8;                 // 4x8 blocks across n
      const uint32_t blk = xcd + 8u * (slot >> 5);           // block index
      const uint32_t in = slot & 31u;
      tm = (blk / blocks_n) * 4u + (in >> 3);
      tn = (blk % blocks_n) * 8u + (in & 7u);
    } else {
      tm = id / tiles_n;
      tn = id % tiles_n;
    }
  }
  const uint32_t m0 = tm * TILE, n0 = tn * TILE;
  const uint32_t ktiles = (k + kK - 1) / kK;
  const uint32_t k_last = k - (ktiles - 1) * kK;  // valid k in the last tile (a multiple of 8)

  const uint32_t rows_a = m - m0 < TILE ? m - m0 : TILE, rows_b = n - n0 < TILE ? n - n0 : TILE;
  const __amdgpu_buffer_rsrc_t pa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a + (uint64_t)m0 * k), (short)0, rows_a * k * 2u, 0x00020000);
  const __amdgpu_buffer_rsrc_t pb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(b + (uint64_t)n0 * k), (short)0, rows_b * k * 2u, 0x00020000);
  uint32_t voff[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const uint32_t row = (wave * kLoads + j) * 8u + (lane >> 3);
    voff[j] = row * k * 2u + ((lane & 7u) ^ ((row >> 1) & 7u)) * 16u;
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Fragment reads (v_mfma_f32_16x16x32_bf16): A block i covers rows
  // arow + 16i, lane group g = lane / 16 takes k elements 8g .. 8g+7 of the
  // 32-deep step, i.e. logical chunk 4s + g.
  const uint32_t arow = wm * 64u + (lane & 15u), brow = wn * 64u + (lane & 15u);
  const uint32_t grp = lane >> 4, swz = ((lane & 15u) >> 1) & 7u;  // (row >> 1) & 7 for row % 16 == lane % 16
  bf16x8 fa[4], fb[4];
  auto read_step = [&](const uint16_t* la, int step) {
    const uint16_t* lb = la + TILE * kK;
    const uint32_t chunk = ((uint32_t)step * 4u + grp) ^ swz;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(la + (arow + i * 16u) * kK + chunk * 8u));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      fb[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(lb + (brow + j * 16u) * kK + chunk * 8u));
  };
  // The last tile of a k that is not a multiple of 64: zero this lane's
  // fragments whose 8 k elements lie past k (both operands, so bytes from the
  // next row never meet a product).
  auto mask_step = [&](int step) {
    if ((uint32_t)step * 32u + grp * 8u >= k_last) {
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = as_bf16x8(u32x4{0, 0, 0, 0});
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = as_bf16x8(u32x4{0, 0, 0, 0});
    }
  };
  auto mfma_step = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
  };

  issue_operand_tile<kLoads>(pa, voff, 0, smem, wave_s);
  issue_operand_tile<kLoads>(pb, voff, 0, smem + TILE * kK, wave_s);
  if (ktiles > 1) {
    issue_operand_tile<kLoads>(pa, voff, kK * 2u, smem + kStageElems, wave_s);
    issue_operand_tile<kLoads>(pb, voff, kK * 2u, smem + kStageElems + TILE * kK, wave_s);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kLoads));  // tile 0's loads landed
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  asm volatile("s_barrier" ::: "memory");
  // read after the final barrier, past every ds_write the loop waits for
  if (kSilu && wave_s == 0) silu_table[lane] = table_entry;
  for (uint32_t kt = 0; kt + 1 < ktiles; ++kt) {
    const uint16_t* la = smem + (kt & 1u) * kStageElems;
    read_step(la, 0);
    mfma_step();
    read_step(la, 1);
    mfma_step();
    // Tile kt+1 landed (this wave's loads: vmcnt(0)) and this wave's reads of
    // stage kt retired (lgkmcnt(0)); after the barrier the stage may be
    // refilled.  The LDS drain is asm because the compiler relaxes a builtin
    // wait that no register use needs; the builtin after the barrier is
    // already satisfied and only tells the compiler nothing is outstanding.
    // No memory fence: one would drain the refill issued ahead (vmcnt(0)).
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    if (kt + 2 < ktiles) {
      uint16_t* st = smem + (kt & 1u) * kStageElems;
      issue_operand_tile<kLoads>(pa, voff, (kt + 2) * kK * 2u, st, wave_s);
      issue_operand_tile<kLoads>(pb, voff, (kt + 2) * kK * 2u, st + TILE * kK, wave_s);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  {  // the last tile, masked past k when k is not a multiple of 64
    const uint16_t* la = smem + ((ktiles - 1) & 1u) * kStageElems;
    read_step(la, 0);
    if (kRaggedK && k_last != (uint32_t)kK) mask_step(0);
    mfma_step();
    read_step(la, 1);
    if (kRaggedK && k_last != (uint32_t)kK) mask_step(1);
    mfma_step();
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmLgkm0);
  __syncthreads();  // every wave is done with the operand stages
  // Keep the epilogue out of the last tile's schedule: interleaved, its
  // temporaries meet the fragments and the accumulators and spill.
  __builtin_amdgcn_sched_barrier(0);

  // Epilogue: wave-private 64 x 64 bf16 region (8 KiB) with 128-B rows, chunk
  // q of row r at q ^ (r & 7).  Lanes 2c and 2c+1 hold adjacent columns of
  // rows r and r+1; one exchange lets each write a 32-bit column pair.
  // Lane-derived values come from an opaque copy of the lane index, so none
  // is computed before the loop ends (in the last tile every register holds
  // an accumulator or a fragment); the region base from the scalar wave index.
  uint32_t elane = lane;
  asm volatile("" : "+v"(elane));
  const uint32_t egrp = elane >> 4;
  uint16_t* cst = smem + wave_s * (64u * 64u);
  const bool odd = elane & 1u;
  const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
  // SiLU in two passes, so the hot code stays one straight line: pass 1
  // stores every element's fast value and marks in the wave-uniform `redo`
  // (bit p = 8i + 2j + r/2) the row pairs where some lane's value only
  // silu_f32 narrows right; pass 2 takes the marked pairs one at a time
  // through one shared copy of the reference code and overwrites those
  // lanes' bf16 (LDS writes of one wave land in issue order).
  uint32_t redo = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        float v0 = acc[i][j][r], v1 = acc[i][j][r + 1];
        if (kSilu) {
          uint64_t m0, m1;
          v0 = tiler::silu_bf16_fast_marked(v0, m0);
          v1 = tiler::silu_bf16_fast_marked(v1, m1);
          redo |= (uint32_t)((m0 | m1) != 0) << (i * 8 + j * 2 + r / 2);
        }
        const uint32_t row = i * 16u + egrp * 4u + r + (odd ? 1u : 0u);
        const uint32_t col = j * 16u + ((elane & 15u) & ~1u);
        const uint32_t q = (col >> 3) ^ (row & 7u);
        // Under SiLU a NaN fast value comes only from a marked input (NaN,
        // +-inf, beyond the fast domain), which pass 2 rewrites canonically.
        *reinterpret_cast<uint32_t*>(cst + row * 64u + q * 8u + (col & 7u)) = pack_row_pair<!kSilu>(v0, v1, sel);
      }
  if (kSilu) {
    while (redo != 0) {
      const uint32_t p = (uint32_t)__builtin_ctz(redo);
      redo &= redo - 1u;
      float xs[2];
      accumulator_pair(acc, p, xs[0], xs[1]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        bool exact;
        (void)tiler::silu_bf16_candidate(xs[h], exact);
        if (exact) {
          const uint32_t row = (p >> 3) * 16u + egrp * 4u + (p & 1u) * 2u + (uint32_t)h;
          const uint32_t col = ((p >> 1) & 3u) * 16u + (elane & 15u);
          cst[row * 64u + (((col >> 3) ^ (row & 7u)) * 8u) + (col & 7u)] = narrow_one(tiler::silu_f32(xs[h], silu_table));
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_wave_barrier();
  // from the scalar wave index: a vector copy would be live (or spilled) across the whole loop
  const uint32_t grow0 = m0 + (wave_s / kGrid) * 64u, gcol0 = n0 + (wave_s % kGrid) * 64u;
#pragma unroll 4
  for (int it = 0; it < 64 * 8 / 64; ++it) {
    const uint32_t qid = it * 64u + elane;
    const uint32_t row = qid >> 3, q = qid & 7u;
    if (grow0 + row < m && gcol0 + q * 8u < n) {
      u32x4 v = *reinterpret_cast<const u32x4*>(cst + row * 64u + ((q ^ (row & 7u)) * 8u));
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(c + (uint64_t)(grow0 + row) * n + gcol0 + q * 8u));
    }
  }
}

}  // namespace

#define TILER_CONTRACT_STAGED(TILE, WAVES)                                                          \
  extern "C" __global__ void __launch_bounds__(64 * WAVES)                                          \
      tiler_contract_bf16_t##TILE(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,    \
                                  uint32_t m, uint32_t n, uint32_t k, uint16_t* __restrict__ c) {   \
    contract_bf16_staged_body<TILE, false>(a, b, m, n, k, c);                                       \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(64 * WAVES)                                          \
      tiler_contract_bf16_silu_t##TILE(const uint16_t* __restrict__ a,                              \
                                       const uint16_t* __restrict__ b, uint32_t m, uint32_t n,      \
                                       uint32_t k, uint16_t* __restrict__ c) {                      \
    contract_bf16_staged_body<TILE, true>(a, b, m, n, k, c);                                        \
  }
TILER_CONTRACT_STAGED(256, 16)
TILER_CONTRACT_STAGED(128, 4)

// The same with k a multiple of 64 (no last-tile masking): *_kf.
#define TILER_CONTRACT_STAGED_KF(TILE, WAVES)                                                       \
  extern "C" __global__ void __launch_bounds__(64 * WAVES)                                          \
      tiler_contract_bf16_t##TILE##_kf(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, \
                                       uint32_t m, uint32_t n, uint32_t k, uint16_t* __restrict__ c) { \
    contract_bf16_staged_body<TILE, false, false>(a, b, m, n, k, c);                                \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(64 * WAVES)                                          \
      tiler_contract_bf16_silu_t##TILE##_kf(const uint16_t* __restrict__ a,                         \
                                            const uint16_t* __restrict__ b, uint32_t m, uint32_t n, \
                                            uint32_t k, uint16_t* __restrict__ c) {                 \
    contract_bf16_staged_body<TILE, true, false>(a, b, m, n, k, c);                                 \
  }
TILER_CONTRACT_STAGED_KF(256, 16)
TILER_CONTRACT_STAGED_KF(128, 4)

// ---------------------------------------------------------------------------
// Skinny bf16 contraction (m <= 64: decode-shaped), bandwidth-bound on B.
// One 1024-thread workgroup per 16 columns of n.  The 16 waves split k into
// 32-deep steps (wave w takes steps w, w + 16, ...); per step each lane loads
// its 16 bytes of the B columns straight into registers (every B element is
// used by one MFMA only, so LDS would add nothing) and of each 16-row block of
// A, and issues one v_mfma_f32_16x16x32_bf16 per block.  The 16 partial
// 16 x 16 tiles are added in LDS in ascending wave order; SiLU, one bf16
// narrowing and guarded 2-byte stores follow.  k a multiple of 8, 16-byte
// aligned A and B; rows past m and columns past n read as zeros.
namespace {

template <int MB, bool kSilu>
__device__ __forceinline__ void contract_bf16_skinny_body(const uint16_t* __restrict__ a,
                                                          const uint16_t* __restrict__ b,
                                                          uint32_t m, uint32_t n, uint32_t k,
                                                          uint16_t* __restrict__ c) {
  __shared__ f32x4 red[16][MB][64];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t n0 = blockIdx.x * 16u, col = lane & 15u, grp = lane >> 4;
  const bool bvalid = n0 + col < n;
  const uint16_t* brow = b + (uint64_t)(bvalid ? n0 + col : 0u) * k;
  f32x4 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t steps = (k + 31u) / 32u;
  const u32x4 zero = {0, 0, 0, 0};
#pragma unroll 4
  for (uint32_t s = wave; s < steps; s += 16u) {
    const uint32_t kk = s * 32u + grp * 8u;  // this lane's 8 k elements
    const bool kin = kk < k;
    const u32x4 bv = (bvalid && kin) ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(brow + kk)) : zero;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t row = mb * 16u + col;
      const u32x4 av = (row < m && kin) ? *reinterpret_cast<const u32x4*>(a + (uint64_t)row * k + kk) : zero;
      acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), acc[mb], 0, 0, 0);
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) red[wave][mb][lane] = acc[mb];
  __syncthreads();
  if (wave < (uint32_t)MB) {  // wave w finishes 16-row block w
    f32x4 t = red[0][wave][lane];
#pragma unroll
    for (int v = 1; v < 16; ++v) {
      const f32x4 u = red[v][wave][lane];
      t = f32x4{t.x + u.x, t.y + u.y, t.z + u.z, t.w + u.w};
    }
    const float tv[4] = {t.x, t.y, t.z, t.w};
    const uint32_t colg = n0 + col;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = wave * 16u + grp * 4u + i;
      const float v = kSilu ? tiler::silu_for_bf16(tv[i]) : tv[i];
      if (row < m && colg < n) c[(uint64_t)row * n + colg] = (uint16_t)tiler::bf16_narrow(v);
    }
  }
}

}  // namespace

#define TILER_CONTRACT_SKINNY(MB)                                                                   \
  extern "C" __global__ void __launch_bounds__(1024)                                                \
      tiler_contract_bf16_skinny##MB(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, \
                                     uint32_t m, uint32_t n, uint32_t k, uint16_t* __restrict__ c) { \
    contract_bf16_skinny_body<MB, false>(a, b, m, n, k, c);                                         \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(1024)                                                \
      tiler_contract_bf16_silu_skinny##MB(const uint16_t* __restrict__ a,                           \
                                          const uint16_t* __restrict__ b, uint32_t m, uint32_t n,   \
                                          uint32_t k, uint16_t* __restrict__ c) {                   \
    contract_bf16_skinny_body<MB, true>(a, b, m, n, k, c);                                          \
  }
TILER_CONTRACT_SKINNY(1)
TILER_CONTRACT_SKINNY(2)
TILER_CONTRACT_SKINNY(3)
TILER_CONTRACT_SKINNY(4)

#define TILER_CONTRACT_BF16(NAME, FULLK, SILU)                                                 \
  extern "C" __global__ void __launch_bounds__(256)                                            \
      NAME(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m,         \
           uint32_t n, uint32_t k, uint16_t* __restrict__ c) {                                  \
    contract_bf16_body<FULLK, SILU>(a, b, m, n, k, c, blockIdx.y);                              \
  }
TILER_CONTRACT_BF16(tiler_contract_bf16_g128, true, false)
TILER_CONTRACT_BF16(tiler_contract_bf16_silu_g128, true, true)
TILER_CONTRACT_BF16(tiler_contract_bf16_g128_k, false, false)
TILER_CONTRACT_BF16(tiler_contract_bf16_silu_g128_k, false, true)

// ---------------------------------------------------------------------------
// Batched forms (*_b): the kernels above over a batch of independent
// [m, k] x [n, k] -> [m, n] problems, each operand moved by the batch
// coordinate's strides (a stride of 0 shares an operand across that axis:
// one K for every head).  Batch b is blockIdx.y (staged, skinny) or
// blockIdx.y / m_tiles (g128, whose m tile is blockIdx.y % m_tiles).  The
// planner checks every moved base keeps the alignment the form assumes.
namespace {

__device__ __forceinline__ void batch_offsets(const tiler_geom::BatchGeometry& g, uint32_t batch, uint64_t& oa,
                                              uint64_t& ob, uint64_t& oc) {
  oa = ob = oc = 0;
  uint64_t rem = batch;
#pragma unroll
  for (int d = tiler_geom::kBatchAxes - 1; d >= 0; --d)
    if ((uint32_t)d < g.rank) {
      const uint64_t coord = rem % g.dims[d];
      rem /= g.dims[d];
      oa += coord * g.a_stride[d];
      ob += coord * g.b_stride[d];
      oc += coord * g.c_stride[d];
    }
}

}  // namespace

#define TILER_CONTRACT_BATCHED_STAGED(TILE, WAVES, SILU, NAME)                                      \
  extern "C" __global__ void __launch_bounds__(64 * WAVES)                                          \
      NAME(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m, uint32_t n,  \
           uint32_t k, uint16_t* __restrict__ c, tiler_geom::BatchGeometry g) {                    \
    uint64_t oa, ob, oc;                                                                            \
    batch_offsets(g, blockIdx.y, oa, ob, oc);                                                       \
    contract_bf16_staged_body<TILE, SILU>(a + oa, b + ob, m, n, k, c + oc);                         \
  }
TILER_CONTRACT_BATCHED_STAGED(256, 16, false, tiler_contract_bf16_t256_b)
TILER_CONTRACT_BATCHED_STAGED(256, 16, true, tiler_contract_bf16_silu_t256_b)
TILER_CONTRACT_BATCHED_STAGED(128, 4, false, tiler_contract_bf16_t128_b)
TILER_CONTRACT_BATCHED_STAGED(128, 4, true, tiler_contract_bf16_silu_t128_b)

#define TILER_CONTRACT_BATCHED_SKINNY(MB, SILU, NAME)                                               \
  extern "C" __global__ void __launch_bounds__(1024)                                                \
      NAME(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m, uint32_t n,  \
           uint32_t k, uint16_t* __restrict__ c, tiler_geom::BatchGeometry g) {                    \
    uint64_t oa, ob, oc;                                                                            \
    batch_offsets(g, blockIdx.y, oa, ob, oc);                                                       \
    contract_bf16_skinny_body<MB, SILU>(a + oa, b + ob, m, n, k, c + oc);                           \
  }
TILER_CONTRACT_BATCHED_SKINNY(1, false, tiler_contract_bf16_skinny1_b)
TILER_CONTRACT_BATCHED_SKINNY(2, false, tiler_contract_bf16_skinny2_b)
TILER_CONTRACT_BATCHED_SKINNY(3, false, tiler_contract_bf16_skinny3_b)
TILER_CONTRACT_BATCHED_SKINNY(4, false, tiler_contract_bf16_skinny4_b)
TILER_CONTRACT_BATCHED_SKINNY(1, true, tiler_contract_bf16_silu_skinny1_b)
TILER_CONTRACT_BATCHED_SKINNY(2, true, tiler_contract_bf16_silu_skinny2_b)
TILER_CONTRACT_BATCHED_SKINNY(3, true, tiler_contract_bf16_silu_skinny3_b)
TILER_CONTRACT_BATCHED_SKINNY(4, true, tiler_contract_bf16_silu_skinny4_b)

#define TILER_CONTRACT_BATCHED_G128(NAME, FULLK, SILU)                                              \
  extern "C" __global__ void __launch_bounds__(256)                                                 \
      NAME(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m, uint32_t n,  \
           uint32_t k, uint16_t* __restrict__ c, uint32_t m_tiles, tiler_geom::BatchGeometry g) {  \
    uint64_t oa, ob, oc;                                                                            \
    batch_offsets(g, blockIdx.y / m_tiles, oa, ob, oc);                                             \
    contract_bf16_body<FULLK, SILU>(a + oa, b + ob, m, n, k, c + oc, blockIdx.y % m_tiles);         \
  }
TILER_CONTRACT_BATCHED_G128(tiler_contract_bf16_g128_b, true, false)
TILER_CONTRACT_BATCHED_G128(tiler_contract_bf16_silu_g128_b, true, true)
TILER_CONTRACT_BATCHED_G128(tiler_contract_bf16_g128_k_b, false, false)
TILER_CONTRACT_BATCHED_G128(tiler_contract_bf16_silu_g128_k_b, false, true)
