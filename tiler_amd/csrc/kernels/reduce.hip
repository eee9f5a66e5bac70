// Sum-reduction realizations (the strict-serial-sum-f32 family) for gfx950.
//
// Four topologies, one per ReductionTopology the planner can select
// (tiler-ir/src/schedule/model.rs:1327-1555):
//   * tiler_sum_f32_serial       Serial: one invocation per output, the strict
//                                left fold of tiler-reference/src/evaluate.rs:498-589.
//   * tiler_sum_f32_partials     MultiPass pass 1: one invocation per
//                                (output, partition), evaluate.rs:612-776; pass 2
//                                is tiler_sum_f32_serial over the partials.
//   * tiler_sum_f32_cooperative  CooperativeWorkgroup: one workgroup per output
//                                with a declared (participants, contributors,
//                                rounds, layout) grouping, evaluate.rs:845-1158.
//   * tiler_sum_f32_grid(+final)/ The reassociating two-level tree (a
//     tiler_sum_f32_rows         REASSOCIATE-class contract): wave64 xor
//                                butterflies, an ascending cross-wave fold in LDS
//                                and, for one output, a second one-workgroup
//                                launch combining the workgroup partials.
// The first three are bit-exact with the reference; the tree's exact order is
// its declared grouping, restated by the oracle's grid/row grouped sums.
#include "common.h"

using tiler::canon;

// ---------------------------------------------------------------------------
// Serial: out[o*inner+i] = strict fold over p of x[(o*extent+p)*inner+i].
// Seeding at -0.0 and adding every contributor equals seeding at the first
// contributor bit for bit (-0.0 is the exact additive identity under
// round-to-nearest), NaN payloads aside, which the commit canonicalizes.
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_serial(const float* __restrict__ x, uint64_t outer, uint64_t extent,
                     uint64_t inner, float* __restrict__ out) {
  uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= outer * inner) return;
  uint64_t o = id / inner, i = id - o * inner;
  const float* base = x + o * extent * inner + i;
  float acc = -0.0f;
  for (uint64_t p = 0; p < extent; ++p) acc = acc + base[p * inner];
  out[id] = extent == 0 ? 0.0f : canon(acc);
}

// MultiPass pass 1: partials[r*P + p] = strict fold of
// x[r*extent + p*chunk .. +chunk]; an empty partition commits +0.0.
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_partials(const float* __restrict__ x, uint64_t rows, uint64_t extent,
                       uint64_t partitions, uint64_t chunk, float* __restrict__ partials) {
  uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * partitions) return;
  uint64_t r = id / partitions, p = id - r * partitions;
  const float* base = x + r * extent + p * chunk;
  float acc = -0.0f;
  for (uint64_t w = 0; w < chunk; ++w) acc = acc + base[w];
  partials[id] = chunk == 0 ? 0.0f : canon(acc);
}

// CooperativeWorkgroup: one workgroup per row; blockDim.x == participants.
// Round r: participant p folds cell (RoundMajor r*P+p | ParticipantMajor p*R+r)
// of `chunk` contributors; staged partials go to LDS; participant 0 folds them
// in ascending p and accumulates round totals in ascending r -- the single
// workgroup tree of tiler-metal's cooperative_workgroup_reduction golden.
extern "C" __global__ void __launch_bounds__(1024)
tiler_sum_f32_cooperative(const float* __restrict__ x, uint64_t extent, uint32_t participants,
                          uint64_t chunk, uint64_t rounds, uint32_t participant_major,
                          float* __restrict__ out) {
  __shared__ float staged[1024];
  const uint32_t p = threadIdx.x;
  const float* row = x + (uint64_t)blockIdx.x * extent;
  float total = -0.0f;
  for (uint64_t r = 0; r < rounds; ++r) {
    uint64_t cell = participant_major ? (uint64_t)p * rounds + r : r * participants + p;
    const float* range = row + cell * chunk;
    float partial = -0.0f;
    for (uint64_t w = 0; w < chunk; ++w) partial = partial + range[w];
    staged[p] = partial;
    __syncthreads();
    if (p == 0) {
      float s = -0.0f;
      for (uint32_t q = 0; q < participants; ++q) s = s + staged[q];
      total = total + s;
    }
    __syncthreads();
  }
  if (p == 0) out[blockIdx.x] = canon(total);
}

// ---------------------------------------------------------------------------
// Reassociating tree.
//
// In-workgroup combine of 256 thread partials: per-wave xor butterfly, then the
// four wave sums in ascending wave order.
__device__ __forceinline__ float block_sum256(float v, float* lds4) {
  v = tiler::wave_sum_butterfly(v);
  const uint32_t t = threadIdx.x;
  if ((t & 63u) == 0) lds4[t >> 6] = v;
  __syncthreads();
  float s = lds4[0];
  s = s + lds4[1];
  s = s + lds4[2];
  s = s + lds4[3];
  return s;
}

// One output over n contributors, two launches.  Tile = 1024 elements
// (256 threads x 4); stage 1: workgroup b folds tiles b, b+G, ... in
// ascending (tile, component) order per thread and writes its partial;
// stage 2 (one workgroup): thread t folds partials t, t+256, ..., then the
// same in-workgroup combine.  The kernel boundary orders the partials: no
// device-scope fence is taken per workgroup (each costs an L2 write-back).
template <bool kAligned>
__device__ __forceinline__ void sum_stage1_body(const float* __restrict__ x, uint64_t n,
                                                float* __restrict__ partials) {
  __shared__ float lds4[4];
  const uint32_t t = threadIdx.x, b = blockIdx.x, G = gridDim.x;
  const uint64_t tiles = (n + 1023) >> 10;
  const uint64_t full = n >> 10;
  float acc = -0.0f;
  uint64_t tile = b;
  if (kAligned) {
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
    for (; tile + 3ull * G < full; tile += 4ull * G) {
      f32x4 v0 = __builtin_nontemporal_load(&x4[(tile) * 256 + t]);
      f32x4 v1 = __builtin_nontemporal_load(&x4[(tile + G) * 256 + t]);
      f32x4 v2 = __builtin_nontemporal_load(&x4[(tile + 2ull * G) * 256 + t]);
      f32x4 v3 = __builtin_nontemporal_load(&x4[(tile + 3ull * G) * 256 + t]);
      acc = acc + v0.x; acc = acc + v0.y; acc = acc + v0.z; acc = acc + v0.w;
      acc = acc + v1.x; acc = acc + v1.y; acc = acc + v1.z; acc = acc + v1.w;
      acc = acc + v2.x; acc = acc + v2.y; acc = acc + v2.z; acc = acc + v2.w;
      acc = acc + v3.x; acc = acc + v3.y; acc = acc + v3.z; acc = acc + v3.w;
    }
    for (; tile < full; tile += G) {
      f32x4 v0 = __builtin_nontemporal_load(&x4[tile * 256 + t]);
      acc = acc + v0.x; acc = acc + v0.y; acc = acc + v0.z; acc = acc + v0.w;
    }
  }
  for (; tile < tiles; tile += G) {
    uint64_t base = (tile << 10) + 4ull * t;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (base + e < n) acc = acc + x[base + e];
  }
  float s = block_sum256(acc, lds4);
  if (t == 0) partials[b] = s;
}

extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_grid(const float* __restrict__ x, uint64_t n, float* __restrict__ partials) {
  sum_stage1_body<true>(x, n, partials);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_grid_unaligned(const float* __restrict__ x, uint64_t n,
                             float* __restrict__ partials) {
  sum_stage1_body<false>(x, n, partials);
}
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_grid_final(const float* __restrict__ partials, uint32_t G, uint64_t n,
                         float* __restrict__ out) {
  __shared__ float lds4[4];
  float acc = -0.0f;
  for (uint32_t i = threadIdx.x; i < G; i += 256) acc = acc + partials[i];
  float total = block_sum256(acc, lds4);
  if (threadIdx.x == 0) out[0] = n == 0 ? 0.0f : canon(total);
}

// Many outputs: one 256-thread workgroup per row of `extent` contributors,
// grouping (vec 4, waves 4): thread t folds elements p with (p/4)%256 == t in
// ascending p, then block_sum256.
extern "C" __global__ void __launch_bounds__(256)
tiler_sum_f32_rows(const float* __restrict__ x, uint64_t extent, float* __restrict__ out) {
  __shared__ float lds4[4];
  const uint32_t t = threadIdx.x;
  const float* row = x + (uint64_t)blockIdx.x * extent;
  float acc = -0.0f;
  for (uint64_t base = 0; base < extent; base += 1024) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint64_t p = base + 4ull * t + e;
      if (p < extent) acc = acc + row[p];
    }
  }
  float s = block_sum256(acc, lds4);
  if (t == 0) out[blockIdx.x] = extent == 0 ? 0.0f : canon(s);
}
