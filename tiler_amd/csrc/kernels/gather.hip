// Indirect gather (tied embedding lookup) for gfx950.
//
// tiler-reference/src/structural.rs:513-606 (GatherF32Reference) with the
// bound rule of tiler-ir/src/semantic/gather.rs:438-455: the output is laid
// out [outer | index | inner]; each index selects one whole inner run of the
// source, which is moved byte for byte (no NaN canonicalization, no subnormal
// handling); an index >= extent -- or < 0 for a signed index type -- is never
// clamped or wrapped: the run is not written and the lowest offending index
// position is recorded in `bad` (a device-scope atomic minimum, initialised to
// UINT64_MAX by the host) so the committed dispatch reports the same position
// the reference's refusal names.
//
// One workgroup moves one output run at a time with 16-byte (or narrower)
// vector accesses: for the 8 KiB bf16 rows of the embedding table each of the
// 256 lanes issues two 16-byte loads and two 16-byte stores.
#include "common.h"

template <typename Unit>
__device__ __forceinline__ void gather_body(const Unit* __restrict__ src, uint64_t outer,
                                            uint64_t gathered, uint64_t run_units,
                                            const uint32_t* __restrict__ index, uint64_t count,
                                            uint32_t index_signed, Unit* __restrict__ out,
                                            unsigned long long* __restrict__ bad) {
  const uint64_t total_runs = outer * count;
  for (uint64_t run = blockIdx.x; run < total_runs; run += gridDim.x) {
    const uint64_t o = run / count;
    const uint64_t pos = run - o * count;
    const uint32_t raw = index[pos];
    const bool invalid = index_signed ? ((int32_t)raw < 0 || (uint64_t)(int32_t)raw >= gathered)
                                      : ((uint64_t)raw >= gathered);
    if (invalid) {
      if (threadIdx.x == 0) atomicMin(bad, (unsigned long long)pos);
      continue;
    }
    const Unit* s = src + (o * gathered + raw) * run_units;
    Unit* d = out + run * run_units;
    uint64_t u = threadIdx.x;
    for (; u + 3 * blockDim.x < run_units; u += 4 * blockDim.x) {
      Unit v0 = __builtin_nontemporal_load(&s[u]);
      Unit v1 = __builtin_nontemporal_load(&s[u + blockDim.x]);
      Unit v2 = __builtin_nontemporal_load(&s[u + 2 * blockDim.x]);
      Unit v3 = __builtin_nontemporal_load(&s[u + 3 * blockDim.x]);
      __builtin_nontemporal_store(v0, &d[u]);
      __builtin_nontemporal_store(v1, &d[u + blockDim.x]);
      __builtin_nontemporal_store(v2, &d[u + 2 * blockDim.x]);
      __builtin_nontemporal_store(v3, &d[u + 3 * blockDim.x]);
    }
    for (; u < run_units; u += blockDim.x) __builtin_nontemporal_store(__builtin_nontemporal_load(&s[u]), &d[u]);
  }
}

#define TILER_GATHER(NAME, UNIT)                                                              \
  extern "C" __global__ void __launch_bounds__(256)                                           \
      NAME(const UNIT* __restrict__ src, uint64_t outer, uint64_t gathered, uint64_t run_units, \
           const uint32_t* __restrict__ index, uint64_t count, uint32_t index_signed,         \
           UNIT* __restrict__ out, unsigned long long* __restrict__ bad) {                     \
    gather_body<UNIT>(src, outer, gathered, run_units, index, count, index_signed, out, bad);  \
  }
TILER_GATHER(tiler_gather_u128, u32x4)
TILER_GATHER(tiler_gather_u64, u32x2)
TILER_GATHER(tiler_gather_u32, uint32_t)
TILER_GATHER(tiler_gather_u16, uint16_t)
TILER_GATHER(tiler_gather_u8, uint8_t)
