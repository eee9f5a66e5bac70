// Size of the no-allocation entry point's per-GPU scratch array, and the
// call that resolves its device address (noalloc.hip).
#pragma once

// 8 MiB: the tree sum's workgroup partials (at most 4096 floats) and a
// multi-pass split of up to 2 Mi partials.
#define TILER_HIP_NOALLOC_SCRATCH_BYTES (8u << 20)

#ifdef __cplusplus
extern "C" {
#endif
// hipGetSymbolAddress of the array on the current device; 0 (hipSuccess) or
// the HIP error code.
int tiler_hip_noalloc_scratch_address(void** out);
#ifdef __cplusplus
}
#endif
