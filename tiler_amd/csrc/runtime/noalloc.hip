// The no-allocation entry point's scratch: a file-scope device array each GPU
// holds from the library's load until the process ends.  Host code never
// passes `scratch` itself to a kernel (in host code the name is a host-side
// stand-in, not a device address): tiler_hip_bind resolves the array's device
// address once per device, with that device current, through
// hipGetSymbolAddress, and every use goes through that address.
//
// This translation unit is compiled by hipcc for gfx950 so the runtime
// registers the array; the library's kernels themselves stay in the offline
// code object and take the address as an argument.
#include <hip/hip_runtime.h>

#include "noalloc.h"

static __device__ __align__(256) unsigned char scratch[TILER_HIP_NOALLOC_SCRATCH_BYTES];

extern "C" int tiler_hip_noalloc_scratch_address(void** out) {
  *out = nullptr;
  return (int)hipGetSymbolAddress(out, HIP_SYMBOL(scratch));
}
