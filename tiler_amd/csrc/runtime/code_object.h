// Device-free reading of AMDGPU HSA code objects (ELF64), for
// validate-from-bytes (ADR 0090 item 8; tiler-runtime/src/adapter.rs:341).
#pragma once

#include <cstdint>
#include <string>

namespace tiler_hip {

struct KernelDescriptorFacts {
  uint32_t group_segment_bytes = 0;    // static LDS
  uint32_t private_segment_bytes = 0;  // scratch per lane
  uint32_t kernarg_bytes = 0;
};

// EF_AMDGPU_MACH value of gfx950 in e_flags.
constexpr uint32_t kMachGfx950 = 0x04f;

// Checks that `code` is a little-endian ELF64 AMDGPU HSA code object for
// gfx950 and, when `symbol` is non-null, that it defines the kernel symbol and
// its `.kd` descriptor.  On success fills `facts` from the descriptor.
// Returns an empty string on success, else the first disagreeing fact.
std::string inspect_code_object(const void* code, uint64_t bytes, const char* symbol,
                                KernelDescriptorFacts* facts, bool* absent_symbol);

}  // namespace tiler_hip
