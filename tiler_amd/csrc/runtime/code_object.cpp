// Device-free code-object inspection: ELF64 header, section table, symbol
// tables and the AMDHSA kernel descriptor (group/private segment and kernarg
// sizes at byte offsets 0, 4 and 8 of the 64-byte descriptor).
#include "code_object.h"

#include <cstring>

namespace tiler_hip {
namespace {

template <typename T>
bool read(const uint8_t* base, uint64_t size, uint64_t off, T* out) {
  if (off > size || size - off < sizeof(T)) return false;
  std::memcpy(out, base + off, sizeof(T));
  return true;
}

struct Section {
  uint32_t name, type;
  uint64_t flags, addr, offset, size;
  uint32_t link, info;
  uint64_t align, entsize;
};

bool read_section(const uint8_t* b, uint64_t size, uint64_t off, Section* s) {
  return read(b, size, off + 0, &s->name) && read(b, size, off + 4, &s->type) &&
         read(b, size, off + 8, &s->flags) && read(b, size, off + 16, &s->addr) &&
         read(b, size, off + 24, &s->offset) && read(b, size, off + 32, &s->size) &&
         read(b, size, off + 40, &s->link) && read(b, size, off + 44, &s->info) &&
         read(b, size, off + 48, &s->align) && read(b, size, off + 56, &s->entsize);
}

}  // namespace

std::string inspect_code_object(const void* code, uint64_t bytes, const char* symbol,
                                KernelDescriptorFacts* facts, bool* absent_symbol) {
  if (absent_symbol) *absent_symbol = false;
  const uint8_t* b = static_cast<const uint8_t*>(code);
  if (!b || bytes < 64) return "payload shorter than an ELF64 header";
  if (!(b[0] == 0x7f && b[1] == 'E' && b[2] == 'L' && b[3] == 'F'))
    return "payload is not an ELF object";
  if (b[4] != 2) return "ELF class is not ELF64";
  if (b[5] != 1) return "ELF data is not little-endian";
  if (b[7] != 64) return "ELF OS/ABI is not AMDGPU HSA";
  uint16_t machine = 0;
  uint32_t flags = 0;
  uint64_t shoff = 0;
  uint16_t shentsize = 0, shnum = 0;
  read(b, bytes, 18, &machine);
  read(b, bytes, 48, &flags);
  read(b, bytes, 40, &shoff);
  read(b, bytes, 58, &shentsize);
  read(b, bytes, 60, &shnum);
  if (machine != 224) return "ELF machine is not EM_AMDGPU";
  if ((flags & 0xffu) != kMachGfx950) return "code object targets another processor than gfx950";
  if (!symbol) return "";
  if (shentsize != 64 || shnum == 0 || shoff > bytes ||
      (bytes - shoff) / shentsize < shnum)
    return "section header table out of bounds";

  const std::string want = symbol;
  const std::string want_kd = want + ".kd";
  bool found_fn = false, found_kd = false;
  uint64_t kd_value = 0;
  uint16_t kd_shndx = 0;
  for (uint16_t i = 0; i < shnum; ++i) {
    Section s;
    if (!read_section(b, bytes, shoff + (uint64_t)i * 64, &s)) return "section header unreadable";
    if (s.type != 2 && s.type != 11) continue;  // SHT_SYMTAB / SHT_DYNSYM
    if (s.entsize != 24 || s.offset > bytes || s.size > bytes - s.offset)
      return "symbol table out of bounds";
    Section strtab;
    if (s.link >= shnum || !read_section(b, bytes, shoff + (uint64_t)s.link * 64, &strtab))
      return "symbol string table unreadable";
    if (strtab.offset > bytes || strtab.size > bytes - strtab.offset)
      return "symbol string table out of bounds";
    for (uint64_t e = 0; e < s.size / 24; ++e) {
      uint64_t off = s.offset + e * 24;
      uint32_t name = 0;
      uint8_t info = 0;
      uint16_t shndx = 0;
      uint64_t value = 0;
      read(b, bytes, off, &name);
      read(b, bytes, off + 4, &info);
      read(b, bytes, off + 6, &shndx);
      read(b, bytes, off + 8, &value);
      if (name >= strtab.size) continue;
      const char* nm = reinterpret_cast<const char*>(b + strtab.offset + name);
      uint64_t maxlen = strtab.size - name;
      uint64_t len = 0;
      while (len < maxlen && nm[len]) ++len;
      if (len == maxlen) continue;
      if (len == want.size() && std::memcmp(nm, want.data(), len) == 0 && (info & 0xf) == 2)
        found_fn = true;
      if (len == want_kd.size() && std::memcmp(nm, want_kd.data(), len) == 0 &&
          (info & 0xf) == 1) {
        found_kd = true;
        kd_value = value;
        kd_shndx = shndx;
      }
    }
  }
  if (!found_fn || !found_kd) {
    if (absent_symbol) *absent_symbol = true;
    return "code object does not define kernel " + want + (found_fn ? " descriptor" : "");
  }
  Section kds;
  if (kd_shndx >= shnum || !read_section(b, bytes, shoff + (uint64_t)kd_shndx * 64, &kds))
    return "kernel descriptor section unreadable";
  if (kd_value < kds.addr) return "kernel descriptor outside its section";
  uint64_t file_off = kd_value - kds.addr + kds.offset;
  KernelDescriptorFacts f;
  if (!read(b, bytes, file_off + 0, &f.group_segment_bytes) ||
      !read(b, bytes, file_off + 4, &f.private_segment_bytes) ||
      !read(b, bytes, file_off + 8, &f.kernarg_bytes))
    return "kernel descriptor out of bounds";
  if (facts) *facts = f;
  return "";
}

}  // namespace tiler_hip
