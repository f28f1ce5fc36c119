// codeobj_inspect.hpp -- reads the facts the code-object lifecycle checks out
// of an AMDGPU code object: the ELF header, the kernel descriptor found
// through the symbol table, and the kernel's entry in the NT_AMDGPU_METADATA
// note (a MessagePack map).  The facts are those the reference reads
// (crates/fe2o3-hsaco-finalize/src/lds_gemm_finalizer.rs:70-278: ELF class,
// machine and ABI version, the descriptor's segment sizes and wavefront bit,
// the metadata's kernarg layout, segment sizes, wavefront size, workgroup
// bound and spill counts).
//
// Plain C++ with no HIP dependency, so a CPU build can run it under
// AddressSanitizer and UndefinedBehaviorSanitizer on mutated objects.  Every
// read of the object's bytes is bounds-checked against the buffer first:
//   - a section is used as data (symbol table, string table, descriptor
//     home, note) only when it occupies file bytes (not SHT_NOBITS) that lie
//     inside the buffer;
//   - offsets inside a section are checked with subtractions, never with
//     sums that could wrap.
// A malformed object yields the name of the first fact that could not be
// read; nothing is read outside [b, b + n).
#pragma once

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <utility>
#include <vector>

#include "../../include/fe2o3_mi355x.h"

namespace fe2o3_inspect {

inline uint64_t get_le(const uint8_t* p, int n) {
  uint64_t v = 0;
  for (int i = 0; i < n; ++i) v |= (uint64_t)p[i] << (8 * i);
  return v;
}

// A small MessagePack reader for the NT_AMDGPU_METADATA note (maps, arrays,
// strings, integers, booleans, nil).
struct MsgValue {
  enum Kind { kNil, kBool, kUInt, kInt, kStr, kArr, kMap } kind = kNil;
  uint64_t u = 0;
  int64_t i = 0;
  std::string s;
  std::vector<MsgValue> items;
  std::vector<std::pair<std::string, MsgValue>> fields;
  const MsgValue* get(const char* key) const {
    for (const auto& f : fields)
      if (f.first == key) return &f.second;
    return nullptr;
  }
  bool uint_value(uint64_t* out) const {
    if (kind == kUInt) {
      *out = u;
      return true;
    }
    if (kind == kInt && i >= 0) {
      *out = (uint64_t)i;
      return true;
    }
    return false;
  }
};

class MsgReader {
 public:
  MsgReader(const uint8_t* p, size_t n) : p_(p), n_(n) {}
  bool read(MsgValue* v, int depth = 0) {
    if (depth > 16 || pos_ >= n_) return false;
    const uint8_t t = p_[pos_++];
    if (t <= 0x7f) return set_uint(v, t);
    if (t >= 0xe0) {
      v->kind = MsgValue::kInt;
      v->i = (int8_t)t;
      return true;
    }
    if ((t & 0xf0) == 0x80) return read_map(v, t & 0x0f, depth);
    if ((t & 0xf0) == 0x90) return read_arr(v, t & 0x0f, depth);
    if ((t & 0xe0) == 0xa0) return read_str(v, t & 0x1f);
    uint64_t x;
    switch (t) {
      case 0xc0: v->kind = MsgValue::kNil; return true;
      case 0xc2: v->kind = MsgValue::kBool; v->u = 0; return true;
      case 0xc3: v->kind = MsgValue::kBool; v->u = 1; return true;
      case 0xcc: return be(1, &x) && set_uint(v, x);
      case 0xcd: return be(2, &x) && set_uint(v, x);
      case 0xce: return be(4, &x) && set_uint(v, x);
      case 0xcf: return be(8, &x) && set_uint(v, x);
      case 0xd0: if (!be(1, &x)) return false; v->kind = MsgValue::kInt; v->i = (int8_t)x; return true;
      case 0xd1: if (!be(2, &x)) return false; v->kind = MsgValue::kInt; v->i = (int16_t)x; return true;
      case 0xd2: if (!be(4, &x)) return false; v->kind = MsgValue::kInt; v->i = (int32_t)x; return true;
      case 0xd3: if (!be(8, &x)) return false; v->kind = MsgValue::kInt; v->i = (int64_t)(x); return true;
      case 0xd9: return be(1, &x) && read_str(v, x);
      case 0xda: return be(2, &x) && read_str(v, x);
      case 0xdb: return be(4, &x) && read_str(v, x);
      case 0xdc: return be(2, &x) && read_arr(v, x, depth);
      case 0xdd: return be(4, &x) && read_arr(v, x, depth);
      case 0xde: return be(2, &x) && read_map(v, x, depth);
      case 0xdf: return be(4, &x) && read_map(v, x, depth);
      default: return false;  // binary, ext and float forms do not occur in the note
    }
  }

 private:
  static bool set_uint(MsgValue* v, uint64_t x) {
    v->kind = MsgValue::kUInt;
    v->u = x;
    return true;
  }
  bool be(int bytes, uint64_t* out) {
    if (n_ - pos_ < (size_t)bytes) return false;
    uint64_t x = 0;
    for (int i = 0; i < bytes; ++i) x = x << 8 | p_[pos_++];
    *out = x;
    return true;
  }
  bool read_str(MsgValue* v, uint64_t len) {
    if (n_ - pos_ < len) return false;
    v->kind = MsgValue::kStr;
    v->s.assign(reinterpret_cast<const char*>(p_ + pos_), (size_t)len);
    pos_ += len;
    return true;
  }
  // every element takes at least one byte, so a count beyond the bytes left
  // is malformed (and would otherwise size a vector from untrusted input)
  bool read_arr(MsgValue* v, uint64_t count, int depth) {
    if (count > n_ - pos_) return false;
    v->kind = MsgValue::kArr;
    v->items.resize((size_t)count);
    for (auto& it : v->items)
      if (!read(&it, depth + 1)) return false;
    return true;
  }
  bool read_map(MsgValue* v, uint64_t count, int depth) {
    if (count > (n_ - pos_) / 2) return false;
    v->kind = MsgValue::kMap;
    v->fields.resize((size_t)count);
    for (auto& f : v->fields) {
      MsgValue key;
      if (!read(&key, depth + 1) || key.kind != MsgValue::kStr) return false;
      f.first = std::move(key.s);
      if (!read(&f.second, depth + 1)) return false;
    }
    return true;
  }
  const uint8_t* p_;
  size_t n_;
  size_t pos_ = 0;
};

constexpr uint16_t kEmAmdgpu = 224;
constexpr uint8_t kOsAbiAmdgpuHsa = 64;
constexpr uint32_t kMachMask = 0xffu, kMachGfx950 = 0x4fu;
constexpr uint32_t kNtAmdgpuMetadata = 32;
constexpr uint32_t kShtSymtab = 2, kShtNote = 7, kShtNobits = 8, kShtDynsym = 11;

struct Section {
  uint32_t name, type;
  uint64_t addr, offset, size;
  uint32_t link;
  uint64_t entsize;
  bool in_file;  // occupies bytes [offset, offset + size) inside the buffer
};

// The ELF header and section table; "" on success, else the fact that
// could not be read.
inline const char* read_sections(const uint8_t* b, size_t n, std::vector<Section>* out) {
  if (b == nullptr || n < 64 || memcmp(b, "\x7f" "ELF", 4) != 0 || b[4] != 2 || b[5] != 1)
    return "ELF header";
  if (get_le(b + 18, 2) != kEmAmdgpu || b[7] != kOsAbiAmdgpuHsa) return "ELF machine";
  const uint64_t shoff = get_le(b + 40, 8);
  const uint64_t shentsize = get_le(b + 58, 2), shnum = get_le(b + 60, 2);
  if (shentsize != 64 || shoff > n || shnum > (n - shoff) / 64) return "section table";
  std::vector<Section>& sec = *out;
  sec.assign(shnum, Section{});
  for (uint64_t i = 0; i < shnum; ++i) {
    const uint8_t* s = b + shoff + 64 * i;
    Section& x = sec[i];
    x = {(uint32_t)get_le(s, 4), (uint32_t)get_le(s + 4, 4), get_le(s + 16, 8), get_le(s + 24, 8),
         get_le(s + 32, 8), (uint32_t)get_le(s + 40, 4), get_le(s + 56, 8), false};
    x.in_file = x.type != kShtNobits && x.offset <= n && x.size <= n - x.offset;
    // a section with file bytes must lie inside the buffer; a NOBITS
    // section has none and can serve as no table or descriptor below
    if (x.type != kShtNobits && !x.in_file) return "section bounds";
  }
  return "";
}

// The NT_AMDGPU_METADATA note's map; "" on success.
inline const char* read_metadata(const uint8_t* b, const std::vector<Section>& sec, MsgValue* md) {
  for (const auto& st : sec) {
    if (st.type != kShtNote) continue;
    if (!st.in_file) return "metadata note";
    uint64_t off = 0;
    while (st.size - off >= 12) {
      const uint8_t* note = b + st.offset + off;
      const uint64_t namesz = get_le(note, 4), descsz = get_le(note + 4, 4), type = get_le(note + 8, 4);
      const uint64_t name_pad = (namesz + 3) & ~3ull, desc_pad = (descsz + 3) & ~3ull;
      if (name_pad + desc_pad > st.size - off - 12) return "metadata note";
      if (type == kNtAmdgpuMetadata && namesz == 7 && memcmp(note + 12, "AMDGPU", 7) == 0) {
        MsgReader r(note + 12 + name_pad, (size_t)descsz);
        if (!r.read(md) || md->kind != MsgValue::kMap) return "metadata";
        return "";
      }
      off += 12 + name_pad + desc_pad;
    }
  }
  return "metadata note";
}

// Returns "" on success, else the first fact that could not be read.
// `kernel` and `descriptor` name the kernel and its descriptor symbol.
inline const char* inspect_code_object(const uint8_t* b, size_t n, const char* kernel,
                                       const char* descriptor, Fe2o3Slice1InspectionV1* out) {
  memset(out, 0, sizeof(*out));
  out->byte_len = n;
  std::vector<Section> sec;
  const char* bad = read_sections(b, n, &sec);
  if (bad[0]) return bad;
  // EI_ABIVERSION: 2, 3, 4 = code object v4, v5, v6.
  out->code_object_version = b[8] + 2u;
  out->e_flags = (uint32_t)get_le(b + 48, 4);
  const uint64_t shnum = sec.size();
  // kernel descriptor through the symbol table
  const uint8_t* kd = nullptr;
  for (const auto& st : sec) {
    if (st.type != kShtSymtab && st.type != kShtDynsym) continue;
    if (st.entsize != 24 || st.link >= shnum || !st.in_file) return "symbol table";
    const Section& strtab = sec[st.link];
    if (!strtab.in_file) return "symbol table";
    for (uint64_t off = 0; st.size - off >= 24; off += 24) {
      const uint8_t* sym = b + st.offset + off;
      const uint64_t name = get_le(sym, 4);
      if (name >= strtab.size) continue;
      const char* nm = reinterpret_cast<const char*>(b + strtab.offset + name);
      const size_t room = (size_t)(strtab.size - name);
      if (strnlen(nm, room) == room || strcmp(nm, descriptor) != 0) continue;
      const uint64_t shndx = get_le(sym + 6, 2);
      const uint64_t value = get_le(sym + 8, 8), size = get_le(sym + 16, 8);
      if (size != 64 || shndx >= shnum) return "kernel descriptor symbol";
      const Section& home = sec[shndx];
      if (!home.in_file || value < home.addr || value - home.addr > home.size ||
          home.size - (value - home.addr) < 64)
        return "kernel descriptor";
      kd = b + home.offset + (value - home.addr);
    }
    if (kd) break;
  }
  if (!kd) return "kernel descriptor symbol";
  out->kd_group_segment_bytes = (uint32_t)get_le(kd + 0, 4);
  out->kd_private_segment_bytes = (uint32_t)get_le(kd + 4, 4);
  out->kd_kernarg_bytes = (uint32_t)get_le(kd + 8, 4);
  // kernel_code_properties bit 10: ENABLE_WAVEFRONT_SIZE32
  out->kd_wavefront_size = (get_le(kd + 56, 2) >> 10 & 1u) ? 32u : 64u;
  // metadata note
  MsgValue md;
  bad = read_metadata(b, sec, &md);
  if (bad[0]) return bad;
  const MsgValue* target = md.get("amdhsa.target");
  if (!target || target->kind != MsgValue::kStr) return "metadata target";
  const std::string triple = "amdgcn-amd-amdhsa--";
  std::string t = target->s.compare(0, triple.size(), triple) == 0 ? target->s.substr(triple.size())
                                                                  : target->s;
  strncpy(out->target, t.c_str(), sizeof(out->target) - 1);
  const MsgValue* kernels = md.get("amdhsa.kernels");
  if (!kernels || kernels->kind != MsgValue::kArr) return "metadata kernels";
  const MsgValue* k = nullptr;
  for (const auto& kk : kernels->items) {
    const MsgValue* name = kk.get(".name");
    if (name && name->kind == MsgValue::kStr && name->s == kernel) k = &kk;
  }
  if (!k) return "metadata kernel";
  const MsgValue* sym = k->get(".symbol");
  if (!sym || sym->kind != MsgValue::kStr || sym->s != descriptor) return "metadata symbol";
  struct {
    const char* key;
    uint32_t* dst;
  } ints[] = {{".kernarg_segment_size", &out->md_kernarg_bytes},
              {".kernarg_segment_align", &out->md_kernarg_alignment},
              {".group_segment_fixed_size", &out->md_group_segment_bytes},
              {".private_segment_fixed_size", &out->md_private_segment_bytes},
              {".wavefront_size", &out->md_wavefront_size},
              {".max_flat_workgroup_size", &out->md_max_flat_workgroup_size},
              {".sgpr_spill_count", &out->sgpr_spills},
              {".vgpr_spill_count", &out->vgpr_spills}};
  for (const auto& f : ints) {
    const MsgValue* v = k->get(f.key);
    uint64_t x;
    if (!v || !v->uint_value(&x) || x > UINT32_MAX) return f.key;
    *f.dst = (uint32_t)x;
  }
  const MsgValue* dyn = k->get(".uses_dynamic_stack");
  out->uses_dynamic_stack = (dyn && dyn->kind == MsgValue::kBool) ? (uint32_t)dyn->u : 0u;
  const MsgValue* args = k->get(".args");
  if (!args || args->kind != MsgValue::kArr) return "metadata args";
  uint64_t explicit_end = 0, implicit_off = out->md_kernarg_bytes;
  for (const auto& a : args->items) {
    const MsgValue* off = a.get(".offset");
    const MsgValue* size = a.get(".size");
    const MsgValue* kind = a.get(".value_kind");
    uint64_t o, s;
    if (!off || !size || !kind || kind->kind != MsgValue::kStr || !off->uint_value(&o) ||
        !size->uint_value(&s) || o > UINT32_MAX || s > UINT32_MAX)
      return "metadata arg";
    if (kind->s.compare(0, 7, "hidden_") == 0) {
      implicit_off = std::min(implicit_off, o);
    } else {
      ++out->explicit_args;
      explicit_end = std::max(explicit_end, o + s);
    }
  }
  if (explicit_end > UINT32_MAX) return "metadata arg";
  out->explicit_bytes = (uint32_t)explicit_end;
  out->implicit_offset = (uint32_t)implicit_off;
  out->implicit_bytes =
      out->md_kernarg_bytes - (uint32_t)std::min<uint64_t>(implicit_off, out->md_kernarg_bytes);
  return "";
}

// inspect_code_object for a code object that holds exactly one kernel,
// whose name and descriptor symbol are read from the metadata first (into
// `kernel` and `descriptor`, NUL-terminated, each of `room` bytes).
inline const char* inspect_single_kernel(const uint8_t* b, size_t n, char* kernel,
                                         char* descriptor, size_t room,
                                         Fe2o3Slice1InspectionV1* out) {
  memset(out, 0, sizeof(*out));
  out->byte_len = n;
  if (room == 0) return "metadata kernel";
  kernel[0] = descriptor[0] = '\0';
  std::vector<Section> sec;
  const char* bad = read_sections(b, n, &sec);
  if (bad[0]) return bad;
  MsgValue md;
  bad = read_metadata(b, sec, &md);
  if (bad[0]) return bad;
  const MsgValue* kernels = md.get("amdhsa.kernels");
  if (!kernels || kernels->kind != MsgValue::kArr) return "metadata kernels";
  if (kernels->items.size() != 1) return "metadata kernel";
  const MsgValue* name = kernels->items[0].get(".name");
  const MsgValue* sym = kernels->items[0].get(".symbol");
  if (!name || name->kind != MsgValue::kStr || name->s.size() >= room) return "metadata kernel";
  if (!sym || sym->kind != MsgValue::kStr || sym->s.size() >= room) return "metadata symbol";
  memcpy(kernel, name->s.c_str(), name->s.size() + 1);
  memcpy(descriptor, sym->s.c_str(), sym->s.size() + 1);
  return inspect_code_object(b, n, kernel, descriptor, out);
}

}  // namespace fe2o3_inspect
