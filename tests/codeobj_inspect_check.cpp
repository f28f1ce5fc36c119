// CPU check of the code-object inspector (fe2o3_amd/csrc/codeobj_inspect.hpp,
// the function the lifecycle's join and the HIP adapter's load_executable
// run on code-object bytes).  Test infrastructure: built with
// AddressSanitizer and UndefinedBehaviorSanitizer and run by
// tests/test_sanitized_host.py, so any read outside the buffer or any
// undefined arithmetic aborts the run.
//   1. The embedded gfx950 code object (argv[1]) parses, with the facts the
//      lifecycle's contract expects.
//   2. Every truncation of it is rejected or parsed without a stray read.
//   3. Targeted corruptions of every section header: the type set to
//      SHT_NOBITS with offsets and sizes past the buffer (the case of a
//      NOBITS section taken as a string table), huge offsets and sizes, every
//      link index, bad entry sizes.
//   4. Symbol values that make (value - addr + 64) wrap, huge name offsets.
//   5. Note headers with huge name and descriptor sizes.
//   6. Random byte mutations (1 to 8 bytes) over the whole object.
// Each buffer is a fresh heap allocation of exactly its length, so ASan sees
// a read one byte past it.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "../fe2o3_amd/csrc/codeobj_inspect.hpp"

static uint64_t state = 0x243F6A8885A308D3ull;
static uint64_t rnd() {
  state ^= state << 13;
  state ^= state >> 7;
  state ^= state << 17;
  return state;
}

static const char* kKernel = "tiled_gemm_lds_v1";
static const char* kDescriptor = "tiled_gemm_lds_v1.kd";
static long runs = 0, accepted = 0, single_mismatches = 0;

static const char* inspect(const std::vector<uint8_t>& v) {
  // exact-size heap copy: a read at v.size() is a heap overflow
  uint8_t* p = (uint8_t*)malloc(v.empty() ? 1 : v.size());
  if (!v.empty()) memcpy(p, v.data(), v.size());
  Fe2o3Slice1InspectionV1 out;
  const char* r = fe2o3_inspect::inspect_code_object(p, v.size(), kKernel, kDescriptor, &out);
  // the single-kernel form (names read from the metadata first) on the same
  // bytes: where the names it reads are the original ones it accepts exactly
  // what the named form accepts, with the same facts (a mutation that renames
  // the kernel is only required not to read out of bounds)
  char kernel[64], descriptor[64];
  Fe2o3Slice1InspectionV1 single;
  const char* rs =
      fe2o3_inspect::inspect_single_kernel(p, v.size(), kernel, descriptor, 64, &single);
  free(p);
  ++runs;
  if (r[0] == 0) ++accepted;
  const bool same_names = rs[0] == 0 && strcmp(kernel, kKernel) == 0 &&
                          strcmp(descriptor, kDescriptor) == 0;
  if ((r[0] == 0) != same_names ||
      (same_names && memcmp(&out, &single, sizeof(out)) != 0))
    ++single_mismatches;
  return r;
}

static void put(std::vector<uint8_t>& v, size_t at, uint64_t x, int bytes) {
  if (at + bytes > v.size()) return;
  for (int i = 0; i < bytes; ++i) v[at + i] = (uint8_t)(x >> (8 * i));
}

int main(int argc, char** argv) {
  if (argc < 2) {
    printf("usage: codeobj_inspect_check CODE_OBJECT\n");
    return 2;
  }
  FILE* f = fopen(argv[1], "rb");
  if (!f) {
    printf("cannot open %s\n", argv[1]);
    return 2;
  }
  std::vector<uint8_t> co;
  int c;
  while ((c = fgetc(f)) != EOF) co.push_back((uint8_t)c);
  fclose(f);

  int failures = 0;
  // 1. the object itself
  {
    uint8_t* p = (uint8_t*)malloc(co.size());
    memcpy(p, co.data(), co.size());
    Fe2o3Slice1InspectionV1 out;
    const char* r = fe2o3_inspect::inspect_code_object(p, co.size(), kKernel, kDescriptor, &out);
    free(p);
    if (r[0] != 0 || out.kd_kernarg_bytes != FE2O3_SLICE1_COMPLETE_KERNARG_BYTES ||
        out.md_kernarg_bytes != FE2O3_SLICE1_COMPLETE_KERNARG_BYTES ||
        out.md_group_segment_bytes != FE2O3_SLICE1_STATIC_LDS_BYTES || out.explicit_args != 3 ||
        out.md_wavefront_size != 64 || out.code_object_version != 6 ||
        strcmp(out.target, "gfx950:xnack-") != 0) {
      printf("FAIL original: '%s' kernarg %u/%u lds %u args %u wave %u cov %u target %s\n", r,
             out.kd_kernarg_bytes, out.md_kernarg_bytes, out.md_group_segment_bytes,
             out.explicit_args, out.md_wavefront_size, out.code_object_version, out.target);
      ++failures;
    }
  }
  // 2. truncations
  for (size_t n = 0; n < co.size(); ++n) {
    std::vector<uint8_t> v(co.begin(), co.begin() + n);
    inspect(v);
  }
  // 3. section headers
  const uint64_t shoff = fe2o3_inspect::get_le(co.data() + 40, 8);
  const uint64_t shnum = fe2o3_inspect::get_le(co.data() + 60, 2);
  const uint64_t huge[] = {co.size(), co.size() + 1, 0x7fffffffull, 0xffffffffull,
                           0x7fffffffffffffffull, 0xffffffffffffffffull, 0xfffffffffffffff0ull};
  for (uint64_t s = 0; s < shnum; ++s) {
    const size_t h = shoff + 64 * s;
    for (uint64_t hv : huge) {
      for (int field : {24, 32}) {  // sh_offset, sh_size
        std::vector<uint8_t> v = co;
        put(v, h + field, hv, 8);
        inspect(v);
        put(v, h + 4, fe2o3_inspect::kShtNobits, 4);  // the same as a NOBITS section
        inspect(v);
      }
      std::vector<uint8_t> v = co;  // NOBITS with both past the buffer
      put(v, h + 4, fe2o3_inspect::kShtNobits, 4);
      put(v, h + 24, hv, 8);
      put(v, h + 32, hv, 8);
      inspect(v);
      // ... and every symbol table linked to it as its string table
      for (uint64_t t = 0; t < shnum; ++t) {
        std::vector<uint8_t> w = v;
        put(w, shoff + 64 * t + 40, s, 4);
        inspect(w);
      }
    }
    for (uint64_t link = 0; link < shnum + 2; ++link) {
      std::vector<uint8_t> v = co;
      put(v, h + 40, link, 4);
      inspect(v);
    }
    for (uint64_t es : {0ull, 1ull, 23ull, 25ull, 0xffffffffffffffffull}) {
      std::vector<uint8_t> v = co;
      put(v, h + 56, es, 8);
      inspect(v);
    }
    for (uint32_t type : {2u, 7u, 8u, 11u}) {  // SYMTAB, NOTE, NOBITS, DYNSYM
      std::vector<uint8_t> v = co;
      put(v, h + 4, type, 4);
      inspect(v);
    }
    for (uint64_t addr : {0ull, 0x1000ull, 0xffffffffffffffc0ull, 0xffffffffffffffffull}) {
      std::vector<uint8_t> v = co;
      put(v, h + 16, addr, 8);
      inspect(v);
    }
  }
  // 4. symbols: every 24-byte entry of every symbol table
  for (uint64_t s = 0; s < shnum; ++s) {
    const uint8_t* hs = co.data() + shoff + 64 * s;
    const uint32_t type = (uint32_t)fe2o3_inspect::get_le(hs + 4, 4);
    if (type != 2 && type != 11) continue;
    const uint64_t off = fe2o3_inspect::get_le(hs + 24, 8), size = fe2o3_inspect::get_le(hs + 32, 8);
    for (uint64_t e = 0; e + 24 <= size && off + e + 24 <= co.size(); e += 24) {
      const size_t at = off + e;
      for (uint64_t val : {0ull, 0xffffffffffffffc0ull, 0xffffffffffffffffull, 0x8000000000000000ull}) {
        std::vector<uint8_t> v = co;
        put(v, at + 8, val, 8);
        inspect(v);
      }
      for (uint64_t name : {0xffffffffull, 0x7fffffffull, 0ull}) {
        std::vector<uint8_t> v = co;
        put(v, at, name, 4);
        inspect(v);
      }
      for (uint64_t ndx : {(uint64_t)0xffff, (uint64_t)shnum, (uint64_t)0}) {
        std::vector<uint8_t> v = co;
        put(v, at + 6, ndx, 2);
        inspect(v);
      }
    }
  }
  // 5. notes
  for (uint64_t s = 0; s < shnum; ++s) {
    const uint8_t* hs = co.data() + shoff + 64 * s;
    if (fe2o3_inspect::get_le(hs + 4, 4) != 7) continue;
    const uint64_t off = fe2o3_inspect::get_le(hs + 24, 8);
    for (uint64_t sz : {0xffffffffull, 0xfffffffdull, 0x7fffffffull, 0ull, 1ull}) {
      for (int field : {0, 4}) {
        std::vector<uint8_t> v = co;
        put(v, off + field, sz, 4);
        inspect(v);
      }
    }
  }
  // 6. random mutations
  for (int it = 0; it < 40000; ++it) {
    std::vector<uint8_t> v = co;
    const int k = 1 + (int)(rnd() % 8);
    for (int j = 0; j < k; ++j) v[rnd() % v.size()] = (uint8_t)rnd();
    inspect(v);
  }
  if (single_mismatches != 0) {
    printf("FAIL single-kernel form disagrees on %ld objects\n", single_mismatches);
    ++failures;
  }
  printf("runs %ld accepted %ld failures %d\n", runs, accepted, failures);
  return failures == 0 ? 0 : 1;
}
