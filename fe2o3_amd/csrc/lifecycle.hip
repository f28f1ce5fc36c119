// lifecycle.hip -- typed, one-shot host lifecycle of the exact 16x16x16 LDS
// GEMM code object (crates/fe2o3-host/src/generated_lds_gemm_lifecycle.rs).
//
// The artifact is codeobj/tiled_gemm_lds_v1.hip built by hipcc into a
// standalone gfx950 code object (v6, xnack-) and embedded here as bytes,
// together with the SHA-256 that the build recorded for them, the SHA-256 of
// the kernel source and the compiler and flags that built it.  Nothing here
// exposes the bytes; they reach a runtime only through an adapter's
// load_executable.
//
// What the reference checks, this file checks in the same order:
//   join   -- the artifact's identities, its contract, the code object's own
//             ELF / kernel-descriptor / metadata facts, the host request's
//             fields and buffer length identities (validate_join :1036,
//             validate_contract :1167);
//   load   -- context identity, environment (target compatibility, HIP
//             ordinal, runtime instance, physical device), load observation
//             (digest, length, runtime, agent), kernel resolution (symbol,
//             304-byte kernarg segment, 16-byte HSA alignment), resources
//             (1024 bytes static LDS, no private segment) (:698-777);
//   dispatch -- implicit-suffix initialization (span, geometry, explicit
//             prefix unchanged), then launch-and-wait (geometry, completion)
//             (:639-696);
//   unload -- terminal, validated, and an unload identity over it (:522-557).
// Failures after a load drop the kernel, then unload once, then release the
// A/B/C leases and the adapter.  An unload failure aborts the process.
//
// SHA-256 is implemented from FIPS 180-4 (the reference uses the sha2
// crate); identities use the reference's framing: each field is preceded by
// its length as a little-endian u64 (hash_field, crates/fe2o3-hsaco-
// finalize/src/lds_gemm_profile_registry.rs:1166-1169).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <utility>
#include <vector>

#include <unistd.h>

#include "../../include/fe2o3_mi355x.h"
#include "codeobj_inspect.hpp"
#include "internal.hpp"

#include "slice1_artifact.inc"
#include "flash_attention_v1_artifact.inc"
#include "row_softmax_v1_artifact.inc"
#include "moe_top2_v1_artifact.inc"

namespace {

// ---- SHA-256 (FIPS 180-4, section 6.2) ------------------------------------------------

// First 32 bits of the fractional parts of the cube roots of the first 64
// primes (FIPS 180-4 section 4.2.2).
constexpr uint32_t kShaK[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u,
    0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu,
    0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu,
    0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau, 0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u,
    0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu,
    0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
    0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u, 0x19a4c116u,
    0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u,
    0xc67178f2u};

class Sha256 {
 public:
  void update(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    total_ += n;
    while (n > 0) {
      const size_t take = std::min(n, sizeof(block_) - fill_);
      std::memcpy(block_ + fill_, p, take);
      fill_ += take;
      p += take;
      n -= take;
      if (fill_ == sizeof(block_)) {
        compress(block_);
        fill_ = 0;
      }
    }
  }
  void finish(uint8_t out[32]) {
    const uint64_t bits = total_ * 8u;
    const uint8_t one = 0x80u, zero = 0u;
    update(&one, 1);
    while (fill_ != 56) update(&zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(len, 8);
    for (int i = 0; i < 8; ++i)
      for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h_[i] >> (24 - 8 * j));
  }

 private:
  static uint32_t rotr(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }
  void compress(const uint8_t* p) {
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
      w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 |
             (uint32_t)p[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
      const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
      const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
      w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
    for (int t = 0; t < 64; ++t) {
      const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
      const uint32_t ch = (e & f) ^ (~e & g);
      const uint32_t t1 = h + S1 + ch + kShaK[t] + w[t];
      const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
      const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
      const uint32_t t2 = S0 + maj;
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h_[0] += a; h_[1] += b; h_[2] += c; h_[3] += d;
    h_[4] += e; h_[5] += f; h_[6] += g; h_[7] += h;
  }
  // First 32 bits of the fractional parts of the square roots of the first
  // 8 primes (FIPS 180-4 section 5.3.3).
  uint32_t h_[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                    0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  uint8_t block_[64];
  size_t fill_ = 0;
  uint64_t total_ = 0;
};

void sha256(const void* data, size_t n, uint8_t out[32]) {
  Sha256 d;
  d.update(data, n);
  d.finish(out);
}

void hash_field(Sha256& d, const void* p, size_t n) {
  uint8_t len[8];
  for (int i = 0; i < 8; ++i) len[i] = (uint8_t)((uint64_t)n >> (8 * i));
  d.update(len, 8);
  d.update(p, n);
}
template <typename T>
void hash_le(Sha256& d, T v) {
  uint8_t b[sizeof(T)];
  for (size_t i = 0; i < sizeof(T); ++i) b[i] = (uint8_t)((uint64_t)v >> (8 * i));
  hash_field(d, b, sizeof(T));
}
void hash_str(Sha256& d, const char* s) { hash_field(d, s, std::strlen(s)); }

void put_le64(uint8_t* p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

// ---- the exact profile ----------------------------------------------------------------

constexpr const char* kTarget = "gfx950:xnack-";
constexpr uint32_t kProfileSlice1 = 1;
constexpr uint32_t kCodeObjectVersion = 6;
constexpr const char* kLogicalName = "tiled_gemm_lds_slice1";
constexpr const char* kKernelSymbol = "tiled_gemm_lds_v1";
constexpr const char* kDescriptorSymbol = "tiled_gemm_lds_v1.kd";
constexpr uint32_t kGrid[3] = {1, 1, 1};
constexpr uint32_t kWorkgroup[3] = {64, 1, 1};
constexpr uint32_t kWavefront = 64;
constexpr uint32_t kExplicitKernarg = FE2O3_SLICE1_EXPLICIT_KERNARG_BYTES;
constexpr uint32_t kCompleteKernarg = FE2O3_SLICE1_COMPLETE_KERNARG_BYTES;
constexpr uint32_t kContractKernargAlign = FE2O3_SLICE1_CONTRACT_KERNARG_ALIGNMENT;
constexpr uint64_t kHsaKernargAlign = FE2O3_SLICE1_HSA_KERNARG_ALIGNMENT;
constexpr uint32_t kStaticLds = FE2O3_SLICE1_STATIC_LDS_BYTES;
constexpr uint32_t kLdsAllocations = 2;
constexpr uint32_t kLdsBytesPerAllocation = 512;
constexpr uint32_t kLdsAlignment = 16;
constexpr uint32_t kPrivateSegment = 0;
constexpr uint32_t kDynamicLds = 0;
constexpr uint64_t kElements = 256;
constexpr char kLengthDomain[] = "FE2O3/EXACT-LDS-GEMM-LENGTH/V1";
constexpr char kProfileDomain[] = "FE2O3/EXACT-LDS-GEMM-PROFILE/V1";
constexpr char kImportDomain[] = "FE2O3/EXACT-LDS-GEMM-COMPILER-IMPORT/V1";
constexpr char kUnloadDomain[] = "FE2O3/EXACT-LDS-GEMM/UNLOAD/V1";
constexpr char kContextDomain[] = "FE2O3/MI355X-HIP-CONTEXT/V1";
constexpr char kRuntimeDomain[] = "FE2O3/MI355X-HIP-RUNTIME-INSTANCE/V1";

enum Role : uint32_t { kRoleA = 1, kRoleB = 2, kRoleC = 3 };
enum Element : uint32_t { kBf16 = 1, kF32 = 2 };

// What load, dispatch and unload check for one embedded code object: the
// exact LDS GEMM, or one of the protected profiles below.  Every profile
// launches grid [1,1,1] x workgroup [64,1,1] with no dynamic LDS, and its
// kernarg is explicit bytes followed by the 256-byte implicit suffix.
struct Spec {
  uint32_t profile;  // FE2O3_PROFILE_*; 0 for the LDS GEMM
  const char* symbol;
  const uint8_t* code;
  size_t code_len;
  uint32_t explicit_bytes, complete_bytes, static_lds;
  const char* unload_domain;
  uint32_t implicit_bytes() const { return complete_bytes - explicit_bytes; }
};

const Spec kSlice1Spec = {0,
                          kKernelSymbol,
                          kSlice1CodeObject,
                          sizeof(kSlice1CodeObject),
                          kExplicitKernarg,
                          kCompleteKernarg,
                          kStaticLds,
                          kUnloadDomain};

// Domain strings are hashed with their terminating NUL, as the reference's
// b"...\0" literals are.
void hash_domain(Sha256& d, const char* domain) { hash_field(d, domain, std::strlen(domain) + 1); }

void length_identity(uint32_t role, uint32_t element, uint64_t elements, uint64_t bytes,
                     uint8_t out[32]) {
  Sha256 d;
  hash_domain(d, kLengthDomain);
  const uint8_t r = (uint8_t)role, e = (uint8_t)element;
  hash_field(d, &r, 1);
  hash_field(d, &e, 1);
  hash_le<uint64_t>(d, elements);
  hash_le<uint64_t>(d, bytes);
  d.finish(out);
}

uint8_t effect_tag(const Fe2o3Slice1BufferContractV1& b) {
  if (b.ownership == 0 && b.access == 0 && b.alias == 0) return 1;
  if (b.ownership == 1 && b.access == 1 && b.alias == 1) return 2;
  return 0;
}

Fe2o3Slice1BufferContractV1 buffer_contract(uint32_t role, uint32_t element, uint64_t elements,
                                            uint64_t element_bytes, bool output) {
  Fe2o3Slice1BufferContractV1 b{};
  b.role = role;
  b.element = element;
  b.elements = elements;
  b.bytes = elements * element_bytes;
  length_identity(role, element, b.elements, b.bytes, b.length_identity);
  b.ownership = output ? 1u : 0u;
  b.access = output ? 1u : 0u;
  b.alias = output ? 1u : 0u;
  return b;
}

// lds_gemm_profile_registry.rs:606-670 (exact_slice1_contract), for gfx950.
Fe2o3Slice1ContractV1 exact_contract() {
  Fe2o3Slice1ContractV1 c{};
  c.profile = kProfileSlice1;
  c.code_object_version = kCodeObjectVersion;
  std::strncpy(c.target, kTarget, sizeof(c.target) - 1);
  for (int i = 0; i < 3; ++i) {
    c.grid[i] = kGrid[i];
    c.workgroup[i] = kWorkgroup[i];
  }
  c.wavefront_size = kWavefront;
  c.explicit_kernarg_bytes = kExplicitKernarg;
  c.complete_kernarg_bytes = kCompleteKernarg;
  c.kernarg_alignment = kContractKernargAlign;
  c.static_lds_bytes = kStaticLds;
  c.lds_allocations = kLdsAllocations;
  c.lds_bytes_per_allocation = kLdsBytesPerAllocation;
  c.lds_alignment = kLdsAlignment;
  c.buffers[0] = buffer_contract(kRoleA, kBf16, kElements, 2, false);
  c.buffers[1] = buffer_contract(kRoleB, kBf16, kElements, 2, false);
  c.buffers[2] = buffer_contract(kRoleC, kF32, kElements, 4, true);
  Sha256 d;
  hash_domain(d, kProfileDomain);
  const uint8_t profile = (uint8_t)kProfileSlice1;
  hash_field(d, &profile, 1);
  hash_str(d, kTarget);
  hash_le<uint16_t>(d, (uint16_t)kCodeObjectVersion);
  hash_str(d, kLogicalName);
  hash_str(d, kKernelSymbol);
  hash_str(d, kDescriptorSymbol);
  hash_le<uint32_t>(d, kExplicitKernarg);
  hash_le<uint32_t>(d, kCompleteKernarg);
  hash_le<uint32_t>(d, kContractKernargAlign);
  uint8_t dims[12];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 4; ++j) dims[4 * i + j] = (uint8_t)(kGrid[i] >> (8 * j));
  hash_field(d, dims, 12);
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 4; ++j) dims[4 * i + j] = (uint8_t)(kWorkgroup[i] >> (8 * j));
  hash_field(d, dims, 12);
  hash_le<uint32_t>(d, kWavefront);
  hash_le<uint32_t>(d, kStaticLds);
  hash_le<uint32_t>(d, kLdsAllocations);
  hash_le<uint32_t>(d, kLdsBytesPerAllocation);
  hash_le<uint32_t>(d, kLdsAlignment);
  for (const auto& b : c.buffers) {
    const uint8_t r = (uint8_t)b.role, tag = effect_tag(b);
    hash_field(d, &r, 1);
    hash_le<uint64_t>(d, b.elements);
    hash_le<uint64_t>(d, b.bytes);
    hash_field(d, b.length_identity, 32);
    hash_field(d, &tag, 1);
  }
  d.finish(c.identity);
  return c;
}

// The compiler import: which source, compiler and flags produced the code
// object, bound to the profile (lds_gemm_profile_registry.rs:1131-1154).
void import_identity(const uint8_t profile_identity[32], uint8_t out[32]) {
  Sha256 d;
  hash_domain(d, kImportDomain);
  hash_field(d, profile_identity, 32);
  hash_field(d, kSlice1SourceDigest, 32);
  hash_str(d, kSlice1Compiler);
  hash_str(d, kSlice1Flags);
  hash_str(d, kTarget);
  d.finish(out);
}

using fe2o3_inspect::kMachGfx950;
using fe2o3_inspect::kMachMask;

// The code object's own facts against the contract; "" when they agree.
const char* inspection_drift(const Fe2o3Slice1InspectionV1& i, const Fe2o3Slice1ContractV1& c) {
  const uint32_t threads = c.workgroup[0] * c.workgroup[1] * c.workgroup[2];
  const struct {
    bool ok;
    const char* field;
  } checks[] = {
      {i.code_object_version == c.code_object_version, "code-object version"},
      {(i.e_flags & kMachMask) == kMachGfx950, "ELF machine"},
      {std::strncmp(i.target, c.target, sizeof(c.target)) == 0, "target"},
      {i.kd_kernarg_bytes == c.complete_kernarg_bytes, "descriptor kernarg size"},
      {i.md_kernarg_bytes == c.complete_kernarg_bytes, "metadata kernarg size"},
      {i.md_kernarg_alignment == c.kernarg_alignment, "metadata kernarg alignment"},
      {i.explicit_args == 3 && i.explicit_bytes == c.explicit_kernarg_bytes, "explicit kernarg"},
      {i.implicit_offset == c.explicit_kernarg_bytes &&
           i.implicit_bytes == c.complete_kernarg_bytes - c.explicit_kernarg_bytes,
       "implicit kernarg"},
      {i.kd_group_segment_bytes == c.static_lds_bytes, "descriptor static LDS"},
      {i.md_group_segment_bytes == c.static_lds_bytes, "metadata static LDS"},
      {i.kd_private_segment_bytes == kPrivateSegment, "descriptor private segment"},
      {i.md_private_segment_bytes == kPrivateSegment, "metadata private segment"},
      {i.kd_wavefront_size == c.wavefront_size, "descriptor wavefront"},
      {i.md_wavefront_size == c.wavefront_size, "metadata wavefront"},
      {i.md_max_flat_workgroup_size == threads, "workgroup size bound"},
      {i.sgpr_spills == 0 && i.vgpr_spills == 0 && i.uses_dynamic_stack == 0, "spills"},
  };
  for (const auto& ch : checks)
    if (!ch.ok) return ch.field;
  return "";
}

// ---- the artifact and the host request ------------------------------------------------

struct Artifact {
  Fe2o3Slice1ArtifactV1 view{};
  const char* inspect_error = "";
  const char* drift = "";
};

const Artifact& artifact() {
  static const Artifact a = [] {
    Artifact x;
    sha256(kSlice1CodeObject, sizeof(kSlice1CodeObject), x.view.finalizer_identity);
    std::memcpy(x.view.build_digest, kSlice1BuildDigest, 32);
    x.view.contract = exact_contract();
    std::memcpy(x.view.profile_identity, x.view.contract.identity, 32);
    import_identity(x.view.profile_identity, x.view.import_identity);
    x.inspect_error =
        fe2o3_inspect::inspect_code_object(kSlice1CodeObject, sizeof(kSlice1CodeObject),
                                           kKernelSymbol, kDescriptorSymbol, &x.view.inspection);
    x.drift = x.inspect_error[0] ? x.inspect_error
                                 : inspection_drift(x.view.inspection, x.view.contract);
    return x;
  }();
  return a;
}

// The generated host request's side of the join: the contract and
// identities it was generated against, and its launch facts.
struct HostFacts {
  Fe2o3Slice1ContractV1 contract;
  uint8_t profile_identity[32];
  uint8_t import_identity[32];
};

const HostFacts& host_facts() {
  static const HostFacts h = [] {
    HostFacts x{};
    x.contract = exact_contract();
    std::memcpy(x.profile_identity, x.contract.identity, 32);
    import_identity(x.profile_identity, x.import_identity);
    return x;
  }();
  return h;
}

void canonical_facts(Fe2o3Slice1JoinFactsV1* f) {
  const Artifact& a = artifact();
  const HostFacts& h = host_facts();
  std::memset(f, 0, sizeof(*f));
  f->import_matches = std::memcmp(a.view.import_identity, h.import_identity, 32) == 0;
  f->profile_matches = std::memcmp(a.view.profile_identity, h.profile_identity, 32) == 0;
  f->contract_matches = std::memcmp(&a.view.contract, &h.contract, sizeof(h.contract)) == 0;
  f->finalized_output_matches = std::memcmp(a.view.finalizer_identity, a.view.build_digest, 32) == 0;
  f->inspection_matches = a.drift[0] == '\0';
  f->contract = a.view.contract;
  std::strncpy(f->host_target, kTarget, sizeof(f->host_target) - 1);
  f->host_profile = kProfileSlice1;
  f->host_profile_identity_matches = std::memcmp(h.profile_identity, f->contract.identity, 32) == 0;
  for (int i = 0; i < 3; ++i) {
    f->host_grid[i] = kGrid[i];
    f->host_workgroup[i] = kWorkgroup[i];
  }
  f->host_static_lds = kStaticLds;
  f->host_dynamic_lds = kDynamicLds;
  f->host_explicit_kernarg = kExplicitKernarg;
  f->host_complete_kernarg = kCompleteKernarg;
  f->host_kernarg_alignment = kContractKernargAlign;
  for (int i = 0; i < 3; ++i)
    std::memcpy(f->host_length_identities[i], h.contract.buffers[i].length_identity, 32);
}

void set_error(Fe2o3Slice1ErrorV1* e, int32_t kind, const char* field = "", int32_t index = -1,
               int32_t adapter_status = 0, uint64_t expected = 0, uint64_t actual = 0) {
  if (!e) return;
  std::memset(e, 0, sizeof(*e));
  e->kind = kind;
  e->index = index;
  e->adapter_status = adapter_status;
  e->expected = expected;
  e->actual = actual;
  std::strncpy(e->field, field, sizeof(e->field) - 1);
}

bool buffer_matches(const Fe2o3Slice1BufferContractV1& actual,
                    const Fe2o3Slice1BufferContractV1& expected) {
  uint8_t li[32];
  length_identity(expected.role, expected.element, expected.elements, expected.bytes, li);
  return actual.role == expected.role && actual.element == expected.element &&
         actual.elements == expected.elements && actual.bytes == expected.bytes &&
         std::memcmp(actual.length_identity, li, 32) == 0 && actual.ownership == expected.ownership &&
         actual.access == expected.access && actual.alias == expected.alias;
}

// validate_join (generated_lds_gemm_lifecycle.rs:1036-1094) and
// validate_contract (:1167-1218), in the reference's order.
int32_t validate_join(const Fe2o3Slice1JoinFactsV1& f, Fe2o3Slice1ErrorV1* err) {
  if (!f.import_matches) return set_error(err, FE2O3_SLICE1_E_IMPORT_IDENTITY), FE2O3_ERR_JOIN;
  if (!f.profile_matches) return set_error(err, FE2O3_SLICE1_E_PROFILE_IDENTITY), FE2O3_ERR_JOIN;
  if (!f.contract_matches) return set_error(err, FE2O3_SLICE1_E_CONTRACT), FE2O3_ERR_JOIN;
  if (!f.finalized_output_matches)
    return set_error(err, FE2O3_SLICE1_E_FINALIZED_OUTPUT, "digest"), FE2O3_ERR_JOIN;
  if (!f.inspection_matches)
    return set_error(err, FE2O3_SLICE1_E_FINALIZED_OUTPUT, "code object inspection"), FE2O3_ERR_JOIN;
  const Fe2o3Slice1ContractV1& c = f.contract;
  const auto eq3 = [](const uint32_t* a, const uint32_t* b) {
    return a[0] == b[0] && a[1] == b[1] && a[2] == b[2];
  };
  const struct {
    bool ok;
    const char* field;
  } contract_checks[] = {
      {c.profile == kProfileSlice1, "profile"},
      {std::strncmp(c.target, kTarget, sizeof(c.target)) == 0, "target"},
      {c.code_object_version == kCodeObjectVersion, "code-object version"},
      {eq3(c.grid, kGrid), "grid"},
      {eq3(c.workgroup, kWorkgroup), "workgroup"},
      {c.wavefront_size == kWavefront, "wavefront"},
      {c.explicit_kernarg_bytes == kExplicitKernarg, "explicit kernarg size"},
      {c.complete_kernarg_bytes == kCompleteKernarg, "complete kernarg size"},
      {c.kernarg_alignment == kContractKernargAlign, "descriptor kernarg alignment"},
      {c.static_lds_bytes == kStaticLds, "static LDS"},
      {c.lds_allocations == kLdsAllocations, "LDS allocation count"},
      {c.lds_bytes_per_allocation == kLdsBytesPerAllocation, "LDS bytes per allocation"},
      {c.lds_alignment == kLdsAlignment, "LDS alignment"},
  };
  for (const auto& ch : contract_checks)
    if (!ch.ok) return set_error(err, FE2O3_SLICE1_E_CONTRACT_FIELD, ch.field), FE2O3_ERR_JOIN;
  const Fe2o3Slice1ContractV1& expected = host_facts().contract;
  for (int i = 0; i < 3; ++i)
    if (!buffer_matches(c.buffers[i], expected.buffers[i]))
      return set_error(err, FE2O3_SLICE1_E_BUFFER_CONTRACT, "", i), FE2O3_ERR_JOIN;
  const struct {
    bool ok;
    const char* field;
  } host_checks[] = {
      {std::strncmp(f.host_target, kTarget, sizeof(f.host_target)) == 0, "target"},
      {f.host_profile == kProfileSlice1, "profile"},
      {f.host_profile_identity_matches != 0, "profile identity"},
      {eq3(f.host_grid, kGrid), "grid"},
      {eq3(f.host_workgroup, kWorkgroup), "workgroup"},
      {f.host_static_lds == kStaticLds, "static LDS"},
      {f.host_dynamic_lds == kDynamicLds, "dynamic LDS"},
      {f.host_explicit_kernarg == kExplicitKernarg, "explicit kernarg size"},
      {f.host_complete_kernarg == kCompleteKernarg, "complete kernarg size"},
      {f.host_kernarg_alignment == kContractKernargAlign, "contract kernarg alignment"},
  };
  for (const auto& ch : host_checks)
    if (!ch.ok) return set_error(err, FE2O3_SLICE1_E_HOST_FIELD, ch.field), FE2O3_ERR_JOIN;
  for (int i = 0; i < 3; ++i)
    if (std::memcmp(f.host_length_identities[i], c.buffers[i].length_identity, 32) != 0)
      return set_error(err, FE2O3_SLICE1_E_HOST_LENGTH_IDENTITY, "", i), FE2O3_ERR_JOIN;
  set_error(err, FE2O3_SLICE1_E_NONE);
  return FE2O3_OK;
}

// ---- process identities ---------------------------------------------------------------

const uint8_t* runtime_instance() {
  static const std::array<uint8_t, 16> id = [] {
    Sha256 d;
    hash_domain(d, kRuntimeDomain);
    hash_le<uint64_t>(d, (uint64_t)getpid());
    hash_le<uint64_t>(d, (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count());
    static int anchor;
    hash_le<uint64_t>(d, (uint64_t)(uintptr_t)&anchor);
    uint8_t full[32];
    d.finish(full);
    std::array<uint8_t, 16> x{};
    std::memcpy(x.data(), full, 16);
    return x;
  }();
  return id.data();
}

void context_identity_for(int32_t device, uint8_t out[16]) {
  Sha256 d;
  hash_domain(d, kContextDomain);
  hash_field(d, runtime_instance(), 16);
  hash_le<int32_t>(d, device);
  uint8_t full[32];
  d.finish(full);
  std::memcpy(out, full, 16);
}

void unload_identity(const char* domain, const Fe2o3Slice1UnloadV1& u, const uint8_t runtime[16],
                     uint64_t agent, uint8_t out[32]) {
  Sha256 d;
  hash_domain(d, domain);
  hash_field(d, u.executable_object, 16);
  hash_field(d, runtime, 16);
  hash_le<uint64_t>(d, agent);
  const uint8_t released = u.released ? 1 : 0;
  hash_field(d, &released, 1);
  d.finish(out);
}

// "gfx950:xnack-" is compatible with an observed "gfx950:sramecc+:xnack-":
// same processor, and every feature the request names has the same setting
// (a feature the device does not report is taken as either setting).
bool target_compatible(const char* requested, const char* observed) {
  auto split = [](const std::string& t) {
    std::vector<std::string> parts;
    size_t start = 0;
    for (;;) {
      const size_t c = t.find(':', start);
      parts.push_back(t.substr(start, c == std::string::npos ? std::string::npos : c - start));
      if (c == std::string::npos) break;
      start = c + 1;
    }
    return parts;
  };
  const auto req = split(requested), obs = split(observed);
  if (req.empty() || obs.empty() || req[0] != obs[0]) return false;
  for (size_t i = 1; i < req.size(); ++i) {
    const std::string& f = req[i];
    if (f.empty()) return false;
    const std::string name = f.substr(0, f.size() - 1);
    for (size_t j = 1; j < obs.size(); ++j)
      if (obs[j].substr(0, obs[j].size() - 1) == name && obs[j] != f) return false;
  }
  return true;
}

bool eq16(const uint8_t* a, const uint8_t* b) { return std::memcmp(a, b, 16) == 0; }
bool geometry_eq(const Fe2o3Slice1GeometryV1& a, const Fe2o3Slice1GeometryV1& b) {
  return std::memcmp(&a, &b, sizeof(a)) == 0;
}
Fe2o3Slice1GeometryV1 exact_geometry() {
  Fe2o3Slice1GeometryV1 g{};
  for (int i = 0; i < 3; ++i) {
    g.grid[i] = kGrid[i];
    g.workgroup[i] = kWorkgroup[i];
  }
  g.dynamic_lds_bytes = kDynamicLds;
  return g;
}

}  // namespace

// ---- the lifecycle handle -------------------------------------------------------------

struct Fe2o3Slice1Lifecycle {
  const Spec* spec = &kSlice1Spec;
  int32_t state = FE2O3_SLICE1_JOINED;
  int32_t device = 0;
  bool leases = true;
  void (*release_leases)(void*) = nullptr;
  void* user = nullptr;
  // the complete kernarg of the profile (spec->complete_bytes of it used)
  alignas(16) uint8_t kernarg[FE2O3_PROTECTED_MAX_COMPLETE_KERNARG_BYTES] = {};
  bool has_adapter = false;
  Fe2o3Slice1AdapterV1 adapter{};
  bool has_executable = false, has_kernel = false;
  uint64_t executable = 0, kernel = 0;
  Fe2o3Slice1EnvironmentV1 environment{};
  Fe2o3Slice1LoadV1 load{};
  Fe2o3Slice1ResolutionV1 resolution{};
  Fe2o3Slice1ResourcesV1 resources{};
  uint8_t dispatch_identity[16] = {};
  Fe2o3Slice1ErrorV1 last_error{};
};

namespace {

void release_leases(Fe2o3Slice1Lifecycle* lc) {
  if (!lc->leases) return;
  lc->leases = false;
  std::memset(lc->kernarg, 0, sizeof(lc->kernarg));
  if (lc->release_leases) lc->release_leases(lc->user);
}

void drop_kernel(Fe2o3Slice1Lifecycle* lc) {
  if (!lc->has_kernel) return;
  lc->has_kernel = false;
  if (lc->adapter.drop_kernel) lc->adapter.drop_kernel(lc->adapter.self, lc->kernel);
}

// terminal_unload (:789-806): an unload the adapter cannot complete, or whose
// observation names another object, runtime or agent, leaves the
// executable's state unknown; the process ends.
Fe2o3Slice1UnloadV1 terminal_unload(Fe2o3Slice1Lifecycle* lc) {
  Fe2o3Slice1UnloadV1 u{};
  lc->has_executable = false;
  const int32_t rc = lc->adapter.unload_executable
                         ? lc->adapter.unload_executable(lc->adapter.self, lc->executable, &u)
                         : -1;
  if (rc != 0) std::abort();
  if (!eq16(u.executable_object, lc->load.executable_object) ||
      !eq16(u.runtime_instance, lc->environment.runtime_instance) ||
      u.agent_handle != lc->environment.agent_handle || !u.released)
    std::abort();
  return u;
}

void drop_adapter(Fe2o3Slice1Lifecycle* lc) {
  if (!lc->has_adapter) return;
  lc->has_adapter = false;
  if (lc->adapter.drop_adapter) lc->adapter.drop_adapter(lc->adapter.self);
}

// Everything a failure at or after load owes: kernel, executable, leases,
// adapter -- in that order -- then the FAILED state.
int32_t fail(Fe2o3Slice1Lifecycle* lc, Fe2o3Slice1ErrorV1* err, int32_t status) {
  drop_kernel(lc);
  if (lc->has_executable) terminal_unload(lc);
  release_leases(lc);
  drop_adapter(lc);
  lc->state = FE2O3_SLICE1_FAILED;
  if (err) lc->last_error = *err;
  return status;
}

int32_t load_error(Fe2o3Slice1Lifecycle* lc, Fe2o3Slice1ErrorV1* err, int32_t kind,
                   const char* field = "", int32_t adapter_status = 0) {
  Fe2o3Slice1ErrorV1 local;
  if (!err) err = &local;
  set_error(err, kind, field, -1, adapter_status);
  return fail(lc, err, FE2O3_ERR_LOAD);
}

int32_t dispatch_error(Fe2o3Slice1Lifecycle* lc, Fe2o3Slice1ErrorV1* err, int32_t kind,
                       const char* field = "", int32_t adapter_status = 0) {
  Fe2o3Slice1ErrorV1 local;
  if (!err) err = &local;
  set_error(err, kind, field, -1, adapter_status);
  return fail(lc, err, FE2O3_ERR_DISPATCH);
}

int32_t state_error(Fe2o3Slice1ErrorV1* err, int32_t state) {
  set_error(err, FE2O3_SLICE1_E_NONE, "state", -1, 0, 0, (uint64_t)state);
  return FE2O3_ERR_STATE;
}

// load_after_context_match (:698-777).
int32_t do_load(Fe2o3Slice1Lifecycle* lc, Fe2o3Slice1ErrorV1* err) {
  Fe2o3Slice1AdapterV1& ad = lc->adapter;
  void* self = ad.self;
  int32_t rc = ad.observe_environment ? ad.observe_environment(self, &lc->environment) : -1;
  if (rc != 0) return load_error(lc, err, FE2O3_SLICE1_E_ENVIRONMENT_ADAPTER, "", rc);
  const Fe2o3Slice1EnvironmentV1& env = lc->environment;
  // validate_environment (:808-846)
  const struct {
    bool ok;
    const char* field;
  } env_checks[] = {
      {target_compatible(kTarget, env.physical_target), "physical-device target"},
      {std::strncmp(env.agent_target, env.physical_target, sizeof(env.agent_target)) == 0,
       "agent target"},
      {env.hip_ordinal == lc->device, "HIP ordinal"},
      {eq16(env.agent_runtime_instance, env.runtime_instance), "runtime instance"},
      {eq16(env.agent_physical_uuid, env.physical_uuid), "physical device"},
  };
  for (const auto& ch : env_checks)
    if (!ch.ok) return load_error(lc, err, FE2O3_SLICE1_E_ENVIRONMENT, ch.field);

  const Spec& spec = *lc->spec;
  uint8_t digest[32];
  sha256(spec.code, spec.code_len, digest);
  rc = ad.load_executable ? ad.load_executable(self, spec.code, spec.code_len, digest,
                                               &lc->executable, &lc->load)
                          : -1;
  if (rc != 0) return load_error(lc, err, FE2O3_SLICE1_E_LOAD_ADAPTER, "", rc);
  lc->has_executable = true;
  if (std::memcmp(lc->load.digest, digest, 32) != 0 || lc->load.byte_len != spec.code_len ||
      !eq16(lc->load.runtime_instance, env.runtime_instance) ||
      lc->load.agent_handle != env.agent_handle)
    return load_error(lc, err, FE2O3_SLICE1_E_LOAD_OBSERVATION, "identity or content observation");

  rc = ad.resolve_kernel ? ad.resolve_kernel(self, lc->executable, spec.symbol, &lc->kernel,
                                             &lc->resolution)
                         : -1;
  if (rc != 0) return load_error(lc, err, FE2O3_SLICE1_E_KERNEL_ADAPTER, "", rc);
  lc->has_kernel = true;
  const Fe2o3Slice1ResolutionV1& res = lc->resolution;
  if (!eq16(res.executable_object, lc->load.executable_object) ||
      strncmp(res.symbol, spec.symbol, sizeof(res.symbol)) != 0 ||
      res.kernarg_segment_bytes != spec.complete_bytes || res.kernarg_alignment != kHsaKernargAlign)
    return load_error(lc, err, FE2O3_SLICE1_E_KERNEL_OBSERVATION,
                      "object, symbol, size, or HSA alignment");

  rc = ad.observe_resources
           ? ad.observe_resources(self, lc->executable, lc->kernel, &lc->resources)
           : -1;
  if (rc != 0) return load_error(lc, err, FE2O3_SLICE1_E_RESOURCE_ADAPTER, "", rc);
  const Fe2o3Slice1ResourcesV1& r = lc->resources;
  if (!eq16(r.executable_object, lc->load.executable_object) ||
      !eq16(r.kernel_object, res.kernel_object) || r.group_segment_bytes != spec.static_lds ||
      r.private_segment_bytes != kPrivateSegment)
    return load_error(lc, err, FE2O3_SLICE1_E_RESOURCE_OBSERVATION,
                      "object, static LDS, or private segment");
  if ((uintptr_t)lc->kernarg % kHsaKernargAlign != 0)
    return load_error(lc, err, FE2O3_SLICE1_E_KERNEL_OBSERVATION, "staging kernarg alignment");
  lc->state = FE2O3_SLICE1_LOADED;
  set_error(err, FE2O3_SLICE1_E_NONE);
  return FE2O3_OK;
}

// LoadedExactStateV1::dispatch_and_wait (:639-696).
int32_t do_dispatch(Fe2o3Slice1Lifecycle* lc, Fe2o3Slice1ErrorV1* err) {
  Fe2o3Slice1AdapterV1& ad = lc->adapter;
  const Spec& spec = *lc->spec;
  const Fe2o3Slice1GeometryV1 geometry = exact_geometry();
  uint8_t explicit_bytes[FE2O3_PROTECTED_MAX_COMPLETE_KERNARG_BYTES];
  std::memcpy(explicit_bytes, lc->kernarg, spec.explicit_bytes);
  Fe2o3Slice1ImplicitV1 imp{};
  int32_t rc = ad.initialize_implicit_kernarg
                   ? ad.initialize_implicit_kernarg(ad.self, lc->executable, lc->kernel, &geometry,
                                                    spec.explicit_bytes, spec.explicit_bytes,
                                                    spec.implicit_bytes(), lc->kernarg,
                                                    spec.complete_bytes, &imp)
                   : -1;
  if (rc != 0) return dispatch_error(lc, err, FE2O3_SLICE1_E_IMPLICIT_ADAPTER, "", rc);
  if (std::memcmp(explicit_bytes, lc->kernarg, spec.explicit_bytes) != 0)
    return dispatch_error(lc, err, FE2O3_SLICE1_E_EXPLICIT_KERNARG_MUTATION);
  if (!eq16(imp.executable_object, lc->load.executable_object) ||
      !eq16(imp.kernel_object, lc->resolution.kernel_object) || !geometry_eq(imp.geometry, geometry) ||
      imp.explicit_bytes != spec.explicit_bytes || imp.implicit_offset != spec.explicit_bytes ||
      imp.implicit_bytes != spec.implicit_bytes() || !imp.completed)
    return dispatch_error(lc, err, FE2O3_SLICE1_E_IMPLICIT_OBSERVATION,
                          "object, geometry, span, or completion");
  Fe2o3Slice1DispatchV1 dsp{};
  rc = ad.launch_and_wait ? ad.launch_and_wait(ad.self, lc->executable, lc->kernel, &geometry,
                                               lc->kernarg, spec.complete_bytes, &dsp)
                          : -1;
  if (rc != 0) return dispatch_error(lc, err, FE2O3_SLICE1_E_DISPATCH_ADAPTER, "", rc);
  if (!eq16(dsp.executable_object, lc->load.executable_object) ||
      !eq16(dsp.kernel_object, lc->resolution.kernel_object) || !geometry_eq(dsp.geometry, geometry) ||
      !dsp.completed)
    return dispatch_error(lc, err, FE2O3_SLICE1_E_DISPATCH_OBSERVATION,
                          "object, geometry, or completion");
  std::memcpy(lc->dispatch_identity, dsp.dispatch_identity, 16);
  // The kernel handle dies before any unload; the dispatch is quiescent, so
  // A, B and C are no longer reachable from the GPU.
  drop_kernel(lc);
  release_leases(lc);
  lc->state = FE2O3_SLICE1_COMPLETED;
  set_error(err, FE2O3_SLICE1_E_NONE);
  return FE2O3_OK;
}

int32_t lifecycle_load(Fe2o3Slice1Lifecycle* lc, const Fe2o3Slice1AdapterV1* adapter,
                       Fe2o3Slice1ErrorV1* error);

// ---- protected profiles ---------------------------------------------------------------
//
// crates/fe2o3-host/src/flash_attention_v1_lifecycle.rs,
// protected_row_softmax_v1_lifecycle.rs and moe_top2_v1_lifecycle.rs: the
// profile constants (:20-32 of each), validate_join's receipt and host
// checks in their order, and the unload identity domains.

constexpr char kReceiptDomain[] = "FE2O3/MI355X-PROTECTED-RECEIPT/V1";
constexpr char kProtectedProfileDomain[] = "FE2O3/MI355X-PROTECTED-PROFILE/V1";
constexpr char kCompilerDomain[] = "FE2O3/MI355X-PROTECTED-COMPILER/V1";
constexpr uint32_t kMaxRegions = FE2O3_PROTECTED_MAX_REGIONS;

struct ProtectedDef {
  Spec spec;
  const char* name;
  const uint8_t* build_digest;
  const uint8_t* source_digest;
  const char* compiler;
  const char* flags;
  uint32_t regions;
  uint64_t elements[kMaxRegions];
  uint32_t element_bytes[kMaxRegions];
  uint32_t writes[kMaxRegions];
  uint32_t shape[4];
  const char* receipt_fields[16];
  const char* host_fields[16];
};

const ProtectedDef kProtected[] = {
    {{FE2O3_PROFILE_FLASH_ATTENTION_V1, "flash_attention_causal_f32_b1_h1_n8_d16_v1",
      kFlashV1CodeObject, sizeof(kFlashV1CodeObject), 64, 320, 0,
      "FE2O3/FLASH-ATTENTION/UNLOAD/V1"},
     "flash_attention_v1", kFlashV1BuildDigest, kFlashV1SourceDigest, kFlashV1Compiler,
     kFlashV1Flags, 4, {128, 128, 128, 128}, {4, 4, 4, 4}, {0, 0, 0, 1}, {1, 1, 8, 16},
     // flash_attention_v1_lifecycle.rs:720-799
     {"identity", "artifact identity", "finalized output", "raw worker output", "target",
      "code-object version", "frontend authority commitment", "OCML provider commitment",
      "finalization", "compiler handoff", "machine identity", "OCML provider closure"},
     {"target", "shape", "argument extent", "grid", "workgroup", "code-object version",
      "explicit ABI", "complete ABI", "ABI alignment", "mask policy"}},
    {{FE2O3_PROFILE_ROW_SOFTMAX_V1, "row_softmax_v1", kSoftmaxV1CodeObject,
      sizeof(kSoftmaxV1CodeObject), 32, 288, 0, "FE2O3/ROW-SOFTMAX/UNLOAD/V1"},
     "row_softmax_v1", kSoftmaxV1BuildDigest, kSoftmaxV1SourceDigest, kSoftmaxV1Compiler,
     kSoftmaxV1Flags, 2, {64, 64}, {4, 4}, {0, 1}, {64, 0, 0, 0},
     // protected_row_softmax_v1_lifecycle.rs:723-777
     {"identity", "admission identity", "artifact identity", "finalized output", "target",
      "row width", "grid", "workgroup", "explicit ABI", "complete ABI"},
     {"target", "row width", "grid", "workgroup", "explicit ABI", "complete ABI",
      "ABI alignment", "activity policy"}},
    {{FE2O3_PROFILE_MOE_TOP2_V1, "moe_top2_route_f32_t8_e4_k2_c4_v1", kMoeTop2V1CodeObject,
      sizeof(kMoeTop2V1CodeObject), 128, 384, 0, "FE2O3/MOE-TOP2/UNLOAD/V1"},
     "moe_top2_v1", kMoeTop2V1BuildDigest, kMoeTop2V1SourceDigest, kMoeTop2V1Compiler,
     kMoeTop2V1Flags, 8, {32, 16, 4, 4, 5, 16, 16, 16}, {4, 4, 4, 4, 4, 4, 4, 4},
     {0, 1, 1, 1, 1, 1, 1, 1}, {8, 4, 2, 4},
     // moe_top2_v1_lifecycle.rs:824-890
     {"identity", "artifact identity", "finalized output", "raw worker output", "target",
      "code-object version", "canonical digest", "source/KIR/compiler profile",
      "upstream LLVM/LLD exchange"},
     {"target", "T/E/K/C profile", "grid", "workgroup", "code-object version", "explicit ABI",
      "complete ABI", "ABI alignment", "routing-only policy"}},
};

const ProtectedDef* protected_def(uint32_t profile) {
  for (const auto& d : kProtected)
    if (d.spec.profile == profile) return &d;
  return nullptr;
}

uint32_t count_fields(const char* const* f) {
  uint32_t n = 0;
  while (n < 16 && f[n] != nullptr) ++n;
  return n;
}

Fe2o3ProtectedProfileV1 profile_view(const ProtectedDef& d) {
  Fe2o3ProtectedProfileV1 v{};
  v.profile = d.spec.profile;
  v.code_object_version = kCodeObjectVersion;
  std::strncpy(v.name, d.name, sizeof(v.name) - 1);
  std::strncpy(v.target, kTarget, sizeof(v.target) - 1);
  std::strncpy(v.symbol, d.spec.symbol, sizeof(v.symbol) - 1);
  for (int i = 0; i < 3; ++i) {
    v.grid[i] = kGrid[i];
    v.workgroup[i] = kWorkgroup[i];
  }
  v.dynamic_lds_bytes = kDynamicLds;
  v.static_lds_bytes = d.spec.static_lds;
  v.private_segment_bytes = kPrivateSegment;
  v.explicit_kernarg_bytes = d.spec.explicit_bytes;
  v.complete_kernarg_bytes = d.spec.complete_bytes;
  v.kernarg_alignment = kContractKernargAlign;
  v.hsa_kernarg_alignment = (uint32_t)kHsaKernargAlign;
  v.regions = d.regions;
  for (uint32_t i = 0; i < d.regions; ++i) {
    v.region_elements[i] = d.elements[i];
    v.region_element_bytes[i] = d.element_bytes[i];
    v.region_writes[i] = d.writes[i];
  }
  std::memcpy(v.shape, d.shape, sizeof(v.shape));
  v.receipt_fields = count_fields(d.receipt_fields);
  v.host_fields = count_fields(d.host_fields);
  for (uint32_t i = 0; i < v.receipt_fields; ++i)
    std::strncpy(v.receipt_field[i], d.receipt_fields[i], sizeof(v.receipt_field[i]) - 1);
  for (uint32_t i = 0; i < v.host_fields; ++i)
    std::strncpy(v.host_field[i], d.host_fields[i], sizeof(v.host_field[i]) - 1);
  return v;
}

bool nonzero32(const uint8_t* p) {
  for (int i = 0; i < 32; ++i)
    if (p[i]) return true;
  return false;
}

struct ProtectedArtifact {
  Fe2o3ProtectedArtifactV1 view{};
  const char* inspect_error = "";
  bool facts_agree = false;  // the code object's own facts against the profile
};

const ProtectedArtifact& protected_artifact(const ProtectedDef& d) {
  static ProtectedArtifact cache[sizeof(kProtected) / sizeof(kProtected[0])];
  static std::once_flag once[sizeof(kProtected) / sizeof(kProtected[0])];
  const size_t slot = (size_t)(&d - kProtected);
  std::call_once(once[slot], [&] {
    ProtectedArtifact& x = cache[slot];
    Fe2o3ProtectedArtifactV1& v = x.view;
    v.profile = profile_view(d);
    sha256(d.spec.code, d.spec.code_len, v.artifact_identity);
    std::memcpy(v.build_digest, d.build_digest, 32);
    std::memcpy(v.source_digest, d.source_digest, 32);
    {
      Sha256 h;
      hash_domain(h, kCompilerDomain);
      hash_str(h, d.compiler);
      hash_str(h, d.flags);
      h.finish(v.compiler_identity);
    }
    {
      Sha256 h;
      hash_domain(h, kProtectedProfileDomain);
      hash_le<uint32_t>(h, d.spec.profile);
      hash_str(h, d.name);
      hash_str(h, kTarget);
      hash_str(h, d.spec.symbol);
      for (int i = 0; i < 3; ++i) hash_le<uint32_t>(h, kGrid[i]);
      for (int i = 0; i < 3; ++i) hash_le<uint32_t>(h, kWorkgroup[i]);
      hash_le<uint32_t>(h, d.spec.explicit_bytes);
      hash_le<uint32_t>(h, d.spec.complete_bytes);
      for (uint32_t i = 0; i < d.regions; ++i) {
        hash_le<uint64_t>(h, d.elements[i]);
        hash_le<uint32_t>(h, d.element_bytes[i]);
        hash_le<uint32_t>(h, d.writes[i]);
      }
      for (int i = 0; i < 4; ++i) hash_le<uint32_t>(h, d.shape[i]);
      h.finish(v.profile_identity);
    }
    {
      Sha256 h;
      hash_domain(h, kReceiptDomain);
      hash_field(h, v.profile_identity, 32);
      hash_field(h, v.artifact_identity, 32);
      hash_field(h, v.source_digest, 32);
      hash_field(h, v.compiler_identity, 32);
      h.finish(v.identity);
    }
    char kernel[64], descriptor[64];
    x.inspect_error = fe2o3_inspect::inspect_single_kernel(d.spec.code, d.spec.code_len, kernel,
                                                           descriptor, sizeof(kernel),
                                                           &v.inspection);
    const Fe2o3Slice1InspectionV1& i = v.inspection;
    x.facts_agree = x.inspect_error[0] == '\0' && std::strcmp(kernel, d.spec.symbol) == 0 &&
                    i.kd_kernarg_bytes == d.spec.complete_bytes &&
                    i.md_kernarg_bytes == d.spec.complete_bytes &&
                    i.explicit_bytes == d.spec.explicit_bytes &&
                    i.explicit_args == d.regions &&
                    i.implicit_offset == d.spec.explicit_bytes &&
                    i.kd_group_segment_bytes == d.spec.static_lds &&
                    i.md_group_segment_bytes == d.spec.static_lds &&
                    i.kd_private_segment_bytes == kPrivateSegment &&
                    i.md_private_segment_bytes == kPrivateSegment &&
                    i.kd_wavefront_size == kWavefront && i.md_wavefront_size == kWavefront &&
                    i.md_max_flat_workgroup_size == kWorkgroup[0];
  });
  return cache[slot];
}

// One receipt check, by the reference's field name, as this library's
// artifact answers it.
bool receipt_check(const ProtectedDef& d, const ProtectedArtifact& a, const char* field) {
  const Fe2o3ProtectedArtifactV1& v = a.view;
  const Fe2o3Slice1InspectionV1& i = v.inspection;
  const bool bytes_recorded = std::memcmp(v.artifact_identity, v.build_digest, 32) == 0;
  const bool closure = a.facts_agree && i.sgpr_spills == 0 && i.vgpr_spills == 0 &&
                       i.uses_dynamic_stack == 0;
  auto is = [&](const char* f) { return std::strcmp(field, f) == 0; };
  if (is("identity")) return nonzero32(v.identity);
  if (is("admission identity")) return nonzero32(v.profile_identity);
  if (is("artifact identity")) return nonzero32(v.artifact_identity);
  if (is("finalized output")) return d.spec.code_len != 0;
  if (is("raw worker output")) return nonzero32(v.build_digest);
  if (is("target")) return std::strcmp(i.target, kTarget) == 0;
  if (is("code-object version")) return i.code_object_version == kCodeObjectVersion;
  if (is("frontend authority commitment") || is("canonical digest"))
    return nonzero32(v.source_digest);
  if (is("OCML provider commitment")) return nonzero32(v.compiler_identity);
  if (is("finalization") || is("source/KIR/compiler profile")) return a.facts_agree;
  if (is("compiler handoff") || is("upstream LLVM/LLD exchange")) return bytes_recorded;
  if (is("machine identity")) return (i.e_flags & fe2o3_inspect::kMachMask) == fe2o3_inspect::kMachGfx950;
  if (is("OCML provider closure")) return closure;
  if (is("row width")) return d.shape[0] == 64;
  if (is("grid")) return a.facts_agree;  // one workgroup: the profile's launch
  if (is("workgroup")) return i.md_max_flat_workgroup_size == kWorkgroup[0];
  if (is("explicit ABI")) return i.explicit_bytes == d.spec.explicit_bytes;
  if (is("complete ABI")) return i.md_kernarg_bytes == d.spec.complete_bytes;
  return false;
}

void protected_canonical_facts(const ProtectedDef& d, Fe2o3ProtectedJoinFactsV1* f) {
  const ProtectedArtifact& a = protected_artifact(d);
  std::memset(f, 0, sizeof(*f));
  f->profile = d.spec.profile;
  for (uint32_t r = 0; r < count_fields(d.receipt_fields); ++r)
    f->receipt[r] = receipt_check(d, a, d.receipt_fields[r]) ? 1 : 0;
  std::strncpy(f->host_target, kTarget, sizeof(f->host_target) - 1);
  std::memcpy(f->host_shape, d.shape, sizeof(f->host_shape));
  f->host_argument_elements = d.elements[0];
  for (int i = 0; i < 3; ++i) {
    f->host_grid[i] = kGrid[i];
    f->host_workgroup[i] = kWorkgroup[i];
  }
  f->host_code_object_version = kCodeObjectVersion;
  f->host_explicit_kernarg = d.spec.explicit_bytes;
  f->host_complete_kernarg = d.spec.complete_bytes;
  f->host_kernarg_alignment = kContractKernargAlign;
  f->host_policy = 1;
}

// validate_join: the receipt fields, then the host fields, in the
// reference's order; the first that does not hold.
int32_t protected_validate_join(const ProtectedDef& d, const Fe2o3ProtectedJoinFactsV1& f,
                                Fe2o3Slice1ErrorV1* err) {
  for (uint32_t r = 0; r < count_fields(d.receipt_fields); ++r)
    if (!f.receipt[r])
      return set_error(err, FE2O3_SLICE1_E_RECEIPT_FIELD, d.receipt_fields[r]), FE2O3_ERR_JOIN;
  for (uint32_t h = 0; h < count_fields(d.host_fields); ++h) {
    const char* field = d.host_fields[h];
    auto is = [&](const char* x) { return std::strcmp(field, x) == 0; };
    bool ok = false;
    if (is("target"))
      ok = std::strncmp(f.host_target, kTarget, sizeof(f.host_target)) == 0;
    else if (is("shape") || is("row width") || is("T/E/K/C profile"))
      ok = std::memcmp(f.host_shape, d.shape, sizeof(f.host_shape)) == 0;
    else if (is("argument extent"))
      ok = f.host_argument_elements == d.elements[0];
    else if (is("grid"))
      ok = f.host_grid[0] == kGrid[0] && f.host_grid[1] == kGrid[1] && f.host_grid[2] == kGrid[2];
    else if (is("workgroup"))
      ok = f.host_workgroup[0] == kWorkgroup[0] && f.host_workgroup[1] == kWorkgroup[1] &&
           f.host_workgroup[2] == kWorkgroup[2];
    else if (is("code-object version"))
      ok = f.host_code_object_version == kCodeObjectVersion;
    else if (is("explicit ABI"))
      ok = f.host_explicit_kernarg == d.spec.explicit_bytes;
    else if (is("complete ABI"))
      ok = f.host_complete_kernarg == d.spec.complete_bytes;
    else if (is("ABI alignment"))
      ok = f.host_kernarg_alignment == kContractKernargAlign;
    else
      ok = f.host_policy == 1;  // the profile's policy field
    if (!ok) return set_error(err, FE2O3_SLICE1_E_HOST_FIELD, field), FE2O3_ERR_JOIN;
  }
  set_error(err, FE2O3_SLICE1_E_NONE);
  return FE2O3_OK;
}

// ---- the HIP adapter ------------------------------------------------------------------

constexpr uint32_t kHipExeMagic = 0x45584531u, kHipKernelMagic = 0x4b524e31u;

struct HipAdapter {
  int32_t device;
  uint64_t agent_handle;
  uint8_t uuid[16];
  char target[64];
  bool observed;
};
struct HipExecutable {
  uint32_t magic;
  hipModule_t module;
  hipStream_t stream;
  uint8_t identity[16];
  // the code object's one kernel, as its own metadata names it
  char kernel[64], descriptor[64];
  Fe2o3Slice1InspectionV1 inspection;
};
struct HipKernel {
  uint32_t magic;
  hipFunction_t function;
  HipExecutable* exe;
  uint8_t identity[16];
};

std::atomic<uint64_t> g_sequence{1};

void object_identity(uint64_t tag, const void* handle, uint8_t out[16]) {
  const uint64_t seq = g_sequence.fetch_add(1);
  put_le64(out, (uint64_t)(uintptr_t)handle ^ (tag << 56));
  put_le64(out + 8, seq);
}

class DeviceScope {
 public:
  explicit DeviceScope(int32_t device) {
    ok_ = hipGetDevice(&prev_) == hipSuccess && hipSetDevice(device) == hipSuccess;
  }
  ~DeviceScope() {
    if (ok_) (void)hipSetDevice(prev_);
  }
  bool ok() const { return ok_; }

 private:
  int prev_ = 0;
  bool ok_ = false;
};

HipExecutable* as_exe(uint64_t h) {
  auto* e = reinterpret_cast<HipExecutable*>((uintptr_t)h);
  return (e && e->magic == kHipExeMagic) ? e : nullptr;
}
HipKernel* as_kernel(uint64_t h) {
  auto* k = reinterpret_cast<HipKernel*>((uintptr_t)h);
  return (k && k->magic == kHipKernelMagic) ? k : nullptr;
}

int32_t hip_context_identity(void* self, uint8_t identity[16]) {
  context_identity_for(static_cast<HipAdapter*>(self)->device, identity);
  return 0;
}

int32_t hip_observe_environment(void* self, Fe2o3Slice1EnvironmentV1* out) {
  auto* a = static_cast<HipAdapter*>(self);
  hipDeviceProp_t prop;
  hipError_t rc = hipGetDeviceProperties(&prop, a->device);
  if (rc != hipSuccess) return (int32_t)rc;
  hipUUID uuid;
  rc = hipDeviceGetUuid(&uuid, a->device);
  if (rc != hipSuccess) return (int32_t)rc;
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out->runtime_instance, runtime_instance(), 16);
  std::strncpy(out->physical_target, prop.gcnArchName, sizeof(out->physical_target) - 1);
  out->hip_ordinal = a->device;
  std::memcpy(out->physical_uuid, uuid.bytes, 16);
  // HIP has one view of the device: the agent is the PCI function it sits on.
  std::strncpy(out->agent_target, prop.gcnArchName, sizeof(out->agent_target) - 1);
  out->agent_handle = (uint64_t)(uint32_t)prop.pciDomainID << 32 |
                      (uint64_t)(uint32_t)prop.pciBusID << 8 | (uint64_t)(uint32_t)prop.pciDeviceID;
  std::memcpy(out->agent_runtime_instance, runtime_instance(), 16);
  std::memcpy(out->agent_physical_uuid, uuid.bytes, 16);
  a->agent_handle = out->agent_handle;
  std::memcpy(a->uuid, uuid.bytes, 16);
  std::strncpy(a->target, prop.gcnArchName, sizeof(a->target) - 1);
  a->observed = true;
  return 0;
}

int32_t hip_load_executable(void* self, const uint8_t* bytes, uint64_t byte_len,
                            const uint8_t* /*digest*/, uint64_t* executable,
                            Fe2o3Slice1LoadV1* out) {
  auto* a = static_cast<HipAdapter*>(self);
  if (!a->observed) return FE2O3_ERR_DEVICE;
  std::unique_ptr<HipExecutable> e(new HipExecutable{});
  e->magic = kHipExeMagic;
  // the object is read (bounds-checked) before the runtime sees it: one
  // kernel, its descriptor and metadata readable
  const char* bad = fe2o3_inspect::inspect_single_kernel(
      bytes, byte_len, e->kernel, e->descriptor, sizeof(e->kernel), &e->inspection);
  if (bad[0]) return FE2O3_ERR_SHAPE;
  DeviceScope scope(a->device);
  if (!scope.ok()) return FE2O3_ERR_DEVICE;
  hipError_t rc = hipModuleLoadData(&e->module, bytes);
  if (rc != hipSuccess) return (int32_t)rc;
  rc = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
  if (rc != hipSuccess) {
    (void)hipModuleUnload(e->module);
    return (int32_t)rc;
  }
  object_identity(1, e->module, e->identity);
  std::memset(out, 0, sizeof(*out));
  sha256(bytes, byte_len, out->digest);  // what was loaded, not what was claimed
  out->byte_len = byte_len;
  std::memcpy(out->runtime_instance, runtime_instance(), 16);
  out->agent_handle = a->agent_handle;
  std::memcpy(out->executable_object, e->identity, 16);
  *executable = (uint64_t)(uintptr_t)e.release();
  return 0;
}

int32_t hip_resolve_kernel(void* self, uint64_t executable, const char* symbol, uint64_t* kernel,
                           Fe2o3Slice1ResolutionV1* out) {
  auto* a = static_cast<HipAdapter*>(self);
  HipExecutable* e = as_exe(executable);
  if (!e) return FE2O3_ERR_NULL;
  DeviceScope scope(a->device);
  if (!scope.ok()) return FE2O3_ERR_DEVICE;
  if (symbol == nullptr || std::strcmp(symbol, e->kernel) != 0) return (int32_t)hipErrorNotFound;
  std::unique_ptr<HipKernel> k(new HipKernel{});
  k->magic = kHipKernelMagic;
  k->exe = e;
  const hipError_t rc = hipModuleGetFunction(&k->function, e->module, symbol);
  if (rc != hipSuccess) return (int32_t)rc;
  object_identity(2, k->function, k->identity);
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out->executable_object, e->identity, 16);
  std::memcpy(out->kernel_object, k->identity, 16);
  std::strncpy(out->symbol, symbol, sizeof(out->symbol) - 1);
  // The kernarg segment as the loaded code object declares it; the
  // dispatch-side alignment is at least the 16 bytes HSA guarantees.
  out->kernarg_segment_bytes = e->inspection.md_kernarg_bytes;
  out->kernarg_alignment = std::max<uint64_t>(kHsaKernargAlign, e->inspection.md_kernarg_alignment);
  *kernel = (uint64_t)(uintptr_t)k.release();
  return 0;
}

int32_t hip_observe_resources(void* self, uint64_t executable, uint64_t kernel,
                              Fe2o3Slice1ResourcesV1* out) {
  auto* a = static_cast<HipAdapter*>(self);
  HipExecutable* e = as_exe(executable);
  HipKernel* k = as_kernel(kernel);
  if (!e || !k || k->exe != e) return FE2O3_ERR_NULL;
  DeviceScope scope(a->device);
  if (!scope.ok()) return FE2O3_ERR_DEVICE;
  int lds = 0, priv = 0;
  hipError_t rc = hipFuncGetAttribute(&lds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, k->function);
  if (rc != hipSuccess) return (int32_t)rc;
  rc = hipFuncGetAttribute(&priv, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, k->function);
  if (rc != hipSuccess) return (int32_t)rc;
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out->executable_object, e->identity, 16);
  std::memcpy(out->kernel_object, k->identity, 16);
  out->group_segment_bytes = (uint32_t)lds;
  out->private_segment_bytes = (uint32_t)priv;
  return 0;
}

// The code object v5/v6 implicit suffix for a dispatch of `g`: block
// counts (u32 at 0, 4, 8), workgroup sizes (u16 at 12, 14, 16), partial
// workgroup remainders (u16 at 18, 20, 22; 0 for whole workgroups), global
// offsets (u64 at 40, 48, 56; 0) and the grid dimensionality (u16 at 64);
// every other byte 0.  The HIP runtime writes the same values when it
// builds the dispatch.
int32_t hip_initialize_implicit(void* /*self*/, uint64_t executable, uint64_t kernel,
                                const Fe2o3Slice1GeometryV1* g, uint64_t explicit_bytes,
                                uint64_t implicit_offset, uint64_t implicit_bytes,
                                uint8_t* kernarg, uint64_t kernarg_bytes,
                                Fe2o3Slice1ImplicitV1* out) {
  HipExecutable* e = as_exe(executable);
  HipKernel* k = as_kernel(kernel);
  if (!e || !k || k->exe != e) return FE2O3_ERR_NULL;
  if (implicit_offset < explicit_bytes || implicit_bytes < 72 ||
      implicit_offset + implicit_bytes > kernarg_bytes)
    return FE2O3_ERR_LENGTH;
  uint8_t* s = kernarg + implicit_offset;
  std::memset(s, 0, (size_t)implicit_bytes);
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 4; ++j) s[4 * i + j] = (uint8_t)(g->grid[i] >> (8 * j));
    s[12 + 2 * i] = (uint8_t)g->workgroup[i];
    s[13 + 2 * i] = (uint8_t)(g->workgroup[i] >> 8);
  }
  const uint16_t dims = (g->grid[2] * g->workgroup[2] > 1) ? 3 : (g->grid[1] * g->workgroup[1] > 1) ? 2 : 1;
  s[64] = (uint8_t)dims;
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out->executable_object, e->identity, 16);
  std::memcpy(out->kernel_object, k->identity, 16);
  out->geometry = *g;
  out->explicit_bytes = explicit_bytes;
  out->implicit_offset = implicit_offset;
  out->implicit_bytes = implicit_bytes;
  out->completed = 1;
  return 0;
}

int32_t hip_launch_and_wait(void* self, uint64_t executable, uint64_t kernel,
                            const Fe2o3Slice1GeometryV1* g, uint8_t* kernarg,
                            uint64_t kernarg_bytes, Fe2o3Slice1DispatchV1* out) {
  auto* a = static_cast<HipAdapter*>(self);
  HipExecutable* e = as_exe(executable);
  HipKernel* k = as_kernel(kernel);
  if (!e || !k || k->exe != e) return FE2O3_ERR_NULL;
  if (kernarg_bytes != e->inspection.md_kernarg_bytes) return FE2O3_ERR_LENGTH;
  DeviceScope scope(a->device);
  if (!scope.ok()) return FE2O3_ERR_DEVICE;
  size_t size = (size_t)kernarg_bytes;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, kernarg, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                    HIP_LAUNCH_PARAM_END};
  hipError_t rc = hipModuleLaunchKernel(k->function, g->grid[0], g->grid[1], g->grid[2],
                                        g->workgroup[0], g->workgroup[1], g->workgroup[2],
                                        g->dynamic_lds_bytes, e->stream, nullptr, config);
  if (rc != hipSuccess) return (int32_t)rc;
  rc = hipStreamSynchronize(e->stream);
  std::memset(out, 0, sizeof(*out));
  object_identity(3, e->stream, out->dispatch_identity);
  std::memcpy(out->executable_object, e->identity, 16);
  std::memcpy(out->kernel_object, k->identity, 16);
  out->geometry = *g;
  out->completed = rc == hipSuccess;
  return rc == hipSuccess ? 0 : (int32_t)rc;
}

void hip_drop_kernel(void* /*self*/, uint64_t kernel) {
  HipKernel* k = as_kernel(kernel);
  if (!k) return;
  k->magic = 0;
  delete k;
}

int32_t hip_unload_executable(void* self, uint64_t executable, Fe2o3Slice1UnloadV1* out) {
  auto* a = static_cast<HipAdapter*>(self);
  HipExecutable* e = as_exe(executable);
  if (!e) return FE2O3_ERR_NULL;
  DeviceScope scope(a->device);
  if (!scope.ok()) return FE2O3_ERR_DEVICE;
  const hipError_t s = hipStreamDestroy(e->stream);
  const hipError_t m = hipModuleUnload(e->module);
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out->executable_object, e->identity, 16);
  std::memcpy(out->runtime_instance, runtime_instance(), 16);
  out->agent_handle = a->agent_handle;
  out->released = s == hipSuccess && m == hipSuccess;
  e->magic = 0;
  delete e;
  return out->released ? 0 : (int32_t)(m != hipSuccess ? m : s);
}

void hip_drop_adapter(void* self) { delete static_cast<HipAdapter*>(self); }

}  // namespace

extern "C" {

int32_t fe2o3_sha256_v1(const void* data, uint64_t len, uint8_t digest[32]) {
  if (!digest || (!data && len)) return FE2O3_ERR_NULL;
  sha256(data, (size_t)len, digest);
  return FE2O3_OK;
}

int32_t fe2o3_lds_gemm_slice1_artifact_v1(Fe2o3Slice1ArtifactV1* out) {
  if (!out) return FE2O3_ERR_NULL;
  *out = artifact().view;
  return FE2O3_OK;
}

int32_t fe2o3_lds_gemm_slice1_join_facts_v1(Fe2o3Slice1JoinFactsV1* out) {
  if (!out) return FE2O3_ERR_NULL;
  canonical_facts(out);
  return FE2O3_OK;
}

int32_t fe2o3_lds_gemm_slice1_validate_join_v1(const Fe2o3Slice1JoinFactsV1* facts,
                                               Fe2o3Slice1ErrorV1* error) {
  if (!facts) return FE2O3_ERR_NULL;
  return validate_join(*facts, error);
}

int32_t fe2o3_lds_gemm_slice1_context_identity_v1(int32_t device, uint8_t identity[16]) {
  if (!identity) return FE2O3_ERR_NULL;
  context_identity_for(device, identity);
  return FE2O3_OK;
}

int32_t fe2o3_lds_gemm_slice1_join_v1(const uint16_t* a, uint64_t a_len, const uint16_t* b,
                                      uint64_t b_len, float* c, uint64_t c_len, int32_t device,
                                      void (*release)(void*), void* user,
                                      Fe2o3Slice1Lifecycle** out, Fe2o3Slice1ErrorV1* error) {
  FE2O3_ENTRY("fe2o3_lds_gemm_slice1_join_v1");
  if (!out) return FE2O3_ERR_NULL;
  *out = nullptr;
  // The leases are released exactly once, also when the join is refused.
  auto refuse = [&](int32_t status) {
    if (release) release(user);
    return status;
  };
  // prepare_regions (generated_lds_gemm.rs:559-670): each region checked in
  // role order, then the output against both inputs.
  const struct {
    const void* p;
    uint64_t len, element_bytes;
  } region[3] = {{a, a_len, 2}, {b, b_len, 2}, {c, c_len, 4}};
  uint64_t start[3], end[3];
  for (int i = 0; i < 3; ++i) {
    if (region[i].len != kElements)
      return set_error(error, FE2O3_SLICE1_E_HOST_LENGTH, "", i, 0, kElements, region[i].len),
             refuse(FE2O3_ERR_JOIN);
    if (!region[i].p) return set_error(error, FE2O3_SLICE1_E_HOST_NULL, "", i), refuse(FE2O3_ERR_JOIN);
    const uint64_t addr = (uint64_t)(uintptr_t)region[i].p;
    if (addr % region[i].element_bytes != 0)
      return set_error(error, FE2O3_SLICE1_E_HOST_ALIGNMENT, "", i, 0, region[i].element_bytes,
                       addr % region[i].element_bytes),
             refuse(FE2O3_ERR_JOIN);
    const uint64_t bytes = kElements * region[i].element_bytes;
    if (addr > UINT64_MAX - bytes)
      return set_error(error, FE2O3_SLICE1_E_HOST_ADDRESS_OVERFLOW, "", i), refuse(FE2O3_ERR_JOIN);
    start[i] = addr;
    end[i] = addr + bytes;
  }
  for (int i = 0; i < 2; ++i)
    if (start[i] < end[2] && start[2] < end[i])
      return set_error(error, FE2O3_SLICE1_E_HOST_OUTPUT_OVERLAP, "", i), refuse(FE2O3_ERR_JOIN);
  Fe2o3Slice1JoinFactsV1 facts;
  canonical_facts(&facts);
  const int32_t rc = validate_join(facts, error);
  if (rc != FE2O3_OK) return refuse(rc);
  auto* lc = new (std::nothrow) Fe2o3Slice1Lifecycle();
  if (!lc) return refuse((int32_t)hipErrorOutOfMemory);
  lc->device = device;
  lc->release_leases = release;
  lc->user = user;
  for (int i = 0; i < 3; ++i) {
    put_le64(lc->kernarg + 16 * i, start[i]);
    put_le64(lc->kernarg + 16 * i + 8, kElements);
  }
  *out = lc;
  set_error(error, FE2O3_SLICE1_E_NONE);
  return FE2O3_OK;
}

int32_t fe2o3_lds_gemm_slice1_hip_adapter_v1(int32_t device, Fe2o3Slice1AdapterV1* out) {
  if (!out) return FE2O3_ERR_NULL;
  auto* a = new (std::nothrow) HipAdapter{};
  if (!a) return (int32_t)hipErrorOutOfMemory;
  a->device = device;
  std::memset(out, 0, sizeof(*out));
  out->self = a;
  out->context_identity = hip_context_identity;
  out->observe_environment = hip_observe_environment;
  out->load_executable = hip_load_executable;
  out->resolve_kernel = hip_resolve_kernel;
  out->observe_resources = hip_observe_resources;
  out->initialize_implicit_kernarg = hip_initialize_implicit;
  out->launch_and_wait = hip_launch_and_wait;
  out->drop_kernel = hip_drop_kernel;
  out->unload_executable = hip_unload_executable;
  out->drop_adapter = hip_drop_adapter;
  return FE2O3_OK;
}

int32_t fe2o3_lds_gemm_slice1_load_v1(Fe2o3Slice1Lifecycle* lc,
                                      const Fe2o3Slice1AdapterV1* adapter,
                                      Fe2o3Slice1ErrorV1* error) {
  FE2O3_ENTRY("fe2o3_lds_gemm_slice1_load_v1");
  if (!lc || !adapter) return FE2O3_ERR_NULL;
  if (lc->spec != &kSlice1Spec) return state_error(error, lc->state);
  return lifecycle_load(lc, adapter, error);
}

}  // extern "C"

namespace {

// The JOINED -> LOADED transition of any handle (load_after_context_match
// after the context check).
int32_t lifecycle_load(Fe2o3Slice1Lifecycle* lc, const Fe2o3Slice1AdapterV1* adapter,
                       Fe2o3Slice1ErrorV1* error) {
  if (lc->state != FE2O3_SLICE1_JOINED) return state_error(error, lc->state);
  lc->adapter = *adapter;
  lc->has_adapter = true;
  uint8_t identity[16] = {}, expected[16];
  context_identity_for(lc->device, expected);
  const int32_t rc = adapter->context_identity ? adapter->context_identity(adapter->self, identity) : -1;
  if (rc != 0 || !eq16(identity, expected))
    return load_error(lc, error, FE2O3_SLICE1_E_CONTEXT_IDENTITY, "", rc);
  return do_load(lc, error);
}

void lifecycle_release(Fe2o3Slice1Lifecycle* lc) {
  drop_kernel(lc);
  if (lc->has_executable) terminal_unload(lc);
  release_leases(lc);
  drop_adapter(lc);
  delete lc;
}

void lifecycle_observe(const Fe2o3Slice1Lifecycle* lc, Fe2o3Slice1ObservationV1* out) {
  std::memset(out, 0, sizeof(*out));
  out->state = lc->state;
  out->leases_retained = lc->leases;
  out->holds_executable = lc->has_executable;
  out->holds_kernel = lc->has_kernel;
  out->environment = lc->environment;
  out->load = lc->load;
  out->resolution = lc->resolution;
  out->resources = lc->resources;
  std::memcpy(out->dispatch_identity, lc->dispatch_identity, 16);
  out->last_error = lc->last_error;
}

}  // namespace

extern "C" {

int32_t fe2o3_lds_gemm_slice1_dispatch_and_wait_v1(Fe2o3Slice1Lifecycle* lc,
                                                   Fe2o3Slice1ErrorV1* error) {
  FE2O3_ENTRY("fe2o3_lds_gemm_slice1_dispatch_and_wait_v1");
  if (!lc) return FE2O3_ERR_NULL;
  if (lc->spec != &kSlice1Spec || lc->state != FE2O3_SLICE1_LOADED)
    return state_error(error, lc->state);
  return do_dispatch(lc, error);
}

int32_t fe2o3_lds_gemm_slice1_unload_v1(Fe2o3Slice1Lifecycle* lc, Fe2o3Slice1ReceiptV1* receipt) {
  if (!lc || !receipt) return FE2O3_ERR_NULL;
  if (lc->spec != &kSlice1Spec || lc->state != FE2O3_SLICE1_COMPLETED) return FE2O3_ERR_STATE;
  const Fe2o3Slice1UnloadV1 u = terminal_unload(lc);
  const Artifact& a = artifact();
  std::memset(receipt, 0, sizeof(*receipt));
  std::memcpy(receipt->finalizer_identity, a.view.finalizer_identity, 32);
  std::memcpy(receipt->import_identity, a.view.import_identity, 32);
  std::memcpy(receipt->profile_identity, a.view.profile_identity, 32);
  std::memcpy(receipt->executable_object, lc->load.executable_object, 16);
  std::memcpy(receipt->kernel_object, lc->resolution.kernel_object, 16);
  std::memcpy(receipt->dispatch_identity, lc->dispatch_identity, 16);
  unload_identity(lc->spec->unload_domain, u, lc->environment.runtime_instance,
                  lc->environment.agent_handle, receipt->unload_identity);
  drop_adapter(lc);
  delete lc;
  return FE2O3_OK;
}

void fe2o3_lds_gemm_slice1_release_v1(Fe2o3Slice1Lifecycle* lc) {
  if (!lc) return;
  lifecycle_release(lc);
}

int32_t fe2o3_lds_gemm_slice1_observe_v1(const Fe2o3Slice1Lifecycle* lc,
                                         Fe2o3Slice1ObservationV1* out) {
  if (!lc || !out) return FE2O3_ERR_NULL;
  lifecycle_observe(lc, out);
  return FE2O3_OK;
}

// ---- protected profiles -----------------------------------------------------------------

int32_t fe2o3_protected_profile_v1(uint32_t profile, Fe2o3ProtectedProfileV1* out) {
  if (!out) return FE2O3_ERR_NULL;
  const ProtectedDef* d = protected_def(profile);
  if (!d) return FE2O3_ERR_SHAPE;
  *out = profile_view(*d);
  return FE2O3_OK;
}

int32_t fe2o3_protected_artifact_v1(uint32_t profile, Fe2o3ProtectedArtifactV1* out) {
  if (!out) return FE2O3_ERR_NULL;
  const ProtectedDef* d = protected_def(profile);
  if (!d) return FE2O3_ERR_SHAPE;
  *out = protected_artifact(*d).view;
  return FE2O3_OK;
}

int32_t fe2o3_protected_join_facts_v1(uint32_t profile, Fe2o3ProtectedJoinFactsV1* out) {
  if (!out) return FE2O3_ERR_NULL;
  const ProtectedDef* d = protected_def(profile);
  if (!d) return FE2O3_ERR_SHAPE;
  protected_canonical_facts(*d, out);
  return FE2O3_OK;
}

int32_t fe2o3_protected_validate_join_v1(const Fe2o3ProtectedJoinFactsV1* facts,
                                         Fe2o3Slice1ErrorV1* error) {
  if (!facts) return FE2O3_ERR_NULL;
  const ProtectedDef* d = protected_def(facts->profile);
  if (!d) return FE2O3_ERR_SHAPE;
  return protected_validate_join(*d, *facts, error);
}

int32_t fe2o3_protected_join_v1(uint32_t profile, const Fe2o3ProtectedRegionV1* regions,
                                uint32_t count, int32_t device, void (*release)(void*),
                                void* user, Fe2o3ProtectedLifecycleV1** out,
                                Fe2o3Slice1ErrorV1* error) {
  FE2O3_ENTRY("fe2o3_protected_join_v1");
  if (!out) return FE2O3_ERR_NULL;
  *out = nullptr;
  auto refuse = [&](int32_t status) {
    if (release) release(user);
    return status;
  };
  const ProtectedDef* d = protected_def(profile);
  if (!d) return set_error(error, FE2O3_SLICE1_E_HOST_FIELD, "profile"), refuse(FE2O3_ERR_JOIN);
  if (!regions || count != d->regions)
    return set_error(error, FE2O3_SLICE1_E_HOST_LENGTH, "regions", -1, 0, d->regions, count),
           refuse(FE2O3_ERR_JOIN);
  // prepare_regions: each region in role order, then the pairs
  uint64_t start[kMaxRegions], end[kMaxRegions];
  for (uint32_t i = 0; i < count; ++i) {
    const uint64_t eb = d->element_bytes[i];
    if (regions[i].elements != d->elements[i])
      return set_error(error, FE2O3_SLICE1_E_HOST_LENGTH, "", (int32_t)i, 0, d->elements[i],
                       regions[i].elements),
             refuse(FE2O3_ERR_JOIN);
    if (!regions[i].address)
      return set_error(error, FE2O3_SLICE1_E_HOST_NULL, "", (int32_t)i), refuse(FE2O3_ERR_JOIN);
    const uint64_t addr = (uint64_t)(uintptr_t)regions[i].address;
    if (addr % eb != 0)
      return set_error(error, FE2O3_SLICE1_E_HOST_ALIGNMENT, "", (int32_t)i, 0, eb, addr % eb),
             refuse(FE2O3_ERR_JOIN);
    const uint64_t bytes = d->elements[i] * eb;
    if (addr > UINT64_MAX - bytes)
      return set_error(error, FE2O3_SLICE1_E_HOST_ADDRESS_OVERFLOW, "", (int32_t)i),
             refuse(FE2O3_ERR_JOIN);
    start[i] = addr;
    end[i] = addr + bytes;
  }
  // a written region overlaps no other; read-only inputs may alias
  for (uint32_t l = 0; l < count; ++l)
    for (uint32_t r = l + 1; r < count; ++r)
      if ((d->writes[l] || d->writes[r]) && start[l] < end[r] && start[r] < end[l])
        return set_error(error, FE2O3_SLICE1_E_HOST_OUTPUT_OVERLAP, "", (int32_t)l, 0, 0, r),
               refuse(FE2O3_ERR_JOIN);
  Fe2o3ProtectedJoinFactsV1 facts;
  protected_canonical_facts(*d, &facts);
  const int32_t rc = protected_validate_join(*d, facts, error);
  if (rc != FE2O3_OK) return refuse(rc);
  auto* lc = new (std::nothrow) Fe2o3Slice1Lifecycle();
  if (!lc) return refuse((int32_t)hipErrorOutOfMemory);
  lc->spec = &d->spec;
  lc->device = device;
  lc->release_leases = release;
  lc->user = user;
  for (uint32_t i = 0; i < count; ++i) {
    put_le64(lc->kernarg + 16 * i, start[i]);
    put_le64(lc->kernarg + 16 * i + 8, d->elements[i]);
  }
  *out = lc;
  set_error(error, FE2O3_SLICE1_E_NONE);
  return FE2O3_OK;
}

int32_t fe2o3_protected_load_v1(Fe2o3ProtectedLifecycleV1* lc,
                                const Fe2o3Slice1AdapterV1* adapter, Fe2o3Slice1ErrorV1* error) {
  FE2O3_ENTRY("fe2o3_protected_load_v1");
  if (!lc || !adapter) return FE2O3_ERR_NULL;
  if (lc->spec == &kSlice1Spec) return state_error(error, lc->state);
  return lifecycle_load(lc, adapter, error);
}

int32_t fe2o3_protected_dispatch_and_wait_v1(Fe2o3ProtectedLifecycleV1* lc,
                                             Fe2o3Slice1ErrorV1* error) {
  FE2O3_ENTRY("fe2o3_protected_dispatch_and_wait_v1");
  if (!lc) return FE2O3_ERR_NULL;
  if (lc->spec == &kSlice1Spec || lc->state != FE2O3_SLICE1_LOADED)
    return state_error(error, lc->state);
  return do_dispatch(lc, error);
}

int32_t fe2o3_protected_unload_v1(Fe2o3ProtectedLifecycleV1* lc, Fe2o3ProtectedReceiptV1* receipt) {
  if (!lc || !receipt) return FE2O3_ERR_NULL;
  if (lc->spec == &kSlice1Spec || lc->state != FE2O3_SLICE1_COMPLETED) return FE2O3_ERR_STATE;
  const Fe2o3Slice1UnloadV1 u = terminal_unload(lc);
  const ProtectedDef* d = protected_def(lc->spec->profile);
  const ProtectedArtifact& a = protected_artifact(*d);
  std::memset(receipt, 0, sizeof(*receipt));
  std::memcpy(receipt->identity, a.view.identity, 32);
  std::memcpy(receipt->artifact_identity, a.view.artifact_identity, 32);
  std::memcpy(receipt->executable_object, lc->load.executable_object, 16);
  std::memcpy(receipt->kernel_object, lc->resolution.kernel_object, 16);
  std::memcpy(receipt->dispatch_identity, lc->dispatch_identity, 16);
  unload_identity(lc->spec->unload_domain, u, lc->environment.runtime_instance,
                  lc->environment.agent_handle, receipt->unload_identity);
  drop_adapter(lc);
  delete lc;
  return FE2O3_OK;
}

void fe2o3_protected_release_v1(Fe2o3ProtectedLifecycleV1* lc) {
  if (!lc) return;
  lifecycle_release(lc);
}

int32_t fe2o3_protected_observe_v1(const Fe2o3ProtectedLifecycleV1* lc,
                                   Fe2o3Slice1ObservationV1* out) {
  if (!lc || !out) return FE2O3_ERR_NULL;
  lifecycle_observe(lc, out);
  return FE2O3_OK;
}

}  // extern "C"
