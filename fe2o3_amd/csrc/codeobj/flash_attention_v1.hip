// flash_attention_v1.hip -- the exact flash-attention profile (causal,
// B1/H1/N8/D16, f32) as a standalone gfx950 code object (code object v6,
// xnack-), the artifact the protected flash-attention lifecycle embeds,
// loads, dispatches and unloads (crates/fe2o3-host/src/
// flash_attention_v1_lifecycle.rs:21-31 for the reference's gfx942 facts).
// Built on its own (hipcc --genco), not linked into the library.
//
// Kernarg ABI (64 explicit bytes, then the 256-byte implicit suffix, 320 in
// all, 8-byte aligned): four regions {u64 address, u64 elements} -- Q, K, V
// (read) and the output (written), 128 f32 each.  Geometry: grid [1,1,1],
// workgroup [64,1,1], no LDS.
//
// The arithmetic is fe2o3_profiles::flash_profile, the routine behind the
// library's fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1.  A region of
// another length is not touched; a dispatch whose implicit arguments do not
// describe the geometry writes quiet NaN to the whole output.
#include "../profiles.hpp"

struct Fe2o3Region {
  const void* address;
  uint64_t elements;
};

extern "C" __global__ void __launch_bounds__(64)
    flash_attention_causal_f32_b1_h1_n8_d16_v1(Fe2o3Region q, Fe2o3Region k, Fe2o3Region v,
                                               Fe2o3Region out) {
  constexpr uint64_t n = fe2o3_profiles::kFlashN * fe2o3_profiles::kFlashD;
  if (q.elements != n || k.elements != n || v.elements != n || out.elements != n) return;
  float* o = static_cast<float*>(const_cast<void*>(out.address));
  const uint8_t* implicit = static_cast<const uint8_t*>(__builtin_amdgcn_implicitarg_ptr());
  const uint32_t block_count_x = *reinterpret_cast<const uint32_t*>(implicit + 0);
  const uint16_t group_size_x = *reinterpret_cast<const uint16_t*>(implicit + 12);
  if (block_count_x != 1u || group_size_x != 64u) {
    o[2 * threadIdx.x] = fe2o3::quiet_nan();
    o[2 * threadIdx.x + 1] = fe2o3::quiet_nan();
    return;
  }
  fe2o3_profiles::flash_profile(static_cast<const float*>(q.address),
                                static_cast<const float*>(k.address),
                                static_cast<const float*>(v.address), o, nullptr);
}
