// moe_top2_v1.hip -- the exact top-2 routing profile (T = 8 tokens, E = 4
// experts, K = 2, capacity 4, f32 logits) as a standalone gfx950 code object
// (code object v6, xnack-), the artifact the protected MoE lifecycle embeds,
// loads, dispatches and unloads (crates/fe2o3-host/src/
// moe_top2_v1_lifecycle.rs:21-32 for the reference's gfx942 facts).  Built
// on its own (hipcc --genco).
//
// Kernarg ABI (128 explicit bytes, then the 256-byte implicit suffix, 384 in
// all, 8-byte aligned): eight regions {u64 address, u64 elements} -- logits
// (read, 32 f32), then top2_experts (16), requested_counts (4),
// admitted_counts (4), expert_offsets (5), route_slots (16), permutation
// (16) and inverse (16), u32, written (examples/moe_top2_v1/src/kernel.rs:
// 102-111).  Geometry: grid [1,1,1], workgroup [64,1,1], no LDS.
//
// The routing is fe2o3_profiles::route_t8_e4 on the wave's lane 0.  A region
// of another length is not touched; a dispatch whose implicit arguments do
// not describe the geometry writes the DROP sentinel to every u32 output.
#include "../profiles.hpp"

struct Fe2o3Region {
  const void* address;
  uint64_t elements;
};

extern "C" __global__ void __launch_bounds__(64) moe_top2_route_f32_t8_e4_k2_c4_v1(
    Fe2o3Region logits, Fe2o3Region top2, Fe2o3Region requested, Fe2o3Region admitted,
    Fe2o3Region offsets, Fe2o3Region slots, Fe2o3Region permutation, Fe2o3Region inverse) {
  using namespace fe2o3_profiles;
  const Fe2o3Region outs[7] = {top2, requested, admitted, offsets, slots, permutation, inverse};
  const uint64_t lens[7] = {kRoutes, kRouteExperts, kRouteExperts, kRouteExperts + 1,
                            kRoutes, kRoutes, kRoutes};
  if (logits.elements != kRouteTokens * kRouteExperts) return;
  for (int i = 0; i < 7; ++i)
    if (outs[i].elements != lens[i]) return;
  auto u32 = [](const Fe2o3Region& r) { return static_cast<uint32_t*>(const_cast<void*>(r.address)); };
  const uint8_t* implicit = static_cast<const uint8_t*>(__builtin_amdgcn_implicitarg_ptr());
  const uint32_t block_count_x = *reinterpret_cast<const uint32_t*>(implicit + 0);
  const uint16_t group_size_x = *reinterpret_cast<const uint16_t*>(implicit + 12);
  if (block_count_x != 1u || group_size_x != 64u) {
    for (int i = 0; i < 7; ++i)
      if (threadIdx.x < lens[i]) u32(outs[i])[threadIdx.x] = kDropRoute;
    return;
  }
  route_t8_e4(static_cast<const float*>(logits.address), u32(top2), u32(requested),
              u32(admitted), u32(offsets), u32(slots), u32(permutation), u32(inverse), nullptr);
}
