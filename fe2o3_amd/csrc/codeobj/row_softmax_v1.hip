// row_softmax_v1.hip -- the exact row-softmax profile (one row of 64 f32)
// as a standalone gfx950 code object (code object v6, xnack-), the artifact
// the protected row-softmax lifecycle embeds, loads, dispatches and unloads
// (crates/fe2o3-host/src/protected_row_softmax_v1_lifecycle.rs:20-31 for the
// reference's gfx942 facts).  Built on its own (hipcc --genco).
//
// Kernarg ABI (32 explicit bytes, then the 256-byte implicit suffix, 288 in
// all, 8-byte aligned): two regions {u64 address, u64 elements} -- the input
// (read) and the output (written), 64 f32 each.  Geometry: grid [1,1,1],
// workgroup [64,1,1], no LDS.
//
// The arithmetic is fe2o3_profiles::softmax_row, the routine behind the
// library's row-softmax entry points for rows it does not hold in
// registers.  A region of another length is not touched; a dispatch whose
// implicit arguments do not describe the geometry writes quiet NaN.
#include "../profiles.hpp"

struct Fe2o3Region {
  const void* address;
  uint64_t elements;
};

extern "C" __global__ void __launch_bounds__(64) row_softmax_v1(Fe2o3Region input,
                                                                Fe2o3Region output) {
  if (input.elements != 64u || output.elements != 64u) return;
  float* y = static_cast<float*>(const_cast<void*>(output.address));
  const uint8_t* implicit = static_cast<const uint8_t*>(__builtin_amdgcn_implicitarg_ptr());
  const uint32_t block_count_x = *reinterpret_cast<const uint32_t*>(implicit + 0);
  const uint16_t group_size_x = *reinterpret_cast<const uint16_t*>(implicit + 12);
  if (block_count_x != 1u || group_size_x != 64u) {
    y[threadIdx.x] = fe2o3::quiet_nan();
    return;
  }
  fe2o3_profiles::softmax_row(static_cast<const float*>(input.address), y, nullptr, 64, nullptr);
}
