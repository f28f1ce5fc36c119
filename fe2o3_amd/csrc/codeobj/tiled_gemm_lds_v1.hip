// tiled_gemm_lds_v1.hip -- the exact 16x16x16 LDS GEMM profile as a
// standalone gfx950 code object (code object v6, xnack-), the artifact that
// the typed host lifecycle in lifecycle.hip embeds, loads, dispatches and
// unloads (crates/fe2o3-host/src/generated_lds_gemm_lifecycle.rs:26-45 for the
// reference's gfx942 contract).  It is built on its own (hipcc --genco), not
// linked into the library's fat binary.
//
// Kernarg ABI (48 explicit bytes, then the 256-byte implicit suffix the
// runtime initializes, 304 bytes in all, 8-byte aligned):
//   offset  0: A region {u64 address, u64 elements}   bf16 bits, row-major 16x16
//   offset 16: B region {u64 address, u64 elements}   bf16 bits, row-major 16x16
//   offset 32: C region {u64 address, u64 elements}   f32, row-major 16x16
// Launch geometry: grid [1,1,1], workgroup [64,1,1], no dynamic LDS.  Static
// LDS: two 512-byte tiles (A as [row][k], B transposed as [n][k]), 16-byte
// aligned, 1024 bytes in all.
//
// The arithmetic is the library's slice-1 tile (one v_mfma_f32_16x16x32_bf16
// with the upper K half zero; output lane l holds column l%16, rows
// 4*(l/16)..+3).  Before writing, the kernel reads the implicit suffix's
// block count and workgroup size (code object v5+ hidden arguments at
// implicit offsets 0 and 12): a dispatch whose implicit arguments do not
// describe this geometry writes quiet NaN to all of C instead of a product.
// A region whose element count is not 256 is not touched at all.
#include <hip/hip_runtime.h>
#include <stdint.h>

struct Fe2o3Region {
  const void* address;
  uint64_t elements;
};

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

extern "C" __global__ void __launch_bounds__(64)
    tiled_gemm_lds_v1(Fe2o3Region a_region, Fe2o3Region b_region, Fe2o3Region c_region) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[16 * 16];
  __shared__ __attribute__((aligned(16))) uint16_t bt_lds[16 * 16];
  if (a_region.elements != 256u || b_region.elements != 256u || c_region.elements != 256u) return;
  const uint16_t* a = static_cast<const uint16_t*>(a_region.address);
  const uint16_t* b = static_cast<const uint16_t*>(b_region.address);
  float* c = static_cast<float*>(const_cast<void*>(c_region.address));
  const uint8_t* implicit = static_cast<const uint8_t*>(__builtin_amdgcn_implicitarg_ptr());
  const uint32_t block_count_x = *reinterpret_cast<const uint32_t*>(implicit + 0);
  const uint16_t group_size_x = *reinterpret_cast<const uint16_t*>(implicit + 12);
  const int l = threadIdx.x;
  // Lane l stages elements 4l .. 4l+3 of each operand with 2-byte loads:
  // the contract only guarantees 2-byte alignment of A and B.
  {
    const int kk = l >> 2, n0 = (l & 3) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a_lds[4 * l + j] = a[4 * l + j];
      bt_lds[(n0 + j) * 16 + kk] = b[4 * l + j];
    }
  }
  __syncthreads();
  bf16x8_t af = {}, bf = {};
  if (l < 32) {
    const int rc = l & 15, chunk = l >> 4;
    af = *reinterpret_cast<const bf16x8_t*>(a_lds + rc * 16 + chunk * 8);
    bf = *reinterpret_cast<const bf16x8_t*>(bt_lds + rc * 16 + chunk * 8);
  }
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, acc, 0, 0, 0);
  const bool geometry_ok = block_count_x == 1u && group_size_x == 64u;
  const float qnan = __builtin_bit_cast(float, 0x7fc00000u);
  const int col = l & 15, row0 = (l >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) c[(row0 + i) * 16 + col] = geometry_ok ? acc[i] : qnan;
}
