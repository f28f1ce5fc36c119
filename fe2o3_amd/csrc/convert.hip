// convert.hip -- Bf16::from_f32 (crates/fe2o3-device/src/half.rs:182-190)
// over a whole device array: round to nearest, ties to even; a NaN keeps its
// sign and high payload bits and is quieted (bit 0x0040).
//
// Each pair of values is one v_cvt_pk_bf16_f32 (common.hpp pack_bf16x2, the
// same narrowing every GEMM, flash and MoE epilogue of the library uses), so
// this entry point is also how the tests sweep that instruction against the
// reference's rule over all 2^32 binary32 patterns.
//
// With x 16-byte and out 8-byte aligned, a thread converts four 4-element
// units per step (one 16-byte load and one 8-byte store each, every wave
// access contiguous); otherwise, and for the last n % 4 elements, one
// element at a time.  HBM-bound: 6 bytes per element.
#include "common.hpp"
#include "internal.hpp"

namespace {

using namespace fe2o3;

template <bool VEC>
__global__ void __launch_bounds__(256) bf16_from_f32_kernel(const float* __restrict__ x,
                                                            uint64_t n, uint16_t* __restrict__ y) {
  const uint64_t t = threadIdx.x, stride = (uint64_t)gridDim.x * 256u;
  uint64_t done = 0;
  if constexpr (VEC) {
    const uint64_t units = n / 4, steps = units / 1024;  // 1024 units per workgroup step
    const f32x4_t* x4 = reinterpret_cast<const f32x4_t*>(x);
    u32x2_t* y4 = reinterpret_cast<u32x2_t*>(y);
    for (uint64_t s = blockIdx.x; s < steps; s += gridDim.x) {
      f32x4_t v[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) v[w] = __builtin_nontemporal_load(x4 + s * 1024 + 256 * w + t);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        u32x2_t p;
        p[0] = pack_bf16x2(v[w][0], v[w][1]);
        p[1] = pack_bf16x2(v[w][2], v[w][3]);
        __builtin_nontemporal_store(p, y4 + s * 1024 + 256 * w + t);
      }
    }
    for (uint64_t u = steps * 1024 + blockIdx.x * 256u + t; u < units; u += stride) {
      const f32x4_t v = x4[u];
      u32x2_t p;
      p[0] = pack_bf16x2(v[0], v[1]);
      p[1] = pack_bf16x2(v[2], v[3]);
      y4[u] = p;
    }
    done = units * 4;
  }
  for (uint64_t i = done + blockIdx.x * 256u + t; i < n; i += stride) y[i] = bf16_bits_from_f32(x[i]);
}

unsigned convert_grid(uint64_t work) {
  const uint64_t g = (work + 4095) / 4096;
  return (unsigned)(g < 8192 ? (g ? g : 1) : 8192);
}

const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_bf16_from_f32", "bf16_from_f32_kernel", (const void*)bf16_from_f32_kernel<true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_bf16_from_f32", "bf16_from_f32_kernel<unaligned>", (const void*)bf16_from_f32_kernel<false>, 256, 0})};

}  // namespace

extern "C" int32_t fe2o3_bf16_from_f32(const float* x, uint64_t x_len, uint16_t* out,
                                       uint64_t out_len, void* stream) {
  FE2O3_ENTRY("fe2o3_bf16_from_f32");
  if (x_len != out_len) return FE2O3_ERR_LENGTH;
  if (x_len == 0) return FE2O3_OK;
  if (!x || !out) return FE2O3_ERR_NULL;
  const hipStream_t s = (hipStream_t)stream;
  if (((uintptr_t)x & 15u) == 0 && ((uintptr_t)out & 7u) == 0)
    bf16_from_f32_kernel<true><<<convert_grid(x_len), 256, 0, s>>>(x, x_len, out);
  else
    bf16_from_f32_kernel<false><<<convert_grid(x_len * 16), 256, 0, s>>>(x, x_len, out);
  return fe2o3_host::after_launch();
}
