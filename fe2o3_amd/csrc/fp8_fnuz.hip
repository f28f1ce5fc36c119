// fp8_fnuz.hip -- the reference's gfx942 FNUZ fp8 value conversions on
// gfx950: Fp8E4M3Fnuz / Fp8E5M2Fnuz ::from_f32 and ::to_f32
// (crates/fe2o3-device/src/fp8.rs:85-95, 193-203, conversion bodies
// :296-381), applied to whole device arrays.
//
// FNUZ has one unsigned zero (0x00), a sole NaN (0x80) and no infinities.
//   * E4M3 FNUZ: 3 fraction bits, bias 8, finite range +-240, smallest
//     subnormal 2^-10.  E5M2 FNUZ: 2 fraction bits, bias 16, +-57344, 2^-17.
//   * Narrowing rounds to nearest, ties to even; a magnitude above the
//     largest finite value saturates to it (0x7f | sign); NaN and +-inf give
//     0x80; whatever rounds to zero, negative zero included, gives 0x00.
//   * Widening is exact; 0x80 widens to the f32 bits 0xffc00000 (negative
//     quiet NaN), as gfx942's native conversion does.
// gfx950's fp8 conversion instructions implement the OCP encodings (bias 7
// and 15, signed zeros), so these are integer conversions (fp8_fnuz.hpp):
// one shift with a ties-to-even correction per element.
//
// The reference's packed Fp8E4M3Fnuzx4 / Fp8E5M2Fnuzx4 (lane i in bits
// 8i..8i+7) is the little-endian 32-bit view of four consecutive codes of
// these byte arrays.
//
// With the f32 array 16-byte and the code array 4-byte aligned, a thread
// converts four 4-element units per step (16-byte f32 and 4-byte code
// accesses, each wave access contiguous), else one element at a time; the
// bound is HBM (5 bytes per element).
#include "common.hpp"
#include "fp8_fnuz.hpp"
#include "internal.hpp"

namespace {

using namespace fe2o3;

// VEC: x 16-byte and q 4-byte aligned.  A workgroup step covers 4096
// elements: unit u = 256 w + t (w = 0..3, t the thread) is the four elements
// 4u .. 4u+3 -- one 16-byte f32 load and one 4-byte store of codes -- so each
// wave access is 1 KiB (or 256 B of codes) contiguous.  The rest (fewer
// than 4096 elements) runs one unit, then one element, per thread.
template <int FMT>
FE2O3_DEVICE uint32_t fnuz_code4(f32x4_t v) {
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) word |= fnuz_code<FMT>(__float_as_uint(v[e])) << (8 * e);
  return word;
}

template <int FMT>
FE2O3_DEVICE u32x4_t fnuz_bits4(uint32_t word) {
  u32x4_t out;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = fnuz_bits<FMT>((word >> (8 * e)) & 0xffu);
  return out;
}

constexpr uint64_t kStepUnits = 1024;  // 4-element units per workgroup step

template <int FMT, bool VEC>
__global__ void __launch_bounds__(256) fnuz_from_f32_kernel(const float* __restrict__ x,
                                                            uint64_t n, uint8_t* __restrict__ q) {
  const uint64_t t = threadIdx.x;
  uint64_t done = 0;
  if constexpr (VEC) {
    const f32x4_t* x4 = reinterpret_cast<const f32x4_t*>(x);
    uint32_t* q4 = reinterpret_cast<uint32_t*>(q);
    const uint64_t units = n / 4, steps = units / kStepUnits;
    for (uint64_t st = blockIdx.x; st < steps; st += gridDim.x) {
      const uint64_t u0 = st * kStepUnits + t;
      f32x4_t v[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) v[w] = __builtin_nontemporal_load(x4 + u0 + 256 * w);
#pragma unroll
      for (int w = 0; w < 4; ++w) __builtin_nontemporal_store(fnuz_code4<FMT>(v[w]), q4 + u0 + 256 * w);
    }
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t u = steps * kStepUnits + blockIdx.x * blockDim.x + t; u < units; u += stride)
      q4[u] = fnuz_code4<FMT>(x4[u]);
    done = units * 4;
  }
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = done + blockIdx.x * blockDim.x + t; i < n; i += stride)
    q[i] = (uint8_t)fnuz_code<FMT>(__float_as_uint(x[i]));
}

template <int FMT, bool VEC>
__global__ void __launch_bounds__(256) fnuz_to_f32_kernel(const uint8_t* __restrict__ q, uint64_t n,
                                                          float* __restrict__ x) {
  const uint64_t t = threadIdx.x;
  uint64_t done = 0;
  if constexpr (VEC) {
    const uint32_t* q4 = reinterpret_cast<const uint32_t*>(q);
    u32x4_t* x4 = reinterpret_cast<u32x4_t*>(x);
    const uint64_t units = n / 4, steps = units / kStepUnits;
    for (uint64_t st = blockIdx.x; st < steps; st += gridDim.x) {
      const uint64_t u0 = st * kStepUnits + t;
      uint32_t c[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) c[w] = __builtin_nontemporal_load(q4 + u0 + 256 * w);
#pragma unroll
      for (int w = 0; w < 4; ++w) __builtin_nontemporal_store(fnuz_bits4<FMT>(c[w]), x4 + u0 + 256 * w);
    }
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t u = steps * kStepUnits + blockIdx.x * blockDim.x + t; u < units; u += stride)
      x4[u] = fnuz_bits4<FMT>(q4[u]);
    done = units * 4;
  }
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = done + blockIdx.x * blockDim.x + t; i < n; i += stride)
    x[i] = __uint_as_float(fnuz_bits<FMT>(q[i]));
}

// one workgroup per 4096-element step, at most 8192 workgroups striding over
// the rest; at least enough threads for the remainder of fewer than 4096
unsigned fnuz_grid(uint64_t n) {
  uint64_t b = (n + 4095) / 4096;
  if (b == 0) b = 1;
  return (unsigned)(b < 8192 ? b : 8192);
}

template <int FMT>
void launch_from(const float* x, uint64_t n, uint8_t* q, bool vec, hipStream_t s) {
  if (vec)
    fnuz_from_f32_kernel<FMT, true><<<fnuz_grid(n), 256, 0, s>>>(x, n, q);
  else
    fnuz_from_f32_kernel<FMT, false><<<fnuz_grid(n * 16), 256, 0, s>>>(x, n, q);
}

template <int FMT>
void launch_to(const uint8_t* q, uint64_t n, float* x, bool vec, hipStream_t s) {
  if (vec)
    fnuz_to_f32_kernel<FMT, true><<<fnuz_grid(n), 256, 0, s>>>(q, n, x);
  else
    fnuz_to_f32_kernel<FMT, false><<<fnuz_grid(n * 16), 256, 0, s>>>(q, n, x);
}

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_from_f32", "fnuz_from_f32_kernel<e4m3>", (const void*)fnuz_from_f32_kernel<0, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_from_f32", "fnuz_from_f32_kernel<e4m3, unaligned>", (const void*)fnuz_from_f32_kernel<0, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_from_f32", "fnuz_from_f32_kernel<e5m2>", (const void*)fnuz_from_f32_kernel<1, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_from_f32", "fnuz_from_f32_kernel<e5m2, unaligned>", (const void*)fnuz_from_f32_kernel<1, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_to_f32", "fnuz_to_f32_kernel<e4m3>", (const void*)fnuz_to_f32_kernel<0, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_to_f32", "fnuz_to_f32_kernel<e4m3, unaligned>", (const void*)fnuz_to_f32_kernel<0, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_to_f32", "fnuz_to_f32_kernel<e5m2>", (const void*)fnuz_to_f32_kernel<1, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_fnuz_to_f32", "fnuz_to_f32_kernel<e5m2, unaligned>", (const void*)fnuz_to_f32_kernel<1, false>, 256, 0})};

// the 4-element unit path: f32 array 16-byte, code array 4-byte aligned
bool aligned_units(const void* f32s, const void* codes) {
  return ((uintptr_t)f32s & 15u) == 0 && ((uintptr_t)codes & 3u) == 0;
}

}  // namespace

extern "C" {

int32_t fe2o3_fp8_fnuz_from_f32(const float* x, uint64_t x_len, uint8_t* q, uint64_t q_len,
                                int32_t format, void* stream) {
  FE2O3_ENTRY("fe2o3_fp8_fnuz_from_f32");
  if (format != FE2O3_FP8_FNUZ_E4M3 && format != FE2O3_FP8_FNUZ_E5M2) return FE2O3_ERR_SHAPE;
  if (x_len != q_len) return FE2O3_ERR_LENGTH;
  if (x_len == 0) return FE2O3_OK;
  if (!x || !q) return FE2O3_ERR_NULL;
  const hipStream_t s = (hipStream_t)stream;
  if (format == FE2O3_FP8_FNUZ_E4M3)
    launch_from<0>(x, x_len, q, aligned_units(x, q), s);
  else
    launch_from<1>(x, x_len, q, aligned_units(x, q), s);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_fp8_fnuz_to_f32(const uint8_t* q, uint64_t q_len, float* x, uint64_t x_len,
                              int32_t format, void* stream) {
  FE2O3_ENTRY("fe2o3_fp8_fnuz_to_f32");
  if (format != FE2O3_FP8_FNUZ_E4M3 && format != FE2O3_FP8_FNUZ_E5M2) return FE2O3_ERR_SHAPE;
  if (x_len != q_len) return FE2O3_ERR_LENGTH;
  if (q_len == 0) return FE2O3_OK;
  if (!x || !q) return FE2O3_ERR_NULL;
  const hipStream_t s = (hipStream_t)stream;
  if (format == FE2O3_FP8_FNUZ_E4M3)
    launch_to<0>(q, q_len, x, aligned_units(x, q), s);
  else
    launch_to<1>(q, q_len, x, aligned_units(x, q), s);
  return fe2o3_host::after_launch();
}

}  // extern "C"
