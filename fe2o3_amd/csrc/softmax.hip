// softmax.hip -- stable row softmax for gfx950.
//
// Semantics (examples/row_softmax_v1/src/kernel.rs:13-42 for the arithmetic,
// examples/row_softmax_v1/src/numerical_contract.rs:130-199 for the mask):
//   max over active elements, w_i = exp(x_i - max) in f32 (OCML expf, as the
//   reference's DeviceMath::exp_f32), sum of w, out_i = w_i / sum (correctly
//   rounded f32 division); masked elements -> +0.  A row without an active
//   element is written as all +0.
//   Non-finite input: the reference's contract rejects a row holding a NaN
//   or an infinity anywhere, masked elements included
//   (examples/row_softmax_v1/src/numerical_contract.rs:145-151).  Such a row
//   is written as all quiet NaN (0x7fc00000) and the device's contract-status
//   word is marked, so the host's next synchronize reports
//   FE2O3_ERR_NONFINITE; other rows are unaffected.  The check is one FMA per
//   element folded into the pass that already holds the row.
//
// One wave64 per row.  Rows of 256*NV columns (NV <= 32) live in registers:
// each lane holds NV float4 chunks loaded with coalesced 16-byte accesses
// (lane l, chunk j -> columns 256*j + 4*l), so the row is read from HBM once
// and written once -- the kernel is HBM-bound at 8 bytes per element.
// Other widths take a strided three-pass path (max, sum, write) per lane.
// Reductions are wave-wide butterflies.
#include "common.hpp"
#include "internal.hpp"
#include "profiles.hpp"

namespace {

using namespace fe2o3;

constexpr int ROWS_PER_BLOCK = 4;  // 4 waves, one row each

template <int NV, bool MASK>
__global__ void __launch_bounds__(256) softmax_reg_kernel(const float* __restrict__ in,
                                                          float* __restrict__ out,
                                                          const uint8_t* __restrict__ mask,
                                                          uint64_t rows,
                                                          uint32_t* __restrict__ status) {
  const uint64_t row = (uint64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint32_t lane = threadIdx.x & 63u;
  constexpr uint32_t cols = 256u * NV;
  const f32x4_t* src = reinterpret_cast<const f32x4_t*>(in + row * cols) + lane;
  f32x4_t x[NV];
  uint32_t act[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) x[j] = __builtin_nontemporal_load(src + 64 * j);
  if (MASK) {
    const uint32_t* msrc = reinterpret_cast<const uint32_t*>(mask + row * cols) + lane;
#pragma unroll
    for (int j = 0; j < NV; ++j) act[j] = msrc[64 * j];
  }
  auto active = [&](int j, int e) -> bool {
    return !MASK || ((act[j] >> (8 * e)) & 0xffu) != 0u;
  };
  float mx = -INFINITY;
  f32x4_t probe = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < NV; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      probe[e] = finite_probe(probe[e], x[j][e]);
      if (active(j, e)) mx = fmaxf(mx, x[j][e]);
    }
  }
  mx = wave_max(mx);
  const float pr = (probe[0] + probe[1]) + (probe[2] + probe[3]);
  const bool rejected = __ballot(pr != pr) != 0ull;
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[j][e] = active(j, e) ? expf(x[j][e] - mx) : 0.0f;
    sum += (x[j][0] + x[j][1]) + (x[j][2] + x[j][3]);
  }
  sum = wave_sum(sum);
  const bool any = mx != -INFINITY;
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(out + row * cols) + lane;
  if (rejected) {
    if (lane == 0) mark_nonfinite(status);
    const float nan = quiet_nan();
#pragma unroll
    for (int j = 0; j < NV; ++j) __builtin_nontemporal_store(f32x4_t{nan, nan, nan, nan}, dst + 64 * j);
    return;
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    f32x4_t y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = any ? x[j][e] / sum : 0.0f;
    __builtin_nontemporal_store(y, dst + 64 * j);
  }
}

__global__ void __launch_bounds__(256) softmax_strided_kernel(const float* __restrict__ in,
                                                              float* __restrict__ out,
                                                              const uint8_t* __restrict__ mask,
                                                              uint64_t rows, uint64_t cols,
                                                              uint32_t* __restrict__ status) {
  const uint64_t row = (uint64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (row >= rows) return;
  fe2o3_profiles::softmax_row(in + row * cols, out + row * cols,
                              mask ? mask + row * cols : nullptr, cols, status);
}

template <int NV>
void launch_reg(const float* in, float* out, const uint8_t* mask, uint64_t rows, dim3 grid,
                uint32_t* status, hipStream_t s) {
  if (mask)
    softmax_reg_kernel<NV, true><<<grid, 256, 0, s>>>(in, out, mask, rows, status);
  else
    softmax_reg_kernel<NV, false><<<grid, 256, 0, s>>>(in, out, mask, rows, status);
}

int32_t row_softmax(const float* input, uint64_t input_len, float* output, uint64_t output_len,
                    const uint8_t* mask, uint64_t mask_len, uint64_t rows, uint64_t cols,
                    void* stream) {
  if (cols == 0) return FE2O3_ERR_SHAPE;
  if (rows > UINT64_MAX / cols) return FE2O3_ERR_OVERFLOW;
  const uint64_t n = rows * cols;
  if (input_len != n || output_len != n || (mask && mask_len != n)) return FE2O3_ERR_LENGTH;
  if (n == 0) return FE2O3_OK;
  if (!input || !output) return FE2O3_ERR_NULL;
  const uint64_t blocks = (rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK;
  if (blocks > 0x7fffffffu) return FE2O3_ERR_SHAPE;
  const dim3 grid((unsigned)blocks);
  hipStream_t s = (hipStream_t)stream;
  uint32_t* status = fe2o3_host::status_word();
  if (status == nullptr) return (int32_t)hipErrorInvalidSymbol;
  const bool aligned = ((uintptr_t)input & 15u) == 0 && ((uintptr_t)output & 15u) == 0 &&
                       (!mask || ((uintptr_t)mask & 3u) == 0);
  if (aligned && cols % 256 == 0 && cols <= 256 * 32) {
    switch (cols / 256) {
      case 1: launch_reg<1>(input, output, mask, rows, grid, status, s); break;
      case 2: launch_reg<2>(input, output, mask, rows, grid, status, s); break;
      case 4: launch_reg<4>(input, output, mask, rows, grid, status, s); break;
      case 8: launch_reg<8>(input, output, mask, rows, grid, status, s); break;
      case 16: launch_reg<16>(input, output, mask, rows, grid, status, s); break;
      case 32: launch_reg<32>(input, output, mask, rows, grid, status, s); break;
      default:
        softmax_strided_kernel<<<grid, 256, 0, s>>>(input, output, mask, rows, cols, status);
        break;
    }
  } else {
    softmax_strided_kernel<<<grid, 256, 0, s>>>(input, output, mask, rows, cols, status);
  }
  return fe2o3_host::after_launch();
}

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax_v1", "softmax_strided_kernel", (const void*)softmax_strided_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<1, false>", (const void*)softmax_reg_kernel<1, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<1, true>", (const void*)softmax_reg_kernel<1, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<2, false>", (const void*)softmax_reg_kernel<2, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<2, true>", (const void*)softmax_reg_kernel<2, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<4, false>", (const void*)softmax_reg_kernel<4, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<4, true>", (const void*)softmax_reg_kernel<4, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<8, false>", (const void*)softmax_reg_kernel<8, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<8, true>", (const void*)softmax_reg_kernel<8, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<16, false>", (const void*)softmax_reg_kernel<16, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<16, true>", (const void*)softmax_reg_kernel<16, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<32, false>", (const void*)softmax_reg_kernel<32, false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_reg_kernel<32, true>", (const void*)softmax_reg_kernel<32, true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_row_softmax", "softmax_strided_kernel", (const void*)softmax_strided_kernel, 256, 0})};

}  // namespace

extern "C" {

int32_t fe2o3_row_softmax_v1(const float* input, uint64_t input_len, float* output,
                             uint64_t output_len, void* stream) {
  FE2O3_ENTRY("fe2o3_row_softmax_v1");
  // examples/row_softmax_v1: exactly one 64-element row.
  if (input_len != 64 || output_len != 64) return FE2O3_ERR_LENGTH;
  return row_softmax(input, input_len, output, output_len, nullptr, 0, 1, 64, stream);
}

int32_t fe2o3_row_softmax(const float* input, uint64_t input_len, float* output,
                          uint64_t output_len, const uint8_t* mask, uint64_t mask_len,
                          uint64_t rows, uint64_t cols, void* stream) {
  FE2O3_ENTRY("fe2o3_row_softmax");
  return row_softmax(input, input_len, output, output_len, mask, mask_len, rows, cols, stream);
}

}  // extern "C"
