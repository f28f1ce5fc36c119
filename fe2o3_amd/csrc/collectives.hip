// collectives.hip -- the reference's wave64 collectives and workgroup
// synchronization profiles as C-ABI entry points, plus a batched form of the
// wave64 collectives for measurement at scale.
//
//   fe2o3_wave64_collectives_v1       examples/wave64_collectives_v1/src/kernel.rs:18-67
//   fe2o3_wave64_collectives_rows     the same per 64-element row, one mask per row
//   fe2o3_lds_reduce_i32_v1           examples/workgroup_sync_v1/src/kernel.rs:18-78
//   fe2o3_scoped_atomic_add_u32_v1    examples/workgroup_sync_v1/src/scoped_atomic.rs:11-32
#include "collectives.hpp"
#include "internal.hpp"

namespace {

using namespace fe2o3;

// One wave: an inactive lane contributes +0 and publishes +0 in all three
// outputs; an active lane publishes the full masked reduction and its
// inclusive / exclusive prefixes in physical lane order.
FE2O3_DEVICE void collectives64(float x, bool active, float* red, float* inc, float* exc) {
  const float c = active ? x : 0.0f;
  const float r = wave_reduce_sum_xor(c);
  const float i = wave_inclusive_scan_sum(c);
  const float e = wave_exclusive_from_inclusive(i);
  *red = active ? r : 0.0f;
  *inc = active ? i : 0.0f;
  *exc = active ? e : 0.0f;
}

__global__ void __launch_bounds__(64) wave64_collectives_kernel(const float* __restrict__ input,
                                                               uint64_t mask,
                                                               float* __restrict__ reduction,
                                                               float* __restrict__ inclusive,
                                                               float* __restrict__ exclusive) {
  const uint32_t lane = threadIdx.x;
  float r, i, e;
  collectives64(input[lane], (mask >> lane) & 1u, &r, &i, &e);
  reduction[lane] = r;
  inclusive[lane] = i;
  exclusive[lane] = e;
}

// Rows of 64: each wave takes groups of ROWS_IN_FLIGHT consecutive rows in a
// grid-stride loop and issues all of a group's loads before any exchange,
// so each wave keeps that many 256-byte row reads in flight (coalesced row
// reads and writes); row r uses masks[r].
constexpr uint32_t ROWS_IN_FLIGHT = 4;

__global__ void __launch_bounds__(256) wave64_collectives_rows_kernel(
    const float* __restrict__ input, const uint64_t* __restrict__ masks, uint64_t rows,
    float* __restrict__ reduction, float* __restrict__ inclusive, float* __restrict__ exclusive) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t waves = (uint64_t)gridDim.x * (blockDim.x / 64u);
  for (uint64_t r0 = ((uint64_t)blockIdx.x * (blockDim.x / 64u) + (threadIdx.x >> 6)) *
                     ROWS_IN_FLIGHT;
       r0 < rows; r0 += waves * ROWS_IN_FLIGHT) {
    float x[ROWS_IN_FLIGHT];
    uint64_t m[ROWS_IN_FLIGHT];
#pragma unroll
    for (uint32_t j = 0; j < ROWS_IN_FLIGHT; ++j) {
      const uint64_t row = r0 + j < rows ? r0 + j : rows - 1;  // clamped reads of a tail group
      x[j] = __builtin_nontemporal_load(input + row * 64u + lane);
      m[j] = masks[row];
    }
#pragma unroll
    for (uint32_t j = 0; j < ROWS_IN_FLIGHT; ++j) {
      if (r0 + j >= rows) break;
      const uint64_t at = (r0 + j) * 64u + lane;
      float r, i, e;
      collectives64(x[j], (m[j] >> lane) & 1u, &r, &i, &e);
      __builtin_nontemporal_store(r, reduction + at);
      __builtin_nontemporal_store(i, inclusive + at);
      __builtin_nontemporal_store(e, exclusive + at);
    }
  }
}

__global__ void __launch_bounds__(64) lds_reduce_i32_kernel(const int32_t* __restrict__ values,
                                                           int32_t* __restrict__ output) {
  __shared__ uint32_t scratch[64];
  const int32_t sum = block_reduce_sum_i32(values[threadIdx.x], scratch, 64u);
  if (threadIdx.x == 0) output[0] = sum;
}

// Relaxed, system-scope atomic add of each eligible lane's value (a vector
// memory atomic: every lane's operand differs).
__global__ void __launch_bounds__(64) scoped_atomic_add_kernel(const uint32_t* __restrict__ values,
                                                              const uint32_t* __restrict__ eligible,
                                                              uint32_t* target) {
  const uint32_t lane = threadIdx.x;
  if (eligible[lane] != 0u)
    __hip_atomic_fetch_add(target, values[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_wave64_collectives_v1", "wave64_collectives_kernel", (const void*)wave64_collectives_kernel, 64, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_wave64_collectives_rows", "wave64_collectives_rows_kernel", (const void*)wave64_collectives_rows_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_lds_reduce_i32_v1", "lds_reduce_i32_kernel", (const void*)lds_reduce_i32_kernel, 64, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_scoped_atomic_add_u32_v1", "scoped_atomic_add_kernel", (const void*)scoped_atomic_add_kernel, 64, 0})};

}  // namespace

extern "C" {

int32_t fe2o3_wave64_collectives_v1(const float* input, uint64_t input_len, uint64_t active_mask,
                                    float* reduction, uint64_t reduction_len, float* inclusive,
                                    uint64_t inclusive_len, float* exclusive,
                                    uint64_t exclusive_len, void* stream) {
  FE2O3_ENTRY("fe2o3_wave64_collectives_v1");
  if (input_len != 64 || reduction_len != 64 || inclusive_len != 64 || exclusive_len != 64)
    return FE2O3_ERR_LENGTH;
  if (!input || !reduction || !inclusive || !exclusive) return FE2O3_ERR_NULL;
  wave64_collectives_kernel<<<1, 64, 0, (hipStream_t)stream>>>(input, active_mask, reduction,
                                                               inclusive, exclusive);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_wave64_collectives_rows(const float* input, uint64_t input_len,
                                      const uint64_t* masks, uint64_t masks_len, float* reduction,
                                      uint64_t reduction_len, float* inclusive,
                                      uint64_t inclusive_len, float* exclusive,
                                      uint64_t exclusive_len, uint64_t rows, void* stream) {
  FE2O3_ENTRY("fe2o3_wave64_collectives_rows");
  if (rows > (UINT64_MAX / 64u)) return FE2O3_ERR_OVERFLOW;
  const uint64_t n = rows * 64u;
  if (input_len != n || masks_len != rows || reduction_len != n || inclusive_len != n ||
      exclusive_len != n)
    return FE2O3_ERR_LENGTH;
  if (rows == 0) return FE2O3_OK;
  if (!input || !masks || !reduction || !inclusive || !exclusive) return FE2O3_ERR_NULL;
  // 4 waves per workgroup, ROWS_IN_FLIGHT rows per wave and step; at most
  // 2048 workgroups (8 per CU), the rest by grid stride
  uint64_t blocks = (rows + 4u * ROWS_IN_FLIGHT - 1u) / (4u * ROWS_IN_FLIGHT);
  if (blocks > 2048u) blocks = 2048u;
  wave64_collectives_rows_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(
      input, masks, rows, reduction, inclusive, exclusive);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_lds_reduce_i32_v1(const int32_t* values, uint64_t values_len, int32_t* output,
                                uint64_t output_len, void* stream) {
  FE2O3_ENTRY("fe2o3_lds_reduce_i32_v1");
  if (values_len != 64 || output_len != 1) return FE2O3_ERR_LENGTH;
  if (!values || !output) return FE2O3_ERR_NULL;
  lds_reduce_i32_kernel<<<1, 64, 0, (hipStream_t)stream>>>(values, output);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_scoped_atomic_add_u32_v1(const uint32_t* values, uint64_t values_len,
                                       const uint32_t* eligible, uint64_t eligible_len,
                                       uint32_t* target, void* stream) {
  FE2O3_ENTRY("fe2o3_scoped_atomic_add_u32_v1");
  if (values_len != 64 || eligible_len != 64) return FE2O3_ERR_LENGTH;
  if (!values || !eligible || !target) return FE2O3_ERR_NULL;
  if (((uintptr_t)target & 3u) != 0) return FE2O3_ERR_ALIGNMENT;
  scoped_atomic_add_kernel<<<1, 64, 0, (hipStream_t)stream>>>(values, eligible, target);
  return fe2o3_host::after_launch();
}

}  // extern "C"
