// collectives.hpp -- wave64 and workgroup collectives for gfx950.
//
// The round structure is fixed, so results are bit-reproducible for any
// finite input, not only for the exact integral corpus of the reference:
//   * reduction: six XOR butterfly rounds, round d adds the value of lane
//     l ^ d (d = 1, 2, 4, 8, 16, 32) -- every lane ends with the same value;
//   * inclusive scan: six Hillis-Steele rounds, round d adds the value of
//     lane l - d to lanes l >= d;
//   * exclusive scan: the inclusive value of lane l - 1, +0 in lane 0.
// These are the orders of examples/wave64_collectives_v1/src/oracle.rs:150-
// 172.  IEEE addition is commutative, so which operand sits on the left does
// not change a bit.  The exchanges use __shfl_xor / __shfl_up, which hipcc
// lowers to DPP, ds_swizzle or ds_bpermute by offset.
#pragma once

#include "common.hpp"

namespace fe2o3 {

FE2O3_DEVICE float wave_reduce_sum_xor(float v) { return wave_sum(v); }

FE2O3_DEVICE float wave_inclusive_scan_sum(float v) {
  const int lane = (int)(threadIdx.x & 63u);
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float t = __shfl_up(v, (unsigned)d, 64);
    if (lane >= d) v = v + t;
  }
  return v;
}

FE2O3_DEVICE float wave_exclusive_from_inclusive(float inclusive) {
  const float t = __shfl_up(inclusive, 1u, 64);
  return (threadIdx.x & 63u) == 0u ? 0.0f : t;
}

// Sum of one int32 per thread of a workgroup of `threads` (a multiple of 64,
// at most 1024) through LDS: every thread publishes its value to its own
// slot, a barrier, then a halving tree with a barrier per level; all threads
// return the total.  Addition wraps (two's complement), so the result is the
// exact sum whenever that sum fits in int32.  `lds` holds `threads` words;
// a final barrier leaves it free for reuse.
FE2O3_DEVICE int32_t block_reduce_sum_i32(int32_t v, uint32_t* lds, uint32_t threads) {
  const uint32_t t = threadIdx.x;
  lds[t] = (uint32_t)v;
  __syncthreads();
  for (uint32_t stride = threads / 2u; stride > 0u; stride >>= 1) {
    if (t < stride) lds[t] = lds[t] + lds[t + stride];
    __syncthreads();
  }
  const int32_t total = (int32_t)lds[0];
  __syncthreads();
  return total;
}

}  // namespace fe2o3
