// gemm_core.hpp -- workgroup-to-tile order shared by the 256x256 GEMM kernels
// (dense bf16, fp8; the pipelined tile itself is gemm_pipe.hpp).
#pragma once

#include "common.hpp"

namespace gemm_core {

// Maps a linear workgroup id onto (tile_m, tile_n).  Workgroups are issued
// round-robin over the 8 XCDs, so id i runs on XCD i % 8; ids are first
// regrouped so that XCD x receives the contiguous range
// [x*tiles/8, (x+1)*tiles/8), then that range is walked in GROUP_M-row
// groups (Triton-style grouped order) so concurrently running workgroups of
// one XCD share A and B panels in its L2.
FE2O3_DEVICE void xcd_tile_order(uint32_t pid, uint32_t tiles_m, uint32_t tiles_n, uint32_t* tm,
                                 uint32_t* tn) {
  const uint32_t total = tiles_m * tiles_n;
  if (total % 8u == 0u) pid = (pid % 8u) * (total / 8u) + pid / 8u;
  constexpr uint32_t GROUP_M = 4;
  const uint32_t in_group = GROUP_M * tiles_n;
  const uint32_t group = pid / in_group;
  const uint32_t first_m = group * GROUP_M;
  const uint32_t size_m = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const uint32_t r = pid % in_group;
  *tm = first_m + r % size_m;
  *tn = r / size_m;
}

}  // namespace gemm_core
