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

// The tail form of a 256 x 256 grid: workgroup 8(4j + q) + x of a launch
// over the tiles first_big .. end of xcd_tile_order's list takes quarter q
// (128 x 128) of tile first_big + 8j + x, so a tile's quarters run on the
// XCD (x) its neighbours in the list ran on.  False when the tile is past
// the grid or the quarter past an edge tile's rows or columns.
FE2O3_DEVICE bool tail_quarter(uint32_t wg, uint32_t first_big, uint32_t m, uint32_t n,
                               uint32_t* tm, uint32_t* tn) {
  const uint32_t x = wg & 7u, q = wg >> 3;
  const uint32_t big = first_big + 8u * (q >> 2) + x;
  const uint32_t big_m = (m + 255u) / 256u, big_n = (n + 255u) / 256u;
  if (big >= big_m * big_n) return false;
  uint32_t btm, btn;
  xcd_tile_order(big, big_m, big_n, &btm, &btn);
  *tm = 2u * btm + ((q & 3u) >> 1);
  *tn = 2u * btn + (q & 1u);
  return *tm * 128u < m && *tn * 128u < n;
}

// Host: whether a 256x256-tile launch whose operands (A and B together) take
// `operand_bytes` stores C through LDS (gemm_pipe::store_bf16_staged).  C
// written straight from the accumulators lands in the caches in part-lines;
// once the operands alone nearly fill the 256 MiB last-level cache, that C
// evicts operand panels that later tiles re-read, and the staged nontemporal
// store is faster (measured: +9% bf16 8192^3, +15% 1024x28672x4096).  With
// smaller operands the staging only adds ~1 us per tile (-1% to -8% on eight
// shapes from 4096^3 to 8192x8192x1024, bf16 and fp8).
constexpr uint64_t kStagedOperandBytes = 192ull << 20;
inline bool staged_epilogue(uint64_t operand_bytes) {
  return operand_bytes >= kStagedOperandBytes;
}

}  // namespace gemm_core
