// tile_plan.hpp -- how the pipelined GEMMs (dense bf16, fp8, general) spread
// their output tiles over the device: the workgroup-to-tile order and the
// launch plan, both from the device's CU and XCD counts as the runtime
// reports them (fe2o3_host::device_topology), not from MI355X constants.
//
// Plain C++ so the same functions compile for gfx950 and for the host (a CPU
// test checks that every plan covers every output block exactly once for
// many shapes and topologies).
#pragma once

#include <stdint.h>

#ifndef FE2O3_HD
#if defined(__HIPCC__)
#define FE2O3_HD __host__ __device__ __forceinline__
#else
#define FE2O3_HD inline
#endif
#endif

namespace tile_plan {

// The device's compute units and XCDs (accelerator complex dies; each has its
// own L2, and the hardware deals workgroup ids round-robin over them).
// MI355X: 256 and 8.
struct Topology {
  uint32_t cus;
  uint32_t xcds;
};

// Maps a linear workgroup id onto (tile_m, tile_n).  Workgroup id i runs on
// XCD i % xcds; ids are first regrouped so that XCD x receives the contiguous
// range [x * tiles / xcds, (x + 1) * tiles / xcds) of the list (when xcds
// divides the tile count; otherwise the list is taken in id order), then the
// list is walked in GROUP_M-row groups (grouped order) so the concurrently
// running workgroups of one XCD share A and B panels in its L2.  A bijection
// of [0, tiles) for any xcds >= 1.
FE2O3_HD void xcd_tile_order(uint32_t pid, uint32_t tiles_m, uint32_t tiles_n, uint32_t xcds,
                             uint32_t* tm, uint32_t* tn) {
  const uint32_t total = tiles_m * tiles_n;
  if (xcds > 1u && total % xcds == 0u) pid = (pid % xcds) * (total / xcds) + pid / xcds;
  constexpr uint32_t GROUP_M = 4;
  const uint32_t in_group = GROUP_M * tiles_n;
  const uint32_t group = pid / in_group;
  const uint32_t first_m = group * GROUP_M;
  const uint32_t size_m = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const uint32_t r = pid % in_group;
  *tm = first_m + r % size_m;
  *tn = r / size_m;
}

// The tail form of a 256 x 256 grid: workgroup xcds * (4j + q) + x of a
// launch over the tiles first_big .. end of xcd_tile_order's list takes
// quarter q (128 x 128) of list entry first_big + xcds * j + x, so a tile's
// quarters run on the XCD (x) that entry would have run on in one launch
// (first_big is a whole number of rounds of CUs, a multiple of xcds when
// the CU count is).  A bijection onto the quarters whatever the counts.
// False when the entry is past the list or the quarter past an edge tile's
// rows or columns.
FE2O3_HD bool tail_quarter(uint32_t wg, uint32_t first_big, uint32_t m, uint32_t n, uint32_t xcds,
                           uint32_t* tm, uint32_t* tn) {
  const uint32_t x = wg % xcds, q = wg / xcds;
  const uint32_t big = first_big + xcds * (q >> 2) + x;
  const uint32_t big_m = (m + 255u) / 256u, big_n = (n + 255u) / 256u;
  if (big >= big_m * big_n) return false;
  uint32_t btm, btn;
  xcd_tile_order(big, big_m, big_n, xcds, &btm, &btn);
  *tm = 2u * btm + ((q & 3u) >> 1);
  *tn = 2u * btn + (q & 1u);
  return *tm * 128u < m && *tn * 128u < n;
}

// Launch plan of an M x N output on a device of `t.cus` CUs:
//   - at most cus / 2 tiles of 256 x 256 (half the CUs or fewer busy): the
//     whole GEMM on 128 x 128 tiles, with three LDS stages while those fit
//     one per CU, else two (two workgroups per CU);
//   - otherwise 256 x 256 tiles; when there are full rounds of `cus` tiles
//     and a last round of at most cus / 2, that last round runs as a second
//     launch of 128 x 128 quarters on all CUs (three stages when the quarters
//     fit one per CU, else two).
struct Plan {
  bool small;            // one launch of 128 x 128 tiles
  int stages;            // LDS stages of the small launch (2 or 3)
  uint64_t grid;         // workgroups of the first launch
  bool tail;             // a second launch of 128 x 128 quarters
  int tail_stages;       // its LDS stages (2 or 3)
  uint64_t tail_grid;    // its workgroups
  uint32_t first_big;    // the first list entry it covers
};

FE2O3_HD Plan plan(uint32_t m, uint32_t n, Topology t) {
  Plan p{};
  const uint64_t cus = t.cus ? t.cus : 1u, xcds = t.xcds ? t.xcds : 1u;
  const uint64_t small_grid = cus / 2u;
  const uint64_t tiles = (uint64_t)((m + 255ull) / 256u) * ((n + 255ull) / 256u);
  if (tiles <= small_grid) {
    p.small = true;
    p.grid = (uint64_t)((m + 127ull) / 128u) * ((n + 127ull) / 128u);
    p.stages = p.grid > cus ? 2 : 3;
    return p;
  }
  const uint64_t full = tiles / cus * cus, rest = tiles - full;
  p.tail = full > 0 && rest > 0 && rest <= small_grid;
  p.grid = p.tail ? full : tiles;
  if (p.tail) {
    p.tail_grid = (rest + xcds - 1u) / xcds * 4u * xcds;
    p.tail_stages = 4u * rest > cus ? 2 : 3;
    p.first_big = (uint32_t)full;
  }
  return p;
}

}  // namespace tile_plan
