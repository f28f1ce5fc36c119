// CPU check of the pipelined GEMMs' launch plan and tile orders
// (fe2o3_amd/csrc/tile_plan.hpp, the functions the dense bf16, fp8 and
// general GEMM entry points and kernels run), for the CU and XCD counts a
// device may report: MI355X (256 CUs, 8 XCDs) and smaller or partitioned
// parts.  Test infrastructure: built with sanitizers and run by
// tests/test_sanitized_host.py.
//   1. Over each plan's launches, every 128 x 128 block of the M x N output
//      is computed exactly once: by the 256 x 256 tile that holds it, by a
//      tail quarter, or by a small-grid tile; no workgroup computes a block
//      outside the output.
//   2. xcd_tile_order is a bijection of [0, tiles) for every XCD count.
//   3. When the XCD count divides the tile count, the workgroups of one XCD
//      take one contiguous piece of the list.
//   4. The plan's shape rules: the small form only when at most half the CUs
//      would have a 256 x 256 tile; a tail only after full rounds and for at
//      most half a round; its quarters run on the XCD of their list entry.
#include <stdint.h>
#include <stdio.h>

#include <vector>

#include "../fe2o3_amd/csrc/tile_plan.hpp"

static long failures = 0, plans = 0;
static void fail(const char* what, uint32_t m, uint32_t n, uint32_t cus, uint32_t xcds) {
  if (failures < 20) printf("FAIL %s: m %u n %u cus %u xcds %u\n", what, m, n, cus, xcds);
  ++failures;
}

static void check(uint32_t m, uint32_t n, tile_plan::Topology t) {
  ++plans;
  const tile_plan::Plan p = tile_plan::plan(m, n, t);
  const uint32_t bm = (m + 127u) / 128u, bn = (n + 127u) / 128u;
  std::vector<uint8_t> hits((size_t)bm * bn, 0);
  const uint32_t tm256 = (m + 255u) / 256u, tn256 = (n + 255u) / 256u;
  const uint64_t tiles = (uint64_t)tm256 * tn256;
  auto hit = [&](uint32_t r, uint32_t c) {
    if (r >= bm || c >= bn) {
      fail("block outside the output", m, n, t.cus, t.xcds);
      return;
    }
    ++hits[(size_t)r * bn + c];
  };
  if (p.small) {
    if (tiles > t.cus / 2) fail("small form with more than half the CUs busy", m, n, t.cus, t.xcds);
    if (p.grid != (uint64_t)bm * bn) fail("small grid size", m, n, t.cus, t.xcds);
    if ((p.stages == 3) != (p.grid <= t.cus)) fail("small stages", m, n, t.cus, t.xcds);
    for (uint64_t wg = 0; wg < p.grid; ++wg) {
      uint32_t tm, tn;
      tile_plan::xcd_tile_order((uint32_t)wg, bm, bn, t.xcds, &tm, &tn);
      hit(tm, tn);
    }
  } else {
    if (tiles <= t.cus / 2) fail("large form with at most half the CUs busy", m, n, t.cus, t.xcds);
    // the 256 x 256 launch: list entries [0, grid)
    for (uint64_t wg = 0; wg < p.grid; ++wg) {
      uint32_t tm, tn;
      tile_plan::xcd_tile_order((uint32_t)wg, tm256, tn256, t.xcds, &tm, &tn);
      for (uint32_t q = 0; q < 4; ++q) {
        const uint32_t r = 2 * tm + q / 2, c = 2 * tn + q % 2;
        if (r < bm && c < bn) hit(r, c);  // an edge tile's missing quarters hold no outputs
      }
    }
    if (p.tail) {
      const uint64_t rest = tiles - p.first_big;
      if (p.first_big % t.cus != 0 || p.first_big == 0 || rest == 0 || rest > t.cus / 2)
        fail("tail shape", m, n, t.cus, t.xcds);
      if (p.grid != p.first_big) fail("tail: first launch covers the full rounds", m, n, t.cus, t.xcds);
      if (p.tail_grid % t.xcds != 0 || p.tail_grid < 4 * rest)
        fail("tail grid", m, n, t.cus, t.xcds);
      if ((p.tail_stages == 3) != (4 * rest <= t.cus)) fail("tail stages", m, n, t.cus, t.xcds);
      for (uint64_t wg = 0; wg < p.tail_grid; ++wg) {
        uint32_t tm, tn;
        if (!tile_plan::tail_quarter((uint32_t)wg, p.first_big, m, n, t.xcds, &tm, &tn)) continue;
        hit(tm, tn);
        // the quarter runs on the XCD its list entry would have run on
        const uint32_t entry = p.first_big + t.xcds * ((uint32_t)(wg / t.xcds) >> 2) +
                               (uint32_t)(wg % t.xcds);
        if (t.cus % t.xcds == 0 && entry % t.xcds != wg % t.xcds)
          fail("tail quarter off its XCD", m, n, t.cus, t.xcds);
      }
    } else if (p.grid != tiles) {
      fail("no tail: one launch over every tile", m, n, t.cus, t.xcds);
    }
  }
  for (size_t i = 0; i < hits.size(); ++i)
    if (hits[i] != 1) {
      fail(hits[i] ? "block computed twice" : "block never computed", m, n, t.cus, t.xcds);
      break;
    }
}

int main() {
  const tile_plan::Topology topos[] = {{256, 8}, {256, 1}, {32, 1}, {64, 2}, {128, 4},
                                       {304, 8}, {80, 8},  {120, 3}, {38, 1}, {1, 1}};
  const uint32_t sizes[] = {1, 100, 127, 128, 129, 255, 256, 257, 511, 512, 1000, 1024,
                            2000, 2048, 3072, 4096, 4100, 6000, 6144, 8192};
  for (const auto& t : topos)
    for (uint32_t m : sizes)
      for (uint32_t n : sizes) check(m, n, t);
  // larger grids: several full rounds with and without a tail
  for (const auto& t : topos)
    for (uint32_t m : {12288u, 14336u, 16384u})
      for (uint32_t n : {4096u, 4608u, 6144u, 14336u}) check(m, n, t);
  // xcd_tile_order: bijection, and contiguous per XCD when xcds divides the count
  for (uint32_t xcds : {1u, 2u, 3u, 4u, 6u, 8u})
    for (uint32_t tmn : {1u, 3u, 7u, 16u, 24u})
      for (uint32_t tnn : {1u, 5u, 8u, 16u, 32u}) {
        const uint32_t total = tmn * tnn;
        std::vector<uint32_t> seen(total, 0);
        for (uint32_t pid = 0; pid < total; ++pid) {
          uint32_t tm, tn;
          tile_plan::xcd_tile_order(pid, tmn, tnn, xcds, &tm, &tn);
          if (tm >= tmn || tn >= tnn) {
            fail("xcd_tile_order out of range", tmn, tnn, 0, xcds);
            continue;
          }
          ++seen[tm * tnn + tn];
        }
        for (uint32_t v : seen)
          if (v != 1) {
            fail("xcd_tile_order not a bijection", tmn, tnn, 0, xcds);
            break;
          }
      }
  printf("plans %ld failures %ld\n", plans, failures);
  return failures == 0 ? 0 : 1;
}
