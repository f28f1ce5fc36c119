// CPU check of the MoE expert-GEMM work list (fe2o3_amd/csrc/moe_tiles.hpp,
// the functions the gate/up and down kernels run on the device).
// Test infrastructure: built and run by tests/test_moe_tiles.py.
//  1. Arbitrary offsets (random words, values beyond the routes, decreasing
//     runs): every workgroup of the launch grid gets a tile inside the
//     workspace rows [0, routes), of 1..288 rows, of an expert in range and
//     an n-block in range.
//  2. Consistent offsets (non-decreasing, total <= routes): over the grid,
//     every tile of the list is run exactly once.
//  3. The lane-parallel form the kernels run (expert_tile_lanes) gives every
//     workgroup the same tile as the serial form.
//  4. Consistent offsets: for every (expert, n-block) the tiles cover the
//     expert's rows exactly once, in ceil(n / 288) tiles whose row counts
//     differ by less than 64, each above 96 rows when there are two or more
//     (no short remainder tile).
// Every case runs for XCD counts 8 (MI355X), 1, 2, 3, 4 and 6: the list's
// split over the XCDs must stay a bijection whatever the device reports.
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <map>
#include <set>
#include <tuple>
#include <vector>

#include "../fe2o3_amd/csrc/moe_tiles.hpp"

static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd() {
  state ^= state << 13;
  state ^= state >> 7;
  state ^= state << 17;
  return (uint32_t)(state >> 11);
}

int main() {
  long long failures = 0, tiles_checked = 0;
  for (int iter = 0; iter < 3000; ++iter) {
    const uint32_t experts = 1 + rnd() % 64;
    const uint32_t routes = 2 * (rnd() % 5000);
    const uint32_t n_blocks = 1 + rnd() % 40;
    std::vector<uint32_t> off(experts + 1);
    const int mode = iter % 4;
    if (mode == 0) {
      for (auto& o : off) o = rnd() * 2654435761u;  // arbitrary words
    } else if (mode == 1) {
      for (auto& o : off) o = rnd() % (routes + 600 + 1);  // unordered, partly beyond routes
    } else {
      // consistent: non-decreasing from 0, total <= routes (mode 3: total == routes)
      std::vector<uint32_t> cnt(experts, 0);
      const uint32_t total = mode == 3 ? routes : (routes ? rnd() % (routes + 1) : 0);
      for (uint32_t i = 0; i < total; ++i) cnt[rnd() % experts] += 1;
      off[0] = 0;
      for (uint32_t e = 0; e < experts; ++e) off[e + 1] = off[e] + cnt[e];
    }
    const uint32_t b = rnd() % experts;
    const uint32_t e_end = b + 1 + rnd() % (experts - b);
    // the device's XCD count: 8 on MI355X, fewer on partitioned parts
    static const uint32_t kXcds[] = {8, 1, 2, 4, 3, 6};
    const uint32_t xcds = kXcds[iter % 6];
    const uint64_t grid = fe2o3::expert_grid(routes, e_end - b, n_blocks, xcds);
    if (grid % xcds != 0) {
      if (failures < 10) printf("grid %llu not a multiple of %u\n", (unsigned long long)grid, xcds);
      ++failures;
    }
    std::set<std::tuple<uint32_t, uint32_t, uint32_t>> seen;
    std::map<std::pair<uint32_t, uint32_t>, std::vector<std::pair<uint32_t, uint32_t>>> spans;
    bool dup = false;
    for (uint64_t blk = 0; blk < grid; ++blk) {
      uint32_t e, row0, rows, nb;
      if (!fe2o3::expert_tile_at(off.data(), b, e_end, routes, n_blocks, (uint32_t)blk, xcds, &e,
                                 &row0, &rows, &nb)) {
        uint32_t e2, r2, n2, b2;
        if (fe2o3::expert_tile_lanes(off.data(), b, e_end, routes, n_blocks, (uint32_t)blk, xcds,
                                     &e2, &r2, &n2, &b2)) {
          if (failures < 10) printf("lanes form has an extra tile: iter %d\n", iter);
          ++failures;
        }
        continue;
      }
      ++tiles_checked;
      uint32_t e2, r2, n2, b2;
      const bool hit2 = fe2o3::expert_tile_lanes(off.data(), b, e_end, routes, n_blocks,
                                                 (uint32_t)blk, xcds, &e2, &r2, &n2, &b2);
      if (!hit2 || e2 != e || r2 != row0 || n2 != rows || b2 != nb) {
        if (failures < 10) printf("lanes form differs: iter %d block %llu\n", iter,
                                  (unsigned long long)blk);
        ++failures;
      }
      if (e < b || e >= e_end || nb >= n_blocks || rows == 0 || rows > 288 ||
          (uint64_t)row0 + rows > routes) {
        if (failures < 10)
          printf("bounds: iter %d block %llu e %u row0 %u rows %u nb %u routes %u\n", iter,
                 (unsigned long long)blk, e, row0, rows, nb, routes);
        ++failures;
      }
      if (!seen.insert(std::make_tuple(e, row0, nb)).second) dup = true;
      spans[{e, nb}].push_back({row0, rows});
    }
    if (mode >= 2) {
      uint64_t want = 0;
      for (uint32_t e = b; e < e_end; ++e) want += (off[e + 1] - off[e] + 287u) / 288u * n_blocks;
      if (dup || seen.size() != want) {
        if (failures < 10)
          printf("coverage: iter %d got %zu tiles want %llu dup %d\n", iter, seen.size(),
                 (unsigned long long)want, (int)dup);
        ++failures;
      }
      for (uint32_t e = b; e < e_end; ++e) {
        const uint32_t n = off[e + 1] - off[e], m_tiles = (n + 287u) / 288u;
        for (uint32_t nb = 0; nb < n_blocks && n > 0; ++nb) {
          auto it = spans.find({e, nb});
          bool ok = it != spans.end() && it->second.size() == m_tiles;
          if (ok) {
            auto v = it->second;
            std::sort(v.begin(), v.end());
            uint32_t at = off[e], lo_rows = 288, hi_rows = 0;
            for (auto& t : v) {
              ok = ok && t.first == at;
              at += t.second;
              lo_rows = std::min(lo_rows, t.second);
              hi_rows = std::max(hi_rows, t.second);
            }
            ok = ok && at == off[e + 1] && hi_rows - lo_rows < 64 &&
                 (m_tiles < 2 || lo_rows > 96);
          }
          if (!ok) {
            if (failures < 10) printf("rows: iter %d expert %u n-block %u n %u\n", iter, e, nb, n);
            ++failures;
          }
        }
      }
    }
  }
  printf("tiles %lld failures %lld\n", tiles_checked, failures);
  return failures == 0 ? 0 : 1;
}
