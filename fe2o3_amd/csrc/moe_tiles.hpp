// moe_tiles.hpp -- the work list of the MoE expert GEMMs.
//
// The tiles of experts [e_begin, e_end) form one list: expert-major, then
// n-block, then the expert's m-tiles, so consecutive entries share a weight
// block and runs of entries share the expert's rows.  An expert of n rows
// has ceil(n / 288) m-tiles (kMaxTileRows), over which its ceil(n / 32)
// 32-row blocks are dealt out evenly (m_tile): 1033 rows are tiles of 288,
// 256, 256 and 233 rows rather than four of 256 and a remainder of 9, and
// every tile runs on an A tile of its own size rounded up to 32 rows.  Workgroup id i
// runs on XCD i % xcds (the device's XCD count, 8 on MI355X); XCD x takes
// the x-th of xcds contiguous pieces of the list in order, so the workgroups
// that share a weight block run at the same time behind one L2.  The grid is sized for the most m-tiles routing can produce;
// entries past the list's end exit at once.
//
// Expert e's rows are offsets[e] .. offsets[e+1] clamped to [0, routes]
// (empty when the offsets decrease): the offsets are device data the host
// cannot validate, and the clamp keeps every tile inside the workspace rows
// [0, routes) for any offsets.
//
// Plain C++ so the same functions compile for gfx950 and for the host (a CPU
// test sweeps arbitrary offsets over every workgroup of the grid).
#pragma once

#include <stdint.h>

#ifndef FE2O3_HD
#if defined(__HIPCC__)
#define FE2O3_HD __host__ __device__ __forceinline__
#else
#define FE2O3_HD inline
#endif
#endif

namespace fe2o3 {

constexpr uint32_t kMaxTileRows = 288;  // rows of the largest expert tile

FE2O3_HD void expert_rows(const uint32_t* offsets, uint32_t e, uint32_t routes, uint32_t* lo,
                          uint32_t* n) {
  const uint32_t a = offsets[e] < routes ? offsets[e] : routes;
  const uint32_t b = offsets[e + 1] < routes ? offsets[e + 1] : routes;
  *lo = a;
  *n = b > a ? b - a : 0u;
}

// m-tiles of an expert of n rows
FE2O3_HD uint32_t expert_m_tiles(uint32_t n) { return (n + kMaxTileRows - 1u) / kMaxTileRows; }

// Rows of m-tile mt (< m_tiles = expert_m_tiles(n)) of an expert whose
// n >= 1 rows start at lo: the first ceil(n/32) % m_tiles tiles take one
// 32-row block more than the others.  Every tile has 1..288 rows (at most
// ceil(ceil(n/32) / m_tiles) <= 9 blocks, and the last starts below n), and
// the tiles cover [lo, lo + n) in order, each row once.
FE2O3_HD void m_tile(uint32_t lo, uint32_t n, uint32_t m_tiles, uint32_t mt, uint32_t* row0,
                     uint32_t* rows) {
  const uint32_t blocks = (n + 31u) / 32u;
  const uint32_t q = blocks / m_tiles, r = blocks % m_tiles;
  const uint32_t off = 32u * (mt * q + (mt < r ? mt : r));
  const uint32_t cap = 32u * (q + (mt < r ? 1u : 0u));
  const uint32_t left = n - off;
  *row0 = lo + off;
  *rows = left < cap ? left : cap;
}

// Entry of workgroup `block` in the list: expert, first row, row count
// (1..288) and n-block; false when the workgroup has no entry.
FE2O3_HD bool expert_tile_at(const uint32_t* offsets, uint32_t e_begin, uint32_t e_end,
                             uint32_t routes, uint32_t n_blocks, uint32_t block, uint32_t xcds,
                             uint32_t* e_out, uint32_t* row0, uint32_t* rows, uint32_t* nb) {
  uint32_t total = 0, lo, n;
  for (uint32_t e = e_begin; e < e_end; ++e) {
    expert_rows(offsets, e, routes, &lo, &n);
    total += expert_m_tiles(n) * n_blocks;
  }
  const uint32_t chunk = (total + xcds - 1u) / xcds;
  const uint32_t slot = block / xcds;
  if (slot >= chunk) return false;
  uint32_t x = (block % xcds) * chunk + slot;
  if (x >= total) return false;
  for (uint32_t e = e_begin; e < e_end; ++e) {
    expert_rows(offsets, e, routes, &lo, &n);
    const uint32_t m_tiles = expert_m_tiles(n);
    if (x < m_tiles * n_blocks) {
      *e_out = e;
      *nb = x / m_tiles;
      m_tile(lo, n, m_tiles, x % m_tiles, row0, rows);
      return true;
    }
    x -= m_tiles * n_blocks;
  }
  return false;
}

// The same lookup in the form the kernels run it, one wave at a time: lane l
// reads expert e_begin + l's bounds (one memory round trip for all experts),
// the lanes' tile counts are prefix-summed, and the entry's expert is the
// number of lanes whose inclusive sum is <= its list index (the sums do not
// decrease).  This host form spells out the 64 lanes as loops; the device
// form (moe.hip) uses a wave scan, a ballot and lane reads, step for step.
// Experts: at most 64.
FE2O3_HD bool expert_tile_lanes(const uint32_t* offsets, uint32_t e_begin, uint32_t e_end,
                                uint32_t routes, uint32_t n_blocks, uint32_t block, uint32_t xcds,
                                uint32_t* e_out, uint32_t* row0, uint32_t* rows, uint32_t* nb) {
  uint32_t lo[64], n[64], incl[64];
  const uint32_t ne = e_end - e_begin;
  uint32_t run = 0;
  for (uint32_t l = 0; l < 64; ++l) {
    lo[l] = n[l] = 0;
    if (l < ne) expert_rows(offsets, e_begin + l, routes, &lo[l], &n[l]);
    run += expert_m_tiles(n[l]) * n_blocks;
    incl[l] = run;
  }
  const uint32_t total = incl[63];
  const uint32_t chunk = (total + xcds - 1u) / xcds;
  const uint32_t slot = block / xcds;
  if (slot >= chunk) return false;
  const uint32_t x = (block % xcds) * chunk + slot;
  if (x >= total) return false;
  uint32_t l = 0;
  for (uint32_t i = 0; i < 64; ++i) l += incl[i] <= x ? 1u : 0u;
  const uint32_t m_tiles = expert_m_tiles(n[l]);
  const uint32_t xi = x - (incl[l] - m_tiles * n_blocks);
  *e_out = e_begin + l;
  *nb = xi / m_tiles;
  m_tile(lo[l], n[l], m_tiles, xi % m_tiles, row0, rows);
  return true;
}

// Grid sizes (workgroups, a multiple of xcds) of the gate/up and down
// launches for experts [e_begin, e_end): routes/288 rounded up plus one
// partial tile per expert bounds the m-tiles of any consistent routing.
FE2O3_HD uint64_t expert_grid(uint64_t routes, uint32_t n_experts, uint32_t n_blocks,
                              uint32_t xcds) {
  const uint64_t m_tiles = (routes + kMaxTileRows - 1u) / kMaxTileRows + n_experts;
  return (m_tiles * n_blocks + xcds - 1u) / xcds * xcds;
}

}  // namespace fe2o3
