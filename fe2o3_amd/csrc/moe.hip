// moe.hip -- top-2 mixture-of-experts for gfx950.
//
// Router (examples/moe_top2_v1/src/kernel.rs:25-202 semantics):
//   1. route_select: one thread per token; running top-2 with
//      candidate_precedes(score, id) = higher score, or equal score and lower
//      id (kernel.rs:25-33); route r = 2*token + rank; gating weights
//      w0 = 1/(1+exp(l1-l0)), w1 = 1 - w0 (w0 in [0.5,1], so the pair sums to
//      exactly 1 as examples/moe_expert_v1/src/pipeline.rs:137-148 requires).
//   2. route_assign: one workgroup per 512 routes; requested = per-expert
//      totals, admitted = min(requested, capacity), offsets = exclusive scan
//      of admitted with the terminal total; each route gets rank = number of
//      earlier routes (lower route id) of its expert, slot = offset + rank
//      when rank < capacity (stable prefix), permutation[slot] = route,
//      inverse[route] = slot, DROP sentinels elsewhere.  Integer work only:
//      bit-identical to the reference's sort-based oracle.
//
// Expert FFN at the BASELINE shape (gate/up SiLU, down, weighted combine):
//   gate/up     Hc = bf16(silu(Xc Wg_e^T) * (Xc Wu_e^T))  per expert e,
//               Xc[slot] = X[permutation[slot] / 2] read in place by the
//               A-tile copies (a gather pass into the workspace first only
//               for an X of 2 GiB or more); one 256x256 MFMA tile whose B
//               rows interleave 32 gate rows and the matching 32 up rows,
//               so gate and up accumulators of the same (row, f) sit in the
//               same lane for the fused epilogue
//   down        Yc = Hc Wd_e^T (fp32)
//   combine     out[t] = bf16((+0 + w0*Yc[inv[2t]]) + w1*Yc[inv[2t+1]]),
//               dropped routes contribute nothing (moe_expert_v1 combine
//               order, examples/moe_expert_v1/src/kernel.rs:98-157).
// Expert row ranges come from the device-resident offsets, so the whole
// layer runs without a host round trip: the grouped GEMM grids are sized
// for the worst case and workgroups beyond the last expert tile exit.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "common.hpp"
#include "gemm_pipe.hpp"
#include "internal.hpp"
#include "moe_tiles.hpp"

namespace {

using namespace fe2o3;
constexpr uint32_t DROP = 0xffffffffu;
constexpr int MAX_EXPERTS = 64;
constexpr int ASSIGN_THREADS = 128;  // 32 KiB of per-thread expert counters

template <typename T>
FE2O3_DEVICE float logit_at(const T* p, uint64_t i);
template <>
FE2O3_DEVICE float logit_at<float>(const float* p, uint64_t i) { return p[i]; }
template <>
FE2O3_DEVICE float logit_at<uint16_t>(const uint16_t* p, uint64_t i) {
  return f32_from_bf16_bits(p[i]);
}

// A token with a NaN or infinite logit is written as top2 = (DROP, DROP)
// and marks the contract-status word; route_assign then rejects the whole
// launch (see there), as the reference's kernel traps on any non-finite
// logit (kernel.rs:118-128).
template <typename T>
__global__ void __launch_bounds__(256) route_select_kernel(const T* __restrict__ logits,
                                                           uint32_t tokens, uint32_t experts,
                                                           uint32_t* __restrict__ top2,
                                                           float* __restrict__ weights,
                                                           uint32_t* __restrict__ status) {
#pragma clang fp contract(off)
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= tokens) return;
  const T* row = logits + (uint64_t)t * experts;
  uint32_t best = DROP, second = DROP;
  float bs = 0.0f, ss = 0.0f, probe = 0.0f;
  for (uint32_t e = 0; e < experts; ++e) probe = finite_probe(probe, logit_at(row, e));
  if (probe != probe) {
    mark_nonfinite(status);
    top2[2ull * t] = DROP;
    top2[2ull * t + 1] = DROP;
    return;
  }
  for (uint32_t e = 0; e < experts; ++e) {
    const float s = logit_at(row, e);
    if (best == DROP || s > bs || (s == bs && e < best)) {
      second = best;
      ss = bs;
      best = e;
      bs = s;
    } else if (second == DROP || s > ss || (s == ss && e < second)) {
      second = e;
      ss = s;
    }
  }
  top2[2ull * t] = best;
  top2[2ull * t + 1] = second;
  if (weights != nullptr) {
    const float w0 = 1.0f / (1.0f + expf(ss - bs));
    weights[2ull * t] = w0;
    weights[2ull * t + 1] = 1.0f - w0;
  }
}

// Slot assignment, one workgroup per RA_ROUTES consecutive routes (one route
// per thread).  Every workgroup first counts, per expert, the routes of the
// whole top2 array and those before its own range, straight from top2 (a few
// tens of KiB read from L2, so the workgroups need no scratch and no
// communication); then each route's stable rank = routes of its expert
// before the workgroup + those in earlier waves of the workgroup + those in
// earlier lanes of its wave (per-expert wave ballots).  requested = totals,
// admitted = min(requested, capacity), offsets = exclusive scan of admitted
// with the terminal total; a route of rank < capacity gets slot
// offsets[e] + rank, permutation[slot] = route, inverse[route] = slot; DROP
// elsewhere.  Integer work only: bit-identical to the reference's sort-based
// oracle for any number of workgroups.
//
// A launch whose route_select rejected any token (an expert id out of range
// in top2) is rejected as a whole: every workgroup sees that entry, and
// every output takes its sentinel -- top2, slots, permutation and inverse
// DROP, route weights +0, requested, admitted and offsets 0 -- so no expert
// receives a route.
constexpr int RA_THREADS = 512, RA_WAVES = RA_THREADS / 64, RA_ROUTES = RA_THREADS;

// For the 64 lanes' experts e (DROP = no route): calls fn(x, mask) once per
// distinct expert x present, mask = the lanes holding x.
template <class Fn>
FE2O3_DEVICE void for_each_expert(uint32_t e, Fn&& fn) {
  uint64_t left = __ballot(e != DROP);
  while (left != 0ull) {
    const int first = (int)__builtin_ctzll(left);
    const uint32_t x = (uint32_t)__builtin_amdgcn_readlane((int)e, first);
    const uint64_t mask = __ballot(e == x);
    fn(x, mask);
    left &= ~mask;
  }
}

// PREFIXED: the per-expert counts before this workgroup and the totals come
// from route_scan_kernel (prefix: (experts + 1) words per workgroup, the
// last unused here; totals: experts words, then the number of workgroups
// that saw a rejected entry) instead of from counting all of top2 here.
template <bool PREFIXED>
__global__ void __launch_bounds__(RA_THREADS) route_assign_kernel(
    uint32_t* __restrict__ top2, uint32_t routes, uint32_t experts, uint32_t capacity,
    uint32_t* __restrict__ requested, uint32_t* __restrict__ admitted,
    uint32_t* __restrict__ offsets, uint32_t* __restrict__ slots,
    uint32_t* __restrict__ permutation, uint32_t* __restrict__ inverse,
    float* __restrict__ weights, const uint32_t* __restrict__ prefix,
    const uint32_t* __restrict__ totals) {
  __shared__ uint32_t total[MAX_EXPERTS], before[MAX_EXPERTS], off_s[MAX_EXPERTS + 1];
  __shared__ uint32_t wave_cnt[RA_WAVES][MAX_EXPERTS];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t start = blockIdx.x * (uint32_t)RA_ROUTES;
  const uint64_t lt = (1ull << lane) - 1ull;
  if constexpr (PREFIXED) {
    if (t < experts) {
      total[t] = totals[t];
      before[t] = prefix[(uint64_t)blockIdx.x * (experts + 1u) + t];
    }
  } else {
    if (t < experts) total[t] = before[t] = 0;
  }
  for (uint32_t i = t; i < RA_WAVES * MAX_EXPERTS; i += RA_THREADS) (&wave_cnt[0][0])[i] = 0;
  __syncthreads();
  // counts over all of top2, 64 routes per wave and chunk; the loads of
  // eight chunks are issued together, then counted
  constexpr int kBatch = 8;
  int rejected = PREFIXED && totals[experts] != 0u;
  for (uint32_t base0 = wave * 64u; !PREFIXED && base0 < routes;
       base0 += kBatch * RA_THREADS) {
    uint32_t ev[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const uint32_t r = base0 + q * RA_THREADS + lane;
      ev[q] = r < routes ? top2[r] : DROP;
      rejected |= r < routes && ev[q] >= experts;
      if (ev[q] >= experts) ev[q] = DROP;  // not an expert: counted nowhere
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const uint32_t base = base0 + q * RA_THREADS;
      for_each_expert(ev[q], [&](uint32_t x, uint64_t mask) {
        if (lane == 0) {
          const uint32_t c = (uint32_t)__builtin_popcountll(mask);
          atomicAdd(&total[x], c);
          if (base < start) atomicAdd(&before[x], c);
        }
      });
    }
  }
  const uint32_t r = start + t;
  if (__syncthreads_or(rejected)) {
    if (r < routes) {
      top2[r] = DROP;
      slots[r] = DROP;
      inverse[r] = DROP;
      permutation[r] = DROP;
      if (weights != nullptr) weights[r] = 0.0f;
    }
    if (blockIdx.x == 0) {
      if (t < experts) requested[t] = admitted[t] = offsets[t] = 0;
      if (t == 0) offsets[experts] = 0;
    }
    return;
  }
  if (t == 0) {  // admitted counts and their exclusive scan (at most 64 experts)
    uint32_t run = 0;
    for (uint32_t x = 0; x < experts; ++x) {
      off_s[x] = run;
      run += total[x] < capacity ? total[x] : capacity;
    }
    off_s[experts] = run;
  }
  // ranks within this wave, and this wave's count per expert
  const uint32_t e = r < routes ? top2[r] : DROP;
  uint32_t rank = 0;
  for_each_expert(e, [&](uint32_t x, uint64_t mask) {
    if (e == x) rank = (uint32_t)__builtin_popcountll(mask & lt);
    if (lane == 0) wave_cnt[wave][x] = (uint32_t)__builtin_popcountll(mask);
  });
  __syncthreads();
  if (blockIdx.x == 0) {
    if (t < experts) {
      requested[t] = total[t];
      admitted[t] = total[t] < capacity ? total[t] : capacity;
      offsets[t] = off_s[t];
    }
    if (t == 0) offsets[experts] = off_s[experts];
  }
  if (r >= routes) return;
  rank += before[e];
  for (uint32_t w = 0; w < wave; ++w) rank += wave_cnt[w][e];
  if (rank < capacity) {
    const uint32_t slot = off_s[e] + rank;
    slots[r] = slot;
    inverse[r] = slot;
    permutation[slot] = r;
  } else {
    slots[r] = DROP;
    inverse[r] = DROP;
  }
  // slots below the accepted total are each written by their route; the rest
  // of the permutation holds the sentinel
  if (r >= off_s[experts]) permutation[r] = DROP;
}

// Slot assignment for many routes, in three kernels whose work is linear in
// the routes (route_assign_kernel<false> has every workgroup count all of
// top2, which grows as routes^2 / 512: 0.33 ms at 2^16 tokens, 8.6 ms at
// 2^19).  route_count_kernel: workgroup b writes its own routes' count per
// expert to counts[b][0 .. experts) and whether any of them holds an entry
// that is not an expert to counts[b][experts].  route_scan_kernel (one
// workgroup): each column's exclusive prefix over the workgroups in place,
// and the column totals.  route_assign_kernel<true> then takes `before` and
// `total` from there: the same numbers the single kernel counts, so the same
// outputs.
__global__ void __launch_bounds__(RA_THREADS) route_count_kernel(
    const uint32_t* __restrict__ top2, uint32_t routes, uint32_t experts,
    uint32_t* __restrict__ counts) {
  __shared__ uint32_t cnt[MAX_EXPERTS];
  const uint32_t t = threadIdx.x, lane = t & 63u;
  if (t < experts) cnt[t] = 0;
  __syncthreads();
  const uint32_t r = blockIdx.x * (uint32_t)RA_ROUTES + t;
  uint32_t e = r < routes ? top2[r] : DROP;
  const int rejected = r < routes && e >= experts;
  if (e >= experts) e = DROP;  // not an expert: counted nowhere
  for_each_expert(e, [&](uint32_t x, uint64_t mask) {
    if (lane == 0) atomicAdd(&cnt[x], (uint32_t)__builtin_popcountll(mask));
  });
  const int any = __syncthreads_or(rejected);
  uint32_t* row = counts + (uint64_t)blockIdx.x * (experts + 1u);
  if (t < experts) row[t] = cnt[t];
  if (t == 0) row[experts] = any ? 1u : 0u;
}

constexpr int RS_THREADS = 1024;
// Routes above which route() takes the three kernels (the single kernel's
// quadratic counting costs more than the two extra launches from here on).
constexpr uint64_t kRouteScanAbove = 8192;

// One workgroup: thread i takes the rows [i * chunk, (i + 1) * chunk) of
// every column in turn: its rows' sum, an exclusive scan of the sums over
// the threads (wave scans, then the waves' sums), then the rows rewritten
// with their exclusive prefixes.  Sums are below 2^32 (at most `routes`).
// A table of at most kScanLdsWords words is first loaded whole into LDS (one
// coalesced pass, where the column-by-column passes over global memory wait
// for it once per column) and scanned there, one wave per column.
constexpr uint32_t kScanLdsWords = 8192;

__global__ void __launch_bounds__(RS_THREADS) route_scan_kernel(uint32_t* __restrict__ counts,
                                                                uint32_t blocks, uint32_t experts,
                                                                uint32_t* __restrict__ totals) {
  __shared__ uint32_t wave_sum[RS_THREADS / 64];
  __shared__ uint32_t table[kScanLdsWords];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t cols = experts + 1u;
  const uint64_t words = (uint64_t)blocks * cols;
  if (words <= kScanLdsWords) {
    for (uint32_t i = t; i < words; i += RS_THREADS) table[i] = counts[i];
    __syncthreads();
    // wave w scans columns w, w + 16, ...: rows in runs of 64 lanes, a
    // running carry between runs
    for (uint32_t c = wave; c < cols; c += RS_THREADS / 64) {
      uint32_t carry = 0;
      for (uint32_t b0 = 0; b0 < blocks; b0 += 64u) {
        const uint32_t b = b0 + lane;
        const uint32_t v = b < blocks ? table[b * cols + c] : 0u;
        uint32_t incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t u = (uint32_t)__shfl_up((int)incl, o, 64);
          if (lane >= (uint32_t)o) incl += u;
        }
        if (b < blocks) counts[(uint64_t)b * cols + c] = carry + incl - v;
        carry += (uint32_t)__shfl((int)incl, 63, 64);
      }
      if (lane == 0) totals[c] = carry;
    }
    return;
  }
  const uint32_t chunk = (blocks + RS_THREADS - 1u) / RS_THREADS;
  const uint32_t b0 = min(t * chunk, blocks), b1 = min(b0 + chunk, blocks);
  for (uint32_t c = 0; c < cols; ++c) {
    uint32_t sum = 0;
    for (uint32_t b = b0; b < b1; ++b) sum += counts[(uint64_t)b * cols + c];
    uint32_t incl = sum;  // inclusive scan within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t v = (uint32_t)__shfl_up((int)incl, o, 64);
      if (lane >= (uint32_t)o) incl += v;
    }
    if (lane == 63) wave_sum[wave] = incl;
    __syncthreads();
    uint32_t run = incl - sum;
    for (uint32_t w = 0; w < wave; ++w) run += wave_sum[w];
    for (uint32_t b = b0; b < b1; ++b) {
      const uint32_t v = counts[(uint64_t)b * cols + c];
      counts[(uint64_t)b * cols + c] = run;
      run += v;
    }
    if (t == RS_THREADS - 1u) totals[c] = run;
    __syncthreads();  // wave_sum is rewritten for the next column
  }
}

// examples/moe_expert_v1/src/kernel.rs:104-157: T=8, K=2, O=16.
__global__ void __launch_bounds__(128) combine_profile_kernel(const float* __restrict__ compact,
                                                              const uint32_t* __restrict__ inverse,
                                                              const float* __restrict__ weights,
                                                              float* __restrict__ combined) {
#pragma clang fp contract(off)
  const uint32_t i = threadIdx.x;  // 0..127
  const uint32_t t = i / 16, o = i % 16;
  float acc = 0.0f;
  for (uint32_t rank = 0; rank < 2; ++rank) {
    const uint32_t route = t * 2 + rank;
    const uint32_t slot = inverse[route];
    if (slot < 16u) {
      const float wv = weights[route] * compact[slot * 16 + o];
      acc = acc + wv;
    }
  }
  combined[i] = acc;
}

// ---- expert FFN -------------------------------------------------------------------------
// Routing arrays live in device memory, where the host cannot validate them
// (fe2o3_moe_routing_check does); every kernel of the FFN clamps what it
// reads from them, so an inconsistent routing gives unspecified outputs but
// no access outside the caller's buffers and the workspace.  A slot whose
// permutation entry is not a route gathers a zero row.
__global__ void __launch_bounds__(256) gather_kernel(const uint16_t* __restrict__ x,
                                                     const uint32_t* __restrict__ permutation,
                                                     const uint32_t* __restrict__ offsets,
                                                     uint32_t experts, uint32_t hidden,
                                                     uint32_t routes,
                                                     uint16_t* __restrict__ xc) {
  const uint32_t slot = blockIdx.x;
  if (slot >= offsets[experts]) return;
  const uint32_t route = permutation[slot];
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(xc + (uint64_t)slot * hidden);
  if (route >= routes) {
    for (uint32_t i = threadIdx.x; i < hidden / 8; i += blockDim.x) dst[i] = u32x4_t{0, 0, 0, 0};
    return;
  }
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(x + (uint64_t)(route >> 1) * hidden);
  for (uint32_t i = threadIdx.x; i < hidden / 8; i += blockDim.x) dst[i] = src[i];
}

// This workgroup's entry of the expert tile list (moe_tiles.hpp), computed
// by each wave as expert_tile_lanes spells out: lane l loads expert
// e_begin + l's row bounds (one memory round trip for all experts, where the
// serial walk took two dependent scalar loads per expert, ~8% of a gate/up
// tile), a wave scan sums the tile counts, a ballot finds the entry's
// expert, and lane reads return its bounds as wave-uniform values.
FE2O3_DEVICE bool expert_tile(const uint32_t* offsets, uint32_t e_begin, uint32_t e_end,
                              uint32_t routes, uint32_t n_blocks, uint32_t xcds, uint32_t* e_out,
                              uint32_t* row0, uint32_t* rows, uint32_t* nb) {
  const uint32_t l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  uint32_t lo = 0, n = 0;
  if (l < e_end - e_begin) expert_rows(offsets, e_begin + l, routes, &lo, &n);
  uint32_t incl = expert_m_tiles(n) * n_blocks;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = (uint32_t)__shfl_up((int)incl, o, 64);
    if (l >= (uint32_t)o) incl += v;
  }
  const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
  const uint32_t chunk = (total + xcds - 1u) / xcds;
  const uint32_t slot = blockIdx.x / xcds;
  if (slot >= chunk) return false;
  const uint32_t x = (blockIdx.x % xcds) * chunk + slot;
  if (x >= total) return false;
  const int le = (int)__builtin_popcountll(__ballot(incl <= x));
  const uint32_t lo_e = (uint32_t)__builtin_amdgcn_readlane((int)lo, le);
  const uint32_t n_e = (uint32_t)__builtin_amdgcn_readlane((int)n, le);
  const uint32_t incl_e = (uint32_t)__builtin_amdgcn_readlane((int)incl, le);
  const uint32_t m_tiles = expert_m_tiles(n_e);
  const uint32_t xi = x - (incl_e - m_tiles * n_blocks);
  *e_out = e_begin + (uint32_t)le;
  *nb = xi / m_tiles;
  m_tile(lo_e, n_e, m_tiles, xi % m_tiles, row0, rows);
  return true;
}

// silu(g) * u = g / (1 + e^-g) * u with the hardware exp2 and reciprocal
// (about one ulp each, far below the bf16 rounding of the product); the
// library expf and IEEE divide cost ~30 instructions per output, a few
// percent of a 256x128 tile.  Limits: g -> +inf gives g, g -> -inf gives -0.
FE2O3_DEVICE float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  const float sg = g * __builtin_amdgcn_rcpf(1.0f + e);
  return sg * u;
}

constexpr int kRowBytes = 128, kStages = 2;  // 64 k per LDS stage, two stages
// two stages of a 288-row A tile and a 256-row B tile: 136 KiB
constexpr int kSmem = kStages * (int)(kMaxTileRows + 256u) * kRowBytes;

// The form a tile of `rows` rows runs on: fn(RPW) with RPW output rows per
// wave, the A tile holding 2 RPW rows = `rows` rounded up to 32, on two 64-k
// stages (the 288-row form keeps its ninth row block's accumulators in
// VGPRs: an expert of up to 1152 rows takes four tiles, not five); fn(0)
// for a tile of at most 64 rows (an expert of at most 64 rows, as the tile
// list deals rows out), which runs 64 rows on four 32-k stages:
// its few MFMAs per stage cannot hide the weight copies' latency, and three
// stages of copies in flight can.  The MFMAs and A copies of a tile are
// those of its own rows; the B copies are the whole n-block's.
template <class Fn>
FE2O3_DEVICE void by_tile_rows(uint32_t rows, Fn&& fn) {
  using std::integral_constant;
  if (rows > 256u) fn(integral_constant<int, 144>{});
  else if (rows > 224u) fn(integral_constant<int, 128>{});
  else if (rows > 192u) fn(integral_constant<int, 112>{});
  else if (rows > 160u) fn(integral_constant<int, 96>{});
  else if (rows > 128u) fn(integral_constant<int, 80>{});
  else if (rows > 96u) fn(integral_constant<int, 64>{});
  else if (rows > 64u) fn(integral_constant<int, 48>{});
  else fn(integral_constant<int, 0>{});
}

// A tile of a gate/up tile read straight from the token matrix x (tokens x
// hidden, x_bytes bytes, below 2^31): tile row r is slot row0 + r of the
// admitted routes, and the slot's permutation entry names its route (token =
// route / 2).  A slot whose entry is not a route (>= routes) loads from an
// offset past x's extent, which the buffer's range check turns into zeros:
// the zero row gather_kernel writes for it.  Rows at or past valid_rows
// repeat the last valid row, as dense_rows does; the bytes in LDS are those
// of the gathered rows, so the products are the same.
template <int ROW_BYTES, int ROWS>
FE2O3_DEVICE gemm_pipe::Rows<ROW_BYTES, gemm_pipe::Geo<ROW_BYTES>::insts(ROWS)> token_rows(
    const uint16_t* x, uint32_t x_bytes, const uint32_t* __restrict__ permutation,
    uint32_t row0, uint32_t valid_rows, uint32_t routes, uint32_t hidden) {
  using G = gemm_pipe::Geo<ROW_BYTES>;
  static_assert(ROWS * ROW_BYTES % 4096 == 0, "whole 1-KiB loads per wave for the tile's rows");
  gemm_pipe::Rows<ROW_BYTES, G::insts(ROWS)> t;
  t.bytes = x_bytes;
  uint32_t route[G::insts(ROWS)];
#pragma unroll
  for (int j = 0; j < G::insts(ROWS); ++j) {
    const uint32_t row = G::inst_row(j);
    route[j] = permutation[row0 + (row < valid_rows ? row : valid_rows - 1u)];
  }
#pragma unroll
  for (int j = 0; j < G::insts(ROWS); ++j) {
    const uint32_t chunk = G::inst_chunk(G::inst_row(j));
    t.base[j] = x;
    t.voff[j] = route[j] < routes ? ((route[j] >> 1) * hidden + chunk * 8u) * 2u
                                  : gemm_pipe::kOutOfRange;
  }
  return t;
}

// One gate/up tile on the pipeline geometry G (ROW_BYTES of k per row and
// stage, STAGES stages, RPW output rows per wave; the A tile holds 2 RPW
// rows; the form by_tile_rows picks).  TOKENS: the A rows come from the token
// matrix through the permutation (token_rows; xa = x); otherwise from the
// gathered rows (xa = xc, row row0 onward).
template <bool TOKENS, int ROW_BYTES, int STAGES, int RPW>
FE2O3_DEVICE void gate_up_tile(const uint16_t* __restrict__ xa, uint32_t x_bytes,
                               const uint32_t* __restrict__ permutation, uint32_t routes,
                               const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu,
                               uint32_t e, uint32_t row0, uint32_t rows, uint32_t nb,
                               uint32_t hidden, uint32_t ffn, uint16_t* __restrict__ hc,
                               uint8_t* smem) {
  using G = gemm_pipe::Geo<ROW_BYTES>;
  const uint32_t f0 = nb * 128u;
  const auto ar = [&] {
    if constexpr (TOKENS)
      return token_rows<ROW_BYTES, 2 * RPW>(xa, x_bytes, permutation, row0, rows, routes, hidden);
    else
      return gemm_pipe::dense_rows<ROW_BYTES, 2 * RPW>(xa + (uint64_t)row0 * hidden, hidden, rows,
                                                       hidden);
  }();
  // B tile row r: 32-row block jb = r/32 belongs to wave column wn = jb/4;
  // within a wave column the blocks are gate f, up f, gate f+32, up f+32 for
  // f = f0 + 64*wn, so each lane's gate and up accumulators of one (row, f)
  // pair up in the epilogue.
  // The buffers are the expert's gate and up matrices.
  gemm_pipe::Rows<ROW_BYTES> br;
  const uint64_t wbase = (uint64_t)e * ffn * hidden;
  br.bytes = ffn * hidden * 2u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
  for (int j = 0; j < G::kInstPerWave; ++j) {
    const uint32_t row = G::inst_row(j);
    // the load's rows lie in one 32-row block: gate or up is wave-uniform
    const uint32_t jb = ((4u * j + wave) * G::kRowsPerInst) >> 5, wn = jb >> 2, jj = jb & 3u;
    const uint32_t f = f0 + wn * 64u + (jj >> 1) * 32u + (row & 31u);
    br.base[j] = ((jj & 1u) ? wu : wg) + wbase;
    br.voff[j] = (f * hidden + G::inst_chunk(row) * 8u) * 2u;
  }
  using Mma = gemm_pipe::Bf16Mma<ROW_BYTES, RPW>;
  typename Mma::Acc acc;
  gemm_pipe::mainloop<Mma, ROW_BYTES, STAGES>(ar, br, hidden, smem, acc);
  // accumulator column j (16 B rows each) of wave column wn: j = 0,1 gate
  // f .. f+31, j = 2,3 up f .. f+31, j = 4,5 gate f+32 .., j = 6,7 up f+32 ..
  // (f = f0 + 64 wn); gate j pairs with up j + 2
  // Lane row g = lane / 16 holds columns 4g .. 4g + 3 of each 16-column
  // block; the blocks sub = 0 and 1 of a half are adjacent, and one
  // v_permlane16_swap per packed word (gemm_pipe::store_bf16_pairs) leaves
  // row g with columns 8 (g / 2) .. + 7 of block g % 2: one 16-byte store per
  // lane, 64 contiguous bytes per output row.  Partner lanes share their
  // output row, so both or neither store.
  const uint32_t r0 = gemm_pipe::acc16_row0<RPW>();
  const uint32_t g = gemm_pipe::lane_id() >> 4;
  const uint32_t wn = gemm_pipe::wave_id() & 1u;
  const uint32_t fl = f0 + 64u * wn + 16u * (g & 1u) + 8u * (g >> 1);
#pragma unroll
  for (int i = 0; i < Mma::kRB; ++i) {
    const uint32_t r = r0 + 16u * i;
    if (r >= rows) continue;
    uint16_t* out_row = hc + (uint64_t)(row0 + r) * ffn;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t w[2][2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const f32x4_t& gv = acc.v[i][4 * half + sub];
        const f32x4_t& uv = acc.v[i][4 * half + sub + 2];
        w[sub][0] = pack_bf16x2(silu_mul(gv[0], uv[0]), silu_mul(gv[1], uv[1]));
        w[sub][1] = pack_bf16x2(silu_mul(gv[2], uv[2]), silu_mul(gv[3], uv[3]));
      }
      const auto s0 = __builtin_amdgcn_permlane16_swap(w[0][0], w[1][0], false, false);
      const auto s1 = __builtin_amdgcn_permlane16_swap(w[0][1], w[1][1], false, false);
      u32x4_t packed;
      packed[0] = s0[0];
      packed[1] = s1[0];
      packed[2] = s0[1];
      packed[3] = s1[1];
      *reinterpret_cast<u32x4_t*>(out_row + fl + half * 32u) = packed;
    }
  }
}

// TOKENS: xa is the token matrix (x_bytes bytes) read through the
// permutation; otherwise the gathered rows xc.
template <bool TOKENS>
__global__ void __launch_bounds__(256, 1) gate_up_kernel(
    const uint16_t* __restrict__ xa, uint32_t x_bytes, const uint32_t* __restrict__ permutation,
    const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu,
    const uint32_t* __restrict__ offsets, uint32_t e_begin, uint32_t e_end, uint32_t hidden,
    uint32_t ffn, uint32_t routes, uint16_t* __restrict__ hc, uint32_t xcds) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  uint32_t e, row0, rows, nb;
  if (!expert_tile(offsets, e_begin, e_end, routes, ffn / 128u, xcds, &e, &row0, &rows, &nb))
    return;
  by_tile_rows(rows, [&](auto rpw) {
    constexpr int R = decltype(rpw)::value;
    if constexpr (R == 0)
      gate_up_tile<TOKENS, 64, 4, 32>(xa, x_bytes, permutation, routes, wg, wu, e, row0, rows, nb,
                                      hidden, ffn, hc, smem);
    else
      gate_up_tile<TOKENS, 128, 2, R>(xa, x_bytes, permutation, routes, wg, wu, e, row0, rows, nb,
                                      hidden, ffn, hc, smem);
  });
}

// One down tile, on the geometry of gate_up_tile.  K is split in `kparts`
// (1 or 2) parts: list entry nb = kparts * n-block + part, and part p writes
// its own fp32 partial at yc + p * routes * hidden, which the combine adds.
template <int ROW_BYTES, int STAGES, int RPW>
FE2O3_DEVICE void down_tile(const uint16_t* __restrict__ hc, const uint16_t* __restrict__ wd,
                            uint32_t e, uint32_t row0, uint32_t rows, uint32_t nb,
                            uint32_t hidden, uint32_t ffn, uint64_t routes, uint32_t kparts,
                            float* __restrict__ yc, uint8_t* smem) {
  const uint32_t n0 = nb / kparts * 256u, kh = nb % kparts, k_half = ffn / kparts;
  const auto ar = gemm_pipe::dense_rows<ROW_BYTES, 2 * RPW>(
      hc + (uint64_t)row0 * ffn + kh * k_half, ffn, rows, k_half);
  const auto br = gemm_pipe::dense_rows<ROW_BYTES>(
      wd + (uint64_t)e * hidden * ffn + (uint64_t)n0 * ffn + kh * k_half, ffn, 256, k_half);
  using Mma = gemm_pipe::Bf16Mma<ROW_BYTES, RPW>;
  typename Mma::Acc acc;
  gemm_pipe::mainloop<Mma, ROW_BYTES, STAGES>(ar, br, k_half, smem, acc);
  float* part = yc + (uint64_t)kh * routes * hidden;
  const uint32_t r0 = gemm_pipe::acc16_row0<RPW>(), c0 = gemm_pipe::acc16_col0();
#pragma unroll
  for (int i = 0; i < Mma::kRB; ++i) {
    const uint32_t r = r0 + 16u * i;
    if (r >= rows) continue;
    float* out_row = part + (uint64_t)(row0 + r) * hidden + n0 + c0;
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<f32x4_t*>(out_row + 16u * j) = acc.v[i][j];
  }
}

// kparts = 2 (split K: twice as many workgroups, each half as long) when
// that fills the grid's last round of tiles better (down_k_parts).
__global__ void __launch_bounds__(256, 1) down_kernel(const uint16_t* __restrict__ hc,
                                                      const uint16_t* __restrict__ wd,
                                                      const uint32_t* __restrict__ offsets,
                                                      uint32_t e_begin, uint32_t e_end,
                                                      uint32_t hidden, uint32_t ffn,
                                                      uint64_t routes, uint32_t kparts,
                                                      float* __restrict__ yc, uint32_t xcds) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  uint32_t e, row0, rows, nb;
  if (!expert_tile(offsets, e_begin, e_end, (uint32_t)routes, kparts * (hidden / 256u), xcds, &e,
                   &row0, &rows, &nb))
    return;
  by_tile_rows(rows, [&](auto rpw) {
    constexpr int R = decltype(rpw)::value;
    if constexpr (R == 0)
      down_tile<64, 4, 32>(hc, wd, e, row0, rows, nb, hidden, ffn, routes, kparts, yc, smem);
    else
      down_tile<128, 2, R>(hc, wd, e, row0, rows, nb, hidden, ffn, routes, kparts, yc, smem);
  });
}

__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ yc,
                                                      const uint32_t* __restrict__ inverse,
                                                      const float* __restrict__ weights,
                                                      uint32_t tokens, uint32_t hidden,
                                                      uint64_t routes, uint32_t kparts,
                                                      uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 4 outputs each
  const uint64_t per_token = hidden / 4u;
  if (idx >= (uint64_t)tokens * per_token) return;
  const uint32_t t = (uint32_t)(idx / per_token);
  const uint32_t h = (uint32_t)(idx % per_token) * 4u;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t rank = 0; rank < 2; ++rank) {
    const uint32_t route = 2u * t + rank;
    const uint32_t slot = inverse[route];
    if (slot >= routes) continue;  // DROP, or not a slot
    const float w = weights[route];
    const f32x4_t y0 = *reinterpret_cast<const f32x4_t*>(yc + (uint64_t)slot * hidden + h);
    f32x4_t y1 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (kparts == 2u)
      y1 = *reinterpret_cast<const f32x4_t*>(yc + routes * hidden + (uint64_t)slot * hidden + h);
#pragma unroll
    for (int z = 0; z < 4; ++z) {
      // the down projection, or the sum of its two k-part partials
      const float y = kparts == 2u ? y0[z] + y1[z] : y0[z];
      const float wv = w * y;
      acc[z] = acc[z] + wv;
    }
  }
  u32x2_t packed;
  packed[0] = pack_bf16x2(acc[0], acc[1]);
  packed[1] = pack_bf16x2(acc[2], acc[3]);
  *reinterpret_cast<u32x2_t*>(out + (uint64_t)t * hidden + h) = packed;
}

struct Workspace {
  uint16_t* xc;
  uint16_t* hc;
  float* yc;
  uint64_t bytes;
};

uint64_t align256(uint64_t v) { return (v + 255u) & ~255ull; }

Workspace carve(void* base, uint32_t tokens, uint32_t hidden, uint32_t ffn) {
  const uint64_t routes = 2ull * tokens;
  Workspace w;
  uint8_t* p = (uint8_t*)base;
  const uint64_t xb = align256(routes * hidden * 2), hb = align256(routes * ffn * 2),
                 yb = align256(2 * routes * hidden * 4);  // up to two k-part partials
  w.xc = (uint16_t*)p;
  w.hc = (uint16_t*)(p + xb);
  w.yc = (float*)(p + xb + hb);
  w.bytes = xb + hb + yb;
  return w;
}

int32_t route(const void* logits, uint64_t logits_len, uint32_t dtype, uint32_t* top2,
              uint64_t top2_len, uint32_t* requested, uint64_t requested_len, uint32_t* admitted,
              uint64_t admitted_len, uint32_t* offsets, uint64_t offsets_len, uint32_t* slots,
              uint64_t slots_len, uint32_t* permutation, uint64_t permutation_len,
              uint32_t* inverse, uint64_t inverse_len, float* weights, uint64_t weights_len,
              uint32_t tokens, uint32_t experts, uint32_t capacity, void* stream) {
  if (experts < 2 || experts > MAX_EXPERTS || dtype > 1) return FE2O3_ERR_SHAPE;
  const uint64_t routes = 2ull * tokens;
  if (routes > 0xfffffffeull) return FE2O3_ERR_OVERFLOW;
  if (logits_len != (uint64_t)tokens * experts || top2_len != routes || slots_len != routes ||
      permutation_len != routes || inverse_len != routes || requested_len != experts ||
      admitted_len != experts || offsets_len != experts + 1ull ||
      (weights && weights_len != routes))
    return FE2O3_ERR_LENGTH;
  if (!requested || !admitted || !offsets) return FE2O3_ERR_NULL;
  if (routes && (!logits || !top2 || !slots || !permutation || !inverse)) return FE2O3_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  uint32_t* status = fe2o3_host::status_word();
  if (status == nullptr) return (int32_t)hipErrorInvalidSymbol;
  if (tokens) {
    const unsigned blocks = (tokens + 255u) / 256u;
    if (dtype == 0)
      route_select_kernel<float><<<blocks, 256, 0, s>>>((const float*)logits, tokens, experts,
                                                        top2, weights, status);
    else
      route_select_kernel<uint16_t><<<blocks, 256, 0, s>>>((const uint16_t*)logits, tokens,
                                                           experts, top2, weights, status);
  }
  const unsigned assign_blocks = routes ? (unsigned)((routes + RA_ROUTES - 1) / RA_ROUTES) : 1u;
  // Many routes: the count / scan / assign kernels, on stream-ordered
  // scratch of (experts + 1) words per workgroup and the totals.  Without
  // scratch on this device, the single kernel.
  if (routes > kRouteScanAbove) {
    void* scratch = nullptr;
    const uint64_t rows = (uint64_t)assign_blocks * (experts + 1u);
    if (fe2o3_host::scratch_alloc(&scratch, (rows + experts + 1u) * 4u, s) == FE2O3_OK) {
      uint32_t* counts = static_cast<uint32_t*>(scratch);
      uint32_t* totals = counts + rows;
      route_count_kernel<<<assign_blocks, RA_THREADS, 0, s>>>(top2, (uint32_t)routes, experts,
                                                               counts);
      route_scan_kernel<<<1, RS_THREADS, 0, s>>>(counts, assign_blocks, experts, totals);
      route_assign_kernel<true><<<assign_blocks, RA_THREADS, 0, s>>>(
          top2, (uint32_t)routes, experts, capacity, requested, admitted, offsets, slots,
          permutation, inverse, weights, counts, totals);
      const int32_t rc = fe2o3_host::after_launch();
      const int32_t free_rc = fe2o3_host::scratch_free(scratch, s);
      return rc != FE2O3_OK ? rc : free_rc;
    }
    (void)hipGetLastError();
  }
  route_assign_kernel<false><<<assign_blocks, RA_THREADS, 0, s>>>(
      top2, (uint32_t)routes, experts, capacity, requested, admitted, offsets, slots, permutation,
      inverse, weights, nullptr, nullptr);
  return fe2o3_host::after_launch();
}

// ---- routing output consistency -------------------------------------------------------
// crates/fe2o3-host/src/moe_routing_expert_bridge_v1.rs:220-389 and the
// compact pack plan (crates/fe2o3-host/src/generated_moe_expert_v1.rs:159-
// 190), over T tokens, E experts and capacity C, on the device.  Each check
// site has a 64-bit key (phase << 58 | position << 3 | sub-check) that
// orders it as the reference's sequential check does; the smallest failing
// key is the reference's first error, and its site writes the record
// {kind, index, expected, actual}.  Exactness for the parallel form: when
// site k is the first failure, every earlier site passed, so what k reads
// (stable ranks from all earlier routes, the slots earlier routes claimed)
// is what the sequential check sees at k.  Every read is bounds-guarded, so
// arbitrary payloads are safe.
enum : uint32_t {
  RC_OK = 0, RC_EXPERT_OUT_OF_RANGE, RC_DUPLICATE_TOKEN_EXPERT, RC_REQUESTED_COUNT, RC_CAPACITY,
  RC_ADMITTED_COUNT, RC_FIRST_OFFSET, RC_NONMONOTONE_OFFSETS, RC_OFFSET_MISMATCH,
  RC_PLAN_OFFSET_ORDER, RC_PLAN_CAPACITY, RC_SLOT_OUT_OF_RANGE, RC_DUPLICATE_SLOT,
  RC_STABLE_SLOT, RC_INVERSE, RC_PERMUTATION, RC_PREFIX_HOLE, RC_PERMUTATION_ROUTE,
  RC_PERMUTATION_TAIL
};
constexpr uint32_t CHECK_MAX_ROUTES = 24576;  // claimed-slot table: 96 KiB of LDS

struct Site {
  uint64_t key = ~0ull;
  uint32_t rec[4] = {0, 0, 0, 0};
  FE2O3_DEVICE void fail(uint64_t k, uint32_t kind, uint32_t index, uint32_t expected,
                         uint32_t actual) {
    if (k < key) {
      key = k;
      rec[0] = kind;
      rec[1] = index;
      rec[2] = expected;
      rec[3] = actual;
    }
  }
};
FE2O3_DEVICE uint64_t site_key(uint32_t phase, uint64_t pos, uint32_t sub) {
  return ((uint64_t)phase << 58) | (pos << 3) | sub;
}

__global__ void __launch_bounds__(ASSIGN_THREADS) routing_check_kernel(
    const uint32_t* __restrict__ top2, const uint32_t* __restrict__ requested,
    const uint32_t* __restrict__ admitted, const uint32_t* __restrict__ offsets,
    const uint32_t* __restrict__ slots, const uint32_t* __restrict__ permutation,
    const uint32_t* __restrict__ inverse, uint32_t tokens, uint32_t experts, uint32_t capacity,
    uint32_t* __restrict__ record) {
  __shared__ uint32_t cnt[MAX_EXPERTS * ASSIGN_THREADS];
  __shared__ unsigned long long best;
  extern __shared__ uint32_t claimant[];  // per slot: the smallest route claiming it
  const uint32_t t = threadIdx.x, routes = 2u * tokens;
  const uint32_t per = (routes + ASSIGN_THREADS - 1) / ASSIGN_THREADS;
  const uint32_t r0 = t * per, r1 = r0 + per < routes ? r0 + per : routes;
  Site site;
  if (t == 0) best = ~0ull;
  for (uint32_t e = 0; e < experts; ++e) cnt[e * ASSIGN_THREADS + t] = 0;
  for (uint32_t s = t; s < routes; s += ASSIGN_THREADS) claimant[s] = DROP;
  __syncthreads();
  // phase 1: top-2 ids in range and distinct per token; per-thread counts
  for (uint32_t tk = t; tk < tokens; tk += ASSIGN_THREADS) {
    const uint32_t a = top2[2 * tk], b = top2[2 * tk + 1];
    if (a >= experts) site.fail(site_key(1, tk, 0), RC_EXPERT_OUT_OF_RANGE, 2 * tk, 0, a);
    else if (b >= experts) site.fail(site_key(1, tk, 1), RC_EXPERT_OUT_OF_RANGE, 2 * tk + 1, 0, b);
    else if (a == b) site.fail(site_key(1, tk, 2), RC_DUPLICATE_TOKEN_EXPERT, tk, 0, a);
  }
  for (uint32_t r = r0; r < r1; ++r) {
    const uint32_t e = top2[r];
    if (e < experts) cnt[e * ASSIGN_THREADS + t] += 1;
  }
  // the slots routes claim (the reference's seen set), smallest route first
  const uint32_t accepted = offsets[experts];
  for (uint32_t r = r0; r < r1; ++r) {
    const uint32_t slot = slots[r];
    if (slot != DROP && slot < accepted && slot < routes) atomicMin(&claimant[slot], r);
  }
  __syncthreads();
  // phases 2-6: counts, capacity, offsets, pack plan (E <= 64, one thread
  // each for the scan of its expert's counts, then one thread in order)
  __shared__ uint32_t total[MAX_EXPERTS];
  if (t < experts) {
    uint32_t run = 0;
    for (uint32_t i = 0; i < ASSIGN_THREADS; ++i) {
      const uint32_t c = cnt[t * ASSIGN_THREADS + i];
      cnt[t * ASSIGN_THREADS + i] = run;  // exclusive prefix: the stable-rank base
      run += c;
    }
    total[t] = run;
  }
  __syncthreads();
  if (t == 0) {
    Site s0;
    for (uint32_t e = 0; e < experts && s0.key == ~0ull; ++e)
      if (requested[e] != total[e]) s0.fail(site_key(2, e, 0), RC_REQUESTED_COUNT, e, total[e], requested[e]);
    for (uint32_t e = 0; e < experts && s0.key == ~0ull; ++e) {
      const uint32_t want = requested[e] < capacity ? requested[e] : capacity;
      if (admitted[e] > capacity) s0.fail(site_key(3, e, 0), RC_CAPACITY, e, 0, admitted[e]);
      else if (admitted[e] != want) s0.fail(site_key(3, e, 1), RC_ADMITTED_COUNT, e, want, admitted[e]);
    }
    if (s0.key == ~0ull && offsets[0] != 0) s0.fail(site_key(4, 0, 0), RC_FIRST_OFFSET, 0, 0, offsets[0]);
    uint32_t cum = 0;
    for (uint32_t e = 0; e < experts && s0.key == ~0ull; ++e) {
      const uint32_t start = offsets[e], end = offsets[e + 1];
      cum += admitted[e];
      if (start > end) s0.fail(site_key(5, e, 0), RC_NONMONOTONE_OFFSETS, e, start, end);
      else if (end != cum) s0.fail(site_key(5, e, 1), RC_OFFSET_MISMATCH, e + 1, cum, end);
    }
    for (uint32_t e = 0; e < experts && s0.key == ~0ull; ++e) {
      const uint32_t start = offsets[e], end = offsets[e + 1];
      if (start > end || end > routes) s0.fail(site_key(6, e, 0), RC_PLAN_OFFSET_ORDER, e, 0, end);
      else if (end - start > capacity) s0.fail(site_key(6, e, 1), RC_PLAN_CAPACITY, e, 0, end - start);
    }
    if (s0.key < site.key) site = s0;
  }
  // phase 7: per route in order -- slot range, duplicate, stable slot,
  // inverse, permutation entry
  for (uint32_t r = r0; r < r1; ++r) {
    const uint32_t e = top2[r];
    if (e >= experts) break;  // phase 1 reports it, and ranks stop being defined
    const uint32_t rank = cnt[e * ASSIGN_THREADS + t]++;
    const uint32_t want = rank < capacity ? offsets[e] + rank : DROP;
    const uint32_t slot = slots[r];
    if (slot != DROP && slot >= accepted) {
      site.fail(site_key(7, r, 0), RC_SLOT_OUT_OF_RANGE, r, accepted, slot);
      break;
    }
    if (slot != DROP && slot < routes && claimant[slot] < r) {
      site.fail(site_key(7, r, 1), RC_DUPLICATE_SLOT, r, 0, slot);
      break;
    }
    if (slot != want) {
      site.fail(site_key(7, r, 2), RC_STABLE_SLOT, r, want, slot);
      break;
    }
    if (inverse[r] != want) {
      site.fail(site_key(7, r, 3), RC_INVERSE, r, want, inverse[r]);
      break;
    }
    if (want != DROP && want < routes && permutation[want] != r) {
      site.fail(site_key(7, r, 4), RC_PERMUTATION, want, r, permutation[want]);
      break;
    }
  }
  // phase 8: every accepted slot claimed, its permutation entry consistent;
  // phase 9: the permutation tail holds the drop sentinel
  const uint32_t acc = accepted < routes ? accepted : routes;
  for (uint32_t s = t; s < acc; s += ASSIGN_THREADS) {
    if (claimant[s] == DROP) { site.fail(site_key(8, s, 0), RC_PREFIX_HOLE, s, 0, 0); continue; }
    const uint32_t r = permutation[s];
    if (r >= routes) site.fail(site_key(8, s, 1), RC_PERMUTATION_ROUTE, s, 0, r);
    else if (slots[r] != s || inverse[r] != s) site.fail(site_key(8, s, 2), RC_PERMUTATION, s, r, r);
  }
  for (uint32_t s = acc + t; s < routes; s += ASSIGN_THREADS)
    if (s >= accepted && permutation[s] != DROP)
      site.fail(site_key(9, s, 0), RC_PERMUTATION_TAIL, s, 0, permutation[s]);
  if (site.key != ~0ull) atomicMin(&best, (unsigned long long)site.key);
  __syncthreads();
  if (best == ~0ull) {
    if (t == 0) record[0] = record[1] = record[2] = record[3] = 0;
  } else if (site.key == best) {
    record[0] = site.rec[0];
    record[1] = site.rec[1];
    record[2] = site.rec[2];
    record[3] = site.rec[3];
  }
}

// The same check for more routes than the single workgroup's LDS table
// holds, over workgroups of RA_ROUTES routes (RA_ROUTES / 2 tokens) on
// stream-ordered scratch: the claimed-slot table (one word per slot, first
// filled with DROP), the per-workgroup expert counts and their prefixes
// (route_count_kernel, route_scan_kernel: the stable ranks), and one site
// per workgroup (the key's two words, then the record).  Every site is
// tested as in routing_check_kernel; that kernel stops a thread's route
// range at its first failure or first out-of-range expert, which skips only
// sites of larger keys (an out-of-range expert is itself a phase-1 failure),
// so the smallest failing key, and the record written, are the same.
constexpr uint32_t kSiteWords = 6;
// routes above which fe2o3_moe_routing_check runs these kernels
constexpr uint64_t kCheckWideAbove = 2048;

FE2O3_DEVICE void block_min_site(const Site& site, uint32_t* __restrict__ out) {
  __shared__ unsigned long long best;
  if (threadIdx.x == 0) best = ~0ull;
  __syncthreads();
  if (site.key != ~0ull) atomicMin(&best, (unsigned long long)site.key);
  __syncthreads();
  const uint64_t k = best;
  if (k == ~0ull ? threadIdx.x == 0 : site.key == k) {
    out[0] = (uint32_t)k;
    out[1] = (uint32_t)(k >> 32);
    for (int i = 0; i < 4; ++i) out[2 + i] = k == ~0ull ? 0u : site.rec[i];
  }
}

__global__ void __launch_bounds__(256) check_fill_kernel(uint32_t* __restrict__ claimant,
                                                         uint32_t routes) {
  for (uint32_t s = blockIdx.x * 256u + threadIdx.x; s < routes; s += gridDim.x * 256u)
    claimant[s] = DROP;
}

// phase 1 for the workgroup's tokens, and its routes' slot claims
__global__ void __launch_bounds__(RA_THREADS) check_claim_kernel(
    const uint32_t* __restrict__ top2, const uint32_t* __restrict__ offsets,
    const uint32_t* __restrict__ slots, uint32_t tokens, uint32_t experts,
    uint32_t* __restrict__ claimant, uint32_t* __restrict__ sites) {
  const uint32_t t = threadIdx.x, routes = 2u * tokens;
  Site site;
  const uint32_t tk = blockIdx.x * (uint32_t)(RA_ROUTES / 2) + t;
  if (t < (uint32_t)(RA_ROUTES / 2) && tk < tokens) {
    const uint32_t a = top2[2 * tk], b = top2[2 * tk + 1];
    if (a >= experts) site.fail(site_key(1, tk, 0), RC_EXPERT_OUT_OF_RANGE, 2 * tk, 0, a);
    else if (b >= experts) site.fail(site_key(1, tk, 1), RC_EXPERT_OUT_OF_RANGE, 2 * tk + 1, 0, b);
    else if (a == b) site.fail(site_key(1, tk, 2), RC_DUPLICATE_TOKEN_EXPERT, tk, 0, a);
  }
  const uint32_t accepted = offsets[experts];
  const uint32_t r = blockIdx.x * (uint32_t)RA_ROUTES + t;
  if (r < routes) {
    const uint32_t slot = slots[r];
    if (slot != DROP && slot < accepted && slot < routes) atomicMin(&claimant[slot], r);
  }
  block_min_site(site, sites + (uint64_t)blockIdx.x * kSiteWords);
}

// phases 2-6 (workgroup 0), 7 for the workgroup's routes and 8-9 for its
// slots; the workgroup's site becomes the smaller of this and the claim
// kernel's
__global__ void __launch_bounds__(RA_THREADS) check_verify_kernel(
    const uint32_t* __restrict__ top2, const uint32_t* __restrict__ requested,
    const uint32_t* __restrict__ admitted, const uint32_t* __restrict__ offsets,
    const uint32_t* __restrict__ slots, const uint32_t* __restrict__ permutation,
    const uint32_t* __restrict__ inverse, uint32_t tokens, uint32_t experts, uint32_t capacity,
    const uint32_t* __restrict__ claimant, const uint32_t* __restrict__ prefix,
    const uint32_t* __restrict__ totals, uint32_t* __restrict__ sites) {
  __shared__ uint32_t wave_cnt[RA_WAVES][MAX_EXPERTS];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, routes = 2u * tokens;
  for (uint32_t i = t; i < RA_WAVES * MAX_EXPERTS; i += RA_THREADS) (&wave_cnt[0][0])[i] = 0;
  Site site;
  if (blockIdx.x == 0 && t == 0) {
    for (uint32_t e = 0; e < experts && site.key == ~0ull; ++e)
      if (requested[e] != totals[e]) site.fail(site_key(2, e, 0), RC_REQUESTED_COUNT, e, totals[e], requested[e]);
    for (uint32_t e = 0; e < experts && site.key == ~0ull; ++e) {
      const uint32_t want = requested[e] < capacity ? requested[e] : capacity;
      if (admitted[e] > capacity) site.fail(site_key(3, e, 0), RC_CAPACITY, e, 0, admitted[e]);
      else if (admitted[e] != want) site.fail(site_key(3, e, 1), RC_ADMITTED_COUNT, e, want, admitted[e]);
    }
    if (site.key == ~0ull && offsets[0] != 0) site.fail(site_key(4, 0, 0), RC_FIRST_OFFSET, 0, 0, offsets[0]);
    uint32_t cum = 0;
    for (uint32_t e = 0; e < experts && site.key == ~0ull; ++e) {
      const uint32_t start = offsets[e], end = offsets[e + 1];
      cum += admitted[e];
      if (start > end) site.fail(site_key(5, e, 0), RC_NONMONOTONE_OFFSETS, e, start, end);
      else if (end != cum) site.fail(site_key(5, e, 1), RC_OFFSET_MISMATCH, e + 1, cum, end);
    }
    for (uint32_t e = 0; e < experts && site.key == ~0ull; ++e) {
      const uint32_t start = offsets[e], end = offsets[e + 1];
      if (start > end || end > routes) site.fail(site_key(6, e, 0), RC_PLAN_OFFSET_ORDER, e, 0, end);
      else if (end - start > capacity) site.fail(site_key(6, e, 1), RC_PLAN_CAPACITY, e, 0, end - start);
    }
  }
  __syncthreads();
  // phase 7: stable rank = this expert's routes in earlier workgroups, in
  // earlier waves, in earlier lanes
  const uint32_t r = blockIdx.x * (uint32_t)RA_ROUTES + t;
  uint32_t e = r < routes ? top2[r] : DROP;
  if (e >= experts) e = DROP;  // phase 1 reports it
  uint32_t rank = 0;
  const uint64_t lt = (1ull << lane) - 1ull;
  for_each_expert(e, [&](uint32_t x, uint64_t mask) {
    if (e == x) rank = (uint32_t)__builtin_popcountll(mask & lt);
    if (lane == 0) wave_cnt[wave][x] = (uint32_t)__builtin_popcountll(mask);
  });
  __syncthreads();
  const uint32_t accepted = offsets[experts];
  if (e != DROP) {
    rank += prefix[(uint64_t)blockIdx.x * (experts + 1u) + e];
    for (uint32_t w = 0; w < wave; ++w) rank += wave_cnt[w][e];
    const uint32_t want = rank < capacity ? offsets[e] + rank : DROP;
    const uint32_t slot = slots[r];
    if (slot != DROP && slot >= accepted)
      site.fail(site_key(7, r, 0), RC_SLOT_OUT_OF_RANGE, r, accepted, slot);
    else if (slot != DROP && slot < routes && claimant[slot] < r)
      site.fail(site_key(7, r, 1), RC_DUPLICATE_SLOT, r, 0, slot);
    else if (slot != want)
      site.fail(site_key(7, r, 2), RC_STABLE_SLOT, r, want, slot);
    else if (inverse[r] != want)
      site.fail(site_key(7, r, 3), RC_INVERSE, r, want, inverse[r]);
    else if (want != DROP && want < routes && permutation[want] != r)
      site.fail(site_key(7, r, 4), RC_PERMUTATION, want, r, permutation[want]);
  }
  // phases 8 and 9 for slot s = r
  const uint32_t acc = accepted < routes ? accepted : routes;
  if (r < acc) {
    if (claimant[r] == DROP) {
      site.fail(site_key(8, r, 0), RC_PREFIX_HOLE, r, 0, 0);
    } else {
      const uint32_t q = permutation[r];
      if (q >= routes) site.fail(site_key(8, r, 1), RC_PERMUTATION_ROUTE, r, 0, q);
      else if (slots[q] != r || inverse[q] != r) site.fail(site_key(8, r, 2), RC_PERMUTATION, r, q, q);
    }
  } else if (r < routes && r >= accepted && permutation[r] != DROP) {
    site.fail(site_key(9, r, 0), RC_PERMUTATION_TAIL, r, 0, permutation[r]);
  }
  // the claim kernel's site of this workgroup competes too
  uint32_t* mine = sites + (uint64_t)blockIdx.x * kSiteWords;
  if (t == 0) {
    const uint64_t k0 = (uint64_t)mine[0] | ((uint64_t)mine[1] << 32);
    if (k0 != ~0ull) site.fail(k0, mine[2], mine[3], mine[4], mine[5]);
  }
  __syncthreads();  // every thread has read `mine` before it is rewritten
  block_min_site(site, mine);
}

// the smallest site over the workgroups, as the record (zeros when none)
__global__ void __launch_bounds__(RS_THREADS) check_reduce_kernel(
    const uint32_t* __restrict__ sites, uint32_t blocks, uint32_t* __restrict__ record) {
  Site site;
  for (uint32_t b = threadIdx.x; b < blocks; b += RS_THREADS) {
    const uint32_t* w = sites + (uint64_t)b * kSiteWords;
    const uint64_t k = (uint64_t)w[0] | ((uint64_t)w[1] << 32);
    if (k != ~0ull) site.fail(k, w[2], w[3], w[4], w[5]);
  }
  __shared__ uint32_t out[kSiteWords];
  block_min_site(site, out);
  __syncthreads();
  if (threadIdx.x < 4) record[threadIdx.x] = out[2 + threadIdx.x];
}

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1", "route_select_kernel<float>", (const void*)route_select_kernel<float>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1", "route_assign_kernel", (const void*)route_assign_kernel<false>, RA_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route", "route_select_kernel<float>", (const void*)route_select_kernel<float>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route", "route_select_kernel<uint16_t>", (const void*)route_select_kernel<uint16_t>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route", "route_assign_kernel", (const void*)route_assign_kernel<false>, RA_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route", "route_count_kernel", (const void*)route_count_kernel, RA_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route", "route_scan_kernel", (const void*)route_scan_kernel, RS_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_top2_route", "route_assign_kernel<prefixed>", (const void*)route_assign_kernel<true>, RA_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_expert_combine_f32_t8_k2_o16_v1", "combine_profile_kernel", (const void*)combine_profile_kernel, 128, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2", "gather_kernel", (const void*)gather_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2", "gate_up_kernel", (const void*)gate_up_kernel<true>, 256, kSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2", "gate_up_kernel<gathered>", (const void*)gate_up_kernel<false>, 256, kSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2", "down_kernel", (const void*)down_kernel, 256, kSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2", "combine_kernel", (const void*)combine_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2_noalloc", "gather_kernel", (const void*)gather_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2_noalloc", "gate_up_kernel", (const void*)gate_up_kernel<true>, 256, kSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2_noalloc", "gate_up_kernel<gathered>", (const void*)gate_up_kernel<false>, 256, kSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2_noalloc", "down_kernel", (const void*)down_kernel, 256, kSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_ffn_top2_noalloc", "combine_kernel", (const void*)combine_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_routing_check", "routing_check_kernel", (const void*)routing_check_kernel, ASSIGN_THREADS, CHECK_MAX_ROUTES * 4}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_routing_check", "check_fill_kernel", (const void*)check_fill_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_routing_check", "route_count_kernel", (const void*)route_count_kernel, RA_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_routing_check", "check_claim_kernel", (const void*)check_claim_kernel, RA_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_routing_check", "route_scan_kernel", (const void*)route_scan_kernel, RS_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_routing_check", "check_verify_kernel", (const void*)check_verify_kernel, RA_THREADS, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_routing_check", "check_reduce_kernel", (const void*)check_reduce_kernel, RS_THREADS, 0})};

// The expert FFN's second stream, one per device, created on first use and
// kept for the life of the process (default priority, non-blocking so that it
// also runs beside a caller's null stream).
struct SideStream {
  std::mutex mu;
  hipStream_t stream = nullptr;
  hipEvent_t ready = nullptr, done = nullptr;
  bool ok = false;
};

SideStream* side_stream() {
  static constexpr int kMaxDevices = 64;
  static SideStream sides[kMaxDevices];
  static std::mutex create_mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  SideStream& sd = sides[dev];
  std::lock_guard<std::mutex> lock(create_mu);
  if (!sd.ok) {
    if (hipStreamCreateWithFlags(&sd.stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&sd.ready, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&sd.done, hipEventDisableTiming) != hipSuccess)
      return nullptr;
    sd.ok = true;
  }
  return &sd;
}

}  // namespace

extern "C" {

int32_t fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1(
    const float* logits, uint64_t logits_len, uint32_t* top2_experts, uint64_t top2_len,
    uint32_t* requested_counts, uint64_t requested_len, uint32_t* admitted_counts,
    uint64_t admitted_len, uint32_t* expert_offsets, uint64_t offsets_len, uint32_t* route_slots,
    uint64_t slots_len, uint32_t* permutation, uint64_t permutation_len, uint32_t* inverse,
    uint64_t inverse_len, void* stream) {
  FE2O3_ENTRY("fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1");
  // examples/moe_top2_v1/src/contract.rs:3-29: T=8, E=4, K=2, C=4
  if (logits_len != 32 || top2_len != 16 || requested_len != 4 || admitted_len != 4 ||
      offsets_len != 5 || slots_len != 16 || permutation_len != 16 || inverse_len != 16)
    return FE2O3_ERR_LENGTH;
  return route(logits, logits_len, 0, top2_experts, top2_len, requested_counts, requested_len,
               admitted_counts, admitted_len, expert_offsets, offsets_len, route_slots, slots_len,
               permutation, permutation_len, inverse, inverse_len, nullptr, 0, 8, 4, 4, stream);
}

int32_t fe2o3_moe_top2_route(const void* logits, uint64_t logits_len, uint32_t logits_dtype,
                             uint32_t* top2_experts, uint64_t top2_len, uint32_t* requested_counts,
                             uint64_t requested_len, uint32_t* admitted_counts,
                             uint64_t admitted_len, uint32_t* expert_offsets, uint64_t offsets_len,
                             uint32_t* route_slots, uint64_t slots_len, uint32_t* permutation,
                             uint64_t permutation_len, uint32_t* inverse, uint64_t inverse_len,
                             float* route_weights, uint64_t weights_len, uint32_t tokens,
                             uint32_t experts, uint32_t capacity, void* stream) {
  FE2O3_ENTRY("fe2o3_moe_top2_route");
  return route(logits, logits_len, logits_dtype, top2_experts, top2_len, requested_counts,
               requested_len, admitted_counts, admitted_len, expert_offsets, offsets_len,
               route_slots, slots_len, permutation, permutation_len, inverse, inverse_len,
               route_weights, weights_len, tokens, experts, capacity, stream);
}

int32_t fe2o3_moe_expert_combine_f32_t8_k2_o16_v1(const float* compact_output,
                                                  uint64_t compact_len, const uint32_t* inverse,
                                                  uint64_t inverse_len,
                                                  const float* route_weights, uint64_t weights_len,
                                                  float* combined_output, uint64_t combined_len,
                                                  void* stream) {
  FE2O3_ENTRY("fe2o3_moe_expert_combine_f32_t8_k2_o16_v1");
  if (compact_len != 256 || inverse_len != 16 || weights_len != 16 || combined_len != 128)
    return FE2O3_ERR_LENGTH;
  if (!compact_output || !inverse || !route_weights || !combined_output) return FE2O3_ERR_NULL;
  combine_profile_kernel<<<1, 128, 0, (hipStream_t)stream>>>(compact_output, inverse,
                                                            route_weights, combined_output);
  return fe2o3_host::after_launch();
}

uint64_t fe2o3_moe_ffn_workspace_bytes(uint32_t tokens, uint32_t hidden, uint32_t ffn,
                                       uint32_t experts) {
  (void)experts;
  return carve(nullptr, tokens, hidden, ffn).bytes;
}

}  // extern "C"

namespace {

// K parts of the down GEMM: 2 (two half-K tiles per output tile, two fp32
// partials) only when that fills the grid's rounds of `cus` tiles better
// than whole-K tiles, each of which counts two half-K rounds.  The m-tile
// count is that of an even routing (experts x expert_m_tiles(routes /
// experts)); routing is device data, and the choice only affects speed.
// Measured in one process (whole K against split K; balanced routings of n
// rows per expert, 8 experts, hidden 4096, FFN 14336): n = 100 +21%,
// 270 +18%, 600 +4% (split kept), n = 300 -1.6%, 1040 -4.1%, 1100 -4.1%,
// 1150 -3.4%, config 5 -3.9% (whole K chosen).
uint32_t down_k_parts(uint64_t routes, uint32_t experts, uint32_t hidden, uint32_t cus) {
  const uint64_t per = (routes + experts - 1u) / experts;
  const uint64_t m = (uint64_t)experts * expert_m_tiles((uint32_t)per);
  const uint64_t t1 = m * (hidden / 256u);  // whole-K tiles
  const uint64_t rounds1 = (t1 + cus - 1u) / cus, rounds2 = (2u * t1 + cus - 1u) / cus;
  return 2u * rounds1 <= rounds2 ? 1u : 2u;
}

// The expert FFN behind both C-ABI entry points.  `split_streams` runs the
// second half of the experts on the per-device side stream (created on
// first use); without it every kernel runs on the caller's stream and the
// call creates nothing.
int32_t ffn_top2(const uint16_t* x, uint64_t x_len, const uint16_t* w_gate, uint64_t w_gate_len,
                 const uint16_t* w_up, uint64_t w_up_len, const uint16_t* w_down,
                 uint64_t w_down_len, uint64_t top2_len, const uint32_t* expert_offsets,
                 uint64_t offsets_len, const uint32_t* permutation, uint64_t permutation_len,
                 const uint32_t* inverse, uint64_t inverse_len, const float* route_weights,
                 uint64_t weights_len, uint16_t* out, uint64_t out_len, void* workspace,
                 uint64_t workspace_bytes, uint32_t tokens, uint32_t hidden, uint32_t ffn,
                 uint32_t experts, bool split_streams, void* stream) {
  if (experts < 1 || experts > MAX_EXPERTS) return FE2O3_ERR_SHAPE;
  // hidden: 256-column output blocks of the down GEMM; ffn: 128-wide gate/up
  // blocks, and each k-half of the down GEMM a whole number of 64-k stages
  if (hidden == 0 || ffn == 0 || hidden % 256 != 0 || ffn % 128 != 0) return FE2O3_ERR_SHAPE;
  const uint64_t routes = 2ull * tokens;
  const uint64_t wsz = (uint64_t)experts * ffn * hidden;
  if (x_len != (uint64_t)tokens * hidden || w_gate_len != wsz || w_up_len != wsz ||
      w_down_len != wsz || top2_len != routes || offsets_len != experts + 1ull ||
      permutation_len != routes || inverse_len != routes || weights_len != routes ||
      out_len != (uint64_t)tokens * hidden)
    return FE2O3_ERR_LENGTH;
  // operand panels of up to 288 rows and one expert's gate/up matrix must
  // fit the 32-bit range of a buffer resource
  if (2ull * kMaxTileRows * ffn >= (1ull << 31) || 2ull * kMaxTileRows * hidden >= (1ull << 31) ||
      2ull * ffn * hidden >= (1ull << 31))
    return FE2O3_ERR_SHAPE;
  if (tokens == 0) return FE2O3_OK;
  const Workspace ws = carve(workspace, tokens, hidden, ffn);
  if (workspace_bytes < ws.bytes) return FE2O3_ERR_WORKSPACE;
  if (!x || !w_gate || !w_up || !w_down || !expert_offsets || !permutation || !inverse ||
      !route_weights || !out || !workspace)
    return FE2O3_ERR_NULL;
  if ((((uintptr_t)x | (uintptr_t)w_gate | (uintptr_t)w_up | (uintptr_t)w_down |
        (uintptr_t)out | (uintptr_t)workspace) & 15u) != 0)
    return FE2O3_ERR_ALIGNMENT;
  static const int32_t lds_rc = fe2o3_host::set_dynamic_lds(
      {(const void*)gate_up_kernel<true>, (const void*)gate_up_kernel<false>,
       (const void*)down_kernel},
      kSmem);
  if (lds_rc != FE2O3_OK) return lds_rc;
  hipStream_t s = (hipStream_t)stream;
  // the most m-tiles any routing yields for experts [b, e): routes/288
  // rounded up, plus one partial tile per expert
  tile_plan::Topology topo;
  const int32_t topo_rc = fe2o3_host::device_topology(&topo);
  if (topo_rc != FE2O3_OK) return topo_rc;
  const uint32_t xcds = topo.xcds;
  const uint32_t kparts = down_k_parts(routes, experts, hidden, topo.cus);
  auto grids = [&](uint32_t n_experts, uint64_t* gu, uint64_t* dn) {
    *gu = expert_grid(routes, n_experts, ffn / 128u, xcds);
    *dn = expert_grid(routes, n_experts, kparts * (hidden / 256u), xcds);
    return *gu <= 0x7fffffffu && *dn <= 0x7fffffffu;
  };
  // The gate/up tiles read the token rows in place, through the permutation,
  // when x fits the 32-bit range of a buffer resource; otherwise from rows
  // gathered into the workspace first.
  const uint64_t x_bytes = (uint64_t)tokens * hidden * 2u;
  const bool tokens_direct = x_bytes < (1ull << 31);
  auto experts_ffn = [&](uint32_t b, uint32_t e, hipStream_t st) {
    uint64_t gu, dn;
    grids(e - b, &gu, &dn);
    if (tokens_direct)
      gate_up_kernel<true><<<(unsigned)gu, 256, kSmem, st>>>(
          x, (uint32_t)x_bytes, permutation, w_gate, w_up, expert_offsets, b, e, hidden, ffn,
          (uint32_t)routes, ws.hc, xcds);
    else
      gate_up_kernel<false><<<(unsigned)gu, 256, kSmem, st>>>(
          ws.xc, 0u, permutation, w_gate, w_up, expert_offsets, b, e, hidden, ffn,
          (uint32_t)routes, ws.hc, xcds);
    down_kernel<<<(unsigned)dn, 256, kSmem, st>>>(ws.hc, w_down, expert_offsets, b, e, hidden,
                                                  ffn, routes, kparts, ws.yc, xcds);
  };
  uint64_t gu_all, dn_all;
  if (!grids(experts, &gu_all, &dn_all)) return FE2O3_ERR_SHAPE;
  if (!tokens_direct)
    gather_kernel<<<(unsigned)routes, 256, 0, s>>>(x, permutation, expert_offsets, experts, hidden,
                                                  (uint32_t)routes, ws.xc);
  // Two halves of the experts, each gate/up then down, on the caller's
  // stream and on a side stream: each grouped GEMM ends in a partly filled
  // round of tiles, which the other half's tiles fill.
  SideStream* side = split_streams && experts >= 2 ? side_stream() : nullptr;
  if (side != nullptr) {
    std::lock_guard<std::mutex> lock(side->mu);  // keeps one call's event waits its own
    const uint32_t half = experts / 2u;
    hipError_t e = hipEventRecord(side->ready, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(side->stream, side->ready, 0);
    if (e != hipSuccess) return (int32_t)e;
    experts_ffn(0u, half, s);
    experts_ffn(half, experts, side->stream);
    e = hipEventRecord(side->done, side->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, side->done, 0);
    if (e != hipSuccess) return (int32_t)e;
  } else {
    experts_ffn(0u, experts, s);
  }
  const uint64_t threads = (uint64_t)tokens * (hidden / 4u);
  combine_kernel<<<(unsigned)((threads + 255u) / 256u), 256, 0, s>>>(ws.yc, inverse, route_weights,
                                                                    tokens, hidden, routes, kparts,
                                                                    out);
  return fe2o3_host::after_launch();
}

// Scratch of the allocation-free FFN entry point: a file-scope device array,
// one copy per device, held from library load to process end.  Host code
// uses only the address hipGetSymbolAddress returns for the current device
// (the array's name on the host is a stand-in, not a device address).
constexpr uint64_t kNoAllocScratchBytes = FE2O3_MOE_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

void* noalloc_scratch() {
  static constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace

extern "C" {

int32_t fe2o3_moe_ffn_top2(const uint16_t* x, uint64_t x_len, const uint16_t* w_gate,
                           uint64_t w_gate_len, const uint16_t* w_up, uint64_t w_up_len,
                           const uint16_t* w_down, uint64_t w_down_len,
                           const uint32_t* top2_experts, uint64_t top2_len,
                           const uint32_t* expert_offsets, uint64_t offsets_len,
                           const uint32_t* permutation, uint64_t permutation_len,
                           const uint32_t* inverse, uint64_t inverse_len,
                           const float* route_weights, uint64_t weights_len, uint16_t* out,
                           uint64_t out_len, void* workspace, uint64_t workspace_bytes,
                           uint32_t tokens, uint32_t hidden, uint32_t ffn, uint32_t experts,
                           void* stream) {
  FE2O3_ENTRY("fe2o3_moe_ffn_top2");
  (void)top2_experts;
  return ffn_top2(x, x_len, w_gate, w_gate_len, w_up, w_up_len, w_down, w_down_len, top2_len,
                  expert_offsets, offsets_len, permutation, permutation_len, inverse, inverse_len,
                  route_weights, weights_len, out, out_len, workspace, workspace_bytes, tokens,
                  hidden, ffn, experts, true, stream);
}

int32_t fe2o3_moe_ffn_top2_noalloc(const uint16_t* x, uint64_t x_len, const uint16_t* w_gate,
                                   uint64_t w_gate_len, const uint16_t* w_up, uint64_t w_up_len,
                                   const uint16_t* w_down, uint64_t w_down_len,
                                   const uint32_t* top2_experts, uint64_t top2_len,
                                   const uint32_t* expert_offsets, uint64_t offsets_len,
                                   const uint32_t* permutation, uint64_t permutation_len,
                                   const uint32_t* inverse, uint64_t inverse_len,
                                   const float* route_weights, uint64_t weights_len,
                                   uint16_t* out, uint64_t out_len, uint32_t tokens,
                                   uint32_t hidden, uint32_t ffn, uint32_t experts,
                                   void* stream) {
  FE2O3_ENTRY("fe2o3_moe_ffn_top2_noalloc");
  (void)top2_experts;
  if (fe2o3_moe_ffn_workspace_bytes(tokens, hidden, ffn, experts) > kNoAllocScratchBytes)
    return FE2O3_ERR_WORKSPACE;
  void* ws = noalloc_scratch();
  if (ws == nullptr) return (int32_t)hipErrorInvalidSymbol;
  return ffn_top2(x, x_len, w_gate, w_gate_len, w_up, w_up_len, w_down, w_down_len, top2_len,
                  expert_offsets, offsets_len, permutation, permutation_len, inverse, inverse_len,
                  route_weights, weights_len, out, out_len, ws, kNoAllocScratchBytes, tokens,
                  hidden, ffn, experts, false, stream);
}

int32_t fe2o3_moe_routing_check(const uint32_t* top2_experts, uint64_t top2_len,
                                const uint32_t* requested_counts, uint64_t requested_len,
                                const uint32_t* admitted_counts, uint64_t admitted_len,
                                const uint32_t* expert_offsets, uint64_t offsets_len,
                                const uint32_t* route_slots, uint64_t slots_len,
                                const uint32_t* permutation, uint64_t permutation_len,
                                const uint32_t* inverse, uint64_t inverse_len, uint32_t tokens,
                                uint32_t experts, uint32_t capacity, uint32_t* record,
                                uint64_t record_len, void* stream) {
  FE2O3_ENTRY("fe2o3_moe_routing_check");
  if (experts < 1 || experts > MAX_EXPERTS) return FE2O3_ERR_SHAPE;
  const uint64_t routes = 2ull * tokens;
  if (routes > 0xFFFFFFFEull) return FE2O3_ERR_SHAPE;
  if (top2_len != routes || slots_len != routes || permutation_len != routes ||
      inverse_len != routes || requested_len != experts || admitted_len != experts ||
      offsets_len != experts + 1ull || record_len != 4)
    return FE2O3_ERR_LENGTH;
  if (!requested_counts || !admitted_counts || !expert_offsets || !record ||
      (routes && (!top2_experts || !route_slots || !permutation || !inverse)))
    return FE2O3_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  // Above kCheckWideAbove routes the workgroups of 256 tokens (35-50 us at
  // config 5, against 119 for one workgroup); without scratch on this
  // device, one workgroup as long as its claimed-slot table fits LDS.
  void* scratch = nullptr;
  const uint32_t blocks = (uint32_t)((routes + RA_ROUTES - 1) / RA_ROUTES);
  const uint64_t count_words = (uint64_t)blocks * (experts + 1u);
  int32_t alloc_rc = FE2O3_OK;
  if (routes > kCheckWideAbove) {
    alloc_rc = fe2o3_host::scratch_alloc(
        &scratch, (routes + count_words + experts + 1u + (uint64_t)blocks * kSiteWords) * 4u, s);
    if (alloc_rc != FE2O3_OK) {
      (void)hipGetLastError();
      if (routes > CHECK_MAX_ROUTES) return alloc_rc;
    }
  }
  if (alloc_rc == FE2O3_OK && scratch != nullptr) {
    uint32_t* claimant = static_cast<uint32_t*>(scratch);
    uint32_t* counts = claimant + routes;
    uint32_t* totals = counts + count_words;
    uint32_t* sites = totals + experts + 1u;
    const uint32_t fill_blocks = (uint32_t)std::min<uint64_t>((routes + 255u) / 256u, 8192u);
    check_fill_kernel<<<fill_blocks, 256, 0, s>>>(claimant, (uint32_t)routes);
    route_count_kernel<<<blocks, RA_THREADS, 0, s>>>(top2_experts, (uint32_t)routes, experts,
                                                     counts);
    check_claim_kernel<<<blocks, RA_THREADS, 0, s>>>(top2_experts, expert_offsets, route_slots,
                                                     tokens, experts, claimant, sites);
    route_scan_kernel<<<1, RS_THREADS, 0, s>>>(counts, blocks, experts, totals);
    check_verify_kernel<<<blocks, RA_THREADS, 0, s>>>(
        top2_experts, requested_counts, admitted_counts, expert_offsets, route_slots, permutation,
        inverse, tokens, experts, capacity, claimant, counts, totals, sites);
    check_reduce_kernel<<<1, RS_THREADS, 0, s>>>(sites, blocks, record);
    const int32_t rc = fe2o3_host::after_launch();
    const int32_t free_rc = fe2o3_host::scratch_free(scratch, s);
    return rc != FE2O3_OK ? rc : free_rc;
  }
  const size_t lds = (size_t)(routes ? routes : 1) * sizeof(uint32_t);
  static const int32_t lds_rc = fe2o3_host::set_dynamic_lds(
      {(const void*)routing_check_kernel}, (int)(CHECK_MAX_ROUTES * sizeof(uint32_t)));
  if (lds_rc != FE2O3_OK) return lds_rc;
  routing_check_kernel<<<1, ASSIGN_THREADS, lds, s>>>(
      top2_experts, requested_counts, admitted_counts, expert_offsets, route_slots, permutation,
      inverse, tokens, experts, capacity, record);
  return fe2o3_host::after_launch();
}

}  // extern "C"
