// profiles.hpp -- the arithmetic of the reference's exact one-wave profiles,
// shared by the library's entry points and the standalone code objects that
// the protected lifecycles load (codeobj/*.hip), so both run the same
// instructions on the same data.
//
// Each routine runs in one wave of 64 lanes.  `status` is the device's
// non-finite counter (mark_nonfinite); a code object has none and passes
// nullptr, and then only the documented sentinel outputs mark the rejection.
#pragma once

#include "common.hpp"

namespace fe2o3_profiles {

using namespace fe2o3;

// ---- flash attention: causal, B1/H1/N8/D16, f32, scale 0.25 ------------------------------
// examples/flash_attention_v1/src/kernel.rs:36-169.  Lane l owns outputs 2l
// and 2l+1 (row (2l)/16, columns (2l)%16 and +1): a sequential strict-f32
// dot product per key and the online recurrence m' = max(m, s);
// w_prev = exp(m - m'); w = exp(s - m'); l = l*w_prev + w;
// n = n*w_prev + v*w (kernel.rs:56-113), exp = OCML expf.  A NaN or an
// infinity anywhere in Q, K or V rejects the whole launch as the
// reference's trap does (kernel.rs:143-146): every output is quiet NaN.
constexpr int kFlashN = 8, kFlashD = 16;

FE2O3_DEVICE void flash_profile(const float* __restrict__ q, const float* __restrict__ k,
                                const float* __restrict__ v, float* __restrict__ out,
                                uint32_t* status) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int first = lane * 2;
  const int row = first / kFlashD, col = first % kFlashD;
  float probe = 0.0f;
  for (int i = first; i < first + 2; ++i)
    probe = finite_probe(finite_probe(finite_probe(probe, q[i]), k[i]), v[i]);
  if (__ballot(probe != probe) != 0ull) {
    if (lane == 0 && status != nullptr) mark_nonfinite(status);
    out[first] = quiet_nan();
    out[first + 1] = quiet_nan();
    return;
  }
  float m = 0.0f, l = 0.0f, n0 = 0.0f, n1 = 0.0f;
  for (int kr = 0; kr <= row; ++kr) {
    float dot = 0.0f;
    for (int f = 0; f < kFlashD; ++f) {
      const float p = q[row * kFlashD + f] * k[kr * kFlashD + f];
      dot = dot + p;
    }
    const float s = dot * 0.25f;
    const float v0 = v[kr * kFlashD + col], v1 = v[kr * kFlashD + col + 1];
    if (kr == 0) {
      m = s;
      l = 1.0f;
      n0 = v0;
      n1 = v1;
    } else {
      const float nm = s > m ? s : m;
      const float wp = expf(m - nm);
      const float wc = expf(s - nm);
      const float t0 = l * wp;
      l = t0 + wc;
      const float a0 = n0 * wp, b0 = v0 * wc;
      n0 = a0 + b0;
      const float a1 = n1 * wp, b1 = v1 * wc;
      n1 = a1 + b1;
      m = nm;
    }
  }
  out[first] = n0 / l;
  out[first + 1] = n1 / l;
}

// ---- row softmax: one row of `cols` f32 per wave ------------------------------------------
// examples/row_softmax_v1/src/kernel.rs:13-42 (max, sum of exp(x - max),
// exp(x - max) / sum) with the row spread over the wave: lane l takes
// columns l, l + 64, ...; max and sum are wave reductions; exp is OCML
// expf.  `mask` (may be null): a column whose byte is 0 is inactive
// (numerical_contract.rs:130-199): it takes no part and its output is 0; a
// row with no active column is all 0.  A non-finite input anywhere in the
// row makes every output of the row quiet NaN.
FE2O3_DEVICE void softmax_row(const float* __restrict__ x, float* __restrict__ y,
                              const uint8_t* __restrict__ m, uint64_t cols, uint32_t* status) {
  const uint32_t lane = threadIdx.x & 63u;
  float mx = -INFINITY, probe = 0.0f;
  for (uint64_t c = lane; c < cols; c += 64) {
    probe = finite_probe(probe, x[c]);
    if (!m || m[c]) mx = fmaxf(mx, x[c]);
  }
  if (__ballot(probe != probe) != 0ull) {
    if (lane == 0 && status != nullptr) mark_nonfinite(status);
    for (uint64_t c = lane; c < cols; c += 64) y[c] = quiet_nan();
    return;
  }
  mx = wave_max(mx);
  float sum = 0.0f;
  for (uint64_t c = lane; c < cols; c += 64)
    if (!m || m[c]) sum += expf(x[c] - mx);
  sum = wave_sum(sum);
  const bool any = mx != -INFINITY;
  for (uint64_t c = lane; c < cols; c += 64)
    y[c] = (any && (!m || m[c])) ? expf(x[c] - mx) / sum : 0.0f;
}

// ---- top-2 routing: T = 8 tokens, E = 4 experts, capacity 4 ------------------------------
// examples/moe_top2_v1/src/kernel.rs:25-205, run by lane 0 of the wave (the
// grid leader) in the reference's order: per token the two best experts
// (higher logit first, an equal logit to the lower expert id); requested
// counts; admitted = min(requested, capacity); offsets = exclusive scan with
// the terminal total; then routes in order take slot offsets[e] + rank
// while their expert's rank is below capacity, else the DROP sentinel.  A
// non-finite logit rejects the launch with the library router's sentinels:
// top2, slots, permutation and inverse DROP; requested, admitted and
// offsets 0.
constexpr uint32_t kRouteTokens = 8, kRouteExperts = 4, kRouteCapacity = 4;
constexpr uint32_t kRoutes = 2 * kRouteTokens;
constexpr uint32_t kDropRoute = 0xffffffffu;

// outputs: top2 [16], requested [4], admitted [4], offsets [5], slots [16],
// permutation [16], inverse [16]
FE2O3_DEVICE void route_t8_e4(const float* __restrict__ logits, uint32_t* __restrict__ top2,
                              uint32_t* __restrict__ requested, uint32_t* __restrict__ admitted,
                              uint32_t* __restrict__ offsets, uint32_t* __restrict__ slots,
                              uint32_t* __restrict__ permutation, uint32_t* __restrict__ inverse,
                              uint32_t* status) {
  if ((threadIdx.x & 63u) != 0u) return;
  bool finite = true;
  for (uint32_t i = 0; i < kRouteTokens * kRouteExperts; ++i)
    finite = finite && __builtin_isfinite(logits[i]);
  if (!finite) {
    if (status != nullptr) mark_nonfinite(status);
    for (uint32_t i = 0; i < kRoutes; ++i)
      top2[i] = slots[i] = permutation[i] = inverse[i] = kDropRoute;
    for (uint32_t e = 0; e < kRouteExperts; ++e) requested[e] = admitted[e] = 0;
    for (uint32_t e = 0; e <= kRouteExperts; ++e) offsets[e] = 0;
    return;
  }
  uint32_t sel[kRoutes], req[kRouteExperts] = {}, adm[kRouteExperts], off[kRouteExperts + 1];
  for (uint32_t t = 0; t < kRouteTokens; ++t) {
    const float* row = logits + t * kRouteExperts;
    // best: a later expert replaces the current only with a strictly higher
    // logit, so an equal logit keeps the lower id
    uint32_t b0 = 0;
    for (uint32_t e = 1; e < kRouteExperts; ++e)
      if (row[e] > row[b0]) b0 = e;
    uint32_t b1 = b0 == 0 ? 1u : 0u;
    for (uint32_t e = 0; e < kRouteExperts; ++e)
      if (e != b0 && row[e] > row[b1]) b1 = e;
    sel[2 * t] = b0;
    sel[2 * t + 1] = b1;
    ++req[b0];
    ++req[b1];
  }
  off[0] = 0;
  for (uint32_t e = 0; e < kRouteExperts; ++e) {
    adm[e] = req[e] > kRouteCapacity ? kRouteCapacity : req[e];
    off[e + 1] = off[e] + adm[e];
  }
  uint32_t slot_of[kRoutes], perm[kRoutes], seen[kRouteExperts] = {};
  for (uint32_t r = 0; r < kRoutes; ++r) slot_of[r] = perm[r] = kDropRoute;
  for (uint32_t r = 0; r < kRoutes; ++r) {
    const uint32_t e = sel[r];
    const uint32_t rank = seen[e]++;
    if (rank < kRouteCapacity) {
      const uint32_t s = off[e] + rank;
      slot_of[r] = s;
      perm[s] = r;
    }
  }
  for (uint32_t r = 0; r < kRoutes; ++r) {
    top2[r] = sel[r];
    slots[r] = slot_of[r];
    permutation[r] = perm[r];
    inverse[r] = slot_of[r];
  }
  for (uint32_t e = 0; e < kRouteExperts; ++e) {
    requested[e] = req[e];
    admitted[e] = adm[e];
    offsets[e] = off[e];
  }
  offsets[kRouteExperts] = off[kRouteExperts];
}

}  // namespace fe2o3_profiles
