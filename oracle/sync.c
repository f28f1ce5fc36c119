/*
 * sync.c -- CPU restatement of the reference's wave64 collectives and
 * workgroup-synchronization oracles, and of the host consistency check over
 * a complete top-2 routing output (the routing -> expert bridge),
 * generalised from the fixed T8/E4/C4 profile to any token count, expert
 * count and capacity.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "fe2o3_oracle.h"

/* ---- wave64 collectives ------------------------------------------------------------------ */

/* examples/wave64_collectives_v1/src/oracle.rs:138-194 (compute_outputs):
 * contributions (+0 for inactive lanes), six XOR butterfly rounds over the
 * complete previous vector, six Hillis-Steele rounds (lane >= d adds lane
 * l - d), exclusive = inclusive of lane l - 1 (+0 in lane 0); inactive lanes
 * publish +0. */
void fe2o3o_wave64_collectives_compute(const float *input, uint64_t mask, float *reduction,
                                       float *inclusive, float *exclusive) {
  float c[64], red[64], inc[64], prev[64];
  for (int l = 0; l < 64; ++l) c[l] = ((mask >> l) & 1u) ? input[l] : 0.0f;
  memcpy(red, c, sizeof c);
  for (int d = 1; d < 64; d <<= 1) {
    memcpy(prev, red, sizeof prev);
    for (int l = 0; l < 64; ++l) red[l] = prev[l] + prev[l ^ d];
  }
  memcpy(inc, c, sizeof c);
  for (int d = 1; d < 64; d <<= 1) {
    memcpy(prev, inc, sizeof prev);
    for (int l = d; l < 64; ++l) inc[l] = prev[l] + prev[l - d];
  }
  for (int l = 0; l < 64; ++l) {
    const int active = (int)((mask >> l) & 1u);
    const float ex = l == 0 ? 0.0f : inc[l - 1];
    reduction[l] = active ? red[l] : 0.0f;
    inclusive[l] = active ? inc[l] : 0.0f;
    exclusive[l] = active ? ex : 0.0f;
  }
}

/* examples/wave64_collectives_v1/src/oracle.rs:106-136, 197-219: every input
 * must be finite (ERR_NONFINITE) and integral in [-1024, 1024]
 * (ERR_ALPHABET, the exact corpus); outputs untouched on rejection. */
int32_t fe2o3o_wave64_collectives_v1(const float *input, uint64_t mask, float *reduction,
                                     float *inclusive, float *exclusive) {
  for (int l = 0; l < 64; ++l) {
    if (!isfinite(input[l])) return FE2O3O_ERR_NONFINITE;
    if (input[l] != truncf(input[l]) || fabsf(input[l]) > 1024.0f) return FE2O3O_ERR_ALPHABET;
  }
  fe2o3o_wave64_collectives_compute(input, mask, reduction, inclusive, exclusive);
  return FE2O3O_OK;
}

/* ---- workgroup synchronization ----------------------------------------------------------- */

/* examples/workgroup_sync_v1/src/contract.rs:192-283 (lds_reduction_oracle_v1):
 * the exact mathematical sum of the 64 values, rejected (ERR_OVERFLOW) when
 * it does not fit int32; output untouched on rejection. */
int32_t fe2o3o_lds_reduce_i32_v1(const int32_t *values, int32_t *output) {
  int64_t sum = 0;
  for (int l = 0; l < 64; ++l) sum += values[l];
  if (sum < INT32_MIN || sum > INT32_MAX) return FE2O3O_ERR_OVERFLOW;
  output[0] = (int32_t)sum;
  return FE2O3O_OK;
}

/* examples/workgroup_sync_v1/src/contract.rs:421-481 (atomic_add_oracle_v1):
 * initial + the values of eligible lanes, exact, rejected (ERR_OVERFLOW)
 * beyond uint32. */
int32_t fe2o3o_atomic_add_u32_v1(uint32_t initial, const uint32_t *values,
                                 const uint32_t *eligible, uint32_t *result) {
  uint64_t sum = initial;
  for (int l = 0; l < 64; ++l)
    if (eligible[l]) sum += values[l];
  if (sum > UINT32_MAX) return FE2O3O_ERR_OVERFLOW;
  result[0] = (uint32_t)sum;
  return FE2O3O_OK;
}

/* ---- routing output consistency --------------------------------------------------------- */

/* crates/fe2o3-host/src/moe_routing_expert_bridge_v1.rs:220-389
 * (check_host_observed_moe_routing_output_v1) and
 * crates/fe2o3-host/src/generated_moe_expert_v1.rs:159-190 (the compact pack
 * plan), for T tokens, E experts and capacity C: the first failing relation
 * in the reference's order is written to record[0..3] = {kind, index,
 * expected, actual}; kind 0 = consistent.  Kinds and fields are listed in
 * fe2o3_oracle.h. */
static void put(uint32_t *rec, uint32_t kind, uint32_t index, uint32_t expected,
                uint32_t actual) {
  rec[0] = kind;
  rec[1] = index;
  rec[2] = expected;
  rec[3] = actual;
}

int32_t fe2o3o_moe_routing_check(const uint32_t *top2, const uint32_t *requested,
                                 const uint32_t *admitted, const uint32_t *offsets,
                                 const uint32_t *slots, const uint32_t *permutation,
                                 const uint32_t *inverse, uint32_t tokens, uint32_t experts,
                                 uint32_t capacity, uint32_t *record) {
  const uint32_t routes = 2u * tokens;
  uint32_t *count = calloc(experts, sizeof(uint32_t));
  uint8_t *seen = calloc(routes ? routes : 1, 1);
  if (!count || !seen) {
    free(count);
    free(seen);
    return FE2O3O_ERR_TOO_LARGE;
  }
  put(record, FE2O3O_RC_OK, 0, 0, 0);
  /* top-2 ids in range and distinct per token; requested counts */
  for (uint32_t t = 0; t < tokens; ++t) {
    const uint32_t a = top2[2 * t], b = top2[2 * t + 1];
    if (a >= experts) { put(record, FE2O3O_RC_EXPERT_OUT_OF_RANGE, 2 * t, 0, a); goto done; }
    count[a]++;
    if (b >= experts) { put(record, FE2O3O_RC_EXPERT_OUT_OF_RANGE, 2 * t + 1, 0, b); goto done; }
    count[b]++;
    if (a == b) { put(record, FE2O3O_RC_DUPLICATE_TOKEN_EXPERT, t, 0, a); goto done; }
  }
  for (uint32_t e = 0; e < experts; ++e)
    if (requested[e] != count[e]) {
      put(record, FE2O3O_RC_REQUESTED_COUNT, e, count[e], requested[e]);
      goto done;
    }
  for (uint32_t e = 0; e < experts; ++e) {
    if (admitted[e] > capacity) { put(record, FE2O3O_RC_CAPACITY, e, 0, admitted[e]); goto done; }
    const uint32_t want = requested[e] < capacity ? requested[e] : capacity;
    if (admitted[e] != want) { put(record, FE2O3O_RC_ADMITTED_COUNT, e, want, admitted[e]); goto done; }
  }
  if (offsets[0] != 0) { put(record, FE2O3O_RC_FIRST_OFFSET, 0, 0, offsets[0]); goto done; }
  {
    uint32_t cum = 0;
    for (uint32_t e = 0; e < experts; ++e) {
      const uint32_t start = offsets[e], end = offsets[e + 1];
      if (start > end) { put(record, FE2O3O_RC_NONMONOTONE_OFFSETS, e, start, end); goto done; }
      cum += admitted[e];
      if (end != cum) { put(record, FE2O3O_RC_OFFSET_MISMATCH, e + 1, cum, end); goto done; }
    }
  }
  /* compact pack plan (generated_moe_expert_v1.rs:159-190) */
  for (uint32_t e = 0; e < experts; ++e) {
    const uint32_t start = offsets[e], end = offsets[e + 1];
    if (start > end || end > routes) { put(record, FE2O3O_RC_PLAN_OFFSET_ORDER, e, 0, end); goto done; }
    if (end - start > capacity) { put(record, FE2O3O_RC_PLAN_CAPACITY, e, 0, end - start); goto done; }
  }
  {
    const uint32_t accepted = offsets[experts];
    memset(count, 0, experts * sizeof(uint32_t)); /* stable ranks */
    for (uint32_t r = 0; r < routes; ++r) {
      const uint32_t e = top2[r];
      const uint32_t rank = count[e]++;
      const uint32_t want = rank < capacity ? offsets[e] + rank : FE2O3O_DROP_ROUTE;
      const uint32_t slot = slots[r];
      if (slot != FE2O3O_DROP_ROUTE && slot >= accepted) {
        put(record, FE2O3O_RC_SLOT_OUT_OF_RANGE, r, accepted, slot);
        goto done;
      }
      if (slot != FE2O3O_DROP_ROUTE) {
        if (seen[slot]) { put(record, FE2O3O_RC_DUPLICATE_SLOT, r, 0, slot); goto done; }
        seen[slot] = 1;
      }
      if (slot != want) { put(record, FE2O3O_RC_STABLE_SLOT, r, want, slot); goto done; }
      if (inverse[r] != want) { put(record, FE2O3O_RC_INVERSE, r, want, inverse[r]); goto done; }
      if (want != FE2O3O_DROP_ROUTE && permutation[want] != r) {
        put(record, FE2O3O_RC_PERMUTATION, want, r, permutation[want]);
        goto done;
      }
    }
    for (uint32_t s = 0; s < accepted; ++s) {
      if (!seen[s]) { put(record, FE2O3O_RC_PREFIX_HOLE, s, 0, 0); goto done; }
      const uint32_t r = permutation[s];
      if (r >= routes) { put(record, FE2O3O_RC_PERMUTATION_ROUTE, s, 0, r); goto done; }
      if (slots[r] != s || inverse[r] != s) { put(record, FE2O3O_RC_PERMUTATION, s, r, r); goto done; }
    }
    for (uint32_t s = accepted; s < routes; ++s)
      if (permutation[s] != FE2O3O_DROP_ROUTE) {
        put(record, FE2O3O_RC_PERMUTATION_TAIL, s, 0, permutation[s]);
        goto done;
      }
  }
done:
  free(count);
  free(seen);
  return FE2O3O_OK;
}
