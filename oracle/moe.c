/*
 * moe.c -- CPU restatement of the reference's top-2 router and expert
 * pipeline oracles, generalised from the fixed T8/E4/K2/C4 profile to any
 * token count, expert count and capacity; plus the SiLU expert FFN of the
 * scaled-up configuration.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "fe2o3_oracle.h"

/* examples/moe_top2_v1/src/oracle.rs:63-82: sort experts by descending score,
 * equal scores by ascending id.  Insertion sort is stable and uses exactly
 * this comparator, so it reproduces the reference's sort_by result. */
static void independent_top2(const float *row, uint32_t experts, uint32_t *out,
                             uint32_t *scratch) {
  for (uint32_t e = 0; e < experts; ++e) scratch[e] = e;
  for (uint32_t i = 1; i < experts; ++i) {
    uint32_t cur = scratch[i];
    int64_t j = (int64_t)i - 1;
    while (j >= 0) {
      uint32_t prev = scratch[j];
      /* descending_score_then_expert(prev, cur) == Greater -> swap */
      int greater = (row[cur] > row[prev]) || (row[cur] == row[prev] && cur < prev);
      if (!greater) break;
      scratch[j + 1] = prev;
      --j;
    }
    scratch[j + 1] = cur;
  }
  out[0] = scratch[0];
  out[1] = scratch[1];
}

/* examples/moe_top2_v1/src/kernel.rs:25-59: running best/second selection
 * with candidate_precedes = higher score, or equal score and lower id. */
static int candidate_precedes(float cs, uint32_t ce, float is, uint32_t ie) {
  return cs > is || (cs == is && ce < ie);
}

void fe2o3o_moe_select_top2_running(const float *logits_row, uint32_t experts,
                                    uint32_t *out) {
  uint32_t best = 0xffffffffu, second = 0xffffffffu;
  for (uint32_t e = 0; e < experts; ++e) {
    float s = logits_row[e];
    if (best == 0xffffffffu || candidate_precedes(s, e, logits_row[best], best)) {
      second = best;
      best = e;
    } else if (second == 0xffffffffu ||
               candidate_precedes(s, e, logits_row[second], second)) {
      second = e;
    }
  }
  out[0] = best;
  out[1] = second;
}

/* examples/moe_top2_v1/src/oracle.rs:90-143 moe_top2_oracle_v1: finite check,
 * top-2 per token (route id = token*2 + rank), requested counts, admitted =
 * min(requested, capacity), exclusive scan with terminal total, stable-prefix
 * slots in route-id order, permutation/inverse, DROP sentinels.  Outputs are
 * staged and committed only on success. */
int32_t fe2o3o_moe_top2_route(const float *logits, uint32_t tokens,
                              uint32_t experts, uint32_t capacity,
                              uint32_t *top2, uint32_t *requested,
                              uint32_t *admitted, uint32_t *offsets,
                              uint32_t *route_slots, uint32_t *permutation,
                              uint32_t *inverse) {
  if (experts < 2) return FE2O3O_ERR_SHAPE;
  uint64_t n_logits = (uint64_t)tokens * experts;
  for (uint64_t i = 0; i < n_logits; ++i)
    if (!isfinite(logits[i])) return FE2O3O_ERR_NONFINITE;
  uint64_t routes = (uint64_t)tokens * 2;
  uint32_t *s_top2 = (uint32_t *)malloc(sizeof(uint32_t) * (routes ? routes : 1));
  uint32_t *s_slots = (uint32_t *)malloc(sizeof(uint32_t) * (routes ? routes : 1));
  uint32_t *s_perm = (uint32_t *)malloc(sizeof(uint32_t) * (routes ? routes : 1));
  uint32_t *s_inv = (uint32_t *)malloc(sizeof(uint32_t) * (routes ? routes : 1));
  uint32_t *s_req = (uint32_t *)calloc(experts, sizeof(uint32_t));
  uint32_t *s_adm = (uint32_t *)calloc(experts, sizeof(uint32_t));
  uint32_t *s_off = (uint32_t *)calloc(experts + 1, sizeof(uint32_t));
  uint32_t *ranks = (uint32_t *)calloc(experts, sizeof(uint32_t));
  uint32_t *scratch = (uint32_t *)malloc(sizeof(uint32_t) * experts);
  for (uint64_t r = 0; r < routes; ++r) s_slots[r] = s_perm[r] = s_inv[r] = FE2O3O_DROP_ROUTE;
  for (uint32_t t = 0; t < tokens; ++t) {
    uint32_t sel[2];
    independent_top2(logits + (uint64_t)t * experts, experts, sel, scratch);
    s_top2[2 * (uint64_t)t] = sel[0];
    s_top2[2 * (uint64_t)t + 1] = sel[1];
    s_req[sel[0]]++;
    s_req[sel[1]]++;
  }
  for (uint32_t e = 0; e < experts; ++e) {
    s_adm[e] = s_req[e] < capacity ? s_req[e] : capacity;
    s_off[e + 1] = s_off[e] + s_adm[e];
  }
  for (uint64_t r = 0; r < routes; ++r) {
    uint32_t e = s_top2[r];
    uint32_t rank = ranks[e]++;
    if (rank < capacity) {
      uint32_t slot = s_off[e] + rank;
      s_slots[r] = slot;
      s_perm[slot] = (uint32_t)r;
      s_inv[r] = slot;
    }
  }
  memcpy(top2, s_top2, sizeof(uint32_t) * routes);
  memcpy(route_slots, s_slots, sizeof(uint32_t) * routes);
  memcpy(permutation, s_perm, sizeof(uint32_t) * routes);
  memcpy(inverse, s_inv, sizeof(uint32_t) * routes);
  memcpy(requested, s_req, sizeof(uint32_t) * experts);
  memcpy(admitted, s_adm, sizeof(uint32_t) * experts);
  memcpy(offsets, s_off, sizeof(uint32_t) * (experts + 1));
  free(s_top2);
  free(s_slots);
  free(s_perm);
  free(s_inv);
  free(s_req);
  free(s_adm);
  free(s_off);
  free(ranks);
  free(scratch);
  return FE2O3O_OK;
}

/* Gating for the selected pair (this build's convention for the scaled-up
 * configuration): softmax over the two selected logits,
 * w0 = 1 / (1 + exp(l1 - l0)) with l0 >= l1, w1 = 1 - w0.  w0 lies in
 * [0.5, 1], so 1 - w0 is exact (Sterbenz) and w0 + w1 == 1.0f exactly. */
void fe2o3o_moe_top2_weights(const float *logits, uint32_t tokens,
                             uint32_t experts, const uint32_t *top2,
                             float *weights) {
  for (uint64_t t = 0; t < tokens; ++t) {
    float l0 = logits[t * experts + top2[2 * t]];
    float l1 = logits[t * experts + top2[2 * t + 1]];
    float w0 = 1.0f / (1.0f + expf(l1 - l0));
    weights[2 * t] = w0;
    weights[2 * t + 1] = 1.0f - w0;
  }
}

/* examples/moe_expert_v1/src/contract.rs:8-23 */
#define MX_T 8
#define MX_E 4
#define MX_H 16
#define MX_O 16
#define MX_TILE 256
#define MX_ROUTES 16

/* examples/moe_expert_v1/src/pipeline.rs:114-149 validate_pipeline_inputs_v1
 * (lengths, finite bf16, route weight pairs finite, nonnegative and summing
 * exactly to 1.0). */
static int32_t validate_expert_inputs(uint64_t act_len, const uint16_t *act,
                                      uint64_t w_len, const uint16_t *w,
                                      uint64_t rw_len, const float *rw) {
  if (act_len != MX_T * MX_H || w_len != MX_E * MX_TILE || rw_len != MX_ROUTES)
    return FE2O3O_ERR_LENGTH;
  for (uint64_t i = 0; i < act_len; ++i)
    if ((act[i] & 0x7f80u) == 0x7f80u) return FE2O3O_ERR_NONFINITE;
  for (uint64_t i = 0; i < w_len; ++i)
    if ((w[i] & 0x7f80u) == 0x7f80u) return FE2O3O_ERR_NONFINITE;
  for (int t = 0; t < MX_T; ++t) {
    float a = rw[2 * t], b = rw[2 * t + 1];
    if (!isfinite(a) || !isfinite(b) || a < 0.0f || b < 0.0f || a + b != 1.0f)
      return FE2O3O_ERR_WEIGHTS;
  }
  return FE2O3O_OK;
}

/* examples/moe_expert_v1/src/oracle.rs:32-90: each accepted route evaluated
 * directly (sequential f32 multiply-add in depth order, bf16 widened exactly),
 * placed in its expert tile row and compact slot, combined as
 * combined += weight * value in route order starting from +0. */
int32_t fe2o3o_moe_expert_independent_v1(
    const float *logits, const uint16_t *activations, uint64_t act_len,
    const uint16_t *weights, uint64_t w_len, const float *route_weights,
    uint64_t rw_len, const uint32_t *top2, const uint32_t *offsets,
    const uint32_t *inverse, float *expert_tiles, float *compact,
    float *combined, float *route_output) {
  (void)logits;
  int32_t rc = validate_expert_inputs(act_len, activations, w_len, weights, rw_len,
                                      route_weights);
  if (rc != 0) return rc;
  float tiles[MX_E * MX_TILE] = {0}, comp[MX_ROUTES * MX_O] = {0};
  float comb[MX_T * MX_O] = {0}, rout[MX_ROUTES * MX_O] = {0};
  for (int r = 0; r < MX_ROUTES; ++r) {
    uint32_t slot = inverse[r];
    if (slot == FE2O3O_DROP_ROUTE) continue;
    int token = r / 2;
    uint32_t e = top2[r];
    uint32_t erow = slot - offsets[e];
    for (int o = 0; o < MX_O; ++o) {
      float value = 0.0f;
      for (int d = 0; d < MX_H; ++d) {
        float p = fe2o3o_bf16_to_f32(activations[token * MX_H + d]) *
                  fe2o3o_bf16_to_f32(weights[e * MX_TILE + d * MX_O + o]);
        value = value + p;
      }
      rout[r * MX_O + o] = value;
      comp[slot * MX_O + o] = value;
      tiles[e * MX_TILE + erow * MX_O + o] = value;
      float wv = route_weights[r] * value;
      comb[token * MX_O + o] = comb[token * MX_O + o] + wv;
    }
  }
  if (expert_tiles) memcpy(expert_tiles, tiles, sizeof(tiles));
  if (compact) memcpy(compact, comp, sizeof(comp));
  if (combined) memcpy(combined, comb, sizeof(comb));
  if (route_output) memcpy(route_output, rout, sizeof(rout));
  return FE2O3O_OK;
}

/* examples/moe_expert_v1/src/pipeline.rs:166-270: compaction into zero-padded
 * per-expert 16x16 tiles, four tile GEMMs, inverse permutation, combine in
 * rank order. */
int32_t fe2o3o_moe_expert_pipeline_v1(
    const float *logits, const uint16_t *activations, uint64_t act_len,
    const uint16_t *weights, uint64_t w_len, const float *route_weights,
    uint64_t rw_len, const uint32_t *top2, const uint32_t *admitted,
    const uint32_t *offsets, const uint32_t *permutation,
    const uint32_t *inverse, uint16_t *activation_tiles, float *expert_tiles,
    float *compact, float *combined) {
  (void)logits;
  (void)admitted;
  int32_t rc = validate_expert_inputs(act_len, activations, w_len, weights, rw_len,
                                      route_weights);
  if (rc != 0) return rc;
  uint16_t at[MX_E * MX_TILE] = {0};
  uint32_t accepted = offsets[MX_E];
  for (uint32_t slot = 0; slot < accepted; ++slot) {
    uint32_t route = permutation[slot];
    int found = -1;
    uint32_t erow = 0;
    for (int e = 0; e < MX_E; ++e) {
      if (offsets[e] <= slot && slot < offsets[e + 1]) {
        found = e;
        erow = slot - offsets[e];
        break;
      }
    }
    if (found < 0 || route >= MX_ROUTES || erow >= 4 || top2[route] != (uint32_t)found ||
        inverse[route] != slot)
      return FE2O3O_ERR_ROUTING;
    uint32_t token = route / 2;
    for (int d = 0; d < MX_H; ++d)
      at[found * MX_TILE + erow * MX_H + d] = activations[token * MX_H + d];
  }
  float tiles[MX_E * MX_TILE];
  for (int e = 0; e < MX_E; ++e) {
    for (int r = 0; r < 16; ++r) {
      for (int o = 0; o < MX_O; ++o) {
        float acc = 0.0f;
        for (int d = 0; d < MX_H; ++d) {
          float p = fe2o3o_bf16_to_f32(at[e * MX_TILE + r * MX_H + d]) *
                    fe2o3o_bf16_to_f32(weights[e * MX_TILE + d * MX_O + o]);
          acc = acc + p;
        }
        tiles[e * MX_TILE + r * MX_O + o] = acc;
      }
    }
  }
  float comp[MX_ROUTES * MX_O] = {0};
  for (uint32_t slot = 0; slot < accepted; ++slot) {
    uint32_t route = permutation[slot];
    uint32_t e = top2[route];
    uint32_t row = slot - offsets[e];
    for (int o = 0; o < MX_O; ++o) comp[slot * MX_O + o] = tiles[e * MX_TILE + row * MX_O + o];
  }
  float comb[MX_T * MX_O];
  for (int t = 0; t < MX_T; ++t) {
    for (int o = 0; o < MX_O; ++o) {
      float acc = 0.0f;
      for (int rank = 0; rank < 2; ++rank) {
        int route = t * 2 + rank;
        uint32_t slot = inverse[route];
        if (slot != FE2O3O_DROP_ROUTE) {
          float wv = route_weights[route] * comp[slot * MX_O + o];
          acc = acc + wv;
        }
      }
      comb[t * MX_O + o] = acc;
    }
  }
  if (activation_tiles) memcpy(activation_tiles, at, sizeof(at));
  if (expert_tiles) memcpy(expert_tiles, tiles, sizeof(tiles));
  if (compact) memcpy(compact, comp, sizeof(comp));
  if (combined) memcpy(combined, comb, sizeof(comb));
  return FE2O3O_OK;
}

/* SiLU expert FFN (not in the reference): g = x.Wg^T, u = x.Wu^T in
 * sequential f32 (same recurrence as the expert GEMM oracle above),
 * hidden = bf16(silu(g) * u) with silu(g) = g / (1 + exp(-g)), then
 * y = hidden.Wd^T in sequential f32.  FB outputs are computed side by side
 * (independent accumulators, each still summed over i = 0, 1, ... in
 * order), which vectorises across outputs without changing any result. */
#define FFN_FB 8
void fe2o3o_moe_ffn_route(const uint16_t *x, const uint16_t *w_gate,
                          const uint16_t *w_up, const uint16_t *w_down,
                          uint32_t h, uint32_t f, uint16_t *hidden, float *y) {
  float *xf = (float *)malloc(sizeof(float) * h);
  float *hf = (float *)malloc(sizeof(float) * f);
  for (uint32_t i = 0; i < h; ++i) xf[i] = fe2o3o_bf16_to_f32(x[i]);
  for (uint32_t j0 = 0; j0 < f; j0 += FFN_FB) {
    const uint32_t nb = f - j0 < FFN_FB ? f - j0 : FFN_FB;
    float g[FFN_FB] = {0}, u[FFN_FB] = {0};
    for (uint32_t i = 0; i < h; ++i) {
      for (uint32_t jj = 0; jj < nb; ++jj) {
        float pg = xf[i] * fe2o3o_bf16_to_f32(w_gate[(uint64_t)(j0 + jj) * h + i]);
        g[jj] = g[jj] + pg;
        float pu = xf[i] * fe2o3o_bf16_to_f32(w_up[(uint64_t)(j0 + jj) * h + i]);
        u[jj] = u[jj] + pu;
      }
    }
    for (uint32_t jj = 0; jj < nb; ++jj) {
      float sg = g[jj] / (1.0f + expf(-g[jj]));
      uint16_t hb = fe2o3o_bf16_from_f32(sg * u[jj]);
      if (hidden) hidden[j0 + jj] = hb;
      hf[j0 + jj] = fe2o3o_bf16_to_f32(hb);
    }
  }
  for (uint32_t i0 = 0; i0 < h; i0 += FFN_FB) {
    const uint32_t nb = h - i0 < FFN_FB ? h - i0 : FFN_FB;
    float acc[FFN_FB] = {0};
    for (uint32_t j = 0; j < f; ++j) {
      for (uint32_t ii = 0; ii < nb; ++ii) {
        float p = hf[j] * fe2o3o_bf16_to_f32(w_down[(uint64_t)(i0 + ii) * f + j]);
        acc[ii] = acc[ii] + p;
      }
    }
    for (uint32_t ii = 0; ii < nb; ++ii) y[i0 + ii] = acc[ii];
  }
  free(xf);
  free(hf);
}

/* fe2o3o_moe_ffn_route for n (token, expert) pairs at once, spread over
 * `threads` OpenMP threads: x [tokens, h]; w_gate, w_up [E, F, H];
 * w_down [E, H, F]; y [n, h] receives each pair's f32 expert output.  The
 * pairs are grouped by expert and each expert's matrices are walked in
 * panels of FFN_PB rows, transposed once to f32, so FFN_PB outputs of a
 * route are accumulated side by side; every output keeps the single-route
 * order (+0, then i = 0, 1, ... with separate rounding), so the results are
 * those of fe2o3o_moe_ffn_route bit for bit. */
#define FFN_PB 16
void fe2o3o_moe_ffn_routes(const uint16_t *x, const uint16_t *w_gate,
                           const uint16_t *w_up, const uint16_t *w_down,
                           uint32_t h, uint32_t f, const uint32_t *tokens,
                           const uint32_t *experts, uint64_t n, float *y,
                           int32_t threads) {
  const uint64_t wsz = (uint64_t)f * h;
  uint32_t max_e = 0;
  for (uint64_t r = 0; r < n; ++r) max_e = experts[r] > max_e ? experts[r] : max_e;
  uint64_t *idx = (uint64_t *)malloc(sizeof(uint64_t) * (n ? n : 1));
  for (uint32_t e = 0; e <= max_e && n; ++e) {
    uint64_t cnt = 0;
    for (uint64_t r = 0; r < n; ++r)
      if (experts[r] == e) idx[cnt++] = r;
    if (cnt == 0) continue;
    const uint16_t *wg = w_gate + e * wsz, *wu = w_up + e * wsz, *wd = w_down + e * wsz;
    float *xf = (float *)malloc(sizeof(float) * cnt * h);
    float *hf = (float *)malloc(sizeof(float) * cnt * f);
    for (uint64_t t = 0; t < cnt; ++t)
      for (uint32_t i = 0; i < h; ++i)
        xf[t * h + i] = fe2o3o_bf16_to_f32(x[(uint64_t)tokens[idx[t]] * h + i]);
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
      float *pg = (float *)malloc(sizeof(float) * (size_t)h * FFN_PB);
      float *pu = (float *)malloc(sizeof(float) * (size_t)h * FFN_PB);
      float *pd = (float *)malloc(sizeof(float) * (size_t)f * FFN_PB);
#pragma omp for schedule(dynamic, 1)
      for (uint32_t j0 = 0; j0 < f; j0 += FFN_PB) {
        const uint32_t nb = f - j0 < FFN_PB ? f - j0 : FFN_PB;
        for (uint32_t i = 0; i < h; ++i)
          for (uint32_t jj = 0; jj < FFN_PB; ++jj) {
            const uint64_t at = (uint64_t)(j0 + jj) * h + i;
            pg[(size_t)i * FFN_PB + jj] = jj < nb ? fe2o3o_bf16_to_f32(wg[at]) : 0.0f;
            pu[(size_t)i * FFN_PB + jj] = jj < nb ? fe2o3o_bf16_to_f32(wu[at]) : 0.0f;
          }
        for (uint64_t t = 0; t < cnt; ++t) {
          float g[FFN_PB], u[FFN_PB];
          for (int jj = 0; jj < FFN_PB; ++jj) g[jj] = u[jj] = 0.0f;
          const float *xr = xf + t * h;
          for (uint32_t i = 0; i < h; ++i) {
            const float xv = xr[i];
            const float *gv = pg + (size_t)i * FFN_PB, *uv = pu + (size_t)i * FFN_PB;
            for (int jj = 0; jj < FFN_PB; ++jj) {
              float a = xv * gv[jj];
              g[jj] = g[jj] + a;
              float b = xv * uv[jj];
              u[jj] = u[jj] + b;
            }
          }
          for (uint32_t jj = 0; jj < nb; ++jj) {
            float sg = g[jj] / (1.0f + expf(-g[jj]));
            hf[t * f + j0 + jj] = fe2o3o_bf16_to_f32(fe2o3o_bf16_from_f32(sg * u[jj]));
          }
        }
      }
#pragma omp for schedule(dynamic, 1)
      for (uint32_t i0 = 0; i0 < h; i0 += FFN_PB) {
        const uint32_t nb = h - i0 < FFN_PB ? h - i0 : FFN_PB;
        for (uint32_t j = 0; j < f; ++j)
          for (uint32_t ii = 0; ii < FFN_PB; ++ii)
            pd[(size_t)j * FFN_PB + ii] =
                ii < nb ? fe2o3o_bf16_to_f32(wd[(uint64_t)(i0 + ii) * f + j]) : 0.0f;
        for (uint64_t t = 0; t < cnt; ++t) {
          float acc[FFN_PB];
          for (int ii = 0; ii < FFN_PB; ++ii) acc[ii] = 0.0f;
          const float *hr = hf + t * f;
          for (uint32_t j = 0; j < f; ++j) {
            const float hv = hr[j];
            const float *dv = pd + (size_t)j * FFN_PB;
            for (int ii = 0; ii < FFN_PB; ++ii) {
              float p = hv * dv[ii];
              acc[ii] = acc[ii] + p;
            }
          }
          for (uint32_t ii = 0; ii < nb; ++ii) y[idx[t] * h + i0 + ii] = acc[ii];
        }
      }
      free(pg);
      free(pu);
      free(pd);
    }
    free(xf);
    free(hf);
  }
  free(idx);
}
