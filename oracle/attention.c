/*
 * attention.c -- CPU restatement of the reference's flash-attention and
 * row-softmax oracles.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).
 * Host exp is glibc exp/expf, the same functions the reference's Rust
 * f64::exp / f32::exp call on linux-gnu.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "fe2o3_oracle.h"

/* examples/flash_attention_v1/src/contract.rs:3-31 */
#define FA_N 8
#define FA_D 16
#define FA_ELEMS (FA_N * FA_D)

/* examples/flash_attention_v1/src/oracle.rs:91-139 strict_f32_scores (scale
 * bits 0x3e800000 = 0.25). */
static int strict_f32_scores(const float *q, const float *k, float scores[FA_N][FA_N]) {
  for (int qr = 0; qr < FA_N; ++qr) {
    for (int kr = 0; kr <= qr; ++kr) {
      float dot = 0.0f;
      for (int f = 0; f < FA_D; ++f) {
        float p = q[qr * FA_D + f] * k[kr * FA_D + f];
        if (!isfinite(p)) return FE2O3O_ERR_INTERMEDIATE;
        dot = dot + p;
        if (!isfinite(dot)) return FE2O3O_ERR_INTERMEDIATE;
      }
      float s = dot * 0.25f;
      if (!isfinite(s)) return FE2O3O_ERR_INTERMEDIATE;
      scores[qr][kr] = s;
    }
  }
  return FE2O3O_OK;
}

/* oracle.rs:140-202 preflight_online_f32: the kernel's online recurrence in
 * strict f32 (host expf surrogate), checked for finiteness only. */
static int preflight_online_f32(float scores[FA_N][FA_N], const float *v) {
  for (int qr = 0; qr < FA_N; ++qr) {
    for (int col = 0; col < FA_D; ++col) {
      float m = 0.0f, l = 0.0f, num = 0.0f;
      for (int kr = 0; kr <= qr; ++kr) {
        float s = scores[qr][kr];
        float val = v[kr * FA_D + col];
        if (kr == 0) {
          m = s;
          l = 1.0f;
          num = val;
          continue;
        }
        float nm = fmaxf(m, s);
        float wp = expf(m - nm);
        float wc = expf(s - nm);
        if (!isfinite(wp) || !isfinite(wc)) return FE2O3O_ERR_INTERMEDIATE;
        float t0 = l * wp;
        l = t0 + wc;
        if (!isfinite(l) || l <= 0.0f) return FE2O3O_ERR_INTERMEDIATE;
        float t1 = num * wp;
        float t2 = val * wc;
        num = t1 + t2;
        if (!isfinite(num)) return FE2O3O_ERR_INTERMEDIATE;
        m = nm;
      }
      if (!isfinite(num / l)) return FE2O3O_ERR_INTERMEDIATE;
    }
  }
  return FE2O3O_OK;
}

/* oracle.rs:222-284 flash_attention_oracle_v1: lengths, finiteness, strict
 * preflight, then the independent two-pass f64 reference; output committed
 * only after every check. */
int32_t fe2o3o_flash_attention_v1(const float *q, uint64_t q_len,
                                  const float *k, uint64_t k_len,
                                  const float *v, uint64_t v_len, float *out,
                                  uint64_t out_len, double *row_maxima,
                                  double *row_denominators) {
  if (q_len != FA_ELEMS || k_len != FA_ELEMS || v_len != FA_ELEMS || out_len != FA_ELEMS)
    return FE2O3O_ERR_LENGTH;
  for (int i = 0; i < FA_ELEMS; ++i)
    if (!isfinite(q[i]) || !isfinite(k[i]) || !isfinite(v[i])) return FE2O3O_ERR_NONFINITE;
  float scores32[FA_N][FA_N];
  int rc = strict_f32_scores(q, k, scores32);
  if (rc != 0) return rc;
  if ((rc = preflight_online_f32(scores32, v)) != 0) return rc;

  float staged[FA_ELEMS];
  double maxima[FA_N], dens[FA_N];
  for (int qr = 0; qr < FA_N; ++qr) {
    double sc[FA_N];
    for (int kr = 0; kr <= qr; ++kr) {
      double dot = 0.0;
      for (int f = 0; f < FA_D; ++f) dot += (double)q[qr * FA_D + f] * (double)k[kr * FA_D + f];
      sc[kr] = dot * 0.25;
    }
    double mx = sc[0];
    for (int kr = 1; kr <= qr; ++kr) mx = fmax(mx, sc[kr]);
    double w[FA_N], den = 0.0;
    for (int kr = 0; kr <= qr; ++kr) {
      w[kr] = exp(sc[kr] - mx);
      den += w[kr];
    }
    maxima[qr] = mx;
    dens[qr] = den;
    for (int col = 0; col < FA_D; ++col) {
      double num = 0.0;
      for (int kr = 0; kr <= qr; ++kr) num += w[kr] * (double)v[kr * FA_D + col];
      float val = (float)(num / den);
      if (!isfinite(val)) return FE2O3O_ERR_INTERMEDIATE;
      staged[qr * FA_D + col] = val;
    }
  }
  memcpy(out, staged, sizeof(staged));
  if (row_maxima) memcpy(row_maxima, maxima, sizeof(maxima));
  if (row_denominators) memcpy(row_denominators, dens, sizeof(dens));
  return FE2O3O_OK;
}

/* The same two-pass f64 reference (oracle.rs:242-277) for the scaled-up
 * [B,H,S,D] bf16 configuration: score = (sum_d q*k in f64) * scale, causal
 * rows see keys 0..=row, then max pass, exp pass, weighted-V pass; output
 * rounded to f32, lse = max + ln(denominator). */
int32_t fe2o3o_flash_attention_rows_bf16(const uint16_t *q, const uint16_t *k,
                                         const uint16_t *v, uint32_t s,
                                         uint32_t d, int32_t causal,
                                         float scale, const uint32_t *bh,
                                         const uint32_t *rows, uint64_t count,
                                         float *out, float *lse,
                                         int32_t threads) {
  int32_t status = FE2O3O_OK;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    double *sc = (double *)malloc(sizeof(double) * s);
    double *qd = (double *)malloc(sizeof(double) * d);
    double *acc = (double *)malloc(sizeof(double) * d);
#pragma omp for schedule(dynamic, 1)
    for (uint64_t r = 0; r < count; ++r) {
      uint64_t head = bh[r];
      uint32_t row = rows[r];
      const uint16_t *qh = q + (head * s + row) * (uint64_t)d;
      const uint16_t *kh = k + head * s * (uint64_t)d;
      const uint16_t *vh = v + head * s * (uint64_t)d;
      uint32_t keys = causal ? row + 1 : s;
      for (uint32_t f = 0; f < d; ++f) qd[f] = (double)fe2o3o_bf16_to_f32(qh[f]);
      for (uint32_t j = 0; j < keys; ++j) {
        const uint16_t *kr = kh + (uint64_t)j * d;
        double dot = 0.0;
        for (uint32_t f = 0; f < d; ++f) dot += qd[f] * (double)fe2o3o_bf16_to_f32(kr[f]);
        sc[j] = dot * (double)scale;
      }
      double mx = sc[0];
      for (uint32_t j = 1; j < keys; ++j) mx = fmax(mx, sc[j]);
      double den = 0.0;
      for (uint32_t f = 0; f < d; ++f) acc[f] = 0.0;
      for (uint32_t j = 0; j < keys; ++j) {
        double w = exp(sc[j] - mx);
        den += w;
        const uint16_t *vr = vh + (uint64_t)j * d;
        for (uint32_t f = 0; f < d; ++f) acc[f] += w * (double)fe2o3o_bf16_to_f32(vr[f]);
      }
      for (uint32_t f = 0; f < d; ++f) {
        float val = (float)(acc[f] / den);
        if (!isfinite(val)) status = FE2O3O_ERR_INTERMEDIATE;
        out[r * d + f] = val;
      }
      if (lse) lse[r] = (float)(mx + log(den));
    }
    free(sc);
    free(qd);
    free(acc);
  }
  return status;
}

/* examples/row_softmax_v1/src/numerical_contract.rs:4 */
#define RS_MAX_ROW 4096u

/* numerical_contract.rs:130-199 row_softmax_oracle_v1. */
int32_t fe2o3o_row_softmax_oracle_v1(const float *input, uint64_t len,
                                     const uint8_t *mask, float *out,
                                     double *state) {
  if (len == 0) return FE2O3O_ERR_EMPTY;
  if (len > RS_MAX_ROW) return FE2O3O_ERR_TOO_LARGE;
  for (uint64_t i = 0; i < len; ++i)
    if (!isfinite(input[i])) return FE2O3O_ERR_NONFINITE;
  uint64_t active = 0;
  for (uint64_t i = 0; i < len; ++i)
    if (!mask || mask[i]) active++;
  if (active == 0) return FE2O3O_ERR_NO_ACTIVE;
  /* reduce(f32::max) over active elements in index order. */
  float mx = 0.0f;
  int first = 1;
  for (uint64_t i = 0; i < len; ++i) {
    if (mask && !mask[i]) continue;
    if (first) {
      mx = input[i];
      first = 0;
    } else {
      mx = fmaxf(mx, input[i]);
    }
  }
  double *w = (double *)calloc(len, sizeof(double));
  float *res = (float *)calloc(len, sizeof(float));
  double mx64 = (double)mx, den = 0.0;
  int32_t rc = FE2O3O_OK;
  for (uint64_t i = 0; i < len; ++i) {
    if (mask && !mask[i]) continue;
    double wt = exp((double)input[i] - mx64);
    if (!isfinite(wt) || wt < 0.0) {
      rc = FE2O3O_ERR_INTERMEDIATE;
      goto done;
    }
    w[i] = wt;
    den += wt;
  }
  if (!isfinite(mx) || !isfinite(den) || den < 1.0) {
    rc = FE2O3O_ERR_INTERMEDIATE;
    goto done;
  }
  for (uint64_t i = 0; i < len; ++i) {
    if (mask && !mask[i]) continue;
    res[i] = (float)(w[i] / den);
    if (!isfinite(res[i]) || res[i] < 0.0f) {
      rc = FE2O3O_ERR_INTERMEDIATE;
      goto done;
    }
  }
  memcpy(out, res, sizeof(float) * len);
  if (state) {
    state[0] = (double)mx;
    state[1] = den;
    state[2] = (double)active;
  }
done:
  free(w);
  free(res);
  return rc;
}

/* numerical_contract.rs:201-257 compare_row_softmax_v1 (masked outputs must be
 * +0.0 bit-exactly; active outputs pass on the abs+rel envelope or on the
 * positive-value ULP distance; the active sum is checked independently). */
int32_t fe2o3o_compare_row_softmax_v1(const float *expected,
                                      const float *actual, uint64_t len,
                                      const uint8_t *mask, float abs_tol,
                                      float rel_tol, float sum_tol,
                                      uint32_t max_ulps, uint64_t *bad_index) {
  if (!(isfinite(abs_tol) && abs_tol >= 0.0f && isfinite(rel_tol) && rel_tol >= 0.0f &&
        isfinite(sum_tol) && sum_tol >= 0.0f))
    return FE2O3O_ERR_POLICY;
  float sum = 0.0f;
  for (uint64_t i = 0; i < len; ++i) {
    float obs = actual[i];
    if (!isfinite(obs) || obs < 0.0f) {
      if (bad_index) *bad_index = i;
      return FE2O3O_ERR_NONFINITE;
    }
    if (mask && !mask[i]) {
      uint32_t bits;
      memcpy(&bits, &obs, 4);
      if (bits != 0) {
        if (bad_index) *bad_index = i;
        return FE2O3O_ERR_MISMATCH;
      }
      continue;
    }
    float ref = expected[i];
    if (!isfinite(ref) || ref < 0.0f) {
      if (bad_index) *bad_index = i;
      return FE2O3O_ERR_NONFINITE;
    }
    float absolute = fabsf(obs - ref);
    float limit = abs_tol + rel_tol * fabsf(ref);
    uint32_t ob, rb;
    memcpy(&ob, &obs, 4);
    memcpy(&rb, &ref, 4);
    uint32_t ulps = ob > rb ? ob - rb : rb - ob;
    if (absolute > limit && ulps > max_ulps) {
      if (bad_index) *bad_index = i;
      return FE2O3O_ERR_MISMATCH;
    }
    sum = sum + obs;
  }
  if (!isfinite(sum) || fabsf(sum - 1.0f) > sum_tol) return FE2O3O_ERR_SUM;
  return FE2O3O_OK;
}

/* examples/row_softmax_v1/src/lib.rs:121-159: f32 max, f32 exp weights,
 * sequential f32 denominator, f32 division (64-element row). */
int32_t fe2o3o_row_softmax_reference_v1(const float *input, float *out) {
  for (int i = 0; i < 64; ++i)
    if (!isfinite(input[i])) return FE2O3O_ERR_NONFINITE;
  float mx = input[0];
  for (int i = 1; i < 64; ++i) mx = fmaxf(mx, input[i]);
  float w[64], den = 0.0f;
  for (int i = 0; i < 64; ++i) {
    w[i] = expf(input[i] - mx);
    den = den + w[i];
  }
  if (!isfinite(mx) || !isfinite(den) || den <= 0.0f) return FE2O3O_ERR_INTERMEDIATE;
  for (int i = 0; i < 64; ++i) out[i] = w[i] / den;
  for (int i = 0; i < 64; ++i)
    if (!isfinite(out[i])) return FE2O3O_ERR_INTERMEDIATE;
  return FE2O3O_OK;
}

int32_t fe2o3o_row_softmax_rows(const float *input, uint64_t rows,
                                uint64_t cols, float *out, int32_t threads) {
  int32_t status = FE2O3O_OK;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (uint64_t r = 0; r < rows; ++r) {
    int32_t rc = fe2o3o_row_softmax_oracle_v1(input + r * cols, cols, NULL,
                                              out + r * cols, NULL);
    if (rc != FE2O3O_OK) status = rc;
  }
  return status;
}

/* Row-by-row check of a device softmax over many rows: for each row the f64
 * oracle (fe2o3o_row_softmax_oracle_v1) and the contract's comparison
 * (fe2o3o_compare_row_softmax_v1) under the given policy, OpenMP over rows.
 * stats[0] = rows failing the comparison, stats[1] = the first failing row
 * (rows if none), stats[2] = max |actual - oracle| over all elements,
 * stats[3] = max |oracle| over all elements, stats[4] = max |f64 row sum of
 * actual - 1|.  Returns the first oracle error (FE2O3O_OK when every row's
 * input is admitted); comparison failures are counted, not returned. */
int32_t fe2o3o_row_softmax_check_rows(const float *input, const float *actual, uint64_t rows,
                                      uint64_t cols, float abs_tol, float rel_tol, float sum_tol,
                                      uint32_t max_ulps, int32_t threads, double *stats) {
  int32_t status = FE2O3O_OK;
  uint64_t failing = 0, first = rows;
  double max_diff = 0.0, max_ref = 0.0, max_sum = 0.0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    float *ref = (float *)malloc(cols * sizeof(float));
    uint64_t my_failing = 0, my_first = rows;
    double my_diff = 0.0, my_ref = 0.0, my_sum = 0.0;
    int32_t my_status = ref ? FE2O3O_OK : FE2O3O_ERR_INTERMEDIATE;
#pragma omp for schedule(static)
    for (uint64_t r = 0; r < rows; ++r) {
      if (!ref) continue;
      const float *x = input + r * cols, *y = actual + r * cols;
      int32_t rc = fe2o3o_row_softmax_oracle_v1(x, cols, NULL, ref, NULL);
      if (rc != FE2O3O_OK) {
        my_status = rc;
        continue;
      }
      if (fe2o3o_compare_row_softmax_v1(ref, y, cols, NULL, abs_tol, rel_tol, sum_tol, max_ulps,
                                        NULL) != FE2O3O_OK) {
        ++my_failing;
        if (r < my_first) my_first = r;
      }
      double sum = 0.0;
      for (uint64_t c = 0; c < cols; ++c) {
        const double d = fabs((double)y[c] - (double)ref[c]);
        if (!isnan(my_diff) && !(d <= my_diff)) my_diff = d; /* a NaN stays the maximum */
        if (fabs((double)ref[c]) > my_ref) my_ref = fabs((double)ref[c]);
        sum += (double)y[c];
      }
      const double e = fabs(sum - 1.0);
      if (!isnan(my_sum) && !(e <= my_sum)) my_sum = e;
    }
    free(ref);
#pragma omp critical
    {
      if (my_status != FE2O3O_OK) status = my_status;
      failing += my_failing;
      if (my_first < first) first = my_first;
      if (!isnan(max_diff) && !(my_diff <= max_diff)) max_diff = my_diff;
      if (my_ref > max_ref) max_ref = my_ref;
      if (!isnan(max_sum) && !(my_sum <= max_sum)) max_sum = my_sum;
    }
  }
  stats[0] = (double)failing;
  stats[1] = (double)first;
  stats[2] = max_diff;
  stats[3] = max_ref;
  stats[4] = max_sum;
  return status;
}
