/*
 * gemm.c -- CPU restatement of the reference's GEMM oracles.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).
 * Compiled with -ffp-contract=off: every `p = x * y; acc = acc + p` below is
 * two separately rounded binary32 operations, as in the reference's
 * black_box'd fp32_product/fp32_sum (examples/tiled_gemm_v1/src/oracle.rs
 * :262-270, numerical_contract.rs:297-305, scalar_gemm_v1/src/harness.rs
 * :79-85).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "fe2o3_oracle.h"

static uint32_t f32_bits(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  return b;
}

static float widen(uint16_t bits) { return fe2o3o_bf16_to_f32(bits); }

/* examples/tiled_gemm_v1/src/oracle.rs:284-320.  Empty output returns without
 * inspecting operands; otherwise exact lengths M*K and K*N are required. */
int32_t fe2o3o_tiled_gemm_arithmetic_v1(uint32_t m, uint32_t n, uint32_t k,
                                        const uint16_t *a, uint64_t a_len,
                                        const uint16_t *b, uint64_t b_len,
                                        float *c) {
  if (m == 0 || n == 0) return FE2O3O_OK;
  if (a_len != (uint64_t)m * k || b_len != (uint64_t)k * n) return FE2O3O_ERR_LENGTH;
  for (uint64_t row = 0; row < m; ++row) {
    for (uint64_t col = 0; col < n; ++col) {
      float acc = 0.0f;
      for (uint64_t d = 0; d < k; ++d) {
        float p = widen(a[row * k + d]) * widen(b[d * n + col]);
        acc = acc + p;
      }
      c[row * n + col] = acc;
    }
  }
  return FE2O3O_OK;
}

/* numerical_contract.rs:139-186: (rows-1)*stride + columns, zero if empty,
 * StrideTooSmall when stride < columns for a nonempty matrix. */
static int32_t checked_extent(uint64_t rows, uint64_t cols, uint64_t stride,
                              uint64_t *out) {
  if (rows == 0 || cols == 0) {
    *out = 0;
    return FE2O3O_OK;
  }
  if (stride < cols) return FE2O3O_ERR_STRIDE;
  if (rows - 1 > (UINT64_MAX - cols) / (stride ? stride : 1)) return FE2O3O_ERR_OVERFLOW;
  *out = (rows - 1) * stride + cols;
  return FE2O3O_OK;
}

int32_t fe2o3o_gemm_spec_checked(uint64_t m, uint64_t n, uint64_t k,
                                 uint64_t lda, uint64_t ldb, uint64_t ldc,
                                 uint64_t *a_len, uint64_t *b_len,
                                 uint64_t *c_len) {
  int32_t rc;
  if ((rc = checked_extent(m, k, lda, a_len)) != 0) return rc;
  if ((rc = checked_extent(k, n, ldb, b_len)) != 0) return rc;
  if ((rc = checked_extent(m, n, ldc, c_len)) != 0) return rc;
  return FE2O3O_OK;
}

/* numerical_contract.rs:272-290 validate_lengths. */
static int32_t validate_lengths(uint64_t m, uint64_t n, uint64_t k,
                                uint64_t lda, uint64_t ldb, uint64_t ldc,
                                uint64_t a_len, uint64_t b_len, uint64_t c_len) {
  uint64_t ea, eb, ec;
  int32_t rc = fe2o3o_gemm_spec_checked(m, n, k, lda, ldb, ldc, &ea, &eb, &ec);
  if (rc != 0) return rc;
  if (ea != a_len || eb != b_len || ec != c_len) return FE2O3O_ERR_LENGTH;
  return FE2O3O_OK;
}

/* numerical_contract.rs:310-331 evaluate_unchecked. */
static void evaluate_unchecked(uint64_t m, uint64_t n, uint64_t k, uint64_t lda,
                               uint64_t ldb, uint64_t ldc, const uint16_t *a,
                               const uint16_t *b, const float *c, float alpha,
                               float beta, float *out) {
  uint64_t o = 0;
  for (uint64_t row = 0; row < m; ++row) {
    for (uint64_t col = 0; col < n; ++col) {
      float acc = 0.0f;
      for (uint64_t d = 0; d < k; ++d) {
        float p = widen(a[row * lda + d]) * widen(b[d * ldb + col]);
        acc = acc + p;
      }
      float product = alpha * acc;
      float initial = beta * c[row * ldc + col];
      out[o++] = product + initial;
    }
  }
}

int32_t fe2o3o_evaluate_source(uint64_t m, uint64_t n, uint64_t k,
                               uint64_t lda, uint64_t ldb, uint64_t ldc,
                               const uint16_t *a, uint64_t a_len,
                               const uint16_t *b, uint64_t b_len,
                               const float *c, uint64_t c_len, float alpha,
                               float beta, float *out) {
  int32_t rc = validate_lengths(m, n, k, lda, ldb, ldc, a_len, b_len, c_len);
  if (rc != 0) return rc;
  evaluate_unchecked(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta, out);
  return FE2O3O_OK;
}

/* numerical_contract.rs:467-498: bf16/f32 unsupported classes. */
static int32_t bf16_class(uint16_t bits) {
  uint16_t e = bits & 0x7f80u, f = bits & 0x007fu;
  if (e == 0x7f80u) return f == 0 ? FE2O3O_ERR_INFINITE : FE2O3O_ERR_NONFINITE;
  if (e == 0 && f != 0) return FE2O3O_ERR_SUBNORMAL;
  return FE2O3O_OK;
}

static int32_t f32_class(float v) {
  if (isnan(v)) return FE2O3O_ERR_NONFINITE;
  if (isinf(v)) return FE2O3O_ERR_INFINITE;
  if (v != 0.0f && fabsf(v) < 1.17549435e-38f) return FE2O3O_ERR_SUBNORMAL;
  return FE2O3O_OK;
}

/* numerical_contract.rs:694-721 build_hardware_expectation and :574-621
 * evaluate_finite: every logical input and every intermediate must be finite
 * normal or signed zero; output only written on success. */
int32_t fe2o3o_build_hardware_expectation(uint64_t m, uint64_t n, uint64_t k,
                                          uint64_t lda, uint64_t ldb,
                                          uint64_t ldc, const uint16_t *a,
                                          uint64_t a_len, const uint16_t *b,
                                          uint64_t b_len, const float *c,
                                          uint64_t c_len, float alpha,
                                          float beta, float *out) {
  int32_t rc = validate_lengths(m, n, k, lda, ldb, ldc, a_len, b_len, c_len);
  if (rc != 0) return rc;
  for (uint64_t r = 0; r < m; ++r)
    for (uint64_t d = 0; d < k; ++d)
      if ((rc = bf16_class(a[r * lda + d])) != 0) return rc;
  for (uint64_t d = 0; d < k; ++d)
    for (uint64_t col = 0; col < n; ++col)
      if ((rc = bf16_class(b[d * ldb + col])) != 0) return rc;
  for (uint64_t r = 0; r < m; ++r)
    for (uint64_t col = 0; col < n; ++col)
      if ((rc = f32_class(c[r * ldc + col])) != 0) return rc;
  if ((rc = f32_class(alpha)) != 0) return rc;
  if ((rc = f32_class(beta)) != 0) return rc;

  uint64_t outputs = m * n;
  float *staged = (float *)malloc(sizeof(float) * (outputs > 0 ? outputs : 1));
  if (!staged) return FE2O3O_ERR_OVERFLOW;
  uint64_t o = 0;
  for (uint64_t row = 0; row < m; ++row) {
    for (uint64_t col = 0; col < n; ++col) {
      float acc = 0.0f;
      for (uint64_t d = 0; d < k; ++d) {
        float p = widen(a[row * lda + d]) * widen(b[d * ldb + col]);
        if (f32_class(p) != 0) goto intermediate;
        acc = acc + p;
        if (f32_class(acc) != 0) goto intermediate;
      }
      float product = alpha * acc;
      if (f32_class(product) != 0) goto intermediate;
      float initial = beta * c[row * ldc + col];
      if (f32_class(initial) != 0) goto intermediate;
      float result = product + initial;
      if (f32_class(result) != 0) goto intermediate;
      staged[o++] = result;
    }
  }
  memcpy(out, staged, sizeof(float) * m * n);
  free(staged);
  return FE2O3O_OK;
intermediate:
  free(staged);
  return FE2O3O_ERR_INTERMEDIATE;
}

/* numerical_contract.rs:879-888: ordered encodings and their distance. */
static uint32_t ordered_f32(uint32_t bits) {
  return (bits & 0x80000000u) == 0 ? (bits | 0x80000000u) : ~bits;
}

uint32_t fe2o3o_ulp_distance(float left, float right) {
  uint32_t l = ordered_f32(f32_bits(left)), r = ordered_f32(f32_bits(right));
  return l > r ? l - r : r - l;
}

/* numerical_contract.rs:640-666 ComparisonPolicy::bounded validation and
 * :890-981 compare_hardware (without the integrity tag, which guards the Rust
 * object against in-process mutation and has no C counterpart). */
int32_t fe2o3o_compare_hardware(const float *expected, const float *observed,
                                uint64_t n, int32_t policy, float max_abs,
                                float max_rel, uint32_t max_ulps, float *report,
                                uint32_t *max_ulp_error, uint64_t *bad_index) {
  if (policy == 1) {
    if (signbit(max_abs) || f32_class(max_abs) != 0) return FE2O3O_ERR_POLICY;
    if (signbit(max_rel) || f32_class(max_rel) != 0) return FE2O3O_ERR_POLICY;
    if (max_abs == 0.0f && max_rel == 0.0f) return FE2O3O_ERR_POLICY;
    if (max_ulps == 0) return FE2O3O_ERR_POLICY;
  }
  float rep_abs = 0.0f, rep_rel = 0.0f;
  uint32_t rep_ulp = 0;
  for (uint64_t i = 0; i < n; ++i) {
    float e = expected[i], a = observed[i];
    if (!isfinite(a)) {
      if (bad_index) *bad_index = i;
      return FE2O3O_ERR_NONFINITE;
    }
    float abs_err = fabsf(a - e);
    float denom = fabsf(e) > 1.17549435e-38f ? fabsf(e) : 1.17549435e-38f;
    float rel_err = abs_err / denom;
    uint32_t ulp = fe2o3o_ulp_distance(e, a);
    if (abs_err > rep_abs) rep_abs = abs_err;
    if (rel_err > rep_rel) rep_rel = rel_err;
    if (ulp > rep_ulp) rep_ulp = ulp;
    int accepted;
    if (policy == 0) {
      accepted = f32_bits(a) == f32_bits(e);
    } else {
      accepted = f32_bits(a) == f32_bits(e) ||
                 (abs_err <= max_abs + max_rel * fabsf(e) && ulp <= max_ulps);
    }
    if (!accepted) {
      if (bad_index) *bad_index = i;
      if (report) {
        report[0] = rep_abs;
        report[1] = rep_rel;
      }
      if (max_ulp_error) *max_ulp_error = rep_ulp;
      return FE2O3O_ERR_MISMATCH;
    }
  }
  if (report) {
    report[0] = rep_abs;
    report[1] = rep_rel;
  }
  if (max_ulp_error) *max_ulp_error = rep_ulp;
  return FE2O3O_OK;
}

/* crates/fe2o3-device/src/tensor.rs:154-159 */
int32_t fe2o3o_row_major_xor4(uint32_t row, uint32_t col, uint32_t *physical) {
  if (row >= 16 || col >= 16) return FE2O3O_ERR_SHAPE;
  *physical = row * 16 + (col ^ ((row & 3u) << 2));
  return FE2O3O_OK;
}

/* examples/tiled_gemm_v1/src/general_reference.rs:171-268.  The plan's
 * storage extents follow general_plan.rs:496-611 (checked_extent per operand,
 * empty output -> no dispatch and empty result). */
int32_t fe2o3o_general_reference_v1(uint32_t m, uint32_t n, uint32_t k,
                                    uint32_t lda, uint32_t ldb, uint32_t ldc,
                                    const uint16_t *a, uint64_t a_len,
                                    const uint16_t *b, uint64_t b_len,
                                    const float *c, uint64_t c_len, float alpha,
                                    float beta, float *out, uint64_t *trace) {
  uint64_t tr[8] = {0};
  uint64_t ea = 0, eb = 0, ec = 0;
  int empty = (m == 0 || n == 0);
  if (!empty) {
    int32_t rc;
    if ((rc = checked_extent(m, k, lda, &ea)) != 0) return rc;
    if ((rc = checked_extent(k, n, ldb, &eb)) != 0) return rc;
    if ((rc = checked_extent(m, n, ldc, &ec)) != 0) return rc;
  }
  if (ea != a_len || eb != b_len || ec != c_len) return FE2O3O_ERR_LENGTH;
  if (empty) {
    if (trace) memcpy(trace, tr, sizeof(tr));
    return FE2O3O_OK;
  }
  uint32_t tile_cols = (n + 15) / 16, tile_rows = (m + 15) / 16;
  uint32_t phases = (k + 15) / 16;
  tr[0] = (uint64_t)tile_cols * tile_rows;
  for (uint32_t gy = 0; gy < tile_rows; ++gy) {
    for (uint32_t gx = 0; gx < tile_cols; ++gx) {
      float acc[256];
      for (int i = 0; i < 256; ++i) acc[i] = 0.0f;
      for (uint32_t ph = 0; ph < phases; ++ph) {
        float a_lds[256], b_lds[256];
        for (int i = 0; i < 256; ++i) a_lds[i] = b_lds[i] = 0.0f;
        for (uint32_t tr_ = 0; tr_ < 16; ++tr_) {
          for (uint32_t td = 0; td < 16; ++td) {
            uint32_t phys;
            fe2o3o_row_major_xor4(tr_, td, &phys);
            uint64_t row = (uint64_t)gy * 16 + tr_, depth = (uint64_t)ph * 16 + td;
            if (row < m && depth < k)
              a_lds[phys] = widen(a[row * lda + depth]);
            else
              tr[4]++;
          }
        }
        for (uint32_t td = 0; td < 16; ++td) {
          for (uint32_t tc = 0; tc < 16; ++tc) {
            uint32_t phys;
            fe2o3o_row_major_xor4(tc, td, &phys);
            uint64_t depth = (uint64_t)ph * 16 + td, col = (uint64_t)gx * 16 + tc;
            if (depth < k && col < n)
              b_lds[phys] = widen(b[depth * ldb + col]);
            else
              tr[5]++;
          }
        }
        tr[1]++;
        tr[2]++;
        for (uint32_t r = 0; r < 16; ++r) {
          for (uint32_t cc = 0; cc < 16; ++cc) {
            for (uint32_t d = 0; d < 16; ++d) {
              uint32_t pa, pb;
              fe2o3o_row_major_xor4(r, d, &pa);
              fe2o3o_row_major_xor4(cc, d, &pb);
              float p = a_lds[pa] * b_lds[pb];
              acc[r * 16 + cc] = acc[r * 16 + cc] + p;
            }
          }
        }
        tr[3]++;
      }
      for (uint32_t r = 0; r < 16; ++r) {
        for (uint32_t cc = 0; cc < 16; ++cc) {
          uint64_t row = (uint64_t)gy * 16 + r, col = (uint64_t)gx * 16 + cc;
          if (row >= m || col >= n) {
            tr[7]++;
            continue;
          }
          float product = alpha * acc[r * 16 + cc];
          float initial = beta * c[row * ldc + col];
          out[row * n + col] = product + initial;
          tr[6]++;
        }
      }
    }
  }
  if (trace) memcpy(trace, tr, sizeof(tr));
  return FE2O3O_OK;
}

/* examples/scalar_gemm_v1/src/harness.rs:87-102 */
void fe2o3o_scalar_gemm(uint32_t m, uint32_t n, uint32_t k, const float *a,
                        const float *b, float *c) {
  for (uint64_t row = 0; row < m; ++row) {
    for (uint64_t col = 0; col < n; ++col) {
      float acc = 0.0f;
      for (uint64_t t = 0; t < k; ++t) {
        float p = a[row * k + t] * b[t * n + col];
        acc = acc + p;
      }
      c[row * n + col] = acc;
    }
  }
}

/* examples/scalar_gemm_v1/src/harness.rs:104-112 */
void fe2o3o_scalar_gemm_inputs(uint64_t a_len, uint64_t b_len, float *a,
                               float *b) {
  for (uint64_t i = 0; i < a_len; ++i)
    a[i] = ((float)((i * 17u) % 29u) - 14.0f) * 0.125f;
  for (uint64_t i = 0; i < b_len; ++i)
    b[i] = ((float)((i * 11u) % 31u) - 15.0f) * 0.0625f;
}

/* Large-shape evaluation of the same per-element recurrence
 * (oracle.rs:306-320): the loops below only change which outputs are
 * computed together (JB independent accumulators, vectorisable across
 * columns); each output still starts at +0 and adds its products in
 * increasing depth order with separate rounding. */
#define JB 16
void fe2o3o_gemm_bf16_nt_rows(uint32_t m, uint32_t n, uint32_t k,
                              const uint16_t *a, const uint16_t *b,
                              uint32_t row_begin, uint32_t row_end, float *out,
                              int32_t threads) {
  (void)m;
  if (row_end <= row_begin) return;
  uint32_t col_blocks = (n + JB - 1) / JB;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    float *bt = (float *)malloc(sizeof(float) * (size_t)k * JB);
    float *arow = (float *)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(dynamic, 1)
    for (uint32_t cb = 0; cb < col_blocks; ++cb) {
      uint32_t c0 = cb * JB;
      uint32_t w = (n - c0) < JB ? (n - c0) : JB;
      for (uint32_t d = 0; d < k; ++d)
        for (uint32_t j = 0; j < JB; ++j)
          bt[(size_t)d * JB + j] = j < w ? widen(b[(size_t)(c0 + j) * k + d]) : 0.0f;
      for (uint32_t row = row_begin; row < row_end; ++row) {
        for (uint32_t d = 0; d < k; ++d) arow[d] = widen(a[(size_t)row * k + d]);
        float acc[JB];
        for (int j = 0; j < JB; ++j) acc[j] = 0.0f;
        for (uint32_t d = 0; d < k; ++d) {
          float av = arow[d];
          const float *bv = bt + (size_t)d * JB;
          for (int j = 0; j < JB; ++j) {
            float p = av * bv[j];
            acc[j] = acc[j] + p;
          }
        }
        float *o = out + (size_t)(row - row_begin) * n + c0;
        for (uint32_t j = 0; j < w; ++j) o[j] = acc[j];
      }
    }
    free(bt);
    free(arow);
  }
}

void fe2o3o_gemm_bf16_nt_points(uint32_t k, const uint16_t *a_rows,
                                const uint16_t *b_cols, uint64_t points,
                                float *out, int32_t threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (uint64_t p = 0; p < points; ++p) {
    const uint16_t *ar = a_rows + p * k;
    const uint16_t *bc = b_cols + p * k;
    float acc = 0.0f;
    for (uint32_t d = 0; d < k; ++d) {
      float prod = widen(ar[d]) * widen(bc[d]);
      acc = acc + prod;
    }
    out[p] = acc;
  }
}

void fe2o3o_gemm_f32_rows(uint32_t m, uint32_t n, uint32_t k, const float *a,
                          const float *b, uint32_t row_begin, uint32_t row_end,
                          float *out, int32_t threads) {
  (void)m;
  if (row_end <= row_begin) return;
  uint32_t col_blocks = (n + JB - 1) / JB;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
  for (uint32_t cb = 0; cb < col_blocks; ++cb) {
    uint32_t c0 = cb * JB;
    uint32_t w = (n - c0) < JB ? (n - c0) : JB;
    for (uint32_t row = row_begin; row < row_end; ++row) {
      float acc[JB];
      for (int j = 0; j < JB; ++j) acc[j] = 0.0f;
      for (uint32_t t = 0; t < k; ++t) {
        float av = a[(size_t)row * k + t];
        const float *bv = b + (size_t)t * n + c0;
        if (w == JB) {
          for (int j = 0; j < JB; ++j) {
            float p = av * bv[j];
            acc[j] = acc[j] + p;
          }
        } else {
          for (uint32_t j = 0; j < w; ++j) {
            float p = av * bv[j];
            acc[j] = acc[j] + p;
          }
        }
      }
      float *o = out + (size_t)(row - row_begin) * n + c0;
      for (uint32_t j = 0; j < w; ++j) o[j] = acc[j];
    }
  }
}
