/*
 * fp8.c -- OCP FP8 E4M3FN ("e4m3fn": bias 7, no infinities, max finite 448,
 * NaN = S.1111.111) encode/decode and the per-tensor-scaled fp8 GEMM oracle.
 *
 * Not in the reference: its only fp8 type is the gfx942 FNUZ encoding
 * (crates/fe2o3-device/src/fp8.rs:53-110, bias 8, max 240), which gfx950's
 * MFMA does not consume.  This restatement follows the OCP 8-bit floating
 * point specification (OFP8, rev 1.0) and is pinned by its closed forms.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "fe2o3_oracle.h"

/* Exact decode: e == 0 -> m * 2^-9 (subnormal), e in 1..15 -> (1 + m/8) *
 * 2^(e-7), except e == 15 && m == 7 -> NaN. */
float fe2o3o_fp8e4m3_to_f32(uint8_t bits) {
  uint32_t s = bits >> 7, e = (bits >> 3) & 0xf, m = bits & 0x7;
  float v;
  if (e == 15 && m == 7) return s ? -NAN : NAN;
  if (e == 0)
    v = ldexpf((float)m, -9);
  else
    v = ldexpf((float)(8 + m), (int)e - 10);
  return s ? -v : v;
}

/* Round-to-nearest-even encode with saturation to +-448 (the OCP "satfinite"
 * conversion); NaN maps to 0x7f with the input sign. */
uint8_t fe2o3o_fp8e4m3_from_f32(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  uint8_t sign = (uint8_t)((bits >> 24) & 0x80);
  if (isnan(value)) return (uint8_t)(sign | 0x7f);
  float a = fabsf(value);
  if (a >= 448.0f) return (uint8_t)(sign | 0x7e);
  /* quantum of the target binade: 2^-9 below 2^-6, else 2^(floor(log2 a)-3) */
  int exp2v;
  frexpf(a, &exp2v); /* a = f * 2^exp2v, f in [0.5, 1) */
  int unbiased = exp2v - 1;
  int q = unbiased < -6 ? -9 : unbiased - 3;
  float scaled = ldexpf(a, -q); /* exact: a is a binary32 value */
  float r = nearbyintf(scaled); /* default rounding mode: ties-to-even */
  float rv = ldexpf(r, q);
  if (rv > 448.0f) rv = 448.0f;
  /* rv is now exactly representable in e4m3: encode it */
  if (rv == 0.0f) return sign;
  int e2;
  frexpf(rv, &e2);
  int ub = e2 - 1;
  if (ub < -6) {
    int m = (int)ldexpf(rv, 9);
    return (uint8_t)(sign | (uint8_t)m);
  }
  int m = (int)ldexpf(rv, -ub + 3) - 8;
  return (uint8_t)(sign | (uint8_t)((ub + 7) << 3) | (uint8_t)m);
}

float fe2o3o_amax_f32(const float *x, uint64_t n, int32_t threads) {
  float amax = 0.0f;
#pragma omp parallel for reduction(max : amax) num_threads(threads > 0 ? threads : 1)
  for (uint64_t i = 0; i < n; ++i) {
    float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  return amax;
}

/* q = e4m3(x / scale) with one correctly rounded f32 division. */
void fe2o3o_quantize_e4m3(const float *x, uint64_t n, float scale,
                          uint8_t *out, int32_t threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (uint64_t i = 0; i < n; ++i) out[i] = fe2o3o_fp8e4m3_from_f32(x[i] / scale);
}

/* acc = sum_k dec(a)*dec(b) in increasing k with separate rounding (each
 * product of two e4m3 values is exact in binary32); c = acc * (sa*sb); the
 * bf16 output is the RNE narrowing of c. */
void fe2o3o_gemm_fp8_points(uint32_t k, const uint8_t *a_rows,
                            const uint8_t *b_cols, uint64_t points,
                            float scale_ab, float *out_f32, uint16_t *out_bf16,
                            int32_t threads) {
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = fe2o3o_fp8e4m3_to_f32((uint8_t)i);
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (uint64_t p = 0; p < points; ++p) {
    const uint8_t *ar = a_rows + p * k;
    const uint8_t *bc = b_cols + p * k;
    float acc = 0.0f;
    for (uint32_t d = 0; d < k; ++d) {
      float prod = lut[ar[d]] * lut[bc[d]];
      acc = acc + prod;
    }
    float c = acc * scale_ab;
    if (out_f32) out_f32[p] = c;
    if (out_bf16) out_bf16[p] = fe2o3o_bf16_from_f32(c);
  }
}

/* Whole output rows row_begin .. row_end-1 of the same recurrence as
 * fe2o3o_gemm_fp8_points (A [m,k], B stored [n,k], both e4m3 bytes):
 * FB8 outputs of a row are accumulated side by side, each from +0 over
 * increasing depth with separate rounding, so every output equals the
 * points form bit for bit.  out_f32 [(row_end-row_begin), n]. */
#define FB8 16
void fe2o3o_gemm_fp8_nt_rows(uint32_t n, uint32_t k, const uint8_t *a, const uint8_t *b,
                             float scale_ab, uint32_t row_begin, uint32_t row_end,
                             float *out_f32, int32_t threads) {
  if (row_end <= row_begin) return;
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = fe2o3o_fp8e4m3_to_f32((uint8_t)i);
  const uint32_t col_blocks = (n + FB8 - 1) / FB8;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    float *bt = (float *)malloc(sizeof(float) * (size_t)k * FB8);
    float *arow = (float *)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(dynamic, 1)
    for (uint32_t cb = 0; cb < col_blocks; ++cb) {
      const uint32_t c0 = cb * FB8, w = (n - c0) < FB8 ? (n - c0) : FB8;
      for (uint32_t d = 0; d < k; ++d)
        for (uint32_t j = 0; j < FB8; ++j)
          bt[(size_t)d * FB8 + j] = j < w ? lut[b[(size_t)(c0 + j) * k + d]] : 0.0f;
      for (uint32_t row = row_begin; row < row_end; ++row) {
        for (uint32_t d = 0; d < k; ++d) arow[d] = lut[a[(size_t)row * k + d]];
        float acc[FB8];
        for (int j = 0; j < FB8; ++j) acc[j] = 0.0f;
        for (uint32_t d = 0; d < k; ++d) {
          const float av = arow[d];
          const float *bv = bt + (size_t)d * FB8;
          for (int j = 0; j < FB8; ++j) {
            float p = av * bv[j];
            acc[j] = acc[j] + p;
          }
        }
        float *o = out_f32 + (size_t)(row - row_begin) * n + c0;
        for (uint32_t j = 0; j < w; ++j) o[j] = acc[j] * scale_ab;
      }
    }
    free(bt);
    free(arow);
  }
}

/* ---- gfx942 FNUZ fp8 (Fp8E4M3Fnuz, Fp8E5M2Fnuz) ----------------------------
 * Restates crates/fe2o3-device/src/fp8.rs:296-381 (f32_to_fnuz, fnuz_to_f32,
 * round_shift_right_ties_even) with the format constants of
 * Fp8E4M3Fnuz::from_f32 / to_f32 (:85-95: 3 fraction bits, bias 8, largest
 * finite 240 = 0x43700000) and Fp8E5M2Fnuz (:193-203: 2 bits, bias 16,
 * 57344 = 0x47600000).  FNUZ: one unsigned zero 0x00, sole NaN 0x80 (widened
 * to the f32 bits 0xffc00000), no infinities; narrowing rounds to nearest,
 * ties to even, saturates finite overflow to +-max, sends NaN and +-inf to
 * 0x80 and everything that rounds to zero (negative zero included) to 0x00.
 * format: 0 = E4M3 FNUZ, 1 = E5M2 FNUZ. */
static void fnuz_format(int32_t format, int *mbits, int *bias, uint32_t *max_bits) {
  if (format == 0) {
    *mbits = 3; *bias = 8; *max_bits = 0x43700000u;
  } else {
    *mbits = 2; *bias = 16; *max_bits = 0x47600000u;
  }
}

/* x / 2^s rounded to nearest, ties to even; x < 2^25 here, so every
 * s >= 64 gives 0. */
static uint64_t shr_rne(uint64_t x, unsigned s) {
  if (s == 0) return x;
  if (s >= 64) return 0; /* x < 2^25: at most 2^-39 of a unit, rounds to 0 */
  uint64_t q = x >> s, r = x & ((1ull << s) - 1ull), half = 1ull << (s - 1);
  return (r > half || (r == half && (q & 1ull))) ? q + 1ull : q;
}

uint8_t fe2o3o_fnuz_from_f32_bits(uint32_t bits, int32_t format) {
  int mb, bias;
  uint32_t maxb;
  fnuz_format(format, &mb, &bias, &maxb);
  const uint32_t mag = bits & 0x7fffffffu;
  const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  if (mag >= 0x7f800000u) return 0x80; /* NaN, +-inf */
  if (mag == 0) return 0;
  if (mag > maxb) return (uint8_t)(sign | 0x7f);
  /* mag = sig * 2^(e - 23); an f32 subnormal (e = -127) is far below every
   * FNUZ quantum and rounds to zero below whichever value sig takes */
  const int e = (int)(mag >> 23) - 127;
  const uint64_t sig = (uint64_t)((mag & 0x7fffffu) | 0x800000u);
  const int emin = 1 - bias; /* exponent of the smallest normal */
  uint32_t code;
  if (e < emin) {
    /* units of the subnormal quantum 2^(emin - mb): sig * 2^(e - 23 - emin + mb) */
    const int s = 23 + emin - mb - e;
    code = (uint32_t)shr_rne(sig, (unsigned)s); /* 2^mb (smallest normal) at most */
    if (code == 0) return 0;
  } else {
    uint64_t m = shr_rne(sig, (unsigned)(23 - mb)); /* in [2^mb, 2^(mb+1)] */
    int ef = e + bias;
    if (m == (1ull << (mb + 1))) {
      m >>= 1;
      ef += 1;
    }
    code = ((uint32_t)ef << mb) | (uint32_t)(m & ((1u << mb) - 1u));
  }
  return (uint8_t)(sign | code);
}

uint32_t fe2o3o_fnuz_to_f32_bits(uint8_t q, int32_t format) {
  int mb, bias;
  uint32_t maxb;
  fnuz_format(format, &mb, &bias, &maxb);
  if (q == 0x80) return 0xffc00000u;
  if (q == 0) return 0;
  /* value = (-1)^s * frac * 2^(emin - mb) (exponent field 0), else
   * (2^mb + frac) * 2^(ef - bias - mb); built as a double, exact, then
   * narrowed (every FNUZ value is an f32 value) */
  const int ef = (q & 0x7f) >> mb, frac = q & ((1 << mb) - 1);
  double v = ef == 0 ? ldexp((double)frac, 1 - bias - mb)
                     : ldexp((double)((1 << mb) + frac), ef - bias - mb);
  float f = (float)((q & 0x80) ? -v : v);
  uint32_t out;
  memcpy(&out, &f, 4);
  return out;
}

void fe2o3o_fnuz_from_f32_array(const float *x, uint64_t n, int32_t format, uint8_t *q) {
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t b;
    memcpy(&b, &x[i], 4);
    q[i] = fe2o3o_fnuz_from_f32_bits(b, format);
  }
}
