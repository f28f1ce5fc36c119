/*
 * common.c -- numeric vocabulary and deterministic input generators.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).
 */
#include <string.h>

#include "fe2o3_oracle.h"

static uint32_t f32_bits(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  return b;
}

static float bits_f32(uint32_t b) {
  float v;
  memcpy(&v, &b, 4);
  return v;
}

/* crates/fe2o3-device/src/half.rs:182-190: RNE narrowing, NaNs keep sign and
 * high payload and are quieted with bit 0x0040. */
uint16_t fe2o3o_bf16_from_f32(float value) {
  uint32_t bits = f32_bits(value);
  if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu) != 0) {
    return (uint16_t)((bits >> 16) | 0x0040u);
  }
  uint32_t lsb = (bits >> 16) & 1u;
  return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}

/* crates/fe2o3-device/src/half.rs:193-195 and
 * examples/tiled_gemm_v1/src/numerical_contract.rs:292-295: exact widening. */
float fe2o3o_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

void fe2o3o_bf16_from_f32_array(const float *in, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = fe2o3o_bf16_from_f32(in[i]);
}

void fe2o3o_bf16_to_f32_array(const uint16_t *in, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = fe2o3o_bf16_to_f32(in[i]);
}

/* examples/tiled_gemm_v1/src/inputs.rs:57-62 (SplitMix64 finaliser). */
uint64_t fe2o3o_mix64(uint64_t value) {
  value += 0x9e3779b97f4a7c15ull;
  value = (value ^ (value >> 30)) * 0xbf58476d1ce4e5b9ull;
  value = (value ^ (value >> 27)) * 0x94d049bb133111ebull;
  return value ^ (value >> 31);
}

static uint64_t rotl64(uint64_t v, unsigned r) {
  return r == 0 ? v : (v << r) | (v >> (64 - r));
}

/* examples/tiled_gemm_v1/src/inputs.rs:12-29: the 16-entry pinned alphabet. */
static const uint16_t kBf16InputPatternV1[16] = {
    0x0000, 0x3d80, 0xbd80, 0x3e00, 0xbe00, 0x3e80, 0xbe80, 0x3f00,
    0xbf00, 0x3f80, 0xbf80, 0x4000, 0xc000, 0x4040, 0xc040, 0x4080};

static const uint64_t kADomainV1 = 0x5d7a91c431e2b80full; /* inputs.rs:31 */
static const uint64_t kBDomainV1 = 0xa2c56e3bce1d47f0ull; /* inputs.rs:32 */

/* inputs.rs:64-70 */
static uint64_t shape_identity(uint32_t m, uint32_t n, uint32_t k) {
  return fe2o3o_mix64((uint64_t)m ^ rotl64((uint64_t)n, 21) ^
                      rotl64((uint64_t)k, 42));
}

/* inputs.rs:72-78 */
static uint16_t generated_value(uint64_t shape_id, uint64_t seed,
                                uint64_t domain, uint64_t index) {
  uint64_t selector =
      fe2o3o_mix64(seed ^ shape_id ^ domain ^ (index * 0xd6e8feb86659fd93ull));
  return kBf16InputPatternV1[selector % 16u];
}

/* inputs.rs:80-88.  Empty output (M==0 or N==0) has zero-length operands
 * (contract.rs:151-160); callers size a/b accordingly. */
void fe2o3o_generate_inputs_v1(uint32_t m, uint32_t n, uint32_t k, uint64_t seed,
                               uint16_t *a, uint16_t *b) {
  if (m == 0 || n == 0) return;
  uint64_t sid = shape_identity(m, n, k);
  uint64_t a_len = (uint64_t)m * k, b_len = (uint64_t)k * n;
  for (uint64_t i = 0; i < a_len; ++i) a[i] = generated_value(sid, seed, kADomainV1, i);
  for (uint64_t i = 0; i < b_len; ++i) b[i] = generated_value(sid, seed, kBDomainV1, i);
}

static int in_alphabet(uint16_t bits) {
  for (int i = 0; i < 16; ++i)
    if (kBf16InputPatternV1[i] == bits) return 1;
  return 0;
}

/* examples/tiled_gemm_v1/src/oracle.rs:199-252: exact lengths, then per
 * element NaN, infinity, subnormal, alphabet, in that order. */
static int32_t validate_operand(uint64_t expected, const uint16_t *v,
                                uint64_t len, uint64_t *index) {
  if (len != expected) {
    *index = len;
    return FE2O3O_ERR_LENGTH;
  }
  for (uint64_t i = 0; i < len; ++i) {
    uint16_t bits = v[i];
    uint16_t e = bits & 0x7f80u, f = bits & 0x007fu;
    *index = i;
    if (e == 0x7f80u && f != 0) return FE2O3O_ERR_NONFINITE;
    if (e == 0x7f80u) return FE2O3O_ERR_INFINITE;
    if (e == 0 && f != 0) return FE2O3O_ERR_SUBNORMAL;
    if (!in_alphabet(bits)) return FE2O3O_ERR_ALPHABET;
  }
  return FE2O3O_OK;
}

int32_t fe2o3o_validate_evidence_inputs_v1(uint32_t m, uint32_t n, uint32_t k,
                                           const uint16_t *a, uint64_t a_len,
                                           const uint16_t *b, uint64_t b_len,
                                           int32_t *operand, uint64_t *index) {
  uint64_t ea = (m == 0 || n == 0) ? 0 : (uint64_t)m * k;
  uint64_t eb = (m == 0 || n == 0) ? 0 : (uint64_t)k * n;
  uint64_t idx = 0;
  int32_t rc = validate_operand(ea, a, a_len, &idx);
  if (rc != FE2O3O_OK) {
    if (operand) *operand = 0;
    if (index) *index = idx;
    return rc;
  }
  rc = validate_operand(eb, b, b_len, &idx);
  if (rc != FE2O3O_OK) {
    if (operand) *operand = 1;
    if (index) *index = idx;
  }
  return rc;
}

/* ---- this build's counter-based generators -------------------------------
 * Not in the reference (it only has the 16-value dyadic alphabet above).  The
 * BASELINE configurations ask for N(0,1) and U[-1,1] inputs; these are
 * produced from integer hashes so the GPU fill kernels reproduce them bit for
 * bit:
 *   hash(i)   = mix64(seed ^ domain ^ i * 0xd6e8feb86659fd93)  (inputs.rs:72)
 *   normal(i) = Irwin-Hall(12): the sum of twelve 16-bit uniforms taken from
 *               hash(3i), hash(3i+1), hash(3i+2), centred and scaled by 2^-16.
 *               Mean 0, variance 1 (to 1e-9), support [-6, 6].  Every step is
 *               exact: the centred integer sum is below 2^20.
 *   uniform(i)= ((hash(i) >> 40) - 2^23) * 2^-23, 24-bit uniform on [-1, 1).
 * A caller scale is applied with one f32 RNE multiply. */
static uint64_t counter_hash(uint64_t seed, uint64_t domain, uint64_t index) {
  return fe2o3o_mix64(seed ^ domain ^ (index * 0xd6e8feb86659fd93ull));
}

float fe2o3o_counter_normal(uint64_t seed, uint64_t domain, uint64_t index) {
  int64_t sum = 0;
  for (uint64_t j = 0; j < 3; ++j) {
    uint64_t h = counter_hash(seed, domain, 3 * index + j);
    sum += (int64_t)(h & 0xffff) + (int64_t)((h >> 16) & 0xffff) +
           (int64_t)((h >> 32) & 0xffff) + (int64_t)(h >> 48);
  }
  int32_t centred = (int32_t)(sum - 393210); /* 12 * 32767.5 */
  return (float)centred * 0x1p-16f;
}

float fe2o3o_counter_uniform_pm1(uint64_t seed, uint64_t domain, uint64_t index) {
  uint64_t h = counter_hash(seed, domain, index);
  int32_t v = (int32_t)(h >> 40) - (1 << 23);
  return (float)v * 0x1p-23f;
}

void fe2o3o_fill_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed,
                             uint64_t domain, float scale, uint64_t first_index) {
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    float x = fe2o3o_counter_normal(seed, domain, first_index + i);
    out[i] = fe2o3o_bf16_from_f32(x * scale);
  }
}

void fe2o3o_fill_normal_f32(float *out, uint64_t n, uint64_t seed,
                            uint64_t domain, float scale, uint64_t first_index) {
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    float x = fe2o3o_counter_normal(seed, domain, first_index + i);
    out[i] = x * scale;
  }
}

void fe2o3o_fill_uniform_f32(float *out, uint64_t n, uint64_t seed,
                             uint64_t domain, uint64_t first_index) {
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i)
    out[i] = fe2o3o_counter_uniform_pm1(seed, domain, first_index + i);
}
