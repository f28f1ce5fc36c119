// fp8_codec.hpp -- OCP FP8 E4M3FN encoding (bias 7, max finite 448, no
// infinities, NaN = S.1111.111) by round-to-nearest-even with saturation to
// +-448, done on the exact binary32 bits with integer arithmetic only.
//
// Plain C++ so the same function compiles for gfx950 (device code) and for
// the host (the CPU test compares it with the oracle over every binary32
// bit pattern).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FE2O3_HD __host__ __device__ __forceinline__
#else
#define FE2O3_HD inline
#endif

namespace fe2o3 {

FE2O3_HD uint8_t e4m3_from_bits(uint32_t bits) {
  const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  const uint32_t mag = bits & 0x7fffffffu;
  if (mag > 0x7f800000u) return (uint8_t)(sign | 0x7f);   // NaN
  if (mag >= 0x43e00000u) return (uint8_t)(sign | 0x7e);  // |x| >= 448 (and inf) saturate
  const int exp = (int)(mag >> 23);                       // biased binary32 exponent
  const uint32_t mant = (mag & 0x7fffffu) | (exp ? 0x800000u : 0u);
  const int unbiased = exp ? exp - 127 : -126;
  // quantum of the target e4m3 binade: 2^-9 when subnormal, else 2^(unbiased-3)
  const int q = unbiased < -6 ? -9 : unbiased - 3;
  // |x| = mant * 2^(unbiased-23); r = round(|x| / 2^q) = round(mant / 2^shift)
  const int shift = q - unbiased + 23;  // >= 20
  uint32_t r = 0;
  if (shift < 32) {  // shift >= 32 leaves mant / 2^shift < 1/2: rounds to 0
    const uint32_t whole = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    r = whole + ((rem > half || (rem == half && (whole & 1u))) ? 1u : 0u);
  }
  if (r == 0) return sign;
  if (unbiased < -6) return (uint8_t)(sign | (r < 8 ? r : 0x08u));  // r == 8 is 2^-6, the first normal
  int e = unbiased + 7;
  if (r == 16) {  // rounding carried into the next binade
    r = 8;
    e += 1;
  }
  uint32_t code = ((uint32_t)e << 3) | (r - 8);
  if (code > 0x7eu) code = 0x7eu;  // values rounding above 448 saturate
  return (uint8_t)(sign | code);
}

// E4M3FN -> bf16 bits, exact: every E4M3 value has at most 4 significant
// bits and an exponent in [-9, 8], which bf16 holds exactly.  NaN
// (S.1111.111) becomes a quiet bf16 NaN of the same sign; subnormals m*2^-9
// are normalized.
FE2O3_HD uint16_t bf16_bits_from_e4m3(uint8_t q) {
  const uint32_t sign = ((uint32_t)q & 0x80u) << 8;
  const uint32_t e = ((uint32_t)q >> 3) & 15u, m = (uint32_t)q & 7u;
  if (e == 15u && m == 7u) return (uint16_t)(sign | 0x7fc0u);
  if (e != 0u) return (uint16_t)(sign | ((e + 120u) << 7) | (m << 4));
  if (m == 0u) return (uint16_t)sign;
  // m * 2^-9 with the leading one of m at bit p (0..2): 2^(p-9) * 1.f
  const uint32_t p = m >= 4u ? 2u : (m >= 2u ? 1u : 0u);
  const uint32_t frac = (m << (3u - p)) & 7u;
  return (uint16_t)(sign | ((p + 118u) << 7) | (frac << 4));
}

}  // namespace fe2o3
