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

// Branch-free (the kernels run it per lane, where a branch per case would
// diverge): the magnitude is clamped to 448 (code 0x7e), which saturates
// larger values and infinities; with E the biased binary32 exponent and sig
// the 24-bit significand, the value in units of the target quantum
// 2^(max(E-127, -6) - 3) is sig >> s, s = 20 + max(121 - E, 0) clamped to 31
// (sig < 2^24, so any shift of 25 or more gives 0), rounded to nearest even
// by adding half a unit less one plus the kept lsb.  The code is then
// (max(E - 121, 0) << 3) + q: a carry into the next binade lands in the
// exponent field, and a subnormal result needs no separate path.  Zero keeps
// its sign (OCP E4M3FN has -0); NaN gives S.1111.111.
FE2O3_HD uint8_t e4m3_from_bits(uint32_t bits) {
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t mag = bits & 0x7fffffffu;
  const uint32_t m = mag < 0x43e00000u ? mag : 0x43e00000u;
  const int E = (int)(m >> 23);
  const uint32_t sig = (m & 0x7fffffu) | 0x800000u;
  int s = 141 - E;
  s = s > 20 ? s : 20;
  s = s < 31 ? s : 31;
  const uint32_t q = (sig + ((1u << (s - 1)) - 1u) + ((sig >> s) & 1u)) >> s;
  const int ef = E - 121;
  const uint32_t code = ((uint32_t)(ef > 0 ? ef : 0) << 3) + q;
  return (uint8_t)(mag > 0x7f800000u ? (sign | 0x7fu) : (sign | code));
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
