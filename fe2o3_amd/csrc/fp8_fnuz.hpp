// fp8_fnuz.hpp -- gfx942 FNUZ fp8 element conversions (the value semantics
// of crates/fe2o3-device/src/fp8.rs:296-381), one code <-> one f32.
//
// Plain C++ so the same functions compile for gfx950 (fp8_fnuz.hip) and for
// the host, where a CPU test checks them on every f32 input against the
// oracle.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FE2O3_HD __host__ __device__ __forceinline__
#else
#define FE2O3_HD inline
#endif

namespace fe2o3 {

// FMT 0: E4M3 FNUZ (3 fraction bits, bias 8, max 240); FMT 1: E5M2 FNUZ (2,
// 16, 57344).  One unsigned zero 0x00, sole NaN 0x80, no infinities.
template <int FMT>
struct Fnuz {
  static constexpr int kMb = FMT == 0 ? 3 : 2;  // fraction bits
  static constexpr int kBias = FMT == 0 ? 8 : 16;
  static constexpr int kEmin = 1 - kBias;       // exponent of the smallest normal
  static constexpr uint32_t kMax = FMT == 0 ? 0x43700000u : 0x47600000u;  // 240, 57344
};

// f32 bits -> FNUZ code: round to nearest, ties to even; a magnitude above
// the largest finite value saturates (it is clamped to that value, whose
// code is 0x7f); NaN and +-inf give 0x80; a result of zero drops the sign.
//   With E the biased f32 exponent and sig the 24-bit significand, the value
//   is sig * 2^(E-150); in units of the target quantum 2^(max(E-127, emin) -
//   mb) it is sig >> s, s = 23 - mb + max(emin + 127 - E, 0), clamped to 31
//   (sig < 2^24, so any shift of 25 or more gives 0), rounded to nearest even
//   by adding half a unit less one plus the kept lsb.  That gives q in
//   [2^mb, 2^(mb+1)] for a normal result (the top value is the carry into
//   the next binade) and in [0, 2^mb] below it; the code is then
//   (max(E - 128 + bias, 0) << mb) + q, so a carry lands in the exponent
//   field.  An f32 subnormal or zero shifts out entirely (q = 0).
//   The sign: code | (sign & (code + 0x7f)) keeps bit 7 exactly when
//   code >= 1 (code <= 0x7f), so zero is unsigned.
template <int FMT>
FE2O3_HD uint32_t fnuz_code(uint32_t bits) {
  using F = Fnuz<FMT>;
  const uint32_t mag = bits & 0x7fffffffu;
  const uint32_t m = mag < F::kMax ? mag : F::kMax;
  const int E = (int)(m >> 23);
  const uint32_t sig = (m & 0x7fffffu) | 0x800000u;
  int s = 23 - F::kMb + (F::kEmin + 127) - E;
  s = s > 23 - F::kMb ? s : 23 - F::kMb;
  s = s < 31 ? s : 31;
  const uint32_t q = (sig + ((1u << (s - 1)) - 1u) + ((sig >> s) & 1u)) >> s;
  const int ef = E - 128 + F::kBias;
  const uint32_t code = ((uint32_t)(ef > 0 ? ef : 0) << F::kMb) + q;
  const uint32_t r = code | (((bits >> 24) & 0x80u) & (code + 0x7fu));
  return mag >= 0x7f800000u ? 0x80u : r;
}

// FNUZ code -> f32 bits, exact: (2^mb + frac) * 2^(ef - bias - mb) for a
// nonzero exponent field ef, frac * 2^(emin - mb) for ef = 0 -- a small
// integer times a power of two in the normal f32 range.  0x80 gives
// 0xffc00000, the negative quiet NaN gfx942 widens it to.
template <int FMT>
FE2O3_HD uint32_t fnuz_bits(uint32_t code) {
  using F = Fnuz<FMT>;
  const uint32_t ef = (code & 0x7fu) >> F::kMb, frac = code & ((1u << F::kMb) - 1u);
  const int k = (ef ? (int)ef : 1) - F::kBias - F::kMb;
  const float m = (float)(ef ? (frac | (1u << F::kMb)) : frac);
  const float p2 = __builtin_bit_cast(float, (uint32_t)(k + 127) << 23);
  const uint32_t v = __builtin_bit_cast(uint32_t, m * p2) | ((code & 0x80u) << 24);
  // 0x80 has m = 0, so v is the sign bit alone: add the quiet-NaN exponent
  // and payload (a mask, not a branch)
  return v | ((0u - (uint32_t)(code == 0x80u)) & 0x7fc00000u);
}

}  // namespace fe2o3
