// common.hpp -- device vocabulary shared by every gfx950 kernel of the
// library: CDNA4 MFMA operand types, bf16 / fp8 conversions, wave64
// reductions, argument validation helpers and status codes.
//
// Everything here is written for gfx950 (CDNA4, wave64) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fe2o3_mi355x.h"

#define FE2O3_DEVICE __device__ __forceinline__

// ---- MFMA operand vectors ---------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// LDS pointer type expected by the global->LDS builtin.
typedef __attribute__((address_space(3))) void lds_void_t;

namespace fe2o3 {

// ---- bf16 ---------------------------------------------------------------------
// Round-to-nearest-even narrowing with NaN quieting, the rule of
// crates/fe2o3-device/src/half.rs:182-190: NaN keeps sign and high payload
// with bit 0x0040 set; every other value rounds (bits + 0x7fff + lsb) >> 16.
FE2O3_DEVICE uint16_t bf16_bits_from_f32(float v) {
  uint32_t bits = __float_as_uint(v);
  if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu) != 0)
    return (uint16_t)((bits >> 16) | 0x0040u);
  uint32_t lsb = (bits >> 16) & 1u;
  return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}

// Exact widening (half.rs:193-195).
FE2O3_DEVICE float f32_from_bf16_bits(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Two f32 -> packed bf16x2 (low half = first), RNE as above.
FE2O3_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)bf16_bits_from_f32(lo) | ((uint32_t)bf16_bits_from_f32(hi) << 16);
}

// ---- OCP FP8 E4M3FN ----------------------------------------------------------------
// Decoding and RNE/satfinite encoding of the OCP 8-bit float (bias 7, max
// finite 448, NaN = S.1111.111, no infinities).  Encoding is done on the
// exact binary32 value with integer arithmetic so it is bit-reproducible.
FE2O3_DEVICE uint8_t e4m3_from_f32(float v) {
  uint32_t bits = __float_as_uint(v);
  uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  uint32_t mag = bits & 0x7fffffffu;
  if (mag > 0x7f800000u) return (uint8_t)(sign | 0x7f);   // NaN
  if (mag >= 0x43e00000u) return (uint8_t)(sign | 0x7e);  // >= 448 (incl. inf) saturates
  int exp = (int)(mag >> 23);                             // biased binary32 exponent
  uint32_t mant = (mag & 0x7fffffu) | (exp ? 0x800000u : 0u);
  int unbiased = exp ? exp - 127 : -126;
  // target quantum exponent: 2^-9 for subnormal e4m3 (unbiased < -6), else unbiased-3
  int q = unbiased < -6 ? -9 : unbiased - 3;
  // value = mant * 2^(unbiased-23); we want round(value / 2^q) = mant >> (q - unbiased + 23)
  int shift = q - unbiased + 23;  // >= 20
  uint32_t r;
  if (shift >= 32) {
    r = 0;
    // ties: only if mant * 2^-shift == 0.5 exactly, impossible for shift >= 32 with mant < 2^24... except
    // mant == 2^(shift-1) which needs shift-1 <= 23; so r = 0 is exact rounding here.
  } else {
    uint32_t whole = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    r = whole + ((rem > half || (rem == half && (whole & 1u))) ? 1u : 0u);
  }
  // r * 2^q is the rounded magnitude; encode it.
  if (r == 0) return sign;
  if (q == -9) {
    // subnormal quantum: r in 1..8; r == 8 is the smallest normal 2^-6 (e=1, m=0)
    if (r < 8) return (uint8_t)(sign | r);
    return (uint8_t)(sign | 0x08);
  }
  // normal: r in 8..16 (16 means carry into the next binade)
  int e = unbiased + 7;
  if (r == 16) {
    r = 8;
    e += 1;
  }
  uint32_t code = ((uint32_t)e << 3) | (r - 8);
  if (code > 0x7eu) code = 0x7eu;  // 464 and above round-to-nearest saturate to 448
  return (uint8_t)(sign | code);
}

// ---- wave64 reductions ---------------------------------------------------------------
// Butterfly over the 64 lanes with DPP row operations for the in-row steps
// (xor 1, 2, 4, 8 within a row of 16 via quad_perm / row_ror patterns are
// expressed through __shfl_xor, which hipcc lowers to DPP for these
// offsets) and the gfx950 permlane swaps for the cross-row steps.
FE2O3_DEVICE float wave_max(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

FE2O3_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// Exchange a value with lane (l ^ 32) using v_permlane32_swap.
FE2O3_DEVICE float swap_half(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]);
}

// ---- explicit counter waits ---------------------------------------------------------
FE2O3_DEVICE void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
FE2O3_DEVICE void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// 16-byte global -> LDS copy (gfx950 global_load_lds_dwordx4): lane i of the
// wave writes its 16 bytes to lds_base + 16*i.  lds_base must be uniform.
FE2O3_DEVICE void g2l_b128(const void* gptr, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gptr, (lds_void_t*)lds_base, 16, 0, 0);
}

}  // namespace fe2o3

// ---- host-side helpers --------------------------------------------------------------
namespace fe2o3_host {

// Records the outcome of the last launch on this thread and maps it onto the
// library's status space (0 or a positive hipError_t).
inline int32_t launch_status() {
  hipError_t e = hipGetLastError();
  return (int32_t)e;
}

inline bool extent_ok(uint64_t rows, uint64_t cols, uint64_t stride, uint64_t* out) {
  if (rows == 0 || cols == 0) {
    *out = 0;
    return true;
  }
  if (stride < cols) return false;
  *out = (rows - 1) * stride + cols;
  return true;
}

}  // namespace fe2o3_host
