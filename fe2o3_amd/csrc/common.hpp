// common.hpp -- device vocabulary shared by every gfx950 kernel of the
// library: CDNA4 MFMA operand types, bf16 / fp8 conversions, wave64
// reductions, argument validation helpers and status codes.
//
// Everything here is written for gfx950 (CDNA4, wave64) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fe2o3_mi355x.h"
#include "fp8_codec.hpp"

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
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

namespace fe2o3 {

// ---- bf16 ---------------------------------------------------------------------
// Round-to-nearest-even narrowing with NaN quieting, the rule of
// crates/fe2o3-device/src/half.rs:182-190: NaN keeps sign and high payload
// with bit 0x0040 set; every other value rounds (bits + 0x7fff + lsb) >> 16.
// gfx950's v_cvt_pk_bf16_f32 computes exactly this rule, two values per
// instruction, under the kernels' floating-point mode (IEEE, f32 denormals
// kept): a GPU sweep of all 2^32 binary32 patterns through each half of the
// instruction found no difference from the rule written out, and
// tests/test_gpu_bf16_convert.py repeats that sweep through
// fe2o3_bf16_from_f32.  Written out, the rule takes ~13 instructions per
// value, 7 of them scalar exec-mask operations around the NaN branch (a
// 256x256 GEMM epilogue: 3,381 instructions per wave, 498 with the
// instruction).  Bit-identical outputs throughout; fp8 GEMM 8192^3 +3%, MoE
// layer +1%, bf16 GEMM 4096^3 +0.5% (its C stores are bound by the write
// path, which hid most of that work).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16x2 (low half = first): one v_cvt_pk_bf16_f32.
FE2O3_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

FE2O3_DEVICE uint16_t bf16_bits_from_f32(float v) {
  return __builtin_bit_cast(uint16_t, (__bf16)v);
}

// Exact widening (half.rs:193-195).
FE2O3_DEVICE float f32_from_bf16_bits(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// ---- OCP FP8 E4M3FN ----------------------------------------------------------------
FE2O3_DEVICE uint8_t e4m3_from_f32(float v) { return e4m3_from_bits(__float_as_uint(v)); }

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

// Exchange a value with lane (l ^ 32) using v_permlane32_swap.  The
// instruction swaps the upper half of its first operand with the lower half
// of its second; with both operands = v, the first result holds v[l-32] in
// lanes 32..63 and the second holds v[l+32] in lanes 0..31.
FE2O3_DEVICE float swap_half(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32u) ? r[0] : r[1]);
}

// ---- finiteness -----------------------------------------------------------------------
// fma(x, 0, acc) leaves acc unchanged (0) for every finite x and makes it NaN
// for a NaN or an infinity (inf * 0 = NaN, and NaN propagates), so one FMA
// per element carries "some element was not finite" through a loop that
// already touches every element.
FE2O3_DEVICE float finite_probe(float acc, float x) { return __builtin_fmaf(x, 0.0f, acc); }

// Counts one rejection in the device's non-finite counter
// (fe2o3_host::status_word) with a vector atomic add; only the rejecting
// path calls it, from one lane.  The counter is never cleared: the host
// reports each change of it once (status_track.hpp).
FE2O3_DEVICE void mark_nonfinite(uint32_t* status) {
  __hip_atomic_fetch_add(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Canonical quiet NaN, the sentinel output of a rejected row or tile.
FE2O3_DEVICE float quiet_nan() { return __uint_as_float(0x7fc00000u); }

// ---- explicit counter waits ---------------------------------------------------------
FE2O3_DEVICE void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
FE2O3_DEVICE void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier that completes this wave's LDS operations first but,
// unlike __syncthreads(), leaves its outstanding global loads (including
// global->LDS copies of later pipeline stages) in flight.  Callers order
// those copies with explicit s_waitcnt vmcnt(N) before the barrier.
FE2O3_DEVICE void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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
