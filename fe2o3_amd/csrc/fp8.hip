// fp8.hip -- per-tensor-scaled OCP fp8 (E4M3FN) quantized GEMM path for
// gfx950: amax reduction, scale = amax / 448, RNE/satfinite quantization,
// and C (bf16) = (scale_a * scale_b) * (A_q . B_q^T) with fp32 accumulation.
//
// The reference has no gfx950 fp8 type (its Fp8E4M3Fnuz,
// crates/fe2o3-device/src/fp8.rs:53-110, is gfx942's FNUZ encoding, bias 8);
// this path follows the OCP 8-bit floating point specification: bias 7, no
// infinities, max finite 448, NaN = S.1111.111, round-to-nearest-even with
// saturation to +-448.
//
// The GEMM reuses the 256x256 tile machinery of the bf16 GEMM: one LDS stage
// is 128 bytes of k per row, i.e. 128 fp8 values, each taken by one
// v_mfma_f32_16x16x128_f8f6f4 (5.0 PFLOP/s dense peak).  Any M
// and N run on it (edge tiles store only their valid rows and columns);
// K not a multiple of 128, or unaligned operands, take a bounds-checked
// 64x64-tile kernel that widens E4M3 to bf16 exactly while staging and
// multiplies on bf16 MFMAs (the products are exact either way); K = 0
// writes +0.
#include "common.hpp"
#include "gemm_core.hpp"
#include "gemm_pipe.hpp"
#include "internal.hpp"

#include <type_traits>

namespace {

using namespace fe2o3;

__global__ void zero_f32_kernel(float* p) { *p = 0.0f; }

// A workgroup step covers 4096 elements as 1024 units of four (unit 256w + t
// for thread t, w = 0..3): four 16-byte loads in flight per thread, each wave
// access 1 KiB contiguous.  The rest
// (fewer than 4096 elements) runs one unit, then one element, per thread.
constexpr uint64_t kStepUnits = 1024;

__global__ void __launch_bounds__(256) amax_kernel(const float* __restrict__ x, uint64_t n,
                                                   float* __restrict__ amax) {
  float m = 0.0f;
  const uint64_t t = threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t units = n / 4, steps = units / kStepUnits;
  const f32x4_t* x4 = reinterpret_cast<const f32x4_t*>(x);
  auto max4 = [](f32x4_t v) {
    return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  };
  for (uint64_t st = blockIdx.x; st < steps; st += gridDim.x) {
    const uint64_t u0 = st * kStepUnits + t;
    f32x4_t v[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = __builtin_nontemporal_load(x4 + u0 + 256 * w);
#pragma unroll
    for (int w = 0; w < 4; ++w) m = fmaxf(m, max4(v[w]));
  }
  for (uint64_t u = steps * kStepUnits + blockIdx.x * blockDim.x + t; u < units; u += stride)
    m = fmaxf(m, max4(x4[u]));
  for (uint64_t i = units * 4 + blockIdx.x * blockDim.x + t; i < n; i += stride)
    m = fmaxf(m, fabsf(x[i]));
  // One device-scope atomic per workgroup: atomics on one address from every
  // wave serialize and cost more than the read of the tensor.
  __shared__ float wave_m[4];
  m = wave_max(m);
  if ((threadIdx.x & 63u) == 0) wave_m[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = fmaxf(fmaxf(wave_m[0], wave_m[1]), fmaxf(wave_m[2], wave_m[3]));
    // |x| >= 0, so the IEEE bit patterns order like unsigned integers
    atomicMax(reinterpret_cast<unsigned int*>(amax), __float_as_uint(m));
  }
}

__global__ void scale_kernel(const float* amax, float* scale) {
  const float a = fmaxf(*amax, 1.17549435e-38f);
  *scale = a / 448.0f;
}

// Same step layout as amax_kernel: four units (16 elements) in flight per
// thread, 16-byte loads and 4-byte stores of codes, each wave access
// contiguous.
__global__ void __launch_bounds__(256) quantize_kernel(const float* __restrict__ x, uint64_t n,
                                                       const float* __restrict__ scale,
                                                       uint8_t* __restrict__ q) {
  const float s = *scale;
  const uint64_t t = threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t units = n / 4, steps = units / kStepUnits;
  const f32x4_t* x4 = reinterpret_cast<const f32x4_t*>(x);
  uint32_t* q4 = reinterpret_cast<uint32_t*>(q);
  auto code4 = [s](f32x4_t v) {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) packed |= (uint32_t)e4m3_from_f32(v[e] / s) << (8 * e);
    return packed;
  };
  for (uint64_t st = blockIdx.x; st < steps; st += gridDim.x) {
    const uint64_t u0 = st * kStepUnits + t;
    f32x4_t v[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = __builtin_nontemporal_load(x4 + u0 + 256 * w);
#pragma unroll
    for (int w = 0; w < 4; ++w) q4[u0 + 256 * w] = code4(v[w]);
  }
  for (uint64_t u = steps * kStepUnits + blockIdx.x * blockDim.x + t; u < units; u += stride)
    q4[u] = code4(x4[u]);
  for (uint64_t i = units * 4 + blockIdx.x * blockDim.x + t; i < n; i += stride)
    q[i] = e4m3_from_f32(x[i] / s);
}

constexpr int kFp8RowBytes = 128, kFp8Stages = 2;
constexpr int kFp8Smem = kFp8Stages * 2 * gemm_pipe::Geo<kFp8RowBytes>::kTileBytes;  // 128 KiB

// STAGED: C leaves through LDS in whole rows with nontemporal stores
// (gemm_pipe::store_bf16_staged), for operands that stream from HBM.
// EDGE: M or N is not a multiple of 256 (or C is not 16-byte aligned): the
// grid covers ceil(M/256) x ceil(N/256) tiles, operand rows past M (N) repeat
// the last valid row, and each tile stores only its valid rows and columns.
// KT: K is a multiple of 16 but not of 128; the last stage is partial and
// its chunks past K load zeros (gemm_pipe::Rows MASK), whose products are
// zero (the generic kernel's zero padding of its last k step).
template <bool STAGED, bool EDGE, bool KT = false>
__global__ void __launch_bounds__(256, 1) gemm_fp8_kernel(const uint8_t* __restrict__ a,
                                                          const uint8_t* __restrict__ b,
                                                          const float* __restrict__ scale_a,
                                                          const float* __restrict__ scale_b,
                                                          uint16_t* __restrict__ c, uint32_t m,
                                                          uint32_t n, uint32_t k, uint32_t xcds) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const uint32_t tiles_m = EDGE ? (m + 255u) / 256u : m / 256u;
  const uint32_t tiles_n = EDGE ? (n + 255u) / 256u : n / 256u;
  uint32_t tm, tn;
  gemm_core::xcd_tile_order(blockIdx.x, tiles_m, tiles_n, xcds, &tm, &tn);
  const uint32_t rows_a = EDGE ? min(256u, m - tm * 256u) : 256u;
  const uint32_t rows_b = EDGE ? min(256u, n - tn * 256u) : 256u;
  const uint32_t k16 = k / 2;  // rows addressed in 16-bit units
  const uint16_t* a16 = reinterpret_cast<const uint16_t*>(a + (uint64_t)tm * 256 * k);
  const uint16_t* b16 = reinterpret_cast<const uint16_t*>(b + (uint64_t)tn * 256 * k);
  const auto ar = gemm_pipe::dense_rows<kFp8RowBytes, 256, KT>(a16, k16, rows_a, k16);
  const auto br = gemm_pipe::dense_rows<kFp8RowBytes, 256, KT>(b16, k16, rows_b, k16);
  // the wave index, read before the K loop: the epilogue needs no thread id
  const uint32_t wave = gemm_pipe::wave_id();
  gemm_pipe::Acc16 acc;
  gemm_pipe::mainloop<gemm_pipe::Fp8Mma16<kFp8RowBytes>, kFp8RowBytes, kFp8Stages, KT>(
      ar, br, k16, smem, acc);
  const float sab = scale_a[0] * scale_b[0];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc.v[i][j][e] *= sab;
  uint16_t* c_tile = c + (uint64_t)tm * 256 * n + (uint64_t)tn * 256;
  if constexpr (EDGE)
    gemm_pipe::store_bf16_edge(acc, c_tile, n, rows_a, rows_b, wave);
  else if constexpr (STAGED)
    gemm_pipe::store_bf16_staged(acc, smem, c_tile, n, wave);
  else
    gemm_pipe::store_bf16(acc, c_tile, n, wave);
}

// The small-grid form: 128 x 128 tiles (Fp8Mma16 with 4 x 4 MFMA tiles per
// wave) for GEMMs whose 256 x 256 tiles would leave most CUs idle; three
// 128-k stages (96 KiB) while the tiles fit one per CU, else two (64 KiB,
// two workgroups per CU).  Every
// output gets the MFMAs of the 256 x 256 tile in the same k order, and the
// same scaling, so C is bit-identical to it.  WHOLE: M and N multiples of
// 128 and C 16-byte aligned; otherwise rows past M (N) repeat the last valid
// row and only valid elements are stored.
template <int STAGES>
constexpr int kFp8SmallSmem = STAGES * 2 * 128 * kFp8RowBytes;
//
// TAIL: the last, partial round of a 256 x 256 grid (tiles first_big .. end
// of gemm_core::xcd_tile_order's list), each as four 128 x 128 quarters
// (gemm_core::tail_quarter).
template <int STAGES, bool WHOLE, bool TAIL = false, bool KT = false>
__global__ void __launch_bounds__(256, STAGES == 2 ? 2 : 1) gemm_fp8_128_kernel(
    const uint8_t* __restrict__ a, const uint8_t* __restrict__ b, const float* __restrict__ scale_a,
    const float* __restrict__ scale_b, uint16_t* __restrict__ c, uint32_t m, uint32_t n,
    uint32_t k, uint32_t xcds, uint32_t first_big = 0) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  uint32_t tm, tn;
  if constexpr (TAIL) {
    if (!gemm_core::tail_quarter(blockIdx.x, first_big, m, n, xcds, &tm, &tn)) return;
  } else {
    gemm_core::xcd_tile_order(blockIdx.x, (m + 127u) / 128u, (n + 127u) / 128u, xcds, &tm, &tn);
  }
  const uint32_t rows_a = WHOLE ? 128u : min(128u, m - tm * 128u);
  const uint32_t rows_b = WHOLE ? 128u : min(128u, n - tn * 128u);
  const uint32_t k16 = k / 2;  // rows addressed in 16-bit units
  const uint16_t* a16 = reinterpret_cast<const uint16_t*>(a + (uint64_t)tm * 128 * k);
  const uint16_t* b16 = reinterpret_cast<const uint16_t*>(b + (uint64_t)tn * 128 * k);
  const auto ar = gemm_pipe::dense_rows<kFp8RowBytes, 128, KT>(a16, k16, rows_a, k16);
  const auto br = gemm_pipe::dense_rows<kFp8RowBytes, 128, KT>(b16, k16, rows_b, k16);
  using Mma = gemm_pipe::Fp8Mma16<kFp8RowBytes, 4, 4>;
  typename Mma::Acc acc;
  gemm_pipe::mainloop<Mma, kFp8RowBytes, STAGES, KT>(ar, br, k16, smem, acc);
  const float sab = scale_a[0] * scale_b[0];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc.v[i][j][e] *= sab;
  gemm_pipe::store_bf16_128<WHOLE>(acc, c + (uint64_t)tm * 128 * n + (uint64_t)tn * 128, n,
                                   rows_a, rows_b);
}

// ---- operand rows the tile cannot read in place ------------------------------------------
// Rows of `cols` E4M3 bytes, `ld` apart from src (any alignment: K not a
// multiple of 16, or a base off a 16-byte boundary), copied into rows of
// dst_cols bytes (a multiple of 16; zeros, E4M3 +0, from cols on) at an
// aligned dst.  16 bytes per thread and step: one load where the piece lies
// inside the row (gfx950 global loads take any alignment), byte by byte at
// the row's end; one 16-byte store.
__global__ void __launch_bounds__(256) repack_bytes_kernel(const uint8_t* __restrict__ src,
                                                           uint32_t rows, uint32_t cols,
                                                           uint32_t ld, uint8_t* __restrict__ dst,
                                                           uint32_t dst_cols) {
  const uint64_t per_row = dst_cols / 16u, groups = (uint64_t)rows * per_row;
  for (uint64_t g = (uint64_t)blockIdx.x * 256u + threadIdx.x; g < groups;
       g += (uint64_t)gridDim.x * 256u) {
    const uint64_t r = g / per_row;
    const uint32_t c0 = (uint32_t)(g % per_row) * 16u;
    const uint8_t* row = src + r * ld;
    u32x4_t p;
    if (c0 + 16u <= cols) {
      __builtin_memcpy(&p, row + c0, 16);
    } else {
      uint8_t v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = c0 + e < cols ? row[c0 + e] : (uint8_t)0;
      __builtin_memcpy(&p, v, 16);
    }
    *reinterpret_cast<u32x4_t*>(dst + r * dst_cols + c0) = p;
  }
}

int32_t repack_bytes(const uint8_t* src, uint32_t rows, uint32_t cols, uint8_t* dst,
                     uint32_t dst_cols, hipStream_t s) {
  const uint64_t g = ((uint64_t)rows * (dst_cols / 16u) + 255u) / 256u;
  repack_bytes_kernel<<<(unsigned)(g < 16384u ? g : 16384u), 256, 0, s>>>(src, rows, cols, cols,
                                                                          dst, dst_cols);
  return fe2o3_host::after_launch();
}

constexpr uint32_t kRepackMin = 128;  // outputs at least this in M and N repack

// ---- any shape ---------------------------------------------------------------------------
// 64x64 output tiles, 32 k per step; each operand element is widened to bf16
// (exact) on its way to LDS, zero outside m x k / n x k, and four waves (2x2,
// 32x32 each) multiply with v_mfma_f32_16x16x32_bf16.  The scale product is
// applied to the fp32 sums, as on the fast path.
constexpr int G8_BM = 64, G8_BN = 64, G8_BK = 32, G8_LDK = G8_BK + 8;

__global__ void __launch_bounds__(256) gemm_fp8_generic_kernel(
    const uint8_t* __restrict__ a, const uint8_t* __restrict__ b, const float* __restrict__ scale_a,
    const float* __restrict__ scale_b, uint16_t* __restrict__ c, uint32_t m, uint32_t n,
    uint32_t k) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[G8_BM * G8_LDK];
  __shared__ __attribute__((aligned(16))) uint16_t b_lds[G8_BN * G8_LDK];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint64_t row0 = (uint64_t)blockIdx.y * G8_BM, col0 = (uint64_t)blockIdx.x * G8_BN;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (uint64_t k0 = 0; k0 < k; k0 += G8_BK) {
    const int r = t >> 2, d0 = (t & 3) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint64_t gd = k0 + d0 + e;
      const uint64_t ga = row0 + r, gb = col0 + r;
      a_lds[r * G8_LDK + d0 + e] = (ga < m && gd < k) ? bf16_bits_from_e4m3(a[ga * k + gd]) : 0;
      b_lds[r * G8_LDK + d0 + e] = (gb < n && gd < k) ? bf16_bits_from_e4m3(b[gb * k + gd]) : 0;
    }
    __syncthreads();
    const int rc = lane & 15, chunk = lane >> 4;
    bf16x8_t af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      af[i] = *reinterpret_cast<const bf16x8_t*>(a_lds + (wm * 32 + i * 16 + rc) * G8_LDK + chunk * 8);
      bf[i] = *reinterpret_cast<const bf16x8_t*>(b_lds + (wn * 32 + i * 16 + rc) * G8_LDK + chunk * 8);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }
  const float sab = scale_a[0] * scale_b[0];
  const int col_in = lane & 15, row_in = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t gr = row0 + wm * 32 + i * 16 + row_in + e;
        const uint64_t gc = col0 + wn * 32 + j * 16 + col_in;
        if (gr < m && gc < n) c[gr * n + gc] = bf16_bits_from_f32(acc[i][j][e] * sab);
      }
}

__global__ void __launch_bounds__(256) zero_fill_bf16_kernel(uint16_t* __restrict__ c, uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) c[i] = 0;
}

// one workgroup per 4096-element step, at most 8192 striding over the rest
unsigned grid_for(uint64_t n) {
  uint64_t b = (n + 4095) / 4096;
  if (b == 0) b = 1;
  return (unsigned)(b < 8192 ? b : 8192);
}

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_amax_f32", "zero_f32_kernel", (const void*)zero_f32_kernel, 1, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_amax_f32", "amax_kernel", (const void*)amax_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_fp8_scale_from_amax", "scale_kernel", (const void*)scale_kernel, 1, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_quantize_e4m3", "quantize_kernel", (const void*)quantize_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_kernel", (const void*)gemm_fp8_kernel<false, false>, 256, kFp8Smem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_kernel<staged>", (const void*)gemm_fp8_kernel<true, false>, 256, kFp8Smem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_kernel<edge>", (const void*)gemm_fp8_kernel<false, true>, 256, kFp8Smem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_kernel<edge, k tail>", (const void*)gemm_fp8_kernel<false, true, true>, 256, kFp8Smem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_kernel<k tail>", (const void*)gemm_fp8_kernel<false, false, true>, 256, kFp8Smem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2, k tail>", (const void*)gemm_fp8_128_kernel<2, true, false, true>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3, k tail>", (const void*)gemm_fp8_128_kernel<3, true, false, true>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2, tail, k tail>", (const void*)gemm_fp8_128_kernel<2, true, true, true>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3, tail, k tail>", (const void*)gemm_fp8_128_kernel<3, true, true, true>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2>", (const void*)gemm_fp8_128_kernel<2, true>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2, edge>", (const void*)gemm_fp8_128_kernel<2, false>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3>", (const void*)gemm_fp8_128_kernel<3, true>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3, edge>", (const void*)gemm_fp8_128_kernel<3, false>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2, tail>", (const void*)gemm_fp8_128_kernel<2, true, true>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2, edge, tail>", (const void*)gemm_fp8_128_kernel<2, false, true>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3, tail>", (const void*)gemm_fp8_128_kernel<3, true, true>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3, edge, tail>", (const void*)gemm_fp8_128_kernel<3, false, true>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2, edge, k tail>", (const void*)gemm_fp8_128_kernel<2, false, false, true>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3, edge, k tail>", (const void*)gemm_fp8_128_kernel<3, false, false, true>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<2, edge, tail, k tail>", (const void*)gemm_fp8_128_kernel<2, false, true, true>, 256, kFp8SmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_128_kernel<3, edge, tail, k tail>", (const void*)gemm_fp8_128_kernel<3, false, true, true>, 256, kFp8SmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "gemm_fp8_generic_kernel", (const void*)gemm_fp8_generic_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "repack_bytes_kernel", (const void*)repack_bytes_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_fp8_nt", "zero_fill_bf16_kernel", (const void*)zero_fill_bf16_kernel, 256, 0})};

}  // namespace

namespace {

// Raises every fast-path kernel's dynamic-LDS limit once per process.
int32_t set_fp8_lds() {
  static const int32_t rc = [] {
    int32_t r = fe2o3_host::set_dynamic_lds(
        {(const void*)gemm_fp8_kernel<false, false>, (const void*)gemm_fp8_kernel<true, false>,
         (const void*)gemm_fp8_kernel<false, true>, (const void*)gemm_fp8_kernel<false, true, true>,
         (const void*)gemm_fp8_kernel<false, false, true>},
        kFp8Smem);
    if (r == FE2O3_OK)
      r = fe2o3_host::set_dynamic_lds(
          {(const void*)gemm_fp8_128_kernel<2, true>, (const void*)gemm_fp8_128_kernel<2, false>,
           (const void*)gemm_fp8_128_kernel<2, true, true>,
           (const void*)gemm_fp8_128_kernel<2, false, true>,
           (const void*)gemm_fp8_128_kernel<2, false, false, true>,
           (const void*)gemm_fp8_128_kernel<2, false, true, true>,
           (const void*)gemm_fp8_128_kernel<2, true, false, true>,
           (const void*)gemm_fp8_128_kernel<2, true, true, true>},
          kFp8SmallSmem<2>);
    if (r == FE2O3_OK)
      r = fe2o3_host::set_dynamic_lds(
          {(const void*)gemm_fp8_128_kernel<3, true>, (const void*)gemm_fp8_128_kernel<3, false>,
           (const void*)gemm_fp8_128_kernel<3, true, true>,
           (const void*)gemm_fp8_128_kernel<3, false, true>,
           (const void*)gemm_fp8_128_kernel<3, false, false, true>,
           (const void*)gemm_fp8_128_kernel<3, false, true, true>,
           (const void*)gemm_fp8_128_kernel<3, true, false, true>,
           (const void*)gemm_fp8_128_kernel<3, true, true, true>},
          kFp8SmallSmem<3>);
    return r;
  }();
  return rc;
}

// The launches of `plan` (tile_plan.hpp).  KT: K not a multiple of 128 (a
// partial last stage in every tile).
template <bool KT>
int32_t launch_fp8(const uint8_t* a, const uint8_t* b, const float* sa, const float* sb,
                   uint16_t* c, uint32_t m, uint32_t n, uint32_t k, const tile_plan::Plan& plan,
                   uint32_t xcds, hipStream_t s) {
  const bool whole = m % 256 == 0 && n % 256 == 0 && ((uintptr_t)c & 15u) == 0;
  const bool whole128 = m % 128 == 0 && n % 128 == 0 && ((uintptr_t)c & 15u) == 0;
  // one launch of 128 x 128 tiles: the whole GEMM (TAIL false) or the tail
  // round's quarters
  auto small = [&](auto stages, auto tail, unsigned grid, uint32_t first) {
    constexpr int S = decltype(stages)::value;
    constexpr bool T = decltype(tail)::value;
    if (whole128)
      gemm_fp8_128_kernel<S, true, T, KT><<<grid, 256, kFp8SmallSmem<S>, s>>>(a, b, sa, sb, c, m,
                                                                              n, k, xcds, first);
    else
      gemm_fp8_128_kernel<S, false, T, KT><<<grid, 256, kFp8SmallSmem<S>, s>>>(a, b, sa, sb, c, m,
                                                                               n, k, xcds, first);
    return fe2o3_host::after_launch();
  };
  using Two = std::integral_constant<int, 2>;
  using Three = std::integral_constant<int, 3>;
  using Whole = std::false_type;
  using Tail = std::true_type;
  if (plan.small)  // 256 x 256 tiles would leave most CUs idle
    return plan.stages == 2 ? small(Two{}, Whole{}, (unsigned)plan.grid, 0u)
                            : small(Three{}, Whole{}, (unsigned)plan.grid, 0u);
  const unsigned big = (unsigned)plan.grid;
  if (!whole)
    gemm_fp8_kernel<false, true, KT><<<big, 256, kFp8Smem, s>>>(a, b, sa, sb, c, m, n, k, xcds);
  else if (!KT && gemm_core::staged_epilogue(((uint64_t)m + n) * k))
    gemm_fp8_kernel<true, false><<<big, 256, kFp8Smem, s>>>(a, b, sa, sb, c, m, n, k, xcds);
  else
    gemm_fp8_kernel<false, false, KT><<<big, 256, kFp8Smem, s>>>(a, b, sa, sb, c, m, n, k, xcds);
  const int32_t big_rc = fe2o3_host::after_launch();
  if (big_rc != FE2O3_OK || !plan.tail) return big_rc;
  // the last round of at most half the CUs' tiles as 128 x 128 quarters; two
  // per CU when there are more quarters than CUs
  return plan.tail_stages == 2
             ? small(Two{}, Tail{}, (unsigned)plan.tail_grid, plan.first_big)
             : small(Three{}, Tail{}, (unsigned)plan.tail_grid, plan.first_big);
}

}  // namespace

extern "C" {

int32_t fe2o3_amax_f32(const float* x, uint64_t x_len, float* amax, void* stream) {
  FE2O3_ENTRY("fe2o3_amax_f32");
  if (!amax || (x_len && !x)) return FE2O3_ERR_NULL;
  if (((uintptr_t)x & 15u) != 0) return FE2O3_ERR_ALIGNMENT;
  hipStream_t s = (hipStream_t)stream;
  zero_f32_kernel<<<1, 1, 0, s>>>(amax);
  // at most 1024 workgroups (4 per CU), each striding over the tensor
  if (x_len) amax_kernel<<<std::min(grid_for(x_len), 1024u), 256, 0, s>>>(x, x_len, amax);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_fp8_scale_from_amax(const float* amax, float* scale, void* stream) {
  FE2O3_ENTRY("fe2o3_fp8_scale_from_amax");
  if (!amax || !scale) return FE2O3_ERR_NULL;
  scale_kernel<<<1, 1, 0, (hipStream_t)stream>>>(amax, scale);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_quantize_e4m3(const float* x, uint64_t x_len, const float* scale, uint8_t* q,
                            uint64_t q_len, void* stream) {
  FE2O3_ENTRY("fe2o3_quantize_e4m3");
  if (x_len != q_len) return FE2O3_ERR_LENGTH;
  if (x_len == 0) return FE2O3_OK;
  if (!x || !scale || !q) return FE2O3_ERR_NULL;
  if (((uintptr_t)x & 15u) != 0 || ((uintptr_t)q & 3u) != 0) return FE2O3_ERR_ALIGNMENT;
  quantize_kernel<<<grid_for(x_len), 256, 0, (hipStream_t)stream>>>(x, x_len, scale, q);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_gemm_fp8_nt(const uint8_t* a, uint64_t a_len, const uint8_t* b, uint64_t b_len,
                          const float* scale_a, const float* scale_b, uint16_t* c, uint64_t c_len,
                          uint32_t m, uint32_t n, uint32_t k, void* stream) {
  FE2O3_ENTRY("fe2o3_gemm_fp8_nt");
  if (a_len != (uint64_t)m * k || b_len != (uint64_t)n * k || c_len != (uint64_t)m * n)
    return FE2O3_ERR_LENGTH;
  if (c_len == 0) return FE2O3_OK;
  if ((a_len && !a) || (b_len && !b) || !c || !scale_a || !scale_b) return FE2O3_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  if (k == 0) {  // the empty sum: +0 (a fill kernel, so the launch can be captured)
    const uint64_t blocks = (c_len + 255) / 256;
    zero_fill_bf16_kernel<<<(unsigned)(blocks < 4096u ? blocks : 4096u), 256, 0, s>>>(c, c_len);
    return fe2o3_host::after_launch();
  }
  // fast path: 16-byte operand rows (K a multiple of 16) and a 256-row fp8
  // panel (256 * k bytes) within its buffer resource's 32-bit range; K not a
  // multiple of 128 takes the edge tiles with a partial last stage
  const bool aligned_a = ((uintptr_t)a & 15u) == 0, aligned_b = ((uintptr_t)b & 15u) == 0;
  const bool fast = k % 16 == 0 && 256ull * k < (1ull << 31) && aligned_a && aligned_b;
  // Rows the tile cannot read in place (K not a multiple of 16, or A or B
  // off a 16-byte boundary) are first copied into aligned rows of kp = K
  // rounded up to 16, zeros from K on, in stream-ordered scratch; the tile
  // then runs on kp, whose zeros fall where its partial last stage puts
  // zeros anyway, so an operand that is only misaligned gives the bits of
  // the aligned one.  Outputs below 128 x 128, and devices without
  // stream-ordered scratch, take the generic kernel.
  const uint32_t kp = (k + 15u) & ~15u;
  const bool repack = !fast && m >= kRepackMin && n >= kRepackMin && 256ull * kp < (1ull << 31);
  void* scratch = nullptr;
  if (repack) {
    const bool ra = k % 16 != 0 || !aligned_a, rb = k % 16 != 0 || !aligned_b;
    const uint64_t a_bytes = ra ? (uint64_t)m * kp : 0, b_bytes = rb ? (uint64_t)n * kp : 0;
    if (fe2o3_host::scratch_alloc(&scratch, a_bytes + b_bytes, s) != FE2O3_OK) {
      (void)hipGetLastError();  // no stream-ordered scratch: the generic kernel
      scratch = nullptr;
    }
  }
  if (!fast && scratch == nullptr) {
    const dim3 grid((n + G8_BN - 1) / G8_BN, (m + G8_BM - 1) / G8_BM);
    if (grid.y > 65535u) return FE2O3_ERR_SHAPE;
    gemm_fp8_generic_kernel<<<grid, 256, 0, s>>>(a, b, scale_a, scale_b, c, m, n, k);
    return fe2o3_host::after_launch();
  }
  // every kernel's LDS limit is raised before anything is launched, so a
  // failure leaves C untouched
  int32_t rc = set_fp8_lds();
  tile_plan::Topology topo;
  if (rc == FE2O3_OK) rc = fe2o3_host::device_topology(&topo);
  const tile_plan::Plan plan = rc == FE2O3_OK ? tile_plan::plan(m, n, topo) : tile_plan::Plan{};
  if (rc == FE2O3_OK && (plan.grid > 0x7fffffffu || plan.tail_grid > 0x7fffffffu))
    rc = FE2O3_ERR_SHAPE;
  const uint8_t* ta = a;
  const uint8_t* tb = b;
  uint32_t tk = k;
  if (rc == FE2O3_OK && scratch != nullptr) {
    const bool ra = k % 16 != 0 || !aligned_a, rb = k % 16 != 0 || !aligned_b;
    uint8_t* ap = static_cast<uint8_t*>(scratch);
    uint8_t* bp = ap + (ra ? (uint64_t)m * kp : 0);
    if (ra) rc = repack_bytes(a, m, k, ap, kp, s);
    if (rb && rc == FE2O3_OK) rc = repack_bytes(b, n, k, bp, kp, s);
    ta = ra ? ap : a;
    tb = rb ? bp : b;
    tk = kp;
  }
  if (rc == FE2O3_OK)
    rc = tk % 128 != 0 ? launch_fp8<true>(ta, tb, scale_a, scale_b, c, m, n, tk, plan, topo.xcds, s)
                       : launch_fp8<false>(ta, tb, scale_a, scale_b, c, m, n, tk, plan, topo.xcds, s);
  if (scratch != nullptr) {
    const int32_t free_rc = fe2o3_host::scratch_free(scratch, s);
    if (rc == FE2O3_OK) rc = free_rc;
  }
  return rc;
}

}  // extern "C"
