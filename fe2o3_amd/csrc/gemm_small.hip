// gemm_small.hip -- the reference's fixed-profile and general GEMM kernels,
// rebuilt for gfx950:
//   * tiled_gemm_lds_slice1 / moe_expert_gemm_bf16_m16_n16_k16: one 16x16x16
//     bf16 tile, one wave64, LDS staging, one v_mfma_f32_16x16x32_bf16 with
//     the upper K half zero;
//   * tiled_gemm_general_v1: any m, n, k, strides, alpha/beta; 64x64 output
//     tiles per 256-thread workgroup, guarded zero-filled loads, MFMA
//     16x16x32 bf16, unfused alpha/beta epilogue;
//   * scalar_gemm_v1: f32, the reference's per-output sequential unfused
//     recurrence, LDS-tiled and register-blocked (4x4 outputs per thread),
//     bit-identical to the scalar oracle.
#include "common.hpp"
#include "gemm_core.hpp"
#include "gemm_pipe.hpp"
#include "internal.hpp"

namespace {

using namespace fe2o3;

// ---- 16x16x16 bf16 tile ------------------------------------------------------------
// A row-major [16 rows][16 k]; B row-major [16 k][16 n]; C row-major f32.
// LDS holds A as [row][k] and B transposed as [n][k] so both MFMA operands
// are one 16-byte read: lane l < 32 reads row/col l%16, k-chunk l/16 (8 k
// values); lanes 32..63 feed zeros for the unused upper K half.  The output
// fragment of lane l is column l%16, rows 4*(l/16)+i (i = 0..3), i.e. the
// reference's Blocked<Index1D,16,4> ownership
// (crates/fe2o3-device/src/thread.rs:569-600) of the row-major C tile.
__global__ void __launch_bounds__(64) tile16_bf16_kernel(const uint16_t* __restrict__ a,
                                                         const uint16_t* __restrict__ b,
                                                         float* __restrict__ c) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[16 * 16];
  __shared__ __attribute__((aligned(16))) uint16_t bt_lds[16 * 16];
  const int l = threadIdx.x;
  // stage: lane l owns elements 4l..4l+3 of each operand
  {
    const uint2 av = *reinterpret_cast<const uint2*>(a + 4 * l);
    *reinterpret_cast<uint2*>(a_lds + 4 * l) = av;
    const uint2 bv = *reinterpret_cast<const uint2*>(b + 4 * l);
    const int kk = l >> 2, n0 = (l & 3) * 4;
    bt_lds[(n0 + 0) * 16 + kk] = (uint16_t)(bv.x & 0xffffu);
    bt_lds[(n0 + 1) * 16 + kk] = (uint16_t)(bv.x >> 16);
    bt_lds[(n0 + 2) * 16 + kk] = (uint16_t)(bv.y & 0xffffu);
    bt_lds[(n0 + 3) * 16 + kk] = (uint16_t)(bv.y >> 16);
  }
  __syncthreads();
  bf16x8_t af = {}, bf = {};
  if (l < 32) {
    const int rc = l & 15, chunk = l >> 4;
    af = *reinterpret_cast<const bf16x8_t*>(a_lds + rc * 16 + chunk * 8);
    bf = *reinterpret_cast<const bf16x8_t*>(bt_lds + rc * 16 + chunk * 8);
  }
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, acc, 0, 0, 0);
  const int col = l & 15, row0 = (l >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) c[(row0 + i) * 16 + col] = acc[i];
}

// ---- exact-tile multi-tile GEMM (tiled_gemm_v1 plan) ---------------------------------
// C[M,N] f32 = A[M,K] bf16 (row-major) * B[K,N] bf16 (row-major), M, N, K
// multiples of 16.  One wave64 per 16x16 output tile, as the reference's plan
// assigns (examples/tiled_gemm_v1/src/contract.rs:387-427); workgroup id ->
// (tile column, tile row) = (id % tile_cols, id / tile_cols).  Each
// v_mfma_f32_16x16x32_bf16 consumes two 16-deep reduction tiles; with an odd
// count the last MFMA's upper half is zero.  Operand lanes: A row l%16 and
// B column l%16, k chunk 8*(l/16) .. +7 of the 32-deep step, read straight
// from global memory (a chunk lies wholly inside or wholly past K).  The
// output lane map is tile16_bf16_kernel's.
__global__ void __launch_bounds__(64) tiled_v1_kernel(const uint16_t* __restrict__ a,
                                                      const uint16_t* __restrict__ b,
                                                      float* __restrict__ c, uint32_t n,
                                                      uint32_t k, uint32_t tile_cols) {
  const uint32_t l = threadIdx.x;
  const uint32_t tr = blockIdx.x / tile_cols, tc = blockIdx.x % tile_cols;
  const uint32_t rc = l & 15u, chunk = l >> 4;
  const uint16_t* arow = a + (uint64_t)(tr * 16u + rc) * k;
  const uint16_t* bcol = b + tc * 16u + rc;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t kk = 0; kk < k; kk += 32u) {
    const uint32_t k0 = kk + 8u * chunk;
    bf16x8_t af = {}, bf = {};
    if (k0 < k) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        af[i] = __builtin_bit_cast(__bf16, arow[k0 + i]);
        bf[i] = __builtin_bit_cast(__bf16, bcol[(uint64_t)(k0 + i) * n]);
      }
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, acc, 0, 0, 0);
  }
  float* ctile = c + (uint64_t)(tr * 16u + 4u * chunk) * n + tc * 16u + rc;
#pragma unroll
  for (int i = 0; i < 4; ++i) ctile[(uint64_t)i * n] = acc[i];
}

// +0 fill of the plan's K = 0 case (a kernel rather than a memset, so the
// call can sit inside a captured graph).
__global__ void __launch_bounds__(256) zero_fill_kernel(float* __restrict__ c, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u)
    c[i] = 0.0f;
}

// ---- general bf16 GEMM with alpha/beta -----------------------------------------------
// C[r*ldc+j] = alpha * (A B)[r][j] + beta * C[r*ldc+j] for r < m, j < n.
// A row-major (lda), B row-major [k][n] (ldb).  Workgroup tile 64x64, K step
// 32, four waves in a 2x2 arrangement each owning 32x32 (2x2 MFMA tiles).
constexpr int G_BM = 64, G_BN = 64, G_BK = 32;
constexpr int G_LDK = G_BK + 8;  // padded LDS row (bf16 elements), 80 bytes

// Two global-transfer schedules of the same kernel, as the reference has two
// (crates/dialect-schedule/src/general_gemm.rs:13-38): VEC_A = false stages
// every A and B element with a masked scalar load; VEC_A = true loads each
// full, in-range, 8-byte-aligned group of 4 A elements with one 8-byte load
// and falls back to masked scalar loads for the rest (tails, misaligned
// rows); B stays scalar.  The staged tiles, hence the results, are the same.
template <bool VEC_A>
__global__ void __launch_bounds__(256) gemm_general_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, float* __restrict__ c,
    uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, float alpha,
    float beta) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[G_BM * G_LDK];
  __shared__ __attribute__((aligned(16))) uint16_t bt_lds[G_BN * G_LDK];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint64_t row0 = (uint64_t)blockIdx.y * G_BM, col0 = (uint64_t)blockIdx.x * G_BN;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const uint32_t phases = (k + G_BK - 1) / G_BK;
  for (uint32_t ph = 0; ph < phases; ++ph) {
    const uint64_t k0 = (uint64_t)ph * G_BK;
    // A: thread t loads row t/4, depths (t%4)*8 .. +7 (zero outside m x k)
    {
      const int r = t >> 2, d0 = (t & 3) * 8;
      const uint64_t gr = row0 + r;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const uint64_t gd0 = k0 + d0 + 4 * v;
        const uint64_t idx = gr * lda + gd0;
        if (VEC_A && gr < m && gd0 + 4 <= k && (((uintptr_t)(a + idx)) & 7u) == 0) {
          *reinterpret_cast<uint2*>(a_lds + r * G_LDK + d0 + 4 * v) =
              *reinterpret_cast<const uint2*>(a + idx);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint64_t gd = gd0 + e;
            a_lds[r * G_LDK + d0 + 4 * v + e] = (gr < m && gd < k) ? a[gr * lda + gd] : (uint16_t)0;
          }
        }
      }
    }
    // B: thread t loads depth t/8, columns (t%8)*8 .. +7, stored transposed
    {
      const int d = t >> 3, n0 = (t & 7) * 8;
      const uint64_t gd = k0 + d;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint64_t gc = col0 + n0 + e;
        bt_lds[(n0 + e) * G_LDK + d] = (gd < k && gc < n) ? b[gd * ldb + gc] : (uint16_t)0;
      }
    }
    __syncthreads();
    const int rc = lane & 15, chunk = lane >> 4;
    bf16x8_t af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      af[i] = *reinterpret_cast<const bf16x8_t*>(a_lds + (wm * 32 + i * 16 + rc) * G_LDK + chunk * 8);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      bf[j] = *reinterpret_cast<const bf16x8_t*>(bt_lds + (wn * 32 + j * 16 + rc) * G_LDK + chunk * 8);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }
  // epilogue: alpha * acc and beta * C rounded separately, then added
  // (examples/tiled_gemm_v1/src/numerical_contract.rs:310-331 order).
  {
#pragma clang fp contract(off)
    const int col_in = lane & 15, row_in = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint64_t gr = row0 + wm * 32 + i * 16 + row_in + e;
          const uint64_t gc = col0 + wn * 32 + j * 16 + col_in;
          if (gr < m && gc < n) {
            float* p = c + gr * ldc + gc;
            const float product = alpha * acc[i][j][e];
            const float initial = beta * *p;
            *p = product + initial;
          }
        }
  }
}

// ---- scalar f32 GEMM (sequential, unfused) -----------------------------------------
// Workgroup tile 16x16, 256 threads, one output per thread, whose accumulator
// follows acc = acc + a*b over t = 0..k-1 in order.  One output per thread
// (rather than a register block) spreads a 256^3 problem over 256 workgroups;
// the k loop runs in LDS chunks of 256, so k <= 256 waits for global memory
// once.
constexpr int S_BM = 16, S_BN = 16, S_BK = 256;

__global__ void __launch_bounds__(256) scalar_gemm_kernel(const float* __restrict__ a,
                                                          const float* __restrict__ b,
                                                          float* __restrict__ c, uint32_t m,
                                                          uint32_t n, uint32_t k) {
#pragma clang fp contract(off)
  // Both tiles k-contiguous per row (B transposed on the way in), rows padded
  // to 260 floats: 16-byte reads of 4 consecutive depths, conflict-free.
  constexpr int LD = S_BK + 4;
  __shared__ __attribute__((aligned(16))) float a_lds[S_BM][LD];   // [row][depth]
  __shared__ __attribute__((aligned(16))) float bt_lds[S_BN][LD];  // [col][depth]
  const int t = threadIdx.x;
  const int tr = t >> 4, tc = t & 15;  // thread owns output (row0 + tr, col0 + tc)
  // linear workgroup id over (row tile, column tile), column tiles fastest
  const uint32_t tiles_n = (uint32_t)(((uint64_t)n + S_BN - 1) / S_BN);
  const uint64_t row0 = (uint64_t)(blockIdx.x / tiles_n) * S_BM;
  const uint64_t col0 = (uint64_t)(blockIdx.x % tiles_n) * S_BN;
  float acc = 0.0f;
  for (uint64_t k0 = 0; k0 < k; k0 += S_BK) {
    // A tile 16 rows x 256 depths and B tile 256 depths x 16 cols, 16 values each per thread
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = t + 256 * e;
      const int ar = i >> 8, ad = i & 255;
      const uint64_t gr = row0 + ar, gd = k0 + ad;
      a_lds[ar][ad] = (gr < m && gd < k) ? a[gr * k + gd] : 0.0f;
      const int bd = i >> 4, bc = i & 15;
      const uint64_t gbd = k0 + bd, gc = col0 + bc;
      bt_lds[bc][bd] = (gbd < k && gc < n) ? b[gbd * n + gc] : 0.0f;
    }
    __syncthreads();
    const int depth = (k - k0) < (uint64_t)S_BK ? (int)(k - k0) : S_BK;
    if (depth == S_BK) {
#pragma unroll 16
      for (int d = 0; d < S_BK; d += 4) {
        const f32x4_t av = *reinterpret_cast<const f32x4_t*>(&a_lds[tr][d]);
        const f32x4_t bv = *reinterpret_cast<const f32x4_t*>(&bt_lds[tc][d]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = av[e] * bv[e];
          acc = acc + p;
        }
      }
    } else {
      for (int d = 0; d < depth; ++d) {
        const float p = a_lds[tr][d] * bt_lds[tc][d];
        acc = acc + p;
      }
    }
    __syncthreads();
  }
  const uint64_t gr = row0 + tr, gc = col0 + tc;
  if (gr < m && gc < n) c[gr * n + gc] = acc;
}

bool aligned(const void* p, uintptr_t bytes) { return ((uintptr_t)p & (bytes - 1)) == 0; }

int32_t tile16(const uint16_t* a, uint64_t a_len, const uint16_t* b, uint64_t b_len, float* c,
               uint64_t c_len, void* stream) {
  if (a_len != 256 || b_len != 256 || c_len != 256) return FE2O3_ERR_LENGTH;
  if (!a || !b || !c) return FE2O3_ERR_NULL;
  if (!aligned(a, 8) || !aligned(b, 8) || !aligned(c, 4)) return FE2O3_ERR_ALIGNMENT;
  tile16_bf16_kernel<<<1, 64, 0, (hipStream_t)stream>>>(a, b, c);
  return fe2o3_host::after_launch();
}

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_tiled_gemm_lds_slice1_v1", "tile16_bf16_kernel", (const void*)tile16_bf16_kernel, 64, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_moe_expert_gemm_bf16_m16_n16_k16_v1", "tile16_bf16_kernel", (const void*)tile16_bf16_kernel, 64, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_tiled_gemm_v1", "tiled_v1_kernel", (const void*)tiled_v1_kernel, 64, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_tiled_gemm_v1", "zero_fill_kernel", (const void*)zero_fill_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_tiled_gemm_general_v1", "gemm_general_kernel<false>", (const void*)gemm_general_kernel<false>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_tiled_gemm_general_vector_a_v1", "gemm_general_kernel<true>", (const void*)gemm_general_kernel<true>, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_scalar_gemm_v1", "scalar_gemm_kernel", (const void*)scalar_gemm_kernel, 256, 0})};

}  // namespace

extern "C" {

int32_t fe2o3_tiled_gemm_lds_slice1_v1(const uint16_t* a, uint64_t a_len, const uint16_t* b,
                                       uint64_t b_len, float* c, uint64_t c_len, void* stream) {
  FE2O3_ENTRY("fe2o3_tiled_gemm_lds_slice1_v1");
  return tile16(a, a_len, b, b_len, c, c_len, stream);
}

int32_t fe2o3_moe_expert_gemm_bf16_m16_n16_k16_v1(const uint16_t* activations,
                                                  uint64_t activations_len,
                                                  const uint16_t* weights, uint64_t weights_len,
                                                  float* output, uint64_t output_len,
                                                  void* stream) {
  FE2O3_ENTRY("fe2o3_moe_expert_gemm_bf16_m16_n16_k16_v1");
  return tile16(activations, activations_len, weights, weights_len, output, output_len, stream);
}

int32_t fe2o3_tiled_gemm_v1(const uint16_t* a, uint64_t a_len, const uint16_t* b, uint64_t b_len,
                            float* c, uint64_t c_len, uint32_t m, uint32_t n, uint32_t k,
                            void* stream) {
  FE2O3_ENTRY("fe2o3_tiled_gemm_v1");
  // ShapeV1::checked (contract.rs:145-179): an empty output needs no
  // operand buffers; otherwise byte extents of A, B, C in that order
  if (m == 0 || n == 0) {
    if (a_len != 0 || b_len != 0 || c_len != 0) return FE2O3_ERR_LENGTH;
    return FE2O3_OK;  // NoDispatchEmptyOutput
  }
  const uint64_t ea = (uint64_t)m * k, eb = (uint64_t)k * n, ec = (uint64_t)m * n;
  if (ea > UINT64_MAX / 2 || eb > UINT64_MAX / 2 || ec > UINT64_MAX / 4) return FE2O3_ERR_OVERFLOW;
  if (a_len != ea || b_len != eb || c_len != ec) return FE2O3_ERR_LENGTH;
  // plan_v1 (contract.rs:387-427), in its order
  if (m % 16u != 0) return FE2O3_ERR_M_TAIL;
  if (n % 16u != 0) return FE2O3_ERR_N_TAIL;
  if (k != 0 && k % 16u != 0) return FE2O3_ERR_K_TAIL;
  if ((uint64_t)(n / 16u) * 64u > UINT32_MAX) return FE2O3_ERR_OVERFLOW;  // AQL grid x
  if (!c || (k != 0 && (!a || !b))) return FE2O3_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  if (k == 0) {  // HostFillPositiveZero
    const uint64_t blocks = (ec + 255u) / 256u;
    zero_fill_kernel<<<(unsigned)(blocks < 4096u ? blocks : 4096u), 256, 0, s>>>(c, ec);
    return fe2o3_host::after_launch();
  }
  const uint64_t tiles = (uint64_t)(m / 16u) * (n / 16u);
  if (tiles > 0x7fffffffu) return FE2O3_ERR_SHAPE;
  tiled_v1_kernel<<<(unsigned)tiles, 64, 0, s>>>(a, b, c, n, k, n / 16u);
  return fe2o3_host::after_launch();
}

}  // extern "C"

namespace {

// ---- general GEMM on the pipelined tile ----------------------------------------------
// The same contract on the 256x256 MFMA tile of gemm_pipe.hpp: A's rows
// (lda apart) are k-contiguous as the tile wants; B is stored [k][n], so its
// 64-k stages arrive as 64 rows of 256 columns and the MFMA fragments are
// read with the transposing LDS read (gemm_pipe::Bf16MmaKN).  Rows past m
// and columns past n repeat the last valid ones and are not stored.  Each
// accumulator receives the same 16x16x32 MFMAs over the same k slices in the
// same order as in gemm_general_kernel, so both give the same bits.  The
// epilogue is that kernel's: alpha * sum and beta * C rounded separately,
// then added.
constexpr int kGpRowBytes = 128, kGpStages = 2;
constexpr int kGpSmem = kGpStages * 2 * gemm_pipe::Geo<kGpRowBytes>::kTileBytes;  // 128 KiB

// C = alpha * acc + beta * C over one tile of TM x TN outputs (rows x cols
// valid), accumulators Acc16T<RB, CB> of waves holding RPW rows by CPW
// columns.  Per 16-row block: every C load of the lane first (one wait),
// then the products and stores.  Whole-width tiles of a 16-byte aligned C
// with ldc % 4 == 0 move 4 columns per access; otherwise element by element,
// the loads of columns past n clamped to the last valid one (not stored).
template <int TN, int RPW, int CPW, class Acc>
FE2O3_DEVICE void general_epilogue(const Acc& acc, float* c_tile, uint32_t rows, uint32_t cols,
                                   uint32_t ldc, bool c_aligned, float alpha, float beta) {
#pragma clang fp contract(off)
  constexpr int RB = RPW / 16, CB = CPW / 16;
  const uint32_t row0 = gemm_pipe::acc16_row0<RPW>(), col0 = gemm_pipe::acc16_col0<CPW>();
  const bool vec = cols == (uint32_t)TN && ldc % 4u == 0u && c_aligned;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const uint32_t r = row0 + 16u * i;
    if (r >= rows) continue;
    float* out = c_tile + (uint64_t)r * ldc;
    if (vec) {
      f32x4_t cv[CB];
#pragma unroll
      for (int j = 0; j < CB; ++j) cv[j] = *reinterpret_cast<const f32x4_t*>(out + col0 + 16u * j);
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        f32x4_t y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float product = alpha * acc.v[i][j][e];
          const float initial = beta * cv[j][e];
          y[e] = product + initial;
        }
        *reinterpret_cast<f32x4_t*>(out + col0 + 16u * j) = y;
      }
    } else {
      float cv[CB][4];
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) cv[j][e] = out[min(col0 + 16u * j + e, cols - 1u)];
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t col = col0 + 16u * j + e;
          if (col < cols) {
            const float product = alpha * acc.v[i][j][e];
            const float initial = beta * cv[j][e];
            out[col] = product + initial;
          }
        }
    }
  }
}

// k: A's k extent and the K loop's; kb: B's rows (its k extent), at most k
// and more than k - 64.  KT: k or kb is not a multiple of 64; A's chunks
// past k and B's rows past kb load zeros (gemm_pipe::Rows MASK), so each
// accumulator gets the staged kernel's zero-padded 32-k blocks.
template <bool KT = false>
__global__ void __launch_bounds__(256, 1) gemm_general_pipe_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, float* __restrict__ c,
    uint32_t m, uint32_t n, uint32_t k, uint32_t kb, uint32_t lda, uint32_t ldb, uint32_t ldc,
    float alpha, float beta, uint32_t xcds) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const uint32_t tiles_m = (m + 255u) / 256u, tiles_n = (n + 255u) / 256u;
  uint32_t tm, tn;
  gemm_core::xcd_tile_order(blockIdx.x, tiles_m, tiles_n, xcds, &tm, &tn);
  const uint32_t rows = min(256u, m - tm * 256u), cols = min(256u, n - tn * 256u);
  const auto ar =
      gemm_pipe::dense_rows<kGpRowBytes, 256, KT>(a + (uint64_t)tm * 256u * lda, lda, rows, k);
  const auto br = gemm_pipe::kn_rows<KT>(b + (uint64_t)tn * 256u, ldb, cols, kb);
  gemm_pipe::Acc16 acc;
  gemm_pipe::mainloop<gemm_pipe::Bf16MmaKN, kGpRowBytes, kGpStages, KT>(ar, br, k, smem, acc);
  general_epilogue<256, 128, 128>(acc, c + (uint64_t)tm * 256u * ldc + (uint64_t)tn * 256u, rows,
                                  cols, ldc, ((uintptr_t)c & 15u) == 0u, alpha, beta);
}

// The same GEMM on 128 x 128 tiles (Bf16MmaKN64), for problems whose
// 256 x 256 tiles would not fill the CUs: two stages (64 KiB of LDS, two
// workgroups per CU) when there are more tiles than CUs, else three (96 KiB,
// one workgroup per CU, copies two stages ahead: +24% at 2048^3, -5% at
// 4096 x 2048 x 2048 where two workgroups per CU pay more).  The k order of
// every output's MFMAs is that of the 256 x 256 tile, so C is bit-identical
// to it.
template <int STAGES>
constexpr int kGp64Smem =
    STAGES * (128 * kGpRowBytes + gemm_pipe::Bf16MmaKN64::kBTileBytes);
// TAIL: the last, partial round of a 256 x 256 grid (tiles first_big .. end
// of gemm_core::xcd_tile_order's list), each as four 128 x 128 quarters
// (gemm_core::tail_quarter).
// k, kb, KT: as for gemm_general_pipe_kernel.
template <int STAGES, bool TAIL = false, bool KT = false>
__global__ void __launch_bounds__(256, STAGES == 2 ? 2 : 1) gemm_general_pipe128_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, float* __restrict__ c,
    uint32_t m, uint32_t n, uint32_t k, uint32_t kb, uint32_t lda, uint32_t ldb, uint32_t ldc,
    float alpha, float beta, uint32_t xcds, uint32_t first_big = 0) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  uint32_t tm, tn;
  if constexpr (TAIL) {
    if (!gemm_core::tail_quarter(blockIdx.x, first_big, m, n, xcds, &tm, &tn)) return;
  } else {
    gemm_core::xcd_tile_order(blockIdx.x, (m + 127u) / 128u, (n + 127u) / 128u, xcds, &tm, &tn);
  }
  const uint32_t rows = min(128u, m - tm * 128u), cols = min(128u, n - tn * 128u);
  const auto ar =
      gemm_pipe::dense_rows<kGpRowBytes, 128, KT>(a + (uint64_t)tm * 128u * lda, lda, rows, k);
  const auto br = gemm_pipe::kn_rows128<KT>(b + (uint64_t)tn * 128u, ldb, cols, kb);
  gemm_pipe::Bf16MmaKN64::Acc acc;
  gemm_pipe::mainloop<gemm_pipe::Bf16MmaKN64, kGpRowBytes, STAGES, KT>(ar, br, k, smem, acc);
  general_epilogue<128, 64, 64>(acc, c + (uint64_t)tm * 128u * ldc + (uint64_t)tn * 128u, rows,
                                cols, ldc, ((uintptr_t)c & 15u) == 0u, alpha, beta);
}

// ---- operands the pipelined tile cannot read directly ---------------------------
// Rows that are not 16-byte aligned (A or B two bytes past a boundary, a
// stride that is not a multiple of 8) or an A whose K is not a multiple of
// 8 are first copied into aligned scratch rows: A as [m][kp] with kp = K
// rounded up to 64 and zeros from K on, B as [K][np] with np = N rounded up
// to 8.  The pipelined tile then reads the copies; its products are the same
// MFMAs over the same zero-padded 32-k blocks.  8 elements (16 bytes) per
// thread per step, written as one 16-byte store.  A whole 8-element piece
// of a source row is read as one 16-byte load at its own (2-byte) alignment
// (gfx950 global loads take any alignment); the piece that holds a row's
// end is read element by element.
__global__ void __launch_bounds__(256) repack_rows_kernel(const uint16_t* __restrict__ src,
                                                          uint32_t rows, uint32_t cols,
                                                          uint32_t ld, uint16_t* __restrict__ dst,
                                                          uint32_t dst_cols) {
  const uint64_t per_row = dst_cols / 8u, groups = (uint64_t)rows * per_row;
  for (uint64_t g = (uint64_t)blockIdx.x * 256u + threadIdx.x; g < groups;
       g += (uint64_t)gridDim.x * 256u) {
    const uint64_t r = g / per_row;
    const uint32_t c0 = (uint32_t)(g % per_row) * 8u;
    const uint16_t* row = src + r * ld;
    u32x4_t p;
    if (c0 + 8u <= cols) {
      __builtin_memcpy(&p, row + c0, 16);
    } else {
      uint16_t v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = c0 + e < cols ? row[c0 + e] : (uint16_t)0;
#pragma unroll
      for (int q = 0; q < 4; ++q) p[q] = (uint32_t)v[2 * q] | ((uint32_t)v[2 * q + 1] << 16);
    }
    *reinterpret_cast<u32x4_t*>(dst + r * dst_cols + c0) = p;
  }
}

#define FE2O3_GENERAL_PIPE_KERNELS(entry)                                                        \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe_kernel", (const void*)gemm_general_pipe_kernel<false>, 256, kGpSmem}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe_kernel<k tail>", (const void*)gemm_general_pipe_kernel<true>, 256, kGpSmem}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<2>", (const void*)gemm_general_pipe128_kernel<2>, 256, kGp64Smem<2>}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<3>", (const void*)gemm_general_pipe128_kernel<3>, 256, kGp64Smem<3>}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<2, tail>", (const void*)gemm_general_pipe128_kernel<2, true>, 256, kGp64Smem<2>}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<3, tail>", (const void*)gemm_general_pipe128_kernel<3, true>, 256, kGp64Smem<3>}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<2, k tail>", (const void*)gemm_general_pipe128_kernel<2, false, true>, 256, kGp64Smem<2>}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<3, k tail>", (const void*)gemm_general_pipe128_kernel<3, false, true>, 256, kGp64Smem<3>}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<2, tail, k tail>", (const void*)gemm_general_pipe128_kernel<2, true, true>, 256, kGp64Smem<2>}), \
  fe2o3_host::KernelRegistrar({entry, "gemm_general_pipe128_kernel<3, tail, k tail>", (const void*)gemm_general_pipe128_kernel<3, true, true>, 256, kGp64Smem<3>}), \
  fe2o3_host::KernelRegistrar({entry, "repack_rows_kernel", (const void*)repack_rows_kernel, 256, 0})

const fe2o3_host::KernelRegistrar kRegisteredPipe[] = {
    FE2O3_GENERAL_PIPE_KERNELS("fe2o3_tiled_gemm_general_v1"),
    FE2O3_GENERAL_PIPE_KERNELS("fe2o3_tiled_gemm_general_vector_a_v1"),
    // fe2o3_gemm_bf16_nt repacks misaligned operand rows with it (gemm_bf16.hip)
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "repack_rows_kernel", (const void*)repack_rows_kernel, 256, 0})};

// Raises every pipelined kernel's dynamic-LDS limit once per process.
int32_t set_general_lds() {
  static const int32_t rc = [] {
    int32_t r = fe2o3_host::set_dynamic_lds(
        {(const void*)gemm_general_pipe_kernel<false>, (const void*)gemm_general_pipe_kernel<true>},
        kGpSmem);
    if (r == FE2O3_OK)
      r = fe2o3_host::set_dynamic_lds({(const void*)gemm_general_pipe128_kernel<2>,
                                       (const void*)gemm_general_pipe128_kernel<2, true>,
                                       (const void*)gemm_general_pipe128_kernel<2, false, true>,
                                       (const void*)gemm_general_pipe128_kernel<2, true, true>},
                                      kGp64Smem<2>);
    if (r == FE2O3_OK)
      r = fe2o3_host::set_dynamic_lds({(const void*)gemm_general_pipe128_kernel<3>,
                                       (const void*)gemm_general_pipe128_kernel<3, true>,
                                       (const void*)gemm_general_pipe128_kernel<3, false, true>,
                                       (const void*)gemm_general_pipe128_kernel<3, true, true>},
                                      kGp64Smem<3>);
    return r;
  }();
  return rc;
}

// The launches of `plan` over A (lda, k) and B (ldb, kb rows); KT: k or kb
// is not a multiple of 64.
template <bool KT>
int32_t launch_general_pipe(const uint16_t* a, const uint16_t* b, float* c, uint32_t m,
                            uint32_t n, uint32_t k, uint32_t kb, uint32_t lda, uint32_t ldb,
                            uint32_t ldc, float alpha, float beta, const tile_plan::Plan& plan,
                            uint32_t xcds, hipStream_t s) {
  if (plan.small) {  // 256 x 256 tiles would leave most CUs idle
    if (plan.stages == 2)
      gemm_general_pipe128_kernel<2, false, KT><<<(unsigned)plan.grid, 256, kGp64Smem<2>, s>>>(
          a, b, c, m, n, k, kb, lda, ldb, ldc, alpha, beta, xcds);
    else
      gemm_general_pipe128_kernel<3, false, KT><<<(unsigned)plan.grid, 256, kGp64Smem<3>, s>>>(
          a, b, c, m, n, k, kb, lda, ldb, ldc, alpha, beta, xcds);
    return fe2o3_host::after_launch();
  }
  gemm_general_pipe_kernel<KT><<<(unsigned)plan.grid, 256, kGpSmem, s>>>(
      a, b, c, m, n, k, kb, lda, ldb, ldc, alpha, beta, xcds);
  const int32_t big_rc = fe2o3_host::after_launch();
  if (big_rc != FE2O3_OK || !plan.tail) return big_rc;
  // the last round of at most half the CUs' tiles as 128 x 128 quarters
  if (plan.tail_stages == 2)  // more quarters than CUs: two per CU
    gemm_general_pipe128_kernel<2, true, KT><<<(unsigned)plan.tail_grid, 256, kGp64Smem<2>, s>>>(
        a, b, c, m, n, k, kb, lda, ldb, ldc, alpha, beta, xcds, plan.first_big);
  else
    gemm_general_pipe128_kernel<3, true, KT><<<(unsigned)plan.tail_grid, 256, kGp64Smem<3>, s>>>(
        a, b, c, m, n, k, kb, lda, ldb, ldc, alpha, beta, xcds, plan.first_big);
  return fe2o3_host::after_launch();
}

// Whether the pipelined tile reads an operand in place: 16-byte aligned
// rows, and its 256-row (A) or K-row (B) panel within a buffer resource's
// 32-bit range.  A also needs K a multiple of 8 (chunks past K are masked
// whole).
bool a_direct(const uint16_t* a, uint32_t k, uint32_t lda) {
  return k % 8 == 0 && lda % 8 == 0 && ((uintptr_t)a & 15u) == 0 &&
         (255ull * lda + k) * 2 < (1ull << 31);
}
bool b_direct(const uint16_t* b, uint32_t k, uint32_t ldb) {
  return ldb % 8 == 0 && ((uintptr_t)b & 15u) == 0 &&
         ((uint64_t)(k - 1) * ldb + 256) * 2 < (1ull << 31);
}

// Operands the tile cannot read in place are repacked (repack_rows_kernel)
// when M and N are at least one 128 x 128 tile; smaller problems stay on
// the staged kernel.
constexpr uint32_t kRepackMin = 128;

template <bool VEC_A>
int32_t general_gemm(const uint16_t* a, uint64_t a_len, const uint16_t* b, uint64_t b_len,
                     float* c, uint64_t c_len, uint32_t m, uint32_t n, uint32_t k, uint32_t lda,
                     uint32_t ldb, uint32_t ldc, float alpha, float beta, void* stream) {
  // examples/tiled_gemm_general_v1/src/kernel.rs:80-89
  if ((m != 0 && k != 0 && lda < k) || (k != 0 && n != 0 && ldb < n) ||
      (m != 0 && n != 0 && ldc < n))
    return FE2O3_ERR_STRIDE;
  uint64_t ea, eb, ec;
  fe2o3_host::extent_ok(m, k, lda, &ea);
  fe2o3_host::extent_ok(k, n, ldb, &eb);
  fe2o3_host::extent_ok(m, n, ldc, &ec);
  if (a_len < ea || b_len < eb || c_len < ec) return FE2O3_ERR_LENGTH;
  if (m == 0 || n == 0) return FE2O3_OK;  // empty output: no dispatch
  if ((ea && !a) || (eb && !b) || !c) return FE2O3_ERR_NULL;
  const bool ad = k != 0 && a_direct(a, k, lda), bd = k != 0 && b_direct(b, k, ldb);
  const bool repack = k != 0 && (!ad || !bd) && m >= kRepackMin && n >= kRepackMin;
  if (k != 0 && ((ad && bd) || repack)) {
    // every kernel's LDS limit is raised before anything is launched, so a
    // failure leaves C untouched
    const int32_t lds_rc = set_general_lds();
    if (lds_rc != FE2O3_OK) return lds_rc;
    tile_plan::Topology topo;
    const int32_t topo_rc = fe2o3_host::device_topology(&topo);
    if (topo_rc != FE2O3_OK) return topo_rc;
    const tile_plan::Plan plan = tile_plan::plan(m, n, topo);
    if (plan.grid > 0x7fffffffu || plan.tail_grid > 0x7fffffffu) return FE2O3_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    if (!repack) {
      if (k % 64 != 0)
        return launch_general_pipe<true>(a, b, c, m, n, k, k, lda, ldb, ldc, alpha, beta, plan,
                                         topo.xcds, s);
      return launch_general_pipe<false>(a, b, c, m, n, k, k, lda, ldb, ldc, alpha, beta, plan,
                                        topo.xcds, s);
    }
    // repack what cannot be read in place into one stream-ordered scratch
    // block: A as [m][kp] (zeros from K on), B as [K][np]
    const uint32_t kp = (k + 63u) & ~63u, np = (n + 7u) & ~7u;
    const uint64_t a_elems = ad ? 0 : (uint64_t)m * kp, b_elems = bd ? 0 : (uint64_t)k * np;
    if ((!ad && 256ull * kp * 2 >= (1ull << 31)) ||
        (!bd && ((uint64_t)(k - 1) * np + 256) * 2 >= (1ull << 31)))
      return FE2O3_ERR_SHAPE;
    void* scratch = nullptr;
    int32_t rc = fe2o3_host::scratch_alloc(&scratch, (a_elems + b_elems) * 2, s);
    if (rc != FE2O3_OK) {
      // no stream-ordered scratch on this device or process: the staged
      // kernel reads the operands as they are
      (void)hipGetLastError();
      goto staged;
    }
    uint16_t* ap = static_cast<uint16_t*>(scratch);
    uint16_t* bp = ap + a_elems;
    auto grid = [](uint64_t groups) {
      const uint64_t g = (groups + 255) / 256;
      return (unsigned)(g < 16384 ? g : 16384);
    };
    if (!ad) repack_rows_kernel<<<grid((uint64_t)m * (kp / 8)), 256, 0, s>>>(a, m, k, lda, ap, kp);
    if (!bd) repack_rows_kernel<<<grid((uint64_t)k * (np / 8)), 256, 0, s>>>(b, k, n, ldb, bp, np);
    rc = fe2o3_host::after_launch();
    if (rc == FE2O3_OK) {
      const uint16_t* ra = ad ? a : ap;
      const uint16_t* rb = bd ? b : bp;
      const uint32_t rlda = ad ? lda : kp, rldb = bd ? ldb : np;
      // a repacked A holds zeros up to kp: the K loop runs whole stages over
      // it; an A read in place masks its chunks past K.  B's rows past K
      // are masked either way.
      const uint32_t kloop = ad ? k : kp;
      rc = k % 64 != 0
               ? launch_general_pipe<true>(ra, rb, c, m, n, kloop, k, rlda, rldb, ldc, alpha,
                                           beta, plan, topo.xcds, s)
               : launch_general_pipe<false>(ra, rb, c, m, n, kloop, k, rlda, rldb, ldc, alpha,
                                            beta, plan, topo.xcds, s);
    }
    const int32_t free_rc = fe2o3_host::scratch_free(scratch, s);
    return rc != FE2O3_OK ? rc : free_rc;
  }
staged:
  dim3 grid((n + G_BN - 1) / G_BN, (m + G_BM - 1) / G_BM);
  if (grid.y > 65535u) return FE2O3_ERR_SHAPE;
  gemm_general_kernel<VEC_A><<<grid, 256, 0, (hipStream_t)stream>>>(a, b, c, m, n, k, lda, ldb,
                                                                    ldc, alpha, beta);
  return fe2o3_host::after_launch();
}

}  // namespace

namespace fe2o3_host {

int32_t repack_bf16_rows(const uint16_t* src, uint32_t rows, uint32_t cols, uint32_t ld,
                         uint16_t* dst, uint32_t dst_cols, hipStream_t s) {
  const uint64_t g = ((uint64_t)rows * (dst_cols / 8u) + 255u) / 256u;
  repack_rows_kernel<<<(unsigned)(g < 16384u ? g : 16384u), 256, 0, s>>>(src, rows, cols, ld, dst,
                                                                         dst_cols);
  return after_launch();
}

}  // namespace fe2o3_host

extern "C" {

int32_t fe2o3_tiled_gemm_general_v1(const uint16_t* a, uint64_t a_len, const uint16_t* b,
                                    uint64_t b_len, float* c, uint64_t c_len, uint32_t m,
                                    uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb,
                                    uint32_t ldc, float alpha, float beta, void* stream) {
  FE2O3_ENTRY("fe2o3_tiled_gemm_general_v1");
  return general_gemm<false>(a, a_len, b, b_len, c, c_len, m, n, k, lda, ldb, ldc, alpha, beta,
                             stream);
}

int32_t fe2o3_tiled_gemm_general_vector_a_v1(const uint16_t* a, uint64_t a_len,
                                             const uint16_t* b, uint64_t b_len, float* c,
                                             uint64_t c_len, uint32_t m, uint32_t n, uint32_t k,
                                             uint32_t lda, uint32_t ldb, uint32_t ldc,
                                             float alpha, float beta, void* stream) {
  FE2O3_ENTRY("fe2o3_tiled_gemm_general_vector_a_v1");
  return general_gemm<true>(a, a_len, b, b_len, c, c_len, m, n, k, lda, ldb, ldc, alpha, beta,
                            stream);
}

int32_t fe2o3_scalar_gemm_v1(const float* a, uint64_t a_len, const float* b, uint64_t b_len,
                             float* c, uint64_t c_len, uint32_t m, uint32_t n, uint32_t k,
                             void* stream) {
  FE2O3_ENTRY("fe2o3_scalar_gemm_v1");
  const uint64_t ea = (uint64_t)m * k, eb = (uint64_t)k * n, ec = (uint64_t)m * n;
  if (a_len < ea || b_len < eb || c_len < ec) return FE2O3_ERR_LENGTH;
  if (ec == 0) return FE2O3_OK;
  if ((ea && !a) || (eb && !b) || !c) return FE2O3_ERR_NULL;
  const uint64_t tiles = (((uint64_t)m + S_BM - 1) / S_BM) * (((uint64_t)n + S_BN - 1) / S_BN);
  if (tiles > 0x7fffffffu) return FE2O3_ERR_SHAPE;
  scalar_gemm_kernel<<<(unsigned)tiles, 256, 0, (hipStream_t)stream>>>(a, b, c, m, n, k);
  return fe2o3_host::after_launch();
}

}  // extern "C"
