// gemm_bf16.hip -- bf16 "NT" GEMM for gfx950: C[m,n] (bf16, row-major) =
// A[m,k] (row-major) * B^T with B stored [n,k] (k contiguous, i.e. the
// BASELINE's column-major B), fp32 accumulation, RNE bf16 output.
//
// Fast path (k a multiple of 8 below 2^22, A and B 16-byte aligned): the
// 256x256 pipelined MFMA tile of gemm_pipe.hpp with 64 k per LDS stage and
// two stages, workgroups ordered XCD-aware (gemm_core.hpp); m or n not a
// multiple of 256 (or an unaligned C) runs its edge form, and k not a
// multiple of 64 either form with a partial last stage.  Any other shape
// (k not a multiple of 8, misaligned A or B) uses a bounds-checked
// 64x64-tile MFMA kernel.
#include "common.hpp"
#include "gemm_core.hpp"
#include "gemm_pipe.hpp"
#include "internal.hpp"

#include <type_traits>

namespace {

using namespace fe2o3;

// ---- generic path -------------------------------------------------------------------
constexpr int N_BM = 64, N_BN = 64, N_BK = 32, N_LDK = N_BK + 8;

__global__ void __launch_bounds__(256) gemm_bf16_nt_generic_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint16_t* __restrict__ c,
    uint32_t m, uint32_t n, uint32_t k) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[N_BM * N_LDK];
  __shared__ __attribute__((aligned(16))) uint16_t b_lds[N_BN * N_LDK];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint64_t row0 = (uint64_t)blockIdx.y * N_BM, col0 = (uint64_t)blockIdx.x * N_BN;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (uint64_t k0 = 0; k0 < k; k0 += N_BK) {
    const int r = t >> 2, d0 = (t & 3) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint64_t gd = k0 + d0 + e;
      const uint64_t ga = row0 + r, gb = col0 + r;
      a_lds[r * N_LDK + d0 + e] = (ga < m && gd < k) ? a[ga * k + gd] : (uint16_t)0;
      b_lds[r * N_LDK + d0 + e] = (gb < n && gd < k) ? b[gb * k + gd] : (uint16_t)0;
    }
    __syncthreads();
    const int rc = lane & 15, chunk = lane >> 4;
    bf16x8_t af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      af[i] = *reinterpret_cast<const bf16x8_t*>(a_lds + (wm * 32 + i * 16 + rc) * N_LDK + chunk * 8);
      bf[i] = *reinterpret_cast<const bf16x8_t*>(b_lds + (wn * 32 + i * 16 + rc) * N_LDK + chunk * 8);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }
  const int col_in = lane & 15, row_in = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t gr = row0 + wm * 32 + i * 16 + row_in + e;
        const uint64_t gc = col0 + wn * 32 + j * 16 + col_in;
        if (gr < m && gc < n) c[gr * n + gc] = bf16_bits_from_f32(acc[i][j][e]);
      }
}

// ---- fast path ----------------------------------------------------------------------------
// 256x256 tiles, 64 k per LDS stage (128-byte rows), two stages, 16x16x32
// MFMAs in a fixed issue order (gemm_pipe.hpp).
constexpr int kRowBytes = 128, kStages = 2;
constexpr int kFastSmem = kStages * 2 * gemm_pipe::Geo<kRowBytes>::kTileBytes;  // 128 KiB

// STAGED: C leaves through LDS in whole rows with nontemporal stores
// (gemm_pipe::store_bf16_staged), for operands that stream from HBM.
// EDGE: M or N is not a multiple of 256; the grid covers ceil(M/256) x
// ceil(N/256) tiles, operand rows past M (N) repeat the last valid row
// (their products reach only outputs that are not stored), and each tile
// stores only its valid rows and columns, element by element.
//
// KT: K is a multiple of 8 but not of 64; the last stage is partial and its
// chunks past K load zeros (gemm_pipe::Rows MASK), the zero padding the
// generic kernel gives its last k step, so C is bit-identical to it.
template <bool STAGED, bool EDGE, bool KT = false>
__global__ void __launch_bounds__(256, 1) gemm_bf16_nt_256_kernel(const uint16_t* __restrict__ a,
                                                                   const uint16_t* __restrict__ b,
                                                                   uint16_t* __restrict__ c,
                                                                   uint32_t m, uint32_t n,
                                                                   uint32_t k, uint32_t xcds) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const uint32_t tiles_m = EDGE ? (m + 255u) / 256u : m / 256u;
  const uint32_t tiles_n = EDGE ? (n + 255u) / 256u : n / 256u;
  uint32_t tm, tn;
  gemm_core::xcd_tile_order(blockIdx.x, tiles_m, tiles_n, xcds, &tm, &tn);
  const uint32_t rows_a = EDGE ? min(256u, m - tm * 256u) : 256u;
  const uint32_t rows_b = EDGE ? min(256u, n - tn * 256u) : 256u;
  const auto ar =
      gemm_pipe::dense_rows<kRowBytes, 256, KT>(a + (uint64_t)tm * 256 * k, k, rows_a, k);
  const auto br =
      gemm_pipe::dense_rows<kRowBytes, 256, KT>(b + (uint64_t)tn * 256 * k, k, rows_b, k);
  gemm_pipe::Acc16 acc;
  gemm_pipe::mainloop<gemm_pipe::Bf16Mma<kRowBytes>, kRowBytes, kStages, KT>(ar, br, k, smem,
                                                                              acc);
  uint16_t* c_tile = c + (uint64_t)tm * 256 * n + (uint64_t)tn * 256;
  if constexpr (EDGE)
    gemm_pipe::store_bf16_edge(acc, c_tile, n, rows_a, rows_b);
  else if constexpr (STAGED)
    gemm_pipe::store_bf16_staged(acc, smem, c_tile, n);
  else
    gemm_pipe::store_bf16(acc, c_tile, n);
}

// The small-grid form: 128 x 128 tiles (Bf16Mma64) for GEMMs whose 256 x 256
// tiles would leave most CUs idle; three 64-k stages (96 KiB) while the
// tiles fit one per CU, else two (64 KiB, two workgroups per CU).  Every
// output gets the MFMAs of the 256 x 256 tile in the same k order, so C is
// bit-identical to it.  WHOLE: M and N multiples of 128 and C 16-byte
// aligned; otherwise rows past M (N) repeat the last valid row and only
// valid elements are stored.
template <int STAGES>
constexpr int kSmallSmem = STAGES * (128 * kRowBytes + gemm_pipe::Bf16Mma64::kBTileBytes);
//
// TAIL: the last, partial round of a 256 x 256 grid (tiles first_big .. end
// of gemm_core::xcd_tile_order's list), each as four 128 x 128 quarters
// (gemm_core::tail_quarter).
template <int STAGES, bool WHOLE, bool TAIL = false, bool KT = false>
__global__ void __launch_bounds__(256, STAGES == 2 ? 2 : 1) gemm_bf16_nt_128_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint16_t* __restrict__ c,
    uint32_t m, uint32_t n, uint32_t k, uint32_t xcds, uint32_t first_big = 0) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  uint32_t tm, tn;
  if constexpr (TAIL) {
    if (!gemm_core::tail_quarter(blockIdx.x, first_big, m, n, xcds, &tm, &tn)) return;
  } else {
    gemm_core::xcd_tile_order(blockIdx.x, (m + 127u) / 128u, (n + 127u) / 128u, xcds, &tm, &tn);
  }
  const uint32_t rows_a = WHOLE ? 128u : min(128u, m - tm * 128u);
  const uint32_t rows_b = WHOLE ? 128u : min(128u, n - tn * 128u);
  const auto ar =
      gemm_pipe::dense_rows<kRowBytes, 128, KT>(a + (uint64_t)tm * 128 * k, k, rows_a, k);
  const auto br =
      gemm_pipe::dense_rows<kRowBytes, 128, KT>(b + (uint64_t)tn * 128 * k, k, rows_b, k);
  gemm_pipe::Bf16Mma64::Acc acc;
  gemm_pipe::mainloop<gemm_pipe::Bf16Mma64, kRowBytes, STAGES, KT>(ar, br, k, smem, acc);
  gemm_pipe::store_bf16_128<WHOLE>(acc, c + (uint64_t)tm * 128 * n + (uint64_t)tn * 128, n,
                                   rows_a, rows_b);
}

// K = 0: C is all +0 (an empty sum).  A grid-stride fill kernel rather than
// a memset node, so a caller may capture the launch in a HIP graph.
__global__ void __launch_bounds__(256) zero_fill_bf16_kernel(uint16_t* __restrict__ c, uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) c[i] = 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_256_kernel", (const void*)gemm_bf16_nt_256_kernel<false, false>, 256, kFastSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_256_kernel<staged>", (const void*)gemm_bf16_nt_256_kernel<true, false>, 256, kFastSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_256_kernel<edge>", (const void*)gemm_bf16_nt_256_kernel<false, true>, 256, kFastSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2>", (const void*)gemm_bf16_nt_128_kernel<2, true>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2, edge>", (const void*)gemm_bf16_nt_128_kernel<2, false>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3>", (const void*)gemm_bf16_nt_128_kernel<3, true>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3, edge>", (const void*)gemm_bf16_nt_128_kernel<3, false>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2, tail>", (const void*)gemm_bf16_nt_128_kernel<2, true, true>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2, edge, tail>", (const void*)gemm_bf16_nt_128_kernel<2, false, true>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3, tail>", (const void*)gemm_bf16_nt_128_kernel<3, true, true>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3, edge, tail>", (const void*)gemm_bf16_nt_128_kernel<3, false, true>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_256_kernel<edge, k tail>", (const void*)gemm_bf16_nt_256_kernel<false, true, true>, 256, kFastSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_256_kernel<k tail>", (const void*)gemm_bf16_nt_256_kernel<false, false, true>, 256, kFastSmem}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2, k tail>", (const void*)gemm_bf16_nt_128_kernel<2, true, false, true>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3, k tail>", (const void*)gemm_bf16_nt_128_kernel<3, true, false, true>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2, tail, k tail>", (const void*)gemm_bf16_nt_128_kernel<2, true, true, true>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3, tail, k tail>", (const void*)gemm_bf16_nt_128_kernel<3, true, true, true>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2, edge, k tail>", (const void*)gemm_bf16_nt_128_kernel<2, false, false, true>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3, edge, k tail>", (const void*)gemm_bf16_nt_128_kernel<3, false, false, true>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<2, edge, tail, k tail>", (const void*)gemm_bf16_nt_128_kernel<2, false, true, true>, 256, kSmallSmem<2>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_128_kernel<3, edge, tail, k tail>", (const void*)gemm_bf16_nt_128_kernel<3, false, true, true>, 256, kSmallSmem<3>}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "gemm_bf16_nt_generic_kernel", (const void*)gemm_bf16_nt_generic_kernel, 256, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_gemm_bf16_nt", "zero_fill_bf16_kernel", (const void*)zero_fill_bf16_kernel, 256, 0})};

// Raises every fast-path kernel's dynamic-LDS limit once per process.
int32_t set_fast_lds() {
  static const int32_t rc = [] {
    int32_t r = fe2o3_host::set_dynamic_lds(
        {(const void*)gemm_bf16_nt_256_kernel<false, false>,
         (const void*)gemm_bf16_nt_256_kernel<true, false>,
         (const void*)gemm_bf16_nt_256_kernel<false, true>,
         (const void*)gemm_bf16_nt_256_kernel<false, true, true>,
         (const void*)gemm_bf16_nt_256_kernel<false, false, true>},
        kFastSmem);
    if (r == FE2O3_OK)
      r = fe2o3_host::set_dynamic_lds(
          {(const void*)gemm_bf16_nt_128_kernel<2, true>,
           (const void*)gemm_bf16_nt_128_kernel<2, false>,
           (const void*)gemm_bf16_nt_128_kernel<2, true, true>,
           (const void*)gemm_bf16_nt_128_kernel<2, false, true>,
           (const void*)gemm_bf16_nt_128_kernel<2, false, false, true>,
           (const void*)gemm_bf16_nt_128_kernel<2, false, true, true>,
           (const void*)gemm_bf16_nt_128_kernel<2, true, false, true>,
           (const void*)gemm_bf16_nt_128_kernel<2, true, true, true>},
          kSmallSmem<2>);
    if (r == FE2O3_OK)
      r = fe2o3_host::set_dynamic_lds(
          {(const void*)gemm_bf16_nt_128_kernel<3, true>,
           (const void*)gemm_bf16_nt_128_kernel<3, false>,
           (const void*)gemm_bf16_nt_128_kernel<3, true, true>,
           (const void*)gemm_bf16_nt_128_kernel<3, false, true>,
           (const void*)gemm_bf16_nt_128_kernel<3, false, false, true>,
           (const void*)gemm_bf16_nt_128_kernel<3, false, true, true>,
           (const void*)gemm_bf16_nt_128_kernel<3, true, false, true>,
           (const void*)gemm_bf16_nt_128_kernel<3, true, true, true>},
          kSmallSmem<3>);
    return r;
  }();
  return rc;
}

// The launches of `plan` (tile_plan.hpp).  KT: K not a multiple of 64 (a
// partial last stage in every tile).
template <bool KT>
int32_t launch_fast(const uint16_t* a, const uint16_t* b, uint16_t* c, uint32_t m, uint32_t n,
                    uint32_t k, const tile_plan::Plan& plan, uint32_t xcds, hipStream_t s) {
  const bool whole = m % 256 == 0 && n % 256 == 0 && aligned16(c);
  const bool whole128 = m % 128 == 0 && n % 128 == 0 && aligned16(c);
  // one launch of 128 x 128 tiles: the whole GEMM (TAIL false) or the tail
  // round's quarters
  auto small = [&](auto stages, auto tail, unsigned grid, uint32_t first) {
    constexpr int S = decltype(stages)::value;
    constexpr bool T = decltype(tail)::value;
    if (whole128)
      gemm_bf16_nt_128_kernel<S, true, T, KT><<<grid, 256, kSmallSmem<S>, s>>>(a, b, c, m, n, k,
                                                                               xcds, first);
    else
      gemm_bf16_nt_128_kernel<S, false, T, KT><<<grid, 256, kSmallSmem<S>, s>>>(a, b, c, m, n, k,
                                                                                xcds, first);
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
    gemm_bf16_nt_256_kernel<false, true, KT><<<big, 256, kFastSmem, s>>>(a, b, c, m, n, k, xcds);
  else if (!KT && gemm_core::staged_epilogue(((uint64_t)m + n) * k * 2u))
    gemm_bf16_nt_256_kernel<true, false><<<big, 256, kFastSmem, s>>>(a, b, c, m, n, k, xcds);
  else
    gemm_bf16_nt_256_kernel<false, false, KT><<<big, 256, kFastSmem, s>>>(a, b, c, m, n, k, xcds);
  const int32_t big_rc = fe2o3_host::after_launch();
  if (big_rc != FE2O3_OK || !plan.tail) return big_rc;
  // the last round of at most half the CUs' tiles as 128 x 128 quarters; two
  // per CU when there are more quarters than CUs
  return plan.tail_stages == 2
             ? small(Two{}, Tail{}, (unsigned)plan.tail_grid, plan.first_big)
             : small(Three{}, Tail{}, (unsigned)plan.tail_grid, plan.first_big);
}

}  // namespace

namespace {
constexpr uint32_t kRepackMin = 128;  // outputs at least this in M and N repack
}  // namespace

extern "C" int32_t fe2o3_gemm_bf16_nt(const uint16_t* a, uint64_t a_len, const uint16_t* b,
                                      uint64_t b_len, uint16_t* c, uint64_t c_len, uint32_t m,
                                      uint32_t n, uint32_t k, void* stream) {
  FE2O3_ENTRY("fe2o3_gemm_bf16_nt");
  if (a_len != (uint64_t)m * k || b_len != (uint64_t)n * k || c_len != (uint64_t)m * n)
    return FE2O3_ERR_LENGTH;
  if (c_len == 0) return FE2O3_OK;
  if ((a_len && !a) || (b_len && !b) || !c) return FE2O3_ERR_NULL;
  if (k == 0) {
    const uint64_t blocks = (c_len + 255) / 256;
    zero_fill_bf16_kernel<<<(unsigned)(blocks < 4096u ? blocks : 4096u), 256, 0,
                            (hipStream_t)stream>>>(c, c_len);
    return fe2o3_host::after_launch();
  }
  // fast path: 16-byte operand rows (K a multiple of 8), and a 256-row panel
  // (512 * k bytes) inside the 32-bit range of its buffer resource; whole
  // tiles with a 16-byte aligned C take the plain tile, any other M and N
  // the edge tile; K not a multiple of 64 the same tiles with a partial last
  // stage (KT)
  const bool fast = k % 8 == 0 && 512ull * k < (1ull << 31) && aligned16(a) && aligned16(b);
  if (fast) {
    const int32_t lds_rc = set_fast_lds();  // before any launch: a failure leaves C untouched
    if (lds_rc != FE2O3_OK) return lds_rc;
    tile_plan::Topology topo;
    const int32_t topo_rc = fe2o3_host::device_topology(&topo);
    if (topo_rc != FE2O3_OK) return topo_rc;
    const tile_plan::Plan plan = tile_plan::plan(m, n, topo);
    if (plan.grid > 0x7fffffffu || plan.tail_grid > 0x7fffffffu) return FE2O3_ERR_SHAPE;
    if (k % gemm_pipe::Geo<kRowBytes>::kK16 != 0)
      return launch_fast<true>(a, b, c, m, n, k, plan, topo.xcds, (hipStream_t)stream);
    return launch_fast<false>(a, b, c, m, n, k, plan, topo.xcds, (hipStream_t)stream);
  }
  // Rows the tile cannot read in place (K not a multiple of 8, or A or B two
  // bytes past a 16-byte boundary) are first copied into aligned rows of kp
  // = K rounded up to 8, zeros from K on, in stream-ordered scratch; the
  // tile then runs on kp, whose zeros fall where its partial last stage
  // puts zeros anyway, so an operand that is only misaligned gives the bits
  // of the aligned one.  Outputs below 128 x 128, and devices without
  // stream-ordered scratch, take the generic kernel.
  const uint32_t kp = (k + 7u) & ~7u;
  hipStream_t s = (hipStream_t)stream;
  if (m >= kRepackMin && n >= kRepackMin && 512ull * kp < (1ull << 31)) {
    const bool ra = k % 8 != 0 || !aligned16(a), rb = k % 8 != 0 || !aligned16(b);
    const int32_t lds_rc = set_fast_lds();
    if (lds_rc != FE2O3_OK) return lds_rc;
    tile_plan::Topology topo;
    const int32_t topo_rc = fe2o3_host::device_topology(&topo);
    if (topo_rc != FE2O3_OK) return topo_rc;
    const tile_plan::Plan plan = tile_plan::plan(m, n, topo);
    if (plan.grid > 0x7fffffffu || plan.tail_grid > 0x7fffffffu) return FE2O3_ERR_SHAPE;
    const uint64_t a_elems = ra ? (uint64_t)m * kp : 0, b_elems = rb ? (uint64_t)n * kp : 0;
    void* scratch = nullptr;
    if (fe2o3_host::scratch_alloc(&scratch, (a_elems + b_elems) * 2u, s) == FE2O3_OK) {
      uint16_t* ap = static_cast<uint16_t*>(scratch);
      uint16_t* bp = ap + a_elems;
      int32_t rc = FE2O3_OK;
      if (ra) rc = fe2o3_host::repack_bf16_rows(a, m, k, k, ap, kp, s);
      if (rb && rc == FE2O3_OK) rc = fe2o3_host::repack_bf16_rows(b, n, k, k, bp, kp, s);
      if (rc == FE2O3_OK)
        rc = kp % gemm_pipe::Geo<kRowBytes>::kK16 != 0
                 ? launch_fast<true>(ra ? ap : a, rb ? bp : b, c, m, n, kp, plan, topo.xcds, s)
                 : launch_fast<false>(ra ? ap : a, rb ? bp : b, c, m, n, kp, plan, topo.xcds, s);
      const int32_t free_rc = fe2o3_host::scratch_free(scratch, s);
      return rc != FE2O3_OK ? rc : free_rc;
    }
    (void)hipGetLastError();  // no stream-ordered scratch: the generic kernel
  }
  dim3 grid((n + N_BN - 1) / N_BN, (m + N_BM - 1) / N_BM);
  if (grid.y > 65535u) return FE2O3_ERR_SHAPE;
  gemm_bf16_nt_generic_kernel<<<grid, 256, 0, s>>>(a, b, c, m, n, k);
  return fe2o3_host::after_launch();
}
