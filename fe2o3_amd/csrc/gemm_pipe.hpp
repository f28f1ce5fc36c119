// gemm_pipe.hpp -- multi-stage 256x256 MFMA GEMM pipeline for gfx950.
//
// Same workgroup tile as gemm_core.hpp (256 threads = 4 waves in 2x2, each
// wave 128x128 as 4x4 v_mfma_f32_32x32x16_bf16 tiles, D = B_frag x A_frag)
// but with a parameterized LDS stage:
//   ROW_BYTES  bytes of k per tile row per stage (128: 64 bf16; 64: 32 bf16)
//   STAGES     LDS stages in flight (STAGES * 2 * 256 * ROW_BYTES bytes)
// Stage kt+STAGES-1 is issued (global_load_lds_dwordx4, 16 bytes per lane)
// while stage kt is consumed, so each load has STAGES-1 stages of MFMA work
// to land.  Each thread waits with s_waitcnt vmcnt(N) for exactly its own
// loads of the next stage (N = loads it issued after that stage), then one
// barrier per stage publishes every wave's loads.
//
// LDS layout per operand tile: [256 rows][ROW_BYTES], 16-byte chunk c of row
// r stored at position c ^ swz(r):
//   ROW_BYTES 128: swz(r) = (r ^ (r >> 3)) & 7
//   ROW_BYTES  64: swz(r) = ((r >> 1) ^ (r >> 3)) & 3
// Both keep the MFMA operand reads (32 consecutive rows, one chunk) free of
// bank conflicts whether the LDS serves 8 or 16 lanes of a 16-byte read per
// cycle (measured: SQ_LDS_BANK_CONFLICT = 0).
#pragma once

#include "common.hpp"

namespace gemm_pipe {

using namespace fe2o3;

template <int ROW_BYTES>
struct Geo {
  static_assert(ROW_BYTES == 128 || ROW_BYTES == 64, "row of 128 or 64 bytes");
  static constexpr int kChunks = ROW_BYTES / 16;             // 16-byte chunks per row
  static constexpr int kRowsPerInst = 1024 / ROW_BYTES;      // rows per 1 KiB load
  static constexpr int kTileBytes = 256 * ROW_BYTES;         // one operand tile
  static constexpr int kInstPerWave = kTileBytes / 1024 / 4; // loads per wave per tile
  static constexpr int kK16 = ROW_BYTES / 2;                 // 16-bit k units per stage

  static FE2O3_DEVICE uint32_t swz(uint32_t r) {
    if (ROW_BYTES == 128) return (r ^ (r >> 3)) & 7u;
    return ((r >> 1) ^ (r >> 3)) & 3u;
  }
  // tile row moved by this thread in load j; the instruction covers rows
  // [(4j + w) * kRowsPerInst, +kRowsPerInst)
  static FE2O3_DEVICE uint32_t inst_row(int j) {
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    return (4u * j + w) * kRowsPerInst + lane / kChunks;
  }
  static FE2O3_DEVICE uint32_t inst_chunk(uint32_t row) {
    return ((threadIdx.x & 63u) % kChunks) ^ swz(row);
  }
};

struct Acc {
  f32x16_t v[4][4];
};

FE2O3_DEVICE void zero(Acc& acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc.v[i][j][e] = 0.0f;
}

// Per-thread source rows of one operand tile: for load j, an element offset
// from base[j] of the chunk this thread moves at k = 0.
template <int ROW_BYTES>
struct Rows {
  const uint16_t* base[Geo<ROW_BYTES>::kInstPerWave];
  uint32_t off[Geo<ROW_BYTES>::kInstPerWave];
};

// Dense operand: rows `ld` elements apart from `base`; rows at or beyond
// valid_rows are clamped to the last valid row (their products only reach
// outputs that are never stored).
template <int ROW_BYTES>
FE2O3_DEVICE Rows<ROW_BYTES> dense_rows(const uint16_t* base, uint32_t ld, uint32_t valid_rows) {
  using G = Geo<ROW_BYTES>;
  Rows<ROW_BYTES> t;
#pragma unroll
  for (int j = 0; j < G::kInstPerWave; ++j) {
    uint32_t row = G::inst_row(j);
    const uint32_t chunk = G::inst_chunk(row);
    if (row >= valid_rows) row = valid_rows - 1u;
    t.base[j] = base;
    t.off[j] = row * ld + chunk * 8u;
  }
  return t;
}

template <int ROW_BYTES>
FE2O3_DEVICE void issue(const Rows<ROW_BYTES>& rows, uint32_t k16, uint8_t* lds_tile) {
  using G = Geo<ROW_BYTES>;
  const uint32_t w = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < G::kInstPerWave; ++j)
    g2l_b128(rows.base[j] + k16 + rows.off[j], lds_tile + (4u * j + w) * 1024u);
}

// bf16 operands: substeps of 16 k (32 bytes of each row) per stage.
template <int ROW_BYTES>
struct MmaBf16 {
  using G = Geo<ROW_BYTES>;
  static constexpr int kSubsteps = ROW_BYTES / 32;
  struct Frags {
    bf16x8_t a[4], b[4];
  };
  static FE2O3_DEVICE void load(const uint8_t* a_tile, const uint8_t* b_tile, int s, Frags& f) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t lr = lane & 31u, g = lane >> 5;
    const uint32_t c = 2u * (uint32_t)s + g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t ra = wm * 128u + i * 32u + lr;
      const uint32_t rb = wn * 128u + i * 32u + lr;
      f.a[i] = *reinterpret_cast<const bf16x8_t*>(a_tile + ra * ROW_BYTES + ((c ^ G::swz(ra)) << 4));
      f.b[i] = *reinterpret_cast<const bf16x8_t*>(b_tile + rb * ROW_BYTES + ((c ^ G::swz(rb)) << 4));
    }
  }
  static FE2O3_DEVICE void mma(const Frags& f, Acc& acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc.v[i][j], 0, 0, 0);
  }
};

// OCP fp8 e4m3 operands: substeps of 64 k (64 bytes of each row, two
// 16-byte chunks per lane) issuing v_mfma_scale_f32_32x32x64_f8f6f4 with both
// formats e4m3 (cbsz = blgp = 0) and unit E8M0 block scales (127 = 2^0).
template <int ROW_BYTES>
struct MmaFp8 {
  using G = Geo<ROW_BYTES>;
  static constexpr int kSubsteps = ROW_BYTES / 64;
  struct Frags {
    i32x8_t a[4], b[4];
  };
  static FE2O3_DEVICE i32x8_t read32(const uint8_t* tile, uint32_t r, uint32_t c0) {
    const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(tile + r * ROW_BYTES + ((c0 ^ G::swz(r)) << 4));
    const i32x4_t hi =
        *reinterpret_cast<const i32x4_t*>(tile + r * ROW_BYTES + (((c0 + 1u) ^ G::swz(r)) << 4));
    i32x8_t v;
    v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
    v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
    return v;
  }
  static FE2O3_DEVICE void load(const uint8_t* a_tile, const uint8_t* b_tile, int s, Frags& f) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t lr = lane & 31u, g = lane >> 5;
    const uint32_t c0 = 4u * (uint32_t)s + 2u * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f.a[i] = read32(a_tile, wm * 128u + i * 32u + lr, c0);
      f.b[i] = read32(b_tile, wn * 128u + i * 32u + lr, c0);
    }
  }
  static FE2O3_DEVICE void mma(const Frags& f, Acc& acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc.v[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[j], f.a[i], acc.v[i][j],
                                                                      0, 0, 0, 127, 0, 127);
  }
};

template <int N>
FE2O3_DEVICE void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Loads j in [J0, J1) of one operand tile.
template <int ROW_BYTES, int J0, int J1>
FE2O3_DEVICE void issue_part(const Rows<ROW_BYTES>& rows, uint32_t k16, uint8_t* lds_tile) {
  const uint32_t w = threadIdx.x >> 6;
#pragma unroll
  for (int j = J0; j < J1; ++j)
    g2l_b128(rows.base[j] + k16 + rows.off[j], lds_tile + (4u * j + w) * 1024u);
}

// Scheduling pattern for one substep: 16 MFMAs, each followed by up to one
// global->LDS load and one LDS fragment read, so the MFMA pipe never waits
// behind a burst of memory instructions and every fragment read is issued a
// full substep before the MFMAs that consume it.
template <int V, int D>
FE2O3_DEVICE void interleave() {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA
    if (i < V) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // VMEM
    if (i < D) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
  }
}

// One substep S_ of K step kt: issue this substep's share of the look-ahead
// stage's global->LDS copies (all of them in substep 0 with two stages, since
// they must land within the step; an equal share per substep otherwise),
// read the next substep's fragments (or, in the last substep, wait for the
// next stage and cross the barrier first), then the 16 MFMAs of this substep.
template <class Mma, int ROW_BYTES, int STAGES, int S_>
struct Substep {
  using G = Geo<ROW_BYTES>;
  static constexpr int S = Mma::kSubsteps;
  static constexpr int NJ = G::kInstPerWave;
  static constexpr int LPS = 2 * NJ;
  static constexpr int J0 = STAGES == 2 ? 0 : S_ * NJ / S;
  static constexpr int J1 = STAGES == 2 ? (S_ == 0 ? NJ : 0) : (S_ + 1) * NJ / S;
  static FE2O3_DEVICE void run(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br, uint32_t ka,
                               uint8_t* dst, const uint8_t* cur, const uint8_t* next,
                               typename Mma::Frags* f, Acc& acc) {
    issue_part<ROW_BYTES, J0, J1>(ar, ka, dst);
    issue_part<ROW_BYTES, J0, J1>(br, ka, dst + G::kTileBytes);
    if constexpr (S_ + 1 < S) {
      Mma::load(cur, cur + G::kTileBytes, S_ + 1, f[(S_ + 1) & 1]);
    } else {
      wait_vmcnt<(STAGES - 2) * LPS>();
      lds_barrier();
      Mma::load(next, next + G::kTileBytes, 0, f[S & 1]);
    }
    Mma::mma(f[S_ & 1], acc);
    interleave<2 * (J1 - J0), sizeof(typename Mma::Frags) / 16>();  // 16-byte LDS reads
    // close the scheduling region: MFMAs of the next substep (whose operands
    // are read above) must not be hoisted into this one
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (S_ + 1 < S)
      Substep<Mma, ROW_BYTES, STAGES, S_ + 1>::run(ar, br, ka, dst, cur, next, f, acc);
  }
};

// K loop over k16 16-bit units per row (a multiple of Geo::kK16, at least
// one stage).  The body is branch-free: the look-ahead stage index is
// clamped for its source address while its destination buffer always
// advances, so past the end the copies land in a buffer nobody reads again
// and every iteration issues the same number of loads (a constant vmcnt).
template <class Mma, int ROW_BYTES, int STAGES>
FE2O3_DEVICE void mainloop(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br, uint32_t k16,
                           uint8_t* smem, Acc& acc) {
  using G = Geo<ROW_BYTES>;
  constexpr int NJ = G::kInstPerWave;
  constexpr int LPS = 2 * NJ;
  constexpr uint32_t kStageBytes = 2u * G::kTileBytes;
  static_assert(STAGES >= 2 && (STAGES - 2) * LPS <= 63, "stages");
  static_assert(STAGES == 2 || NJ % Mma::kSubsteps == 0, "even split of the loads");
  static_assert(Mma::kSubsteps % 2 == 0, "fragment buffers alternate within a stage");
  const int steps = (int)(k16 / G::kK16);
  auto buf = [&](int st) { return smem + (uint32_t)(st % STAGES) * kStageBytes; };
  auto kofs = [&](int st) { return (uint32_t)(st < steps ? st : steps - 1) * G::kK16; };
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st) {
    issue_part<ROW_BYTES, 0, NJ>(ar, kofs(st), buf(st));
    issue_part<ROW_BYTES, 0, NJ>(br, kofs(st), buf(st) + G::kTileBytes);
  }
  wait_vmcnt<(STAGES - 2) * LPS>();
  lds_barrier();
  typename Mma::Frags f[2];
  Mma::load(buf(0), buf(0) + G::kTileBytes, 0, f[0]);
  for (int kt = 0; kt < steps; ++kt)
    Substep<Mma, ROW_BYTES, STAGES, 0>::run(ar, br, kofs(kt + STAGES - 1), buf(kt + STAGES - 1),
                                            buf(kt), buf(kt + 1), f, acc);
}

// Output coordinates of accumulator (i, j, e) of this lane: tile row
// wm*128 + 32i + lane%32, tile column wn*128 + 32j + 8(e/4) + 4(lane/32) + e%4.
FE2O3_DEVICE uint32_t acc_row(int i) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  return (wave >> 1) * 128u + i * 32u + (lane & 31u);
}
FE2O3_DEVICE uint32_t acc_col(int j, int q) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  return (wave & 1u) * 128u + j * 32u + 8u * q + 4u * (lane >> 5);
}

FE2O3_DEVICE void store_bf16(const Acc& acc, uint16_t* c_tile, uint64_t ldc,
                             uint32_t valid_rows = 256) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t row = acc_row(i);
    if (row >= valid_rows) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x2_t packed;
        packed[0] = pack_bf16x2(acc.v[i][j][4 * q + 0], acc.v[i][j][4 * q + 1]);
        packed[1] = pack_bf16x2(acc.v[i][j][4 * q + 2], acc.v[i][j][4 * q + 3]);
        *reinterpret_cast<u32x2_t*>(c_tile + (uint64_t)row * ldc + acc_col(j, q)) = packed;
      }
  }
}

}  // namespace gemm_pipe
