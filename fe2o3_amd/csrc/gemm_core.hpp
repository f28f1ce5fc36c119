// gemm_core.hpp -- the 256x256x64 bf16 MFMA main loop shared by the dense
// NT GEMM and the grouped MoE expert GEMMs.
//
// Tile geometry (one 256-thread workgroup, 4 waves in 2x2):
//   wave (wm, wn) owns output rows wm*128 + [0,128) and columns
//   wn*128 + [0,128), as 4x4 tiles of v_mfma_f32_32x32x16_bf16.
// LDS layout per stage: A tile then B tile, each [256 rows][64 k] bf16 with
//   128-byte rows; 16-byte chunk c of row r sits at position c ^ swz(r),
//   swz(r) = (r ^ (r >> 3)) & 7.
// Global -> LDS: wave w, instruction j (0..7) moves rows (4j + w)*8 .. +7 of
//   each tile, lane l taking row +l/8 and LDS position l%8 (so it fetches
//   logical chunk (l%8) ^ swz(row)): every instruction reads eight full
//   128-byte row segments.
// MFMA issue order: D = B_frag x A_frag so that lane l ends with output
//   column block rows n = 8*(e/4) + 4*(l/32) + e%4 (e = 0..15) of output
//   row m = l%32: four consecutive n per lane for 8-byte bf16 stores.
#pragma once

#include "common.hpp"

namespace gemm_core {

using namespace fe2o3;

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kTileBytes = 256 * 64 * 2;          // 32 KiB per operand tile
constexpr int kStageBytes = 2 * kTileBytes;       // A + B
constexpr int kSmemBytes256 = 2 * kStageBytes;    // two stages = 128 KiB

struct Acc256 {
  f32x16_t v[4][4];
};

FE2O3_DEVICE void zero(Acc256& acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc.v[i][j][e] = 0.0f;
}

FE2O3_DEVICE uint32_t swz(uint32_t r) { return (r ^ (r >> 3)) & 7u; }

// Maps a linear workgroup id onto (tile_m, tile_n).  Workgroups are issued
// round-robin over the 8 XCDs, so id i runs on XCD i % 8; ids are first
// regrouped so that XCD x receives the contiguous range
// [x*tiles/8, (x+1)*tiles/8), then that range is walked in GROUP_M-row
// groups (Triton-style grouped order) so concurrently running workgroups of
// one XCD share A and B panels in its L2.
FE2O3_DEVICE void xcd_tile_order(uint32_t pid, uint32_t tiles_m, uint32_t tiles_n, uint32_t* tm,
                                 uint32_t* tn) {
  const uint32_t total = tiles_m * tiles_n;
  if (total % 8u == 0u) pid = (pid % 8u) * (total / 8u) + pid / 8u;
  constexpr uint32_t GROUP_M = 4;
  const uint32_t in_group = GROUP_M * tiles_n;
  const uint32_t group = pid / in_group;
  const uint32_t first_m = group * GROUP_M;
  const uint32_t size_m = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const uint32_t r = pid % in_group;
  *tm = first_m + r % size_m;
  *tn = r / size_m;
}

// Per-thread source rows of one operand tile.  Instruction j moves tile rows
// [32j, 32j+32) (rows (4j + w)*8 + lane/8 for wave w), so each instruction has
// a workgroup-uniform base pointer base[j]; off[j] is the 32-bit element
// offset from it of the 16-byte chunk this thread moves (k offset 0).
struct TileRows {
  const uint16_t* base[8];
  uint32_t off[8];
};

FE2O3_DEVICE uint32_t tile_row(int j) {
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  return (4u * j + w) * 8u + (lane >> 3);
}

FE2O3_DEVICE uint32_t tile_chunk(uint32_t row) { return ((threadIdx.x & 63u) & 7u) ^ swz(row); }

// Dense operand: tile rows start at `base`, consecutive rows `ld` apart;
// rows at or beyond `valid_rows` are clamped to the last valid row (their
// values only feed outputs that are never stored).
FE2O3_DEVICE TileRows dense_rows(const uint16_t* base, uint32_t ld, uint32_t valid_rows) {
  TileRows t;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t row = tile_row(j);
    const uint32_t chunk = tile_chunk(row);
    if (row >= valid_rows) row = valid_rows - 1u;
    t.base[j] = base;
    t.off[j] = row * ld + chunk * 8u;
  }
  return t;
}

FE2O3_DEVICE void issue_tile(const TileRows& rows, uint32_t k0, uint8_t* lds_tile) {
  const uint32_t w = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    g2l_b128(rows.base[j] + k0 + rows.off[j], lds_tile + (4u * j + w) * 1024u);
}

// MFMA policies.  Each LDS stage holds 128 bytes of k per tile row: 64 bf16
// or 128 fp8 values.  A policy knows how many k-substeps a stage has, how a
// wave reads its operand fragments for one substep, and the MFMA it issues.

// bf16: 4 substeps of 16 k; per substep 4 A and 4 B 16-byte reads and 16
// v_mfma_f32_32x32x16_bf16 per wave.
struct MmaBf16 {
  static constexpr int kSubsteps = 4;
  struct Frags {
    bf16x8_t a[4], b[4];
  };
  static FE2O3_DEVICE void load(const uint8_t* stage, int s, Frags& f) {
    const uint8_t* a_tile = stage;
    const uint8_t* b_tile = stage + kTileBytes;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t lr = lane & 31u, g = lane >> 5;
    const uint32_t c = 2u * (uint32_t)s + g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t ra = wm * 128u + i * 32u + lr;
      const uint32_t rb = wn * 128u + i * 32u + lr;
      f.a[i] = *reinterpret_cast<const bf16x8_t*>(a_tile + ra * 128u + ((c ^ swz(ra)) << 4));
      f.b[i] = *reinterpret_cast<const bf16x8_t*>(b_tile + rb * 128u + ((c ^ swz(rb)) << 4));
    }
  }
  static FE2O3_DEVICE void mma(const Frags& f, Acc256& acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc.v[i][j], 0, 0, 0);
  }
};

// OCP fp8 e4m3: 2 substeps of 64 k; per substep each lane reads 32 bytes
// (two 16-byte chunks) per operand fragment and the wave issues 16
// v_mfma_scale_f32_32x32x64_f8f6f4 with both formats e4m3 (cbsz = blgp = 0)
// and unit E8M0 block scales (127 = 2^0).
struct MmaFp8 {
  static constexpr int kSubsteps = 2;
  struct Frags {
    i32x8_t a[4], b[4];
  };
  static FE2O3_DEVICE i32x8_t read32(const uint8_t* tile, uint32_t r, uint32_t c0) {
    const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(tile + r * 128u + ((c0 ^ swz(r)) << 4));
    const i32x4_t hi =
        *reinterpret_cast<const i32x4_t*>(tile + r * 128u + (((c0 + 1u) ^ swz(r)) << 4));
    i32x8_t v;
    v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
    v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
    return v;
  }
  static FE2O3_DEVICE void load(const uint8_t* stage, int s, Frags& f) {
    const uint8_t* a_tile = stage;
    const uint8_t* b_tile = stage + kTileBytes;
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
  static FE2O3_DEVICE void mma(const Frags& f, Acc256& acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc.v[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[j], f.a[i], acc.v[i][j],
                                                                      0, 0, 0, 127, 0, 127);
  }
};

// Full K loop over `k16` 16-bit units of k per row (a multiple of 64: 128
// bytes per stage) with two LDS stages and register double-buffered
// fragments: the reads of substep s+1 are issued before the MFMAs of
// substep s, and the per-step barrier sits before the last substep's MFMAs
// so the first reads of the next stage overlap them.
template <class Mma = MmaBf16>
FE2O3_DEVICE void mainloop(const TileRows& a_rows, const TileRows& b_rows, uint32_t k16,
                           uint8_t* smem, Acc256& acc) {
  constexpr int S = Mma::kSubsteps;
  const uint32_t steps = k16 / BK;
  issue_tile(a_rows, 0, smem);
  issue_tile(b_rows, 0, smem + kTileBytes);
  wait_vmcnt0();
  __syncthreads();
  typename Mma::Frags f[2];
  Mma::load(smem, 0, f[0]);
  for (uint32_t kt = 0; kt < steps; ++kt) {
    const uint8_t* cur = smem + (kt & 1u) * kStageBytes;
    uint8_t* nxt = smem + ((kt + 1) & 1u) * kStageBytes;
    const bool more = kt + 1 < steps;
    if (more) {
      issue_tile(a_rows, (kt + 1) * BK, nxt);
      issue_tile(b_rows, (kt + 1) * BK, nxt + kTileBytes);
    }
#pragma unroll
    for (int s = 0; s + 1 < S; ++s) {
      Mma::load(cur, s + 1, f[(s + 1) & 1]);
      Mma::mma(f[s & 1], acc);
    }
    wait_vmcnt0();
    __syncthreads();
    if (more) Mma::load(nxt, 0, f[S & 1]);
    Mma::mma(f[(S - 1) & 1], acc);
  }
}

FE2O3_DEVICE void mainloop_nt_256(const uint16_t* a_tile_base, const uint16_t* b_tile_base,
                                  uint32_t k, uint32_t lda, uint32_t ldb, uint8_t* smem,
                                  Acc256& acc) {
  const TileRows ar = dense_rows(a_tile_base, lda, 256);
  const TileRows br = dense_rows(b_tile_base, ldb, 256);
  mainloop<MmaBf16>(ar, br, k, smem, acc);
}

// Output coordinates of accumulator (i, j, e) for this lane: tile row
// wm*128 + 32i + lane%32, tile column wn*128 + 32j + 8(e/4) + 4(lane/32) + e%4.
FE2O3_DEVICE uint32_t acc_row(int i) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  return (wave >> 1) * 128u + i * 32u + (lane & 31u);
}
FE2O3_DEVICE uint32_t acc_col(int j, int q) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  return (wave & 1u) * 128u + j * 32u + 8u * q + 4u * (lane >> 5);
}

// bf16 epilogue for a 256x256 tile at c_tile (row stride ldc); rows at or
// beyond valid_rows are not stored.
FE2O3_DEVICE void store_bf16_256(const Acc256& acc, uint16_t* c_tile, uint64_t ldc,
                                 uint32_t valid_rows = 256) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t row = wm * 128u + i * 32u + (lane & 31u);
    if (row >= valid_rows) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t col = wn * 128u + j * 32u + 8u * q + 4u * (lane >> 5);
        u32x2_t packed;
        packed[0] = pack_bf16x2(acc.v[i][j][4 * q + 0], acc.v[i][j][4 * q + 1]);
        packed[1] = pack_bf16x2(acc.v[i][j][4 * q + 2], acc.v[i][j][4 * q + 3]);
        *reinterpret_cast<u32x2_t*>(c_tile + (uint64_t)row * ldc + col) = packed;
      }
  }
}

}  // namespace gemm_core
