// gemm_pipe.hpp -- the 256x256 MFMA GEMM pipeline for gfx950 (bf16 and
// OCP fp8 e4m3 operands).
//
// Workgroup: 256 threads = 4 waves in 2x2, each wave a 128x128 block of the
// output, accumulators in AGPRs.  The instruction is a policy:
//   Bf16Mma  8x8 tiles of v_mfma_f32_16x16x32_bf16 (inline asm, Acc16)
//   Fp8Mma16 8x8 tiles of v_mfma_f32_16x16x128_f8f6f4 (builtin, Acc16)
// Parameters:
//   ROW_BYTES  bytes of k per tile row per stage (128: 64 bf16 / 128 fp8)
//   STAGES     LDS stages in flight (STAGES * 2 * 256 * ROW_BYTES bytes)
//
// Global -> LDS.  Operand tiles are copied with buffer_load_dwordx4 ... lds
// (16 bytes per lane straight into LDS).  Each operand has a buffer resource
// per load slot (wave-uniform) and each thread a fixed byte offset per slot;
// the k offset of a stage is a scalar, and the LDS destination (M0) is
// scalar too, so a copy costs no VALU.
//
// LDS layout.  The A tiles of all stages come first, then the B tiles (A of
// stage p at p * T, B at (STAGES + p) * T, T = 256 * ROW_BYTES).  16-byte
// chunk c of row r is stored at position c ^ swz(r):
//   ROW_BYTES 128: swz(r) = (r & 6) | parity(r & 7)
//   ROW_BYTES  64: swz(r) = ((r >> 1) ^ (r >> 3)) & 3
// A ds_read_b128 is served in four passes of 16 lanes, {8k .. 8k+7} and
// {8k+16 .. 8k+23}, over 64 banks of 4 bytes: a pass is conflict-free when
// its lanes' 16-byte pieces fall on distinct (row parity, chunk position)
// pairs.  Both read patterns pair each row with chunks c and c ^ 1 (bf16
// 16x16x32: 16 rows x chunks 4s + l/16) or c and c ^ 2 (fp8 16x16x128: 16
// rows x chunks 2(l/16) + h), so among the even (odd) rows of each 8 the
// swizzle values must differ in bits {1, 2} and in bits {0, 2}: the values
// of even parity {0, 3, 5, 6} on even rows and {1, 2, 4, 7} on odd rows do.
// Measured SQ_LDS_BANK_CONFLICT = 0 for both; the earlier (r ^ (r >> 2)) & 7
// gave the fp8 pattern 2-way conflicts (3.4e7 cycles per 8192^3 GEMM, LDS
// busy twice as long, at the same throughput).
//
// Fragment reads.  The K loop is unrolled over the STAGES buffers, so the
// stage, tile and row-block offsets of every ds_read are compile-time
// immediates; the per-lane part depends only on (substep, row block mod the
// swizzle period) and is computed once before the loop.
#pragma once

#include <type_traits>

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
  // loads per wave and stage for an operand tile of `rows` rows
  static constexpr int insts(int rows) { return rows * ROW_BYTES / 4096; }

  static FE2O3_DEVICE uint32_t swz(uint32_t r) {
    if (ROW_BYTES == 128) return (r & 6u) | ((r ^ (r >> 1) ^ (r >> 2)) & 1u);
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


// Source of one operand tile of N loads per wave: for load slot j the base
// of its buffer (wave-uniform) and this thread's byte offset of its chunk
// at k = 0; all slots share one buffer extent.  Offsets and extent are
// 32-bit.  The B tile is always 256 rows; the A tile has the policy's
// kARows rows (256, or fewer for short tiles).  KN: the operand is stored
// [k][n] (rows of n, kn_rows) and a stage's k offset `kbytes` (the byte
// offset along a k-contiguous row) becomes kbytes * kmul bytes down the rows.
// MASK: the rows hold k_end bytes of k, not a whole number of stages; a
// chunk at or past k_end (chunk byte offset cbytes[j] along k within its
// stage, plus the stage's kbytes) loads from a VGPR offset past the
// buffer's extent, which the range check turns into 16 zero bytes in LDS.
// The range check covers the VGPR offset only, not the scalar offset soff
// carries, so a stage offset alone never makes a load return zeros: every
// load past the operand's k goes through this mask.  For a [k][n] operand a
// chunk is one k row (cbytes = 2 * its row within the stage).  Dense rows
// have k_end a multiple of 16 bytes, so no chunk straddles it.  The zeros'
// products are zero, the zero padding the staged kernels give a partial k
// step.
constexpr uint32_t kOutOfRange = 0x80000000u;  // past any extent (extents are < 2^31)

// the mask's per-slot chunk offsets and k extent (no members without MASK)
template <bool MASK, int N>
struct RowsMask {
  uint32_t cbytes[N];
  uint32_t k_end;
};
template <int N>
struct RowsMask<false, N> {};

template <int ROW_BYTES, int N = Geo<ROW_BYTES>::kInstPerWave, bool KN = false,
          bool MASK = false>
struct Rows : RowsMask<MASK, N> {
  static constexpr bool kMask = MASK;
  const void* base[N];
  uint32_t bytes;
  uint32_t voff[N];
  uint32_t kmul;
  FE2O3_DEVICE uint32_t soff(uint32_t kbytes) const { return KN ? kbytes * kmul : kbytes; }
  // this lane's offset for load slot j of the stage at kbytes
  FE2O3_DEVICE uint32_t off(int j, uint32_t kbytes) const {
    if constexpr (MASK) return this->cbytes[j] < this->k_end - kbytes ? voff[j] : kOutOfRange;
    else return voff[j];
  }
};

FE2O3_DEVICE __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, the raw-buffer setting for CDNA
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from buffer `r` at voff + soff (soff wave-uniform) into
// LDS at lds + 16 * lane (lds wave-uniform).
FE2O3_DEVICE void b2l_b128(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, voff, soff, 0, 0);
}

// Dense operand: rows `ld` 16-bit elements apart from `base`, k16 elements
// read per row; rows at or beyond valid_rows are clamped to the last valid
// row (their products only reach outputs that are never stored).  The
// caller guarantees ((valid_rows - 1) * ld + k16) * 2 < 2^31.  MASK: k16 is
// a multiple of 8 but not of the stage's k (Rows::off).
template <int ROW_BYTES, int ROWS = 256, bool MASK = false>
FE2O3_DEVICE Rows<ROW_BYTES, Geo<ROW_BYTES>::insts(ROWS), false, MASK> dense_rows(
    const uint16_t* base, uint32_t ld, uint32_t valid_rows, uint32_t k16) {
  using G = Geo<ROW_BYTES>;
  static_assert(ROWS * ROW_BYTES % 4096 == 0, "whole 1-KiB loads per wave for the tile's rows");
  Rows<ROW_BYTES, G::insts(ROWS), false, MASK> t;
  t.bytes = ((valid_rows - 1u) * ld + k16) * 2u;
  if constexpr (MASK) t.k_end = k16 * 2u;
#pragma unroll
  for (int j = 0; j < G::insts(ROWS); ++j) {
    uint32_t row = G::inst_row(j);
    const uint32_t chunk = G::inst_chunk(row);
    if (row >= valid_rows) row = valid_rows - 1u;
    t.base[j] = base;
    t.voff[j] = (row * ld + chunk * 8u) * 2u;
    if constexpr (MASK) t.cbytes[j] = chunk * 16u;
  }
  return t;
}

// Loads j in [J0, J1) of one operand tile into the LDS tile at byte offset
// `tile` of smem, k offset `kbytes` (wave-uniform).
template <int ROW_BYTES, int J0, int J1, int N, bool KN, bool MASK>
FE2O3_DEVICE void issue_part(const Rows<ROW_BYTES, N, KN, MASK>& rows, uint32_t kbytes,
                             uint8_t* smem, uint32_t tile, uint32_t wave) {
#pragma unroll
  for (int j = J0; j < J1; ++j)
    b2l_b128(rsrc(rows.base[j], rows.bytes), smem + tile + (4u * j + wave) * 1024u,
             rows.off(j, kbytes), rows.soff(kbytes));
}

// B stored [k][n] (row-major, ldb elements apart), 256 columns from `base`:
// one stage is 64 k-rows of 512 bytes.  Load j of wave w moves k-rows
// 2(4j + w) and 2(4j + w) + 1; lane l fills LDS chunk position l % 32 of
// k-row 2(4j + w) + l / 32 with global chunk (l % 32) ^ kn_swz(row), i.e.
// columns 8c .. 8c + 7 of chunk c are stored at chunk position c ^
// kn_swz(row).  Columns at or past valid_cols read the last valid chunk
// (their products reach only outputs that are never stored).  The caller
// guarantees ((k16 - 1) * ld + 256) * 2 < 2^31 and 16-byte aligned rows.
FE2O3_DEVICE uint32_t kn_swz(uint32_t krow) {
  // twice a 4-bit row code: the 16 rows one transposing fragment read
  // touches (8g + q, g, q < 4) get 16 different codes, so its 64 lanes'
  // 8-byte pieces fill 32 distinct 16-byte positions of the 512-byte rows
  return 2u * ((krow & 3u) | (((krow >> 3) & 3u) << 2));
}
// MASK: k16 is not a multiple of 64 and the last stage's rows from k16 on
// load zeros (Rows::off).
template <bool MASK = false>
FE2O3_DEVICE Rows<128, 8, true, MASK> kn_rows(const uint16_t* base, uint32_t ld,
                                              uint32_t valid_cols, uint32_t k16) {
  Rows<128, 8, true, MASK> t;
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t last_chunk = (valid_cols - 1u) / 8u;
  t.bytes = ((k16 - 1u) * ld + valid_cols) * 2u;
  t.kmul = ld;  // a stage of 64 k (128 bytes along a k row) is 64 rows of ld elements
  if constexpr (MASK) t.k_end = k16 * 2u;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t krow = 2u * (4u * j + w) + lane / 32u;
    uint32_t chunk = (lane % 32u) ^ kn_swz(krow);
    if (chunk > last_chunk) chunk = last_chunk;
    t.base[j] = base;
    t.voff[j] = (krow * ld + chunk * 8u) * 2u;
    if constexpr (MASK) t.cbytes[j] = 2u * krow;
  }
  return t;
}

// Stage p's A tile (A_ROWS rows) at a(p); its B tile (B_TILE bytes: 256
// rows, or a policy's smaller tile) at b_region + b(p).  Fragment reads add
// a(p) or b(p) (plus the row-block offset) as ds_read immediates; the B
// region's base is folded into the per-lane B offsets, so every immediate
// stays below 64 KiB.
template <int ROW_BYTES, int STAGES, int A_ROWS = 256, int B_TILE = 256 * ROW_BYTES>
struct Lay {
  using G = Geo<ROW_BYTES>;
  static constexpr uint32_t a_tile = (uint32_t)A_ROWS * ROW_BYTES;
  static constexpr uint32_t b_region = (uint32_t)STAGES * a_tile;
  static constexpr uint32_t a(int p) { return (uint32_t)p * a_tile; }
  static constexpr uint32_t b(int p) { return (uint32_t)p * (uint32_t)B_TILE; }
  // largest row-block offset: 16-row block 7 (bf16) > 32-row block 3 (fp8)
  static_assert((STAGES - 1) * B_TILE + 7 * 16 * ROW_BYTES < 65536,
                "fragment read offsets fit the ds_read immediate");
};

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0]+[15:14], expcnt [6:4],
// lgkmcnt [11:8]); as builtins the compiler's own wait tracking sees them
constexpr int waitcnt_imm(int vmcnt, int lgkmcnt) {
  return (vmcnt & 15) | ((vmcnt >> 4) << 14) | (7 << 4) | (lgkmcnt << 8);
}
constexpr int kWaitVm0Lgkm0 = waitcnt_imm(0, 0);
constexpr int kWaitVm0 = waitcnt_imm(0, 15);
constexpr int kWaitLgkm0 = waitcnt_imm(63, 0);

// B stored [k][n] for 128-column tiles (Bf16MmaKN64): one stage is 64 k-rows
// of 256 bytes.  Load j of wave w moves k-rows 4(4j + w) .. +3; lane l fills
// LDS chunk position l % 16 of k-row 4(4j + w) + l / 16 with global chunk
// (l % 16) ^ kn_swz16(row).  Columns at or past valid_cols read the last
// valid chunk (their products reach only outputs that are never stored).
// The caller guarantees ((k16 - 1) * ld + 128) * 2 < 2^31 and 16-byte
// aligned rows.
FE2O3_DEVICE uint32_t kn_swz16(uint32_t krow) {
  // twice a 3-bit row code: the 8 rows a half wave of one transposing read
  // touches (8g + q, g < 2, q < 4) get 8 different codes, so its 32 lanes'
  // 8-byte pieces fill 16 distinct 16-byte positions of the 256-byte rows
  return 2u * ((krow & 3u) | (((krow >> 3) & 1u) << 2));
}
template <bool MASK = false>
FE2O3_DEVICE Rows<128, 4, true, MASK> kn_rows128(const uint16_t* base, uint32_t ld,
                                                 uint32_t valid_cols, uint32_t k16) {
  Rows<128, 4, true, MASK> t;
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t last_chunk = (valid_cols - 1u) / 8u;
  t.bytes = ((k16 - 1u) * ld + valid_cols) * 2u;
  t.kmul = ld;  // a stage of 64 k (128 bytes along a k row) is 64 rows of ld elements
  if constexpr (MASK) t.k_end = k16 * 2u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t krow = 4u * (4u * j + w) + lane / 16u;
    uint32_t chunk = (lane % 16u) ^ kn_swz16(krow);
    if (chunk > last_chunk) chunk = last_chunk;
    t.base[j] = base;
    t.voff[j] = (krow * ld + chunk * 8u) * 2u;
    if constexpr (MASK) t.cbytes[j] = 2u * krow;
  }
  return t;
}

// ---- instruction policies --------------------------------------------------------------------
//
// A policy fixes, per substep (a k slice of one stage): kMfma MFMAs, issued
// as tile I = (I / kTn, I % kTn), row tile outer; kReads fragment read units
// of the next substep, in the order the MFMAs first use them; and how the
// first substep of the K loop writes (rather than adds to) the accumulators.

template <int RB, int CB = 8>
struct Acc16T {  // RB row blocks of 16 x CB column blocks of 16
  f32x4_t v[RB][CB];
};
using Acc16 = Acc16T<8>;

// bf16: v_mfma_f32_16x16x32_bf16, 32 k per substep.  Each wave owns RPW
// output rows (RPW/16 row blocks) by 128 columns; the A tile holds 2 RPW
// rows (256 for full tiles; any multiple of 32 up to 288 for the MoE
// experts' tiles, which then cost the MFMAs and A loads of their rows
// only).  Row blocks 0-7 accumulate in AGPRs (all 256 of them); a ninth
// (RPW = 144) in 32 VGPRs.
// Lane l holds k 8(l/16) .. +7 of row 16i + l%16 of the wave's A rows (a[i])
// and B rows (b[j]); the swizzle of a row depends on its index mod 32, hence
// four lane offsets per operand and substep.  One read unit is one
// ds_read_b128.
//
// The MFMAs are inline asm with the accumulator tied to the destination
// ("+a").  Left to itself the compiler gives this 8x8 tile's MFMAs a
// destination other than their accumulator input and pays for it with
// hundreds of v_accvgpr moves per iteration.  Inline asm hides the MFMAs from
// the compiler's hazard recognizer, so:
//   - the first substep writes the accumulators with srcC = 0 (no VALU write
//     of an accumulator precedes an MFMA);
//   - finish() puts explicit wait states (s_nop) between the last MFMA and
//     the epilogue's VALU reads of the accumulators;
//   - fragment registers are only MFMA sources A and B, read at issue: the
//     LDS reads that overwrite them need no wait states;
//   - accumulators, AGPR or VGPR, are touched by nothing but these MFMAs
//     between the first substep and finish() (tests/test_isa_mfma_acc.py
//     checks the compiled MoE kernels for it).
template <int ROW_BYTES, int RPW = 128>
struct Bf16Mma {
  static_assert(RPW % 16 == 0 && RPW >= 16 && RPW <= 144, "rows per wave");
  using G = Geo<ROW_BYTES>;
  static constexpr int kRB = RPW / 16;
  using Acc = Acc16T<kRB>;
  static constexpr int kSubsteps = ROW_BYTES / 64, kMfma = kRB * 8, kTn = 8, kReads = kRB + 8;
  static constexpr int kARows = 2 * RPW;
  static constexpr bool kBKN = false;
  static constexpr int kBTileBytes = G::kTileBytes;
  static constexpr int kLateSlots = kMfma;  // late copies spread over a whole substep 0
  struct Frags {
    bf16x8_t a[kRB], b[8];
  };
  struct Lanes {
    uint32_t a[kSubsteps][4], b[kSubsteps][4];
  };
  static FE2O3_DEVICE Lanes lanes(uint32_t b_region) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t lr = lane & 15u, g = lane >> 4;
    Lanes l;
#pragma unroll
    for (int s = 0; s < kSubsteps; ++s)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t c = 4u * s + g;
        const uint32_t ra = wm * RPW + p * 16u + lr, rb = wn * 128u + p * 16u + lr;
        l.a[s][p] = (wm * RPW + lr) * ROW_BYTES + ((c ^ G::swz(ra)) << 4);
        l.b[s][p] = b_region + (wn * 128u + lr) * ROW_BYTES + ((c ^ G::swz(rb)) << 4);
      }
    return l;
  }
  // read unit R of substep S from the stage at A_TILE / B_TILE: a0, b0 .. b7, a1 .. a7
  template <uint32_t A_TILE, uint32_t B_TILE, int S, int R>
  static FE2O3_DEVICE void read(const uint8_t* smem, const Lanes& l, Frags& f) {
    static_assert(R >= 0 && R < kReads, "read unit");
    if constexpr (R == 0) {
      f.a[0] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][0] + A_TILE);
    } else if constexpr (R <= 8) {
      constexpr int j = R - 1;
      f.b[j] = *reinterpret_cast<const bf16x8_t*>(smem + l.b[S][j & 3] +
                                                  (B_TILE + j * 16u * ROW_BYTES));
    } else {
      constexpr int i = R - 8;
      f.a[i] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][i & 3] +
                                                  (A_TILE + i * 16u * ROW_BYTES));
    }
  }
  template <bool FIRST, int I>
  static FE2O3_DEVICE void mfma(Acc& acc, const Frags& f) {
    constexpr int i = I / kTn, j = I % kTn;
    if constexpr (FIRST && i < 8)
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                   : "=a"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
    else if constexpr (FIRST)
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                   : "=v"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
    else if constexpr (i < 8)
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                   : "+a"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
    else
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                   : "+v"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
  }
  // wait states between the last MFMA's accumulator write and the VALU reads
  // that follow (an 8-pass MFMA needs at most 18); every accumulator then
  // passes through an empty asm, so no copy of one out of its AGPRs (the
  // epilogue's v_accvgpr_read) can be placed ahead of the wait states
  static FE2O3_DEVICE void finish(Acc& acc) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < kRB; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (i < 8) asm volatile("" : "+a"(acc.v[i][j]));
        else asm volatile("" : "+v"(acc.v[i][j]));
      }
  }
};

// bf16 with B stored [k][n] (kn_rows): the A side is Bf16Mma<128>'s; a B
// fragment (k 8(l/16) .. +7 of column 16j + l%16) is read from the row-major
// LDS tile with two ds_read_b64_tr_b16.  Within each 16-lane group the
// instruction hands lane i element M[4e + i/4][i%4] (e = 0..3) of the 16 x 4
// block whose row r is the 4 bf16 at lane r's address; lane i of group G
// addresses k-row kb + i/4, columns c0 + 4(i%4) (kb = 32s + 8G, c0 the
// fragment's first column), so it receives B[kb + e][c0 + i]: four k of its
// column, and the second read (k-rows + 4, 2048 bytes on) the next four.  The
// per-lane byte offsets of the eight fragments differ by more than a
// constant (kn_swz mixes the column bits), so each substep keeps eight.
struct Bf16MmaKN {
  using A = Bf16Mma<128, 128>;
  using Acc = A::Acc;
  static constexpr int kRB = A::kRB, kSubsteps = A::kSubsteps, kMfma = A::kMfma, kTn = A::kTn;
  static constexpr int kReads = A::kReads;
  static constexpr int kARows = A::kARows;
  static constexpr bool kBKN = true;
  static constexpr int kBTileBytes = A::kBTileBytes;
  static constexpr int kLateSlots = kMfma;
  using Frags = A::Frags;
  struct Lanes {
    uint32_t a[kSubsteps][4], b[kSubsteps][8];
  };
  static FE2O3_DEVICE Lanes lanes(uint32_t b_region) {
    const typename A::Lanes la = A::lanes(b_region);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wn = wave & 1u, g = lane >> 4, i = lane & 15u;
    Lanes l;
#pragma unroll
    for (int s = 0; s < kSubsteps; ++s) {
#pragma unroll
      for (int p = 0; p < 4; ++p) l.a[s][p] = la.a[s][p];
      const uint32_t krow = 32u * s + 8u * g + (i >> 2);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t chunk = wn * 16u + 2u * j + ((i & 3u) >> 1);
        l.b[s][j] = b_region + krow * 512u + ((chunk ^ kn_swz(krow)) << 4) + (i & 1u) * 8u;
      }
    }
    return l;
  }
  template <uint32_t A_TILE, uint32_t B_TILE, int S, int R>
  static FE2O3_DEVICE void read(const uint8_t* smem, const Lanes& l, Frags& f) {
    static_assert(R >= 0 && R < kReads, "read unit");
    if constexpr (R == 0) {
      f.a[0] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][0] + A_TILE);
    } else if constexpr (R <= 8) {
      constexpr int j = R - 1;
      // inline asm: as a builtin the transposing read is taken to alias the
      // global->LDS copies in flight and gets a vmcnt(0) before it, which
      // drains the copy pipeline every substep.  It does not alias them
      // (copies fill the other stage), and its result is waited for with the
      // A read a0 issued before it: the compiler's lgkmcnt wait for a0 at
      // the next substep's first MFMA leaves only the later A reads a1..a7
      // outstanding, and LDS reads complete in order.  The compiled kernel is
      // replayed against that rule by tests/test_isa_lds_waits.py.
      const lds_bf16x4_t* p = (const lds_bf16x4_t*)(smem + l.b[S][j]);
      bf16x4_t lo, hi;
      // early-clobber outputs: the second read takes its address from p
      // after the first is in flight, so lo must not be given p's register
      asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\tds_read_b64_tr_b16 %1, %2 offset:%4"
                   : "=&v"(lo), "=&v"(hi)
                   : "v"(p), "i"(B_TILE), "i"(B_TILE + 2048u));
      f.b[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      constexpr int ii = R - 8;
      f.a[ii] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][ii & 3] +
                                                   (A_TILE + ii * 16u * 128u));
    }
  }
  template <bool FIRST, int I>
  static FE2O3_DEVICE void mfma(Acc& acc, const Frags& f) {
    A::template mfma<FIRST, I>(acc, f);
  }
  static FE2O3_DEVICE void finish(Acc& acc) { A::finish(acc); }
};

// bf16, both operands k-contiguous (dense_rows), 128 x 128 tiles: the small
// grid form of Bf16Mma.  Each wave owns 64 rows by 64 columns (4 x 4 MFMA
// tiles, 64 AGPRs); A and B tiles of 128 rows.  All reads are ds_read_b128,
// in Bf16Mma's order (a0, b0 .. b3, a1 .. a3).
struct Bf16Mma64 {
  using A = Bf16Mma<128, 64>;
  using G = Geo<128>;
  static constexpr int kRB = 4, kTn = 4, kSubsteps = A::kSubsteps, kMfma = 16, kReads = 8;
  static constexpr int kARows = A::kARows;  // 128
  static constexpr bool kBKN = false;
  static constexpr int kBTileBytes = 128 * 128;
  static constexpr int kLateSlots = kMfma;
  using Acc = Acc16T<4, 4>;
  struct Frags {
    bf16x8_t a[4], b[4];
  };
  struct Lanes {
    uint32_t a[kSubsteps][4], b[kSubsteps][4];
  };
  static FE2O3_DEVICE Lanes lanes(uint32_t b_region) {
    const typename A::Lanes la = A::lanes(b_region);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wn = wave & 1u, lr = lane & 15u, g = lane >> 4;
    Lanes l;
#pragma unroll
    for (int s = 0; s < kSubsteps; ++s)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t c = 4u * s + g, rb = wn * 64u + p * 16u + lr;
        l.a[s][p] = la.a[s][p];
        l.b[s][p] = b_region + (wn * 64u + lr) * 128u + ((c ^ G::swz(rb)) << 4);
      }
    return l;
  }
  template <uint32_t A_TILE, uint32_t B_TILE, int S, int R>
  static FE2O3_DEVICE void read(const uint8_t* smem, const Lanes& l, Frags& f) {
    static_assert(R >= 0 && R < kReads, "read unit");
    if constexpr (R == 0) {
      f.a[0] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][0] + A_TILE);
    } else if constexpr (R <= 4) {
      constexpr int j = R - 1;
      f.b[j] = *reinterpret_cast<const bf16x8_t*>(smem + l.b[S][j & 3] +
                                                  (B_TILE + j * 16u * 128u));
    } else {
      constexpr int i = R - 4;
      f.a[i] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][i & 3] +
                                                  (A_TILE + i * 16u * 128u));
    }
  }
  template <bool FIRST, int I>
  static FE2O3_DEVICE void mfma(Acc& acc, const Frags& f) {
    constexpr int i = I / kTn, j = I % kTn;
    if constexpr (FIRST)
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                   : "=a"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
    else
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                   : "+a"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
  }
  static FE2O3_DEVICE void finish(Acc& acc) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc.v[i][j]));
  }
};

// bf16 with B stored [k][n], 128 x 128 tiles: for GEMMs whose 256 x 256
// tiles would leave most CUs idle (a quarter of the output per tile, four
// times the tiles).  Each wave owns 64 rows by 64 columns (4 x 4 MFMA
// tiles, accumulators in 64 AGPRs); the A tile holds 128 rows (the A side
// of Bf16Mma<128, 64>), the B tile 64 k-rows of 128 columns (kn_rows128).
// B fragments are read as in Bf16MmaKN, from 256-byte rows (the second read
// of a fragment 4 k-rows, 1024 bytes, on).
struct Bf16MmaKN64 {
  using A = Bf16Mma<128, 64>;
  static constexpr int kRB = 4, kTn = 4, kSubsteps = A::kSubsteps, kMfma = 16, kReads = 8;
  static constexpr int kARows = A::kARows;  // 128
  static constexpr bool kBKN = true;
  static constexpr int kBTileBytes = 64 * 256;
  static constexpr int kLateSlots = kMfma;
  using Acc = Acc16T<4, 4>;
  struct Frags {
    bf16x8_t a[4], b[4];
  };
  struct Lanes {
    uint32_t a[kSubsteps][4], b[kSubsteps][4];
  };
  static FE2O3_DEVICE Lanes lanes(uint32_t b_region) {
    const typename A::Lanes la = A::lanes(b_region);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wn = wave & 1u, g = lane >> 4, i = lane & 15u;
    Lanes l;
#pragma unroll
    for (int s = 0; s < kSubsteps; ++s) {
#pragma unroll
      for (int p = 0; p < 4; ++p) l.a[s][p] = la.a[s][p];
      const uint32_t krow = 32u * s + 8u * g + (i >> 2);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t chunk = wn * 8u + 2u * j + ((i & 3u) >> 1);
        l.b[s][j] = b_region + krow * 256u + ((chunk ^ kn_swz16(krow)) << 4) + (i & 1u) * 8u;
      }
    }
    return l;
  }
  // read unit R of substep S: a0, b0 .. b3, a1 .. a3 (the order and the
  // inline-asm transposing reads of Bf16MmaKN, for the same reason)
  template <uint32_t A_TILE, uint32_t B_TILE, int S, int R>
  static FE2O3_DEVICE void read(const uint8_t* smem, const Lanes& l, Frags& f) {
    static_assert(R >= 0 && R < kReads, "read unit");
    if constexpr (R == 0) {
      f.a[0] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][0] + A_TILE);
    } else if constexpr (R <= 4) {
      constexpr int j = R - 1;
      const lds_bf16x4_t* p = (const lds_bf16x4_t*)(smem + l.b[S][j]);
      bf16x4_t lo, hi;
      // early-clobber outputs, as in Bf16MmaKN::read
      asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\tds_read_b64_tr_b16 %1, %2 offset:%4"
                   : "=&v"(lo), "=&v"(hi)
                   : "v"(p), "i"(B_TILE), "i"(B_TILE + 1024u));
      f.b[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      constexpr int ii = R - 4;
      f.a[ii] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][ii & 3] +
                                                   (A_TILE + ii * 16u * 128u));
    }
  }
  template <bool FIRST, int I>
  static FE2O3_DEVICE void mfma(Acc& acc, const Frags& f) {
    constexpr int i = I / kTn, j = I % kTn;
    if constexpr (FIRST)
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                   : "=a"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
    else
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                   : "+a"(acc.v[i][j]) : "v"(f.b[j]), "v"(f.a[i]));
  }
  static FE2O3_DEVICE void finish(Acc& acc) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc.v[i][j]));
  }
};

// A fragment of an fp8 operand: 32 bytes of one row, two ds_read_b128 at
// the lane's two chunk offsets plus an immediate.
FE2O3_DEVICE i32x8_t fp8_frag(const uint8_t* smem, const uint32_t (&lo_hi)[2], uint32_t imm) {
  const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(smem + lo_hi[0] + imm);
  const i32x4_t hi = *reinterpret_cast<const i32x4_t*>(smem + lo_hi[1] + imm);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// OCP fp8 e4m3: v_mfma_f32_16x16x128_f8f6f4 with both formats e4m3 (cbsz =
// blgp = 0).  It is the scaled builtin with both scale operands 0, which the
// compiler lowers to the unscaled instruction (no v_mfma_ld_scale prefix, no
// scale register; tests/test_isa_fp8_mfma.py checks the selection).  Each
// wave owns RB x CB tiles of 16 x 16 in the bf16 tile's layout (Acc16T): 8 x
// 8 for 256 x 256 workgroup tiles, 4 x 4 for the 128 x 128 form.  Lane l
// holds k 32(l/16) .. +31 (chunks 2(l/16) and the next) of row 16i + l%16.
//
// One MFMA consumes a whole 128-k stage, so the two substeps of a stage
// split the rows instead of k: substep s runs row blocks [s H, (s+1) H),
// H = RB/2, with the column block outer (MFMA I: j = I / H).  Fragments live
// in two buffers: X (f[FC] of substep 0) holds a0 .. a(H-1) and every b_j for
// the whole stage, Y holds a(H) .. a(RB-1).  Each read overwrites a register
// after the last MFMA that needs its old value:
//   substep 0: b(CB-1) of this stage into X at slot 0 (first needed at slot
//     (CB-1) H); a(H) .. a(RB-1) into Y over [M/8, 7M/8);
//   substep 1, from the barrier (slot M/4, or 0 for 4 x 4): the next
//     stage's b0 and a0 .. a(H-1) into X, then b1 .. b(CB-2), each at or
//     after slot (j+1) H, past this substep's last MFMA of column block j.
// Against 4 x 4 tiles of v_mfma_f32_32x32x64_f8f6f4 with the same copy
// plan: +2.2% at 8192^3, +1.1% at 12288 x 4608 x 8192; with the barrier
// and late copies below, +5-6% at 8192^3.
template <int ROW_BYTES, int RB = 8, int CB = 8>
struct Fp8Mma16 {
  static_assert(ROW_BYTES == 128, "one 16x16x128 MFMA per 128-byte row");
  static_assert(RB % 2 == 0 && CB >= 2, "two row halves, two column blocks");
  using G = Geo<ROW_BYTES>;
  using Acc = Acc16T<RB, CB>;
  static constexpr bool kRowSplit = true;
  static constexpr int kH = RB / 2;
  static constexpr int kSubsteps = 2, kMfma = kH * CB, kTn = CB;
  static constexpr int kARows = 32 * RB;
  static constexpr bool kBKN = false;
  static constexpr int kBTileBytes = 32 * CB * ROW_BYTES;
  // 256 x 256 tiles: the barrier a quarter of the way through substep 1 and
  // the late copies over the first half of substep 0 (8192^3: +2.7-3.3% over
  // halfway and 3/4; an eighth: -1.8%; 3/8: +-0).  128 x 128 tiles: the
  // barrier at the start of substep 1 and the late copies over all of
  // substep 0, since their eight-MFMA substeps leave half a substep too short
  // for the next stage's reads (2048^3: 0.94 -> 0.99 of the 32x32x64 form,
  // 2048^2 x 8192: 1.00 -> 1.04)
  static constexpr int kLateSlots = RB == 8 ? kMfma / 2 : kMfma;
  static constexpr int kBarrier = RB == 8 ? kMfma / 4 : 0;
  struct Frags {
    i32x8_t a[RB], b[CB];
  };
  struct Lanes {
    uint32_t a[2][2], b[2][2];  // [row block parity][chunk]
  };
  static FE2O3_DEVICE Lanes lanes(uint32_t b_region) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t lr = lane & 15u, g = lane >> 4;
    Lanes l;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t c = 2u * g + h;
        const uint32_t ra = wm * 16u * RB + p * 16u + lr, rb = wn * 16u * CB + p * 16u + lr;
        l.a[p][h] = (wm * 16u * RB + lr) * ROW_BYTES + ((c ^ G::swz(ra)) << 4);
        l.b[p][h] = b_region + (wn * 16u * CB + lr) * ROW_BYTES + ((c ^ G::swz(rb)) << 4);
      }
    return l;
  }
  static constexpr uint32_t kRow = 16u * ROW_BYTES;  // one row block
  template <uint32_t A_TILE, int I>
  static FE2O3_DEVICE void read_a(const uint8_t* smem, const Lanes& l, Frags& f) {
    f.a[I] = fp8_frag(smem, l.a[I & 1], A_TILE + I * kRow);
  }
  template <uint32_t B_TILE, int J>
  static FE2O3_DEVICE void read_b(const uint8_t* smem, const Lanes& l, Frags& f) {
    f.b[J] = fp8_frag(smem, l.b[J & 1], B_TILE + J * kRow);
  }
  // substep 0's reads of a(H + u) and their slots
  static constexpr int own_slot(int u) { return kMfma / 8 + u * (kMfma - kMfma / 4) / kH; }
  // substep 1's reads of the next stage: unit 0 is b0, units 1 .. H are
  // a0 .. a(H-1), unit H + j is b_j (j = 1 .. CB-2), spread from the barrier
  // on, none before its register's last use
  static constexpr int kNext = 1 + kH + (CB - 2);
  static constexpr int next_slot(int u) {
    const int base = kBarrier + u * (kMfma - kBarrier) / kNext;
    const int least = u == 0 ? kH : u <= kH ? 0 : (u - kH + 1) * kH;
    return base > least ? base : least;
  }
  static_assert(next_slot(kNext - 1) < kMfma, "every read of the next stage in substep 1");
  template <uint32_t A_TILE, uint32_t B_TILE, int U>
  static FE2O3_DEVICE void next_unit(const uint8_t* smem, const Lanes& l, Frags& f) {
    if constexpr (U == 0) read_b<B_TILE, 0>(smem, l, f);
    else if constexpr (U <= kH) read_a<A_TILE, U - 1>(smem, l, f);
    else read_b<B_TILE, U - kH>(smem, l, f);
  }
  template <uint32_t A_TILE, uint32_t B_TILE, int I, int U = 0>
  static FE2O3_DEVICE void next_reads(const uint8_t* smem, const Lanes& l, Frags& f) {
    if constexpr (U < kNext) {
      if constexpr (I < 0 || next_slot(U) == I) next_unit<A_TILE, B_TILE, U>(smem, l, f);
      next_reads<A_TILE, B_TILE, I, U + 1>(smem, l, f);
    }
  }
  template <uint32_t A_TILE, int I, int U = 0>
  static FE2O3_DEVICE void own_reads(const uint8_t* smem, const Lanes& l, Frags& f) {
    if constexpr (U < kH) {
      if constexpr (own_slot(U) == I) read_a<A_TILE, kH + U>(smem, l, f);
      own_reads<A_TILE, I, U + 1>(smem, l, f);
    }
  }
  // what substep 1 of a step -1 would read, from stage 0 into X
  template <uint32_t A_TILE, uint32_t B_TILE>
  static FE2O3_DEVICE void prologue_reads(const uint8_t* smem, const Lanes& l, Frags& x) {
    next_reads<A_TILE, B_TILE, -1>(smem, l, x);
  }
  // the reads at slot I of substep S (fc: this substep's buffer, fn: the other)
  template <uint32_t A_CUR, uint32_t B_CUR, uint32_t A_NXT, uint32_t B_NXT, int S, int I>
  static FE2O3_DEVICE void reads_at(const uint8_t* smem, const Lanes& l, Frags& fc, Frags& fn) {
    if constexpr (S == 0) {
      if constexpr (I == 0) read_b<B_CUR, CB - 1>(smem, l, fc);
      own_reads<A_CUR, I>(smem, l, fn);
    } else {
      next_reads<A_NXT, B_NXT, I>(smem, l, fn);
    }
  }
  // MFMA I of substep S: substep 0 takes A and B from X (fc); substep 1 its
  // A from Y (fc) and B from X (fn)
  template <bool FIRST, int S, int I>
  static FE2O3_DEVICE void mfma2(Acc& acc, const Frags& fc, const Frags& fn) {
    constexpr int j = I / kH, i = S * kH + I % kH;
    const f32x4_t c = FIRST ? f32x4_t{} : acc.v[i][j];
    const i32x8_t& bj = S == 0 ? fc.b[j] : fn.b[j];
    acc.v[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bj, fc.a[i], c, 0, 0, 0,
                                                                   0, 0, 0);
  }
  static FE2O3_DEVICE void finish(Acc&) {}
};

// ---- the pipeline ----------------------------------------------------------------------------
//
// Two stages (ROW_BYTES 128: 64 bf16 or 128 fp8 of k) in two LDS buffers; a K step is one
// stage, kSubsteps substeps of kMfma MFMAs each.  Every other instruction of
// the step has a fixed slot between two MFMAs (item n of N spread over slots
// [s0, s1) sits after MFMA s0 + n (s1 - s0) / N), the order pinned by
// sched_barrier(0) after every slot.  With M = kMfma, for step t in buffer P:
//   every substep but the last: the next substep's fragment reads over
//     [M/8, 7M/8);
//   substep 0: the second half of stage t+1's copies (the A tile's) into
//     the other buffer over [0, L), L = the policy's kLateSlots;
//   last substep: MFMAs up to M/2; wait for stage t+1's copies and cross the
//     barrier; then stage t+1's first fragment reads over [M/2, M), and the
//     first half of stage t+2's copies (the B tile's) into buffer P over
//     [M/2, M).
// Buffer P is free from that barrier on: every wave's reads of it were issued
// before it and completed (lgkmcnt(0)) at it.  Starting the next copies there
// rather than in the next substep 0 gives them up to two substeps to land,
// which is what operands streamed from HBM need.  The barrier sits halfway
// through the last substep, whose fragments are already in registers, so the
// waves meet with half a substep of MFMAs still to issue.  A policy may move
// it (kBarrier) and place its own fragment reads (Fp8Mma16, whose substeps
// split rows rather than k).

// item n of N over slots [S0, S1): call fn(n) for the items at slot I
template <int N, int S0, int S1, int n = 0>
struct Spread {
  template <int I, class Fn>
  static FE2O3_DEVICE void at(Fn&& fn) {
    if constexpr (n < N) {
      if constexpr (S0 + n * (S1 - S0) / N == I) fn(std::integral_constant<int, n>{});
      Spread<N, S0, S1, n + 1>::template at<I>(fn);
    }
  }
};

// Order of a stage's NA A copies and NB B copies: the B copies first (copy
// c < NB is B slot c), then the A copies, so the early half of a stage (the
// copies started at the barrier, with the longer time to land) is the B
// tile.  In the MoE expert GEMMs B is the expert's weights, streamed from
// HBM, while the token rows of A are re-read by every weight panel from the
// caches: +5.5% on the config-5 layer over alternating A and B, dense bf16
// and fp8 GEMMs within +-0.5%.
template <int NA, int NB>
struct CopyOrder {
  static_assert(NA >= 1 && NB >= 1, "copies of both operands");
  static constexpr int NC = NA + NB;
  static constexpr bool is_a(int c) { return c >= NB; }
  static constexpr int slot(int c) {
    int n = 0;
    for (int x = 0; x < c; ++x)
      if (is_a(x) == is_a(c)) ++n;
    return n;
  }
};

// Copy C of the stage at k offset `kbytes` into LDS buffer `buf`.
template <int ROW_BYTES, int STAGES, int A_ROWS, int C, class RA, class RB>
FE2O3_DEVICE void copy_one(const RA& ar, const RB& br, uint32_t kbytes, uint8_t* smem,
                           uint32_t wave, int buf) {
  constexpr int NA = sizeof(ar.voff) / sizeof(uint32_t), NB = sizeof(br.voff) / sizeof(uint32_t);
  using L = Lay<ROW_BYTES, STAGES, A_ROWS, NB * 4096>;  // NB 1-KiB loads per wave
  using O = CopyOrder<NA, NB>;
  constexpr int j = O::slot(C);
  if constexpr (O::is_a(C))
    b2l_b128(rsrc(ar.base[j], ar.bytes), smem + L::a(buf) + (4u * j + wave) * 1024u,
             ar.off(j, kbytes), kbytes);
  else
    b2l_b128(rsrc(br.base[j], br.bytes), smem + L::b_region + L::b(buf) + (4u * j + wave) * 1024u,
             br.off(j, kbytes), br.soff(kbytes));
}

// Policies whose substeps split the tile's rows instead of k (Fp8Mma16)
// place their own fragment reads and see both fragment buffers.
template <class M, class = void>
struct RowSplit : std::false_type {};
template <class M>
struct RowSplit<M, std::void_t<decltype(M::kRowSplit)>> : std::bool_constant<M::kRowSplit> {};

// The barrier's slot in the last substep: the policy's kBarrier, else M/2.
template <class M, class = void>
struct BarrierAt {
  static constexpr int value = M::kMfma / 2;
};
template <class M>
struct BarrierAt<M, std::void_t<decltype(M::kBarrier)>> {
  static constexpr int value = M::kBarrier;
};

// Substep S_ of a K step held in stage buffer P.  FIRST: the K loop's first
// substep (accumulators written, not added to).  k_next / k_next2: k byte
// offsets of the stages one and two ahead (clamped to the last stage).
// MASK: the operands' rows end inside the last stage (Rows::off).
template <class M, int ROW_BYTES, int STAGES, int P, int S_, bool FIRST, bool MASK = false>
struct Substep {
  using G = Geo<ROW_BYTES>;
  using L = Lay<ROW_BYTES, STAGES, M::kARows, M::kBTileBytes>;
  static constexpr int S = M::kSubsteps, MF = M::kMfma;
  static constexpr int NA = G::insts(M::kARows), NB = M::kBTileBytes / 4096;
  using RA_ = Rows<ROW_BYTES, NA, false, MASK>;
  using RB_ = Rows<ROW_BYTES, NB, M::kBKN, MASK>;
  static constexpr int NC = NA + NB;              // copies per stage and wave
  static constexpr int kEarly = NC / 2;           // copies started at the barrier
  static constexpr int PN = (P + 1) % STAGES;     // buffer of the next step
  static constexpr int PL = (P + STAGES - 1) % STAGES;  // buffer of the late copies' stage
  static constexpr bool LAST = S_ + 1 == S;
  static constexpr int kBarrierAt = BarrierAt<M>::value;
  // late copies: all of substep 0, or its first half when it is also the
  // last substep (every late copy precedes the barrier, every early one
  // follows it, which keeps the wait counts exact)
  static constexpr int kLateTo = LAST ? kBarrierAt : M::kLateSlots;
  // fragment buffers alternate by substep over the whole K loop
  static constexpr int FC = (P * S + S_) & 1, FN = FC ^ 1;
  static constexpr int kReadFrom = LAST ? MF / 2 : MF / 8;
  static constexpr int kReadTo = LAST ? MF : MF - MF / 8;
  // fragments read here: the next substep's, or in the last substep the next stage's first
  static constexpr uint32_t RA = LAST ? L::a(PN) : L::a(P);
  static constexpr uint32_t RB = LAST ? L::b(PN) : L::b(P);
  static constexpr int RS = LAST ? 0 : S_ + 1;

  template <int I>
  static FE2O3_DEVICE void slot(const RA_& ar, const RB_& br,
                                uint32_t k_next, uint32_t k_next2, uint8_t* smem, uint32_t wave,
                                const typename M::Lanes& ln, typename M::Frags* f,
                                typename M::Acc& acc) {
    if constexpr (I < MF) {
      if constexpr (LAST && I == kBarrierAt) {
        // stage t+1 landed: later stages' copies may still be in flight
        __builtin_amdgcn_s_waitcnt(waitcnt_imm((STAGES - 2) * NC, 0));
        __builtin_amdgcn_s_barrier();
      }
      if constexpr (RowSplit<M>::value)
        M::template mfma2<FIRST, S_, I>(acc, f[FC], f[FN]);
      else
        M::template mfma<FIRST && S_ == 0, I>(acc, f[FC]);
      if constexpr (LAST)  // early copies: stage t+STAGES into buffer P
        Spread<kEarly, kBarrierAt, MF>::template at<I>([&](auto n) {
          copy_one<ROW_BYTES, STAGES, M::kARows, decltype(n)::value>(ar, br, k_next2, smem, wave,
                                                                     P);
        });
      if constexpr (S_ == 0)  // late copies: the rest of stage t+STAGES-1
        Spread<NC - kEarly, 0, kLateTo>::template at<I>([&](auto n) {
          copy_one<ROW_BYTES, STAGES, M::kARows, kEarly + decltype(n)::value>(ar, br, k_next,
                                                                              smem, wave, PL);
        });
      if constexpr (RowSplit<M>::value)
        M::template reads_at<L::a(P), L::b(P), L::a(PN), L::b(PN), S_, I>(smem, ln, f[FC], f[FN]);
      else
        Spread<M::kReads, kReadFrom, kReadTo>::template at<I>([&](auto n) {
          M::template read<RA, RB, RS, decltype(n)::value>(smem, ln, f[FN]);
        });
      __builtin_amdgcn_sched_barrier(0);
      slot<I + 1>(ar, br, k_next, k_next2, smem, wave, ln, f, acc);
    }
  }
  static FE2O3_DEVICE void run(const RA_& ar, const RB_& br,
                               uint32_t k_next, uint32_t k_next2, uint8_t* smem, uint32_t wave,
                               const typename M::Lanes& ln, typename M::Frags* f,
                               typename M::Acc& acc) {
    __builtin_amdgcn_sched_barrier(0);
    slot<0>(ar, br, k_next, k_next2, smem, wave, ln, f, acc);
    if constexpr (!LAST)
      Substep<M, ROW_BYTES, STAGES, P, S_ + 1, FIRST, MASK>::run(ar, br, k_next, k_next2, smem,
                                                                 wave, ln, f, acc);
  }
};

// Steps kt .. kt+STAGES-1 in buffers P .. STAGES-1 (TAIL: stop at the last
// step; FIRST: kt is the K loop's first step).
template <class M, int ROW_BYTES, int STAGES, int P, bool TAIL, bool FIRST, bool MASK = false>
struct Steps {
  static FE2O3_DEVICE uint32_t stage_k(int st, int steps) {
    using G = Geo<ROW_BYTES>;
    return __builtin_amdgcn_readfirstlane((uint32_t)(st < steps ? st : steps - 1) *
                                          (G::kK16 * 2u));
  }
  using Sub0 = Substep<M, ROW_BYTES, STAGES, 0, 0, false, MASK>;
  static FE2O3_DEVICE void run(const typename Sub0::RA_& ar, const typename Sub0::RB_& br, int kt,
                               int steps, uint8_t* smem, uint32_t wave,
                               const typename M::Lanes& ln, typename M::Frags* f,
                               typename M::Acc& acc) {
    if (TAIL && kt >= steps) return;
    Substep<M, ROW_BYTES, STAGES, P, 0, FIRST && P == 0, MASK>::run(
        ar, br, stage_k(kt + STAGES - 1, steps), stage_k(kt + STAGES, steps), smem, wave, ln, f,
        acc);
    if constexpr (P + 1 < STAGES)
      Steps<M, ROW_BYTES, STAGES, P + 1, TAIL, FIRST, MASK>::run(ar, br, kt + 1, steps, smem,
                                                                 wave, ln, f, acc);
  }
};

// K loop over k16 16-bit units per row (at least one); every accumulator is
// written (no zeroing beforehand).  k16 is a multiple of Geo::kK16, or, with
// MASK, of 8: the last stage is then partial and its chunks past k16 load
// zeros.
template <class M, int ROW_BYTES, int STAGES, bool MASK = false>
FE2O3_DEVICE void mainloop(
    const typename Substep<M, ROW_BYTES, STAGES, 0, 0, false, MASK>::RA_& ar,
    const typename Substep<M, ROW_BYTES, STAGES, 0, 0, false, MASK>::RB_& br, uint32_t k16,
    uint8_t* smem, typename M::Acc& acc) {
  using G = Geo<ROW_BYTES>;
  using L = Lay<ROW_BYTES, STAGES, M::kARows, M::kBTileBytes>;
  using Sub = Substep<M, ROW_BYTES, STAGES, 0, 0, false, MASK>;
  static_assert((ROW_BYTES == 128 && (STAGES == 2 || STAGES == 3)) ||
                    (ROW_BYTES == 64 && STAGES == 4),
                "two or three 64-k stages, or four 32-k stages");
  static_assert(M::kSubsteps % 2 == 0 || STAGES % 2 == 0,
                "fragment buffers alternate across the unrolled steps");
  constexpr int NA = Sub::NA, NB = Sub::NB;
  const int steps = (int)(MASK ? (k16 + G::kK16 - 1u) / G::kK16 : k16 / G::kK16);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const typename M::Lanes ln = M::lanes(L::b_region);
  // stages 0 .. STAGES-2 whole, and stage STAGES-1's early copies (those a
  // step -1 would issue)
  using St = Steps<M, ROW_BYTES, STAGES, 0, false, false, MASK>;
#pragma unroll
  for (int st = 0; st + 1 < STAGES; ++st) {
    const uint32_t kb = st == 0 ? 0u : St::stage_k(st, steps);
    issue_part<ROW_BYTES, 0, NA>(ar, kb, smem, L::a(st), wave);
    issue_part<ROW_BYTES, 0, NB>(br, kb, smem, L::b_region + L::b(st), wave);
  }
  const uint32_t kl = St::stage_k(STAGES - 1, steps);
  Spread<Sub::kEarly, 0, 1>::template at<0>([&](auto n) {
    copy_one<ROW_BYTES, STAGES, M::kARows, decltype(n)::value>(ar, br, kl, smem, wave,
                                                               STAGES - 1);
  });
  // stage 0 landed
  __builtin_amdgcn_s_waitcnt(waitcnt_imm((STAGES - 2) * Sub::NC + Sub::kEarly, 0));
  __builtin_amdgcn_s_barrier();
  typename M::Frags f[2];
  if constexpr (RowSplit<M>::value)
    M::template prologue_reads<L::a(0), L::b(0)>(smem, ln, f[0]);
  else
    Spread<M::kReads, 0, 1>::template at<0>([&](auto n) {
      M::template read<L::a(0), L::b(0), 0, decltype(n)::value>(smem, ln, f[0]);
    });
  // every first fragment landed.  The wait is inline asm between scheduling
  // barriers: a policy's inline-asm reads are invisible to the compiler's
  // wait tracking, which may otherwise move reads past a builtin wait or
  // drop the wait as redundant (seen with three 128 x 128 stages).
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // the first group bounded (it may hold every step), then whole groups,
  // then the rest; one code path whatever the step count
  Steps<M, ROW_BYTES, STAGES, 0, true, true, MASK>::run(ar, br, 0, steps, smem, wave, ln, f, acc);
  int kt = STAGES;
  for (; kt + STAGES <= steps; kt += STAGES)
    Steps<M, ROW_BYTES, STAGES, 0, false, false, MASK>::run(ar, br, kt, steps, smem, wave, ln, f,
                                                            acc);
  if (kt < steps)  // fewer than STAGES steps left; they start in buffer 0
    Steps<M, ROW_BYTES, STAGES, 0, true, false, MASK>::run(ar, br, kt, steps, smem, wave, ln, f,
                                                           acc);
  __builtin_amdgcn_sched_barrier(0);
  // The last steps' early copies (of clamped stages nobody reads) land
  // before the workgroup can end and its LDS be handed to another, and the
  // last substep's reads of a next stage that does not exist land before
  // the epilogue may reuse their registers (a policy's inline-asm reads are
  // invisible to the compiler's own wait tracking).
  __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
  M::finish(acc);
  __builtin_amdgcn_sched_barrier(0);
}

// ---- epilogue coordinates --------------------------------------------------------------------
// The lane and wave come from mbcnt and a scalar, so nothing derived from
// threadIdx stays live across the K loop.
FE2O3_DEVICE uint32_t lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}
FE2O3_DEVICE uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Acc16T (i, j, e): tile row wm*RPW + 16i + lane%16, tile column
// wn*CPW + 16j + 4(lane/16) + e (CPW = 128, or 64 for Bf16MmaKN64).
// (`w`: the wave index, when the caller read it before the K loop, so that
// the thread id need not stay live across the loop)
template <int RPW = 128>
FE2O3_DEVICE uint32_t acc16_row0(uint32_t w = wave_id()) {
  return (w >> 1) * RPW + (lane_id() & 15u);
}
template <int CPW = 128>  // columns per wave
FE2O3_DEVICE uint32_t acc16_col0(uint32_t w = wave_id()) {
  return (w & 1u) * CPW + 4u * (lane_id() >> 4);
}

// Acc16 (i, j, e) holds column 16j + 4g + e of the wave's block, g = lane /
// 16 (the lane's 16-lane row of the wave).  For a pair of column blocks
// (j, j + 1), v_permlane16_swap exchanges rows 1 and 3 of block j's packed
// values with rows 0 and 2 of block j + 1's: afterwards lanes of row g hold
// columns 8 (g / 2) .. + 7 of block j + g % 2, 16 bytes per lane, and each
// store writes 64 contiguous bytes of 16 rows (half the stores of writing
// the 8-byte pieces in place).
// row0, col0: this lane's first row and column (columns of a pair start
// 32 apart).
template <int RB, int CB>
FE2O3_DEVICE void store_bf16_pairs(const Acc16T<RB, CB>& acc, uint16_t* c_tile, uint64_t ldc,
                                   uint32_t row0, uint32_t col0) {
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int jp = 0; jp < CB / 2; ++jp) {
      const int ja = 2 * jp, jb = 2 * jp + 1;
      const uint32_t y0 = pack_bf16x2(acc.v[i][ja][0], acc.v[i][ja][1]);
      const uint32_t y1 = pack_bf16x2(acc.v[i][ja][2], acc.v[i][ja][3]);
      const uint32_t x0 = pack_bf16x2(acc.v[i][jb][0], acc.v[i][jb][1]);
      const uint32_t x1 = pack_bf16x2(acc.v[i][jb][2], acc.v[i][jb][3]);
      const auto s0 = __builtin_amdgcn_permlane16_swap(y0, x0, false, false);
      const auto s1 = __builtin_amdgcn_permlane16_swap(y1, x1, false, false);
      u32x4_t packed;
      packed[0] = s0[0];
      packed[1] = s1[0];
      packed[2] = s0[1];
      packed[3] = s1[1];
      *reinterpret_cast<u32x4_t*>(c_tile + (uint64_t)(row0 + 16u * i) * ldc + col0 + 32u * jp) =
          packed;
    }
}

FE2O3_DEVICE void store_bf16(const Acc16& acc, uint16_t* c_tile, uint64_t ldc,
                            uint32_t w = wave_id()) {
  const uint32_t g = lane_id() >> 4;
  const uint32_t col0 = (w & 1u) * 128u + 16u * (g & 1u) + 8u * (g >> 1);
  store_bf16_pairs(acc, c_tile, ldc, acc16_row0(w), col0);
}

// Edge tiles (the last tile row or column of a C whose M or N is not a
// multiple of 256): only tile rows < rows_valid and columns < cols_valid are
// written, one 2-byte store per element, so C rows need no alignment.  The
// values are those store_bf16 writes.
FE2O3_DEVICE void store_bf16_edge(const Acc16& acc, uint16_t* c_tile, uint64_t ldc,
                                  uint32_t rows_valid, uint32_t cols_valid,
                                  uint32_t w = wave_id()) {
  const uint32_t row0 = acc16_row0(w), col0 = acc16_col0(w);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t r = row0 + 16u * i;
    if (r >= rows_valid) continue;
    uint16_t* out = c_tile + (uint64_t)r * ldc;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t c = col0 + 16u * j + e;
        if (c < cols_valid) out[c] = bf16_bits_from_f32(acc.v[i][j][e]);
      }
  }
}

// A 128 x 128 tile of Acc16T<4, 4> (waves of 64 x 64): whole tiles of a
// 16-byte aligned C (WHOLE) with store_bf16's pair exchange, 16 bytes per
// lane; otherwise only rows < rows_valid and columns < cols_valid, one
// 2-byte store per element.
template <bool WHOLE>
FE2O3_DEVICE void store_bf16_128(const Acc16T<4, 4>& acc, uint16_t* c_tile, uint64_t ldc,
                                 uint32_t rows_valid, uint32_t cols_valid) {
  if constexpr (WHOLE) {
    const uint32_t g = lane_id() >> 4;
    const uint32_t col0 = (wave_id() & 1u) * 64u + 16u * (g & 1u) + 8u * (g >> 1);
    store_bf16_pairs(acc, c_tile, ldc, acc16_row0<64>(), col0);
    return;
  }
  const uint32_t row0 = acc16_row0<64>(), col0 = acc16_col0<64>();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t r = row0 + 16u * i;
    if (r >= rows_valid) continue;
    uint16_t* out = c_tile + (uint64_t)r * ldc;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t c = col0 + 16u * j + e;
        if (c < cols_valid) out[c] = bf16_bits_from_f32(acc.v[i][j][e]);
      }
  }
}

// Staged stores. Straight from the accumulators, one store instruction writes
// 32 bytes into each of 16 rows, parts of cache
// lines. Here each wave first writes its 128x128 block as bf16 into its own
// 32 KiB of the idle stage buffers (row-major, 256 bytes a row, the 16-byte
// chunks of row r XOR-permuted by r & 15 so that the 16-byte reads are
// conflict-free), then reads 16 bytes per lane, so that one nontemporal store
// writes four whole 256-byte row segments. The detour costs ~1 us per tile;
// it pays where C would otherwise evict operands from the last-level cache
// (gemm_core::staged_epilogue).
FE2O3_DEVICE void stage_bf16(const Acc16& acc, uint8_t* region) {
  const uint32_t l = lane_id(), s = l & 15u;
  const uint32_t wr = s * 256u + ((l >> 4) & 1u) * 8u;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x2_t packed;
      packed[0] = pack_bf16x2(acc.v[i][j][0], acc.v[i][j][1]);
      packed[1] = pack_bf16x2(acc.v[i][j][2], acc.v[i][j][3]);
      const uint32_t chunk = ((2u * j) | (l >> 5)) ^ s;
      *reinterpret_cast<u32x2_t*>(region + 4096u * i + wr + chunk * 16u) = packed;
    }
}

// `smem` needs 128 KiB, and the caller's copies must all have landed.
FE2O3_DEVICE void store_bf16_staged(const Acc16& acc, uint8_t* smem, uint16_t* c_tile,
                                    uint64_t ldc, uint32_t w = wave_id()) {
  const uint32_t l = lane_id();
  uint8_t* region = smem + w * 32768u;
  __syncthreads();  // every wave is past its last fragment read and copy
  stage_bf16(acc, region);
  __syncthreads();  // the wave's lanes read what other lanes wrote
  const uint32_t rr = l >> 4, cc = l & 15u;
  uint16_t* out = c_tile + (uint64_t)((w >> 1) * 128u + rr) * ldc + (w & 1u) * 128u + 8u * cc;
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    const uint32_t r = 4u * p + rr;
    const u32x4_t v =
        *reinterpret_cast<const u32x4_t*>(region + r * 256u + ((cc ^ (r & 15u)) << 4));
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(out + (uint64_t)(4u * p) * ldc));
  }
}

}  // namespace gemm_pipe
