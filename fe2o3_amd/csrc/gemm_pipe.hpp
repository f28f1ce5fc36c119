// gemm_pipe.hpp -- multi-stage 256x256 MFMA GEMM pipelines for gfx950.
//
// Workgroup: 256 threads = 4 waves in 2x2, each wave a 128x128 block of the
// output, accumulators in AGPRs.  Two instruction forms share the copy
// machinery and LDS layout below:
//   bf16  8x8 tiles of v_mfma_f32_16x16x32_bf16, issued in a fixed order
//         (mainloop_bf16, Acc16);
//   fp8   4x4 tiles of v_mfma_scale_f32_32x32x64_f8f6f4 (mainloop, Acc32).
// Parameters:
//   ROW_BYTES  bytes of k per tile row per stage (128: 64 bf16; 64: 32 bf16)
//   STAGES     LDS stages in flight (STAGES * 2 * 256 * ROW_BYTES bytes)
//
// Global -> LDS.  Operand tiles are copied with buffer_load_dwordx4 ... lds
// (16 bytes per lane straight into LDS).  Each operand has a buffer resource
// per load slot (wave-uniform) and each thread a fixed byte offset per slot;
// the k offset of a stage is a scalar, and the LDS destination (M0) is
// scalar too, so a copy costs no VALU.  Stage kt+STAGES-1 is copied while
// stage kt is consumed.  One s_waitcnt vmcnt + one barrier per stage
// publishes every wave's copies.
//
// LDS layout.  The A tiles of all stages come first, then the B tiles (A of
// stage p at p * T, B at (STAGES + p) * T, T = 256 * ROW_BYTES).  16-byte
// chunk c of row r is stored at position c ^ swz(r):
//   ROW_BYTES 128: swz(r) = (r ^ (r >> 3)) & 7
//   ROW_BYTES  64: swz(r) = ((r >> 1) ^ (r >> 3)) & 3
// Both keep the MFMA operand reads (16 or 32 consecutive rows, one chunk)
// free of bank conflicts (measured: SQ_LDS_BANK_CONFLICT = 0).
//
// Fragment reads.  The K loop is unrolled over the STAGES buffers, so the
// stage, tile and row-block offsets of every ds_read are compile-time
// immediates; the per-lane part depends only on (substep, row block mod the
// swizzle period) and is computed once before the loop.
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

// 32x32 accumulators (fp8 path): tile (i, j) of the wave's 4x4
struct Acc32 {
  f32x16_t v[4][4];
};

FE2O3_DEVICE void zero(Acc32& acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc.v[i][j][e] = 0.0f;
}

// Source of one operand tile: for load slot j the base of its buffer
// (wave-uniform) and this thread's byte offset of its chunk at k = 0; all
// slots share one buffer extent.  Offsets and extent are 32-bit.
template <int ROW_BYTES>
struct Rows {
  const void* base[Geo<ROW_BYTES>::kInstPerWave];
  uint32_t bytes;
  uint32_t voff[Geo<ROW_BYTES>::kInstPerWave];
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
// caller guarantees ((valid_rows - 1) * ld + k16) * 2 < 2^31.
template <int ROW_BYTES>
FE2O3_DEVICE Rows<ROW_BYTES> dense_rows(const uint16_t* base, uint32_t ld, uint32_t valid_rows,
                                        uint32_t k16) {
  using G = Geo<ROW_BYTES>;
  Rows<ROW_BYTES> t;
  t.bytes = ((valid_rows - 1u) * ld + k16) * 2u;
#pragma unroll
  for (int j = 0; j < G::kInstPerWave; ++j) {
    uint32_t row = G::inst_row(j);
    const uint32_t chunk = G::inst_chunk(row);
    if (row >= valid_rows) row = valid_rows - 1u;
    t.base[j] = base;
    t.voff[j] = (row * ld + chunk * 8u) * 2u;
  }
  return t;
}

// OCP fp8 e4m3 operands: substeps of 64 k (64 bytes of each row, chunks
// 4s + 2(l/32) and the next one per lane) issuing
// v_mfma_scale_f32_32x32x64_f8f6f4 with both formats e4m3 (cbsz = blgp = 0)
// and unit E8M0 block scales (127 = 2^0).
template <int ROW_BYTES>
struct MmaFp8 {
  using G = Geo<ROW_BYTES>;
  static constexpr int kSubsteps = ROW_BYTES / 64;
  struct Frags {
    i32x8_t a[4], b[4];
  };
  struct Lanes {
    uint32_t a[kSubsteps][2][2], b[kSubsteps][2][2];  // [substep][row parity][chunk]
  };
  static FE2O3_DEVICE Lanes lanes(uint32_t b_region) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t lr = lane & 31u, g = lane >> 5;
    Lanes l;
#pragma unroll
    for (int s = 0; s < kSubsteps; ++s)
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t c = 4u * s + 2u * g + h;
          const uint32_t ra = wm * 128u + p * 32u + lr, rb = wn * 128u + p * 32u + lr;
          l.a[s][p][h] = (wm * 128u + lr) * ROW_BYTES + ((c ^ G::swz(ra)) << 4);
          l.b[s][p][h] = b_region + (wn * 128u + lr) * ROW_BYTES + ((c ^ G::swz(rb)) << 4);
        }
    return l;
  }
  static FE2O3_DEVICE i32x8_t join(i32x4_t lo, i32x4_t hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  template <uint32_t A_TILE, uint32_t B_TILE, int S>
  static FE2O3_DEVICE void load(const uint8_t* smem, const Lanes& l, Frags& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      constexpr uint32_t kRow = 32u * ROW_BYTES;
      f.a[i] = join(*reinterpret_cast<const i32x4_t*>(smem + l.a[S][i & 1][0] + (A_TILE + i * kRow)),
                    *reinterpret_cast<const i32x4_t*>(smem + l.a[S][i & 1][1] + (A_TILE + i * kRow)));
      f.b[i] = join(*reinterpret_cast<const i32x4_t*>(smem + l.b[S][i & 1][0] + (B_TILE + i * kRow)),
                    *reinterpret_cast<const i32x4_t*>(smem + l.b[S][i & 1][1] + (B_TILE + i * kRow)));
    }
  }
  static FE2O3_DEVICE void mma(const Frags& f, Acc32& acc) {
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

// Loads j in [J0, J1) of one operand tile into the LDS tile at byte offset
// `tile` of smem, k offset `kbytes` (wave-uniform).
template <int ROW_BYTES, int J0, int J1>
FE2O3_DEVICE void issue_part(const Rows<ROW_BYTES>& rows, uint32_t kbytes, uint8_t* smem,
                             uint32_t tile, uint32_t wave) {
#pragma unroll
  for (int j = J0; j < J1; ++j)
    b2l_b128(rsrc(rows.base[j], rows.bytes), smem + tile + (4u * j + wave) * 1024u, rows.voff[j],
             kbytes);
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

// Stage p's A tile at a(p); its B tile at b_region + b(p).  Fragment reads
// add a(p) or b(p) (plus the row-block offset) as ds_read immediates; the
// B region's base is folded into the per-lane B offsets, so every immediate
// stays below 64 KiB.
template <int ROW_BYTES, int STAGES>
struct Lay {
  using G = Geo<ROW_BYTES>;
  static constexpr uint32_t b_region = (uint32_t)STAGES * G::kTileBytes;
  static constexpr uint32_t a(int p) { return (uint32_t)p * G::kTileBytes; }
  static constexpr uint32_t b(int p) { return (uint32_t)p * G::kTileBytes; }
  // largest row-block offset: 16-row block 7 (bf16) > 32-row block 3 (fp8)
  static_assert((STAGES - 1) * G::kTileBytes + 7 * 16 * ROW_BYTES < 65536,
                "fragment read offsets fit the ds_read immediate");
};

// One substep S_ of a K step held in stage buffer P: issue this substep's
// share of the look-ahead stage's copies, read the next substep's fragments
// (or, in the last substep, wait for the next stage and cross the barrier
// first), then the substep's 16 MFMAs.
template <class Mma, int ROW_BYTES, int STAGES, int P, int S_>
struct Substep {
  using G = Geo<ROW_BYTES>;
  using L = Lay<ROW_BYTES, STAGES>;
  static constexpr int S = Mma::kSubsteps;
  static constexpr int NJ = G::kInstPerWave;
  static constexpr int LPS = 2 * NJ;
  static constexpr int PL = (P + STAGES - 1) % STAGES;  // look-ahead stage's buffer
  static constexpr int PN = (P + 1) % STAGES;           // next step's buffer
  // substeps that issue look-ahead copies: with two stages the first half
  // (the copies must land within this step), otherwise all of them
  static constexpr int DS = STAGES == 2 ? (S > 1 ? S / 2 : 1) : S;
  static constexpr int J0 = S_ < DS ? S_ * NJ / DS : NJ;
  static constexpr int J1 = S_ < DS ? (S_ + 1) * NJ / DS : NJ;
  static FE2O3_DEVICE void run(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br,
                               uint32_t kbytes, uint8_t* smem, uint32_t wave,
                               const typename Mma::Lanes& ln, typename Mma::Frags* f, Acc32& acc) {
    issue_part<ROW_BYTES, J0, J1>(ar, kbytes, smem, L::a(PL), wave);
    issue_part<ROW_BYTES, J0, J1>(br, kbytes, smem, L::b_region + L::b(PL), wave);
    if constexpr (S_ + 1 < S) {
      Mma::template load<L::a(P), L::b(P), S_ + 1>(smem, ln, f[(S_ + 1) & 1]);
    } else {
      wait_vmcnt<(STAGES - 2) * LPS>();
      lds_barrier();
      Mma::template load<L::a(PN), L::b(PN), 0>(smem, ln, f[S & 1]);
    }
    Mma::mma(f[S_ & 1], acc);
    interleave<2 * (J1 - J0), sizeof(typename Mma::Frags) / 16>();  // 16-byte LDS reads
    // close the scheduling region: MFMAs of the next substep (whose operands
    // are read above) must not be hoisted into this one
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (S_ + 1 < S)
      Substep<Mma, ROW_BYTES, STAGES, P, S_ + 1>::run(ar, br, kbytes, smem, wave, ln, f, acc);
  }
};

// K steps kt, kt+1, ... held in stage buffers P, P+1, ..., STAGES-1.  The
// main loop runs whole groups (TAIL false: no branch inside the group, which
// keeps the register allocation spill-free); the tail (TAIL true) stops at
// the last step.
template <class Mma, int ROW_BYTES, int STAGES, int P, bool TAIL>
struct Steps {
  static FE2O3_DEVICE void run(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br, int kt,
                               int steps, uint8_t* smem, uint32_t wave,
                               const typename Mma::Lanes& ln, typename Mma::Frags* f, Acc32& acc) {
    using G = Geo<ROW_BYTES>;
    if (TAIL && kt >= steps) return;
    // look-ahead stage, clamped to the last one for its source (its copies
    // then land in a buffer nobody reads again)
    const int la = kt + STAGES - 1;
    const uint32_t kbytes =
        __builtin_amdgcn_readfirstlane((uint32_t)(la < steps ? la : steps - 1) * (G::kK16 * 2u));
    Substep<Mma, ROW_BYTES, STAGES, P, 0>::run(ar, br, kbytes, smem, wave, ln, f, acc);
    if constexpr (P + 1 < STAGES)
      Steps<Mma, ROW_BYTES, STAGES, P + 1, TAIL>::run(ar, br, kt + 1, steps, smem, wave, ln, f,
                                                      acc);
  }
};

// K loop over k16 16-bit units per row (a multiple of Geo::kK16, at least
// one stage).  Every step issues the same number of copies (a constant
// vmcnt).
template <class Mma, int ROW_BYTES, int STAGES>
FE2O3_DEVICE void mainloop(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br, uint32_t k16,
                           uint8_t* smem, Acc32& acc) {
  using G = Geo<ROW_BYTES>;
  using L = Lay<ROW_BYTES, STAGES>;
  constexpr int NJ = G::kInstPerWave;
  constexpr int LPS = 2 * NJ;
  static_assert(STAGES >= 2 && (STAGES - 2) * LPS <= 63, "stages");
  static_assert(STAGES == 2 || NJ % Mma::kSubsteps == 0, "even split of the loads");
  static_assert(Mma::kSubsteps % 2 == 0, "fragment buffers alternate within a stage");
  const int steps = (int)(k16 / G::kK16);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const typename Mma::Lanes ln = Mma::lanes(L::b_region);
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st) {
    const uint32_t kb =
        __builtin_amdgcn_readfirstlane((uint32_t)(st < steps ? st : steps - 1) * (G::kK16 * 2u));
    issue_part<ROW_BYTES, 0, NJ>(ar, kb, smem, L::a(st), wave);
    issue_part<ROW_BYTES, 0, NJ>(br, kb, smem, L::b_region + L::b(st), wave);
  }
  wait_vmcnt<(STAGES - 2) * LPS>();
  lds_barrier();
  typename Mma::Frags f[2];
  Mma::template load<L::a(0), L::b(0), 0>(smem, ln, f[0]);
  int kt = 0;
  for (; kt + STAGES <= steps; kt += STAGES)
    Steps<Mma, ROW_BYTES, STAGES, 0, false>::run(ar, br, kt, steps, smem, wave, ln, f, acc);
  if (kt < steps)  // fewer than STAGES steps left; they start in buffer 0
    Steps<Mma, ROW_BYTES, STAGES, 0, true>::run(ar, br, kt, steps, smem, wave, ln, f, acc);
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

FE2O3_DEVICE void store_bf16(const Acc32& acc, uint16_t* c_tile, uint64_t ldc,
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

// ---- bf16: 16x16x32 MFMAs in a fixed issue order ----------------------------------------
//
// Each wave's 128x128 block is 8x8 tiles of v_mfma_f32_16x16x32_bf16, one
// f32x4 accumulator each (256 AGPRs).  A K step (one 64-k stage, ROW_BYTES
// 128, two LDS buffers) is two substeps of 32 k; a substep is 64 MFMAs
// (tile (i, j), i outer), and the step's other instructions sit between them
// at fixed slots, the order pinned by sched_barrier(0) after every slot.  For
// step t in buffer P:
//   substep 0  fragment read r (of 16) of substep 1 after MFMA 8 + 3r; the
//              second half (copies 8-15, A and B alternating) of stage
//              t+1's copies into the other buffer after MFMAs 0, 8, .., 56;
//   substep 1  MFMAs 0-31; wait for stage t+1's copies and cross the
//              barrier; then fragment read r of stage t+1 after MFMA 32 + 2r,
//              and the first half (copies 0-7) of stage t+2's copies into
//              buffer P after MFMAs 32, 36, .., 60.
// Buffer P is free from that barrier on: every wave's reads of it were
// issued before it and completed (lgkmcnt(0)) at it.  Starting the next
// copies there rather than in the next substep 0 gives them up to two
// substeps to land, which is what operands streamed from HBM need (MI355X,
// in one process: 8192^3 +11%, 1024x28672x4096 +12%, MoE layer +10%; the
// 4096^3 case, whose operands stay in the last-level cache, +1%).  The
// barrier sits halfway through the last substep, whose fragments are
// already in registers, so the waves meet with half a substep of MFMAs
// still to issue.
//
// The MFMAs are inline asm with the accumulator tied to the destination
// ("+a").  Left to itself the compiler gives this 8x8 tile's MFMAs a
// destination other than their accumulator input and pays for it with
// hundreds of v_accvgpr moves per iteration.  Inline asm hides the MFMAs from
// the compiler's hazard recognizer, so:
//   - the first substep of the K loop writes the accumulators with srcC = 0
//     (no VALU write of an accumulator precedes an MFMA);
//   - after the loop, explicit wait states (s_nop) separate the last MFMA
//     from the epilogue's VALU reads of the accumulators;
//   - fragment registers are only MFMA sources A and B, read at issue: the
//     LDS reads that overwrite them need no wait states.

struct Acc16 {
  f32x4_t v[8][8];
};

FE2O3_DEVICE void mfma16_acc(f32x4_t& acc, const bf16x8_t& x, const bf16x8_t& y) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(x), "v"(y));
}
FE2O3_DEVICE void mfma16_first(f32x4_t& acc, const bf16x8_t& x, const bf16x8_t& y) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(x), "v"(y));
}

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0]+[15:14], expcnt [6:4],
// lgkmcnt [11:8]); as builtins the compiler's own wait tracking sees them
constexpr int waitcnt_imm(int vmcnt, int lgkmcnt) {
  return (vmcnt & 15) | ((vmcnt >> 4) << 14) | (7 << 4) | (lgkmcnt << 8);
}
constexpr int kWaitVm0Lgkm0 = waitcnt_imm(0, 0);
constexpr int kWaitVm0 = waitcnt_imm(0, 15);
constexpr int kWaitLgkm0 = waitcnt_imm(63, 0);

// Fragments of one substep (32 k): lane l holds k 8(l/16) .. +7 of row
// 16i + l%16 of the wave's 128 A rows (a[i]) and B rows (b[j]).  The
// swizzle of row 16i + r depends on i mod 4, hence four lane offsets per
// operand and substep.
template <int ROW_BYTES>
struct Bf16Frags {
  using G = Geo<ROW_BYTES>;
  static constexpr int kSubsteps = ROW_BYTES / 64;
  bf16x8_t a[8], b[8];
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
        const uint32_t ra = wm * 128u + p * 16u + lr, rb = wn * 128u + p * 16u + lr;
        l.a[s][p] = (wm * 128u + lr) * ROW_BYTES + ((c ^ G::swz(ra)) << 4);
        l.b[s][p] = b_region + (wn * 128u + lr) * ROW_BYTES + ((c ^ G::swz(rb)) << 4);
      }
    return l;
  }
  // Read R (0..15) of substep S from the stage at A_TILE / B_TILE, in the
  // order the MFMAs first use them: a0, b0 .. b7, a1 .. a7.
  template <uint32_t A_TILE, uint32_t B_TILE, int S, int R>
  FE2O3_DEVICE void read(const uint8_t* smem, const Lanes& l) {
    static_assert(R >= 0 && R < 16, "16 reads per substep");
    if constexpr (R == 0) {
      a[0] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][0] + A_TILE);
    } else if constexpr (R <= 8) {
      constexpr int j = R - 1;
      b[j] = *reinterpret_cast<const bf16x8_t*>(smem + l.b[S][j & 3] +
                                                (B_TILE + j * 16u * ROW_BYTES));
    } else {
      constexpr int i = R - 8;
      a[i] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][i & 3] +
                                                (A_TILE + i * 16u * ROW_BYTES));
    }
  }
  template <uint32_t A_TILE, uint32_t B_TILE, int S, int R = 0>
  FE2O3_DEVICE void read_all(const uint8_t* smem, const Lanes& l) {
    if constexpr (R < 16) {
      read<A_TILE, B_TILE, S, R>(smem, l);
      read_all<A_TILE, B_TILE, S, R + 1>(smem, l);
    }
  }
};

// Copy C (0 .. 2*NJ-1: A slot C/2 for even C, B slot C/2 for odd C) of the
// stage at k offset `kbytes` into LDS buffer `buf`.
template <int ROW_BYTES, int STAGES, int C>
FE2O3_DEVICE void copy_one(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br, uint32_t kbytes,
                           uint8_t* smem, uint32_t wave, int buf) {
  using L = Lay<ROW_BYTES, STAGES>;
  constexpr int j = C >> 1;
  const Rows<ROW_BYTES>& rows = (C & 1) ? br : ar;
  const uint32_t tile = (C & 1) ? L::b_region + L::b(buf) : L::a(buf);
  b2l_b128(rsrc(rows.base[j], rows.bytes), smem + tile + (4u * j + wave) * 1024u, rows.voff[j],
           kbytes);
}

// Substep S_ of a K step held in stage buffer P.  FIRST: the K loop's first
// substep (accumulators written, not added to).  k_next / k_next2: k byte
// offsets of the stages one and two ahead (clamped to the last stage).
template <int ROW_BYTES, int STAGES, int P, int S_, bool FIRST>
struct Bf16Substep {
  using G = Geo<ROW_BYTES>;
  using L = Lay<ROW_BYTES, STAGES>;
  using F = Bf16Frags<ROW_BYTES>;
  static constexpr int S = F::kSubsteps;
  static constexpr int NC = 2 * G::kInstPerWave;  // copies per stage and wave (16)
  static constexpr int PN = (P + 1) % STAGES;     // buffer of the next step
  static constexpr bool LAST = S_ + 1 == S;
  // slots
  static constexpr int kBarrierAt = 32;
  static constexpr int kEarly = NC / 2, kEarlyEvery = 4;  // last substep, from the barrier
  static constexpr int kLateEvery = 8;                    // substep 0, from slot 0
  static constexpr int kReadFrom = LAST ? kBarrierAt : 8, kReadEvery = LAST ? 2 : 3;
  static_assert(kBarrierAt + (kEarly - 1) * kEarlyEvery < 64 &&
                    (NC - kEarly - 1) * kLateEvery < 64 && kReadFrom + 15 * kReadEvery < 64,
                "every copy and read has a slot");
  // fragments read here: the next substep's, or in the last substep the next stage's first
  static constexpr uint32_t RA = LAST ? L::a(PN) : L::a(P);
  static constexpr uint32_t RB = LAST ? L::b(PN) : L::b(P);
  static constexpr int RS = LAST ? 0 : S_ + 1;

  template <int I>
  static FE2O3_DEVICE void slot(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br,
                                uint32_t k_next, uint32_t k_next2, uint8_t* smem, uint32_t wave,
                                const typename F::Lanes& ln, F* f, Acc16& acc) {
    if constexpr (I < 64) {
      constexpr int i = I / 8, j = I % 8;
      if constexpr (LAST && I == kBarrierAt) {
        static_assert(STAGES == 2, "the stage waited for holds every outstanding copy");
        __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
        __builtin_amdgcn_s_barrier();
      }
      if constexpr (FIRST && S_ == 0)
        mfma16_first(acc.v[i][j], f[S_ & 1].b[j], f[S_ & 1].a[i]);
      else
        mfma16_acc(acc.v[i][j], f[S_ & 1].b[j], f[S_ & 1].a[i]);
      constexpr int E = I - kBarrierAt;  // early copies: stage t+2 into buffer P
      if constexpr (LAST && E >= 0 && E % kEarlyEvery == 0 && E / kEarlyEvery < kEarly)
        copy_one<ROW_BYTES, STAGES, E / kEarlyEvery>(ar, br, k_next2, smem, wave, P);
      // late copies: the rest of stage t+1 into the other buffer
      if constexpr (S_ == 0 && I % kLateEvery == 0 && I / kLateEvery < NC - kEarly)
        copy_one<ROW_BYTES, STAGES, kEarly + I / kLateEvery>(ar, br, k_next, smem, wave, PN);
      if constexpr (I >= kReadFrom && (I - kReadFrom) % kReadEvery == 0 &&
                    (I - kReadFrom) / kReadEvery < 16)
        f[(S_ + 1) & 1].template read<RA, RB, RS, (I - kReadFrom) / kReadEvery>(smem, ln);
      __builtin_amdgcn_sched_barrier(0);
      slot<I + 1>(ar, br, k_next, k_next2, smem, wave, ln, f, acc);
    }
  }
  static FE2O3_DEVICE void run(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br,
                               uint32_t k_next, uint32_t k_next2, uint8_t* smem, uint32_t wave,
                               const typename F::Lanes& ln, F* f, Acc16& acc) {
    __builtin_amdgcn_sched_barrier(0);
    slot<0>(ar, br, k_next, k_next2, smem, wave, ln, f, acc);
    if constexpr (!LAST)
      Bf16Substep<ROW_BYTES, STAGES, P, S_ + 1, FIRST>::run(ar, br, k_next, k_next2, smem, wave,
                                                            ln, f, acc);
  }
};

// Steps kt .. kt+STAGES-1 in buffers P .. STAGES-1 (TAIL: stop at the last
// step; FIRST: kt is the K loop's first step).
template <int ROW_BYTES, int STAGES, int P, bool TAIL, bool FIRST>
struct Bf16Steps {
  using F = Bf16Frags<ROW_BYTES>;
  static FE2O3_DEVICE uint32_t stage_k(int st, int steps) {
    using G = Geo<ROW_BYTES>;
    return __builtin_amdgcn_readfirstlane((uint32_t)(st < steps ? st : steps - 1) *
                                          (G::kK16 * 2u));
  }
  static FE2O3_DEVICE void run(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br, int kt,
                               int steps, uint8_t* smem, uint32_t wave,
                               const typename F::Lanes& ln, F* f, Acc16& acc) {
    if (TAIL && kt >= steps) return;
    Bf16Substep<ROW_BYTES, STAGES, P, 0, FIRST && P == 0>::run(
        ar, br, stage_k(kt + 1, steps), stage_k(kt + 2, steps), smem, wave, ln, f, acc);
    if constexpr (P + 1 < STAGES)
      Bf16Steps<ROW_BYTES, STAGES, P + 1, TAIL, FIRST>::run(ar, br, kt + 1, steps, smem, wave,
                                                            ln, f, acc);
  }
};

// K loop over k16 bf16 elements per row (a multiple of Geo::kK16, at least
// one stage); every accumulator is written (no zeroing beforehand).
template <int ROW_BYTES, int STAGES>
FE2O3_DEVICE void mainloop_bf16(const Rows<ROW_BYTES>& ar, const Rows<ROW_BYTES>& br,
                                uint32_t k16, uint8_t* smem, Acc16& acc) {
  using G = Geo<ROW_BYTES>;
  using L = Lay<ROW_BYTES, STAGES>;
  using F = Bf16Frags<ROW_BYTES>;
  using Sub = Bf16Substep<ROW_BYTES, STAGES, 0, 0, false>;
  static_assert(ROW_BYTES == 128 && STAGES == 2, "the slot plan is for two 64-k stages");
  constexpr int NJ = G::kInstPerWave;
  const int steps = (int)(k16 / G::kK16);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const typename F::Lanes ln = F::lanes(L::b_region);
  // stage 0 whole, and stage 1's early copies (those a step -1 would issue)
  issue_part<ROW_BYTES, 0, NJ>(ar, 0u, smem, L::a(0), wave);
  issue_part<ROW_BYTES, 0, NJ>(br, 0u, smem, L::b_region + L::b(0), wave);
  const uint32_t k1 = Bf16Steps<ROW_BYTES, STAGES, 0, false, false>::stage_k(1, steps);
  issue_part<ROW_BYTES, 0, Sub::kEarly / 2>(ar, k1, smem, L::a(1), wave);
  issue_part<ROW_BYTES, 0, Sub::kEarly / 2>(br, k1, smem, L::b_region + L::b(1), wave);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(Sub::kEarly, 0));  // stage 0 landed
  __builtin_amdgcn_s_barrier();
  F f[2];
  f[0].template read_all<L::a(0), L::b(0), 0>(smem, ln);
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  int kt = 0;
  if (steps >= STAGES) {
    Bf16Steps<ROW_BYTES, STAGES, 0, false, true>::run(ar, br, 0, steps, smem, wave, ln, f, acc);
    for (kt = STAGES; kt + STAGES <= steps; kt += STAGES)
      Bf16Steps<ROW_BYTES, STAGES, 0, false, false>::run(ar, br, kt, steps, smem, wave, ln, f,
                                                         acc);
    if (kt < steps)  // fewer than STAGES steps left; they start in buffer 0
      Bf16Steps<ROW_BYTES, STAGES, 0, true, false>::run(ar, br, kt, steps, smem, wave, ln, f,
                                                        acc);
  } else {
    Bf16Steps<ROW_BYTES, STAGES, 0, true, true>::run(ar, br, 0, steps, smem, wave, ln, f, acc);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the last steps' early copies (of clamped stages nobody reads) land before
  // the workgroup can end and its LDS be handed to another
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  // wait states between the last MFMA's accumulator write and the VALU reads
  // that follow (an 8-pass MFMA needs at most 18); every accumulator then
  // passes through an empty asm, so no copy of one out of its AGPRs (the
  // epilogue's v_accvgpr_read) can be placed ahead of the wait states
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+a"(acc.v[i][j]));
  __builtin_amdgcn_sched_barrier(0);
}

// Output coordinates of accumulator (i, j, e) of this lane: tile row
// wm*128 + 16i + lane%16, tile column wn*128 + 16j + 4(lane/16) + e.  The
// lane and wave come from mbcnt and a scalar, so nothing derived from
// threadIdx stays live across the K loop.
FE2O3_DEVICE uint32_t acc16_row0() {
  const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  return (wave >> 1) * 128u + (lane & 15u);
}
FE2O3_DEVICE uint32_t acc16_col0() {
  const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  return (wave & 1u) * 128u + 4u * (lane >> 4);
}

FE2O3_DEVICE void store_bf16(const Acc16& acc, uint16_t* c_tile, uint64_t ldc) {
  const uint32_t row0 = acc16_row0(), col0 = acc16_col0();
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x2_t packed;
      packed[0] = pack_bf16x2(acc.v[i][j][0], acc.v[i][j][1]);
      packed[1] = pack_bf16x2(acc.v[i][j][2], acc.v[i][j][3]);
      *reinterpret_cast<u32x2_t*>(c_tile + (uint64_t)(row0 + 16u * i) * ldc + col0 + 16u * j) =
          packed;
    }
}

}  // namespace gemm_pipe
