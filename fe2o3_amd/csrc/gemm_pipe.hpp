// gemm_pipe.hpp -- multi-stage 256x256 MFMA GEMM pipeline for gfx950.
//
// Workgroup: 256 threads = 4 waves in 2x2, each wave 128x128 as 4x4
// v_mfma_f32_32x32x16_bf16 tiles (D = B_frag x A_frag), accumulators in
// AGPRs.  Parameters:
//   ROW_BYTES  bytes of k per tile row per stage (128: 64 bf16; 64: 32 bf16)
//   STAGES     LDS stages in flight (STAGES * 2 * 256 * ROW_BYTES bytes)
//
// Global -> LDS.  Operand tiles are copied with buffer_load_dwordx4 ... lds
// (16 bytes per lane straight into LDS).  Each operand has a buffer resource
// per load slot (wave-uniform) and each thread a fixed byte offset per slot;
// the k offset of a stage is a scalar, and the LDS destination (M0) is
// scalar too, so a copy costs no VALU.  Stage kt+STAGES-1 is copied while
// stage kt is consumed; with two stages the copies are spread over the
// first half of the step's substeps, which leaves the second half for them
// to land.  One s_waitcnt vmcnt + one barrier per stage publishes every
// wave's copies.
//
// LDS layout.  The A tiles of all stages come first, then the B tiles (A of
// stage p at p * T, B at (STAGES + p) * T, T = 256 * ROW_BYTES).  16-byte
// chunk c of row r is stored at position c ^ swz(r):
//   ROW_BYTES 128: swz(r) = (r ^ (r >> 3)) & 7
//   ROW_BYTES  64: swz(r) = ((r >> 1) ^ (r >> 3)) & 3
// Both keep the MFMA operand reads (32 consecutive rows, one chunk) free of
// bank conflicts (measured: SQ_LDS_BANK_CONFLICT = 0).
//
// Fragment reads.  The K loop is unrolled over the STAGES buffers, so the
// stage, tile and 32-row block offsets of every ds_read are compile-time
// immediates; the per-lane part depends only on (substep, row parity) and is
// computed once before the loop (Mma::Lanes).
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

// bf16 operands: substeps of 16 k (32 bytes of each row) per stage.  Lane l
// reads row 32i + l%32 of its wave's half, chunk 2s + l/32; the swizzle of
// row 32i + r depends on i mod 2 only.
template <int ROW_BYTES>
struct MmaBf16 {
  using G = Geo<ROW_BYTES>;
  static constexpr int kSubsteps = ROW_BYTES / 32;
  struct Frags {
    bf16x8_t a[4], b[4];
  };
  struct Lanes {
    uint32_t a[kSubsteps][2], b[kSubsteps][2];
  };
  static FE2O3_DEVICE Lanes lanes(uint32_t b_region) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t lr = lane & 31u, g = lane >> 5;
    Lanes l;
#pragma unroll
    for (int s = 0; s < kSubsteps; ++s)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint32_t c = 2u * s + g;
        const uint32_t ra = wm * 128u + p * 32u + lr, rb = wn * 128u + p * 32u + lr;
        l.a[s][p] = (wm * 128u + lr) * ROW_BYTES + ((c ^ G::swz(ra)) << 4);
        l.b[s][p] = b_region + (wn * 128u + lr) * ROW_BYTES + ((c ^ G::swz(rb)) << 4);
      }
    return l;
  }
  template <uint32_t A_TILE, uint32_t B_TILE, int S>
  static FE2O3_DEVICE void load(const uint8_t* smem, const Lanes& l, Frags& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f.a[i] = *reinterpret_cast<const bf16x8_t*>(smem + l.a[S][i & 1] +
                                                  (A_TILE + i * 32u * ROW_BYTES));
      f.b[i] = *reinterpret_cast<const bf16x8_t*>(smem + l.b[S][i & 1] +
                                                  (B_TILE + i * 32u * ROW_BYTES));
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
// add a(p) or b(p) (plus the 32-row block offset) as ds_read immediates; the
// B region's base is folded into the per-lane B offsets, so every immediate
// stays below 64 KiB.
template <int ROW_BYTES, int STAGES>
struct Lay {
  using G = Geo<ROW_BYTES>;
  static constexpr uint32_t b_region = (uint32_t)STAGES * G::kTileBytes;
  static constexpr uint32_t a(int p) { return (uint32_t)p * G::kTileBytes; }
  static constexpr uint32_t b(int p) { return (uint32_t)p * G::kTileBytes; }
  static_assert((STAGES - 1) * G::kTileBytes + 3 * 32 * ROW_BYTES < 65536,
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
                               const typename Mma::Lanes& ln, typename Mma::Frags* f, Acc& acc) {
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
                               const typename Mma::Lanes& ln, typename Mma::Frags* f, Acc& acc) {
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
                           uint8_t* smem, Acc& acc) {
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
