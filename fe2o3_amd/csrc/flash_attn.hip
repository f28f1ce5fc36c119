// flash_attn.hip -- flash-attention forward for gfx950.
//
// 1. The reference's exact profile (examples/flash_attention_v1/src/kernel.rs
//    :36-169): causal, B1/H1/N8/D16, f32, scale 0.25, one wave64, lane l owns
//    outputs 2l and 2l+1, sequential strict-f32 dot products and the online
//    max/sum recurrence m' = max(m, s); w_prev = exp(m - m');
//    w = exp(s - m'); l = l*w_prev + w; n = n*w_prev + v*w (kernel.rs:56-113),
//    exp = OCML expf as the reference's DeviceMath::exp_f32.
//
// 2. The BASELINE shape: Q, K, V, O bf16 [B, H, S, 128], fp32 online softmax
//    statistics, optional causal mask, LSE output.  Per workgroup: one (b, h)
//    and 128 query rows; 4 waves x 32 query rows; K/V tiles of 64 keys,
//    double-buffered in LDS.
//    * S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (K tile rows as the first
//      operand, the wave's Q rows -- held in registers for the whole loop --
//      as the second), so lane l owns query row l%32 and 16 of the 32 keys of
//      each key block; the other 16 sit in lane l^32.  Row max and row sum are
//      in-lane reductions plus one v_permlane32_swap.
//    * Softmax in the exp2 domain: p = exp2(s*c - m) with c = scale*log2(e)
//      folded into one FMA before v_exp_f32.  The tile's p are computed
//      against the running reference m first; only when some lane's sum of
//      them is not <= 2^8 (every p is at most that sum; the first tile,
//      against m = -inf, gives +inf or NaN) does the tile take its row max,
//      raise m, rescale O and l by exp2(m_old - m_new) and compute its p
//      again.  Most tiles thus skip both the max and the 64 rescale
//      multiplies per lane; p stays <= 256, exact enough in bf16 and fp32.
//    * O^T += V^T P^T: P (bf16) is the second operand straight from the S
//      registers; the V^T operand is read from the row-major V tile with
//      ds_read_b64_tr_b16 (the gfx950 transposing LDS read), two reads per
//      MFMA, so V needs no register transpose.
//    * K and V tiles go global -> LDS with 16-byte buffer loads to LDS (one
//      fixed VGPR offset per thread, tile offsets scalar), chunks
//      XOR-permuted per row against bank conflicts.  The next tile's loads
//      are spread one per two S^T MFMAs rather than issued as a burst
//      (+3%).
//    * Both MFMA runs alternate accumulators (S^T: the two key blocks; PV:
//      the four d blocks), and each LDS operand is read two MFMAs ahead of
//      its MFMA (+3% over the scheduler's read-just-before-use).
//    * Causal: a workgroup runs query tiles r and nq-1-r of one head in
//      turn, so every workgroup does nq+1 key tiles; a wave skips the
//      MFMAs of key tiles that lie entirely above its rows and masks the
//      diagonal tile.
#include "common.hpp"
#include "internal.hpp"
#include "profiles.hpp"

namespace {

using namespace fe2o3;

// ---- exact profile ---------------------------------------------------------------------
constexpr int P_N = fe2o3_profiles::kFlashN, P_D = fe2o3_profiles::kFlashD;

// The profile's arithmetic and its rejection of non-finite inputs are
// fe2o3_profiles::flash_profile (profiles.hpp), shared with the code object
// the protected lifecycle loads.
__global__ void __launch_bounds__(64) flash_profile_kernel(const float* __restrict__ q,
                                                           const float* __restrict__ k,
                                                           const float* __restrict__ v,
                                                           float* __restrict__ out,
                                                           uint32_t* __restrict__ status) {
  fe2o3_profiles::flash_profile(q, k, v, out, status);
}

// ---- BASELINE-shape kernel -------------------------------------------------------------------
constexpr int D = 128;         // head dim
constexpr int BQ = 128;        // query rows per workgroup
constexpr int WAVES = BQ / 32; // one wave per 32 query rows
constexpr int THREADS = WAVES * 64;
static_assert(16 % WAVES == 0 && (4 * WAVES) % 16 == 0, "tile copies split evenly over the waves");
constexpr int BKV = 64;        // keys per tile
constexpr int TILE_BYTES = BKV * D * 2;     // 16 KiB: 64 rows of 256 B
constexpr int STAGE_BYTES = 2 * TILE_BYTES; // K tile then V tile
constexpr int SMEM_BYTES = 2 * STAGE_BYTES; // 64 KiB: two stages
constexpr float RESCALE_SLACK = 8.0f;       // log2 units: p may reach 2^8 before a rescale
constexpr float kLazyBound = 256.0f;          // 2^RESCALE_SLACK

// Both tiles are [64 keys][128 d] bf16 rows of 256 B holding 16 chunks of
// 16 B.  K chunk c of row r sits at c ^ (r & 15): the S^T operand reads (32
// consecutive rows, one chunk) are conflict-free.  V chunk c of row r sits at
// c ^ f(r & 3), f(j) = 2j ^ 4j: the transposing reads below touch 4
// consecutive rows x 2 chunks per 16 lanes and 4 rows x 4 chunks per 32
// lanes; f puts them in 8 distinct chunks mod 8 and 16 distinct chunks mod
// 16, so they are conflict-free whether the LDS serves 128 or 256 bytes of
// a read per cycle.
FE2O3_DEVICE uint32_t swz_k(uint32_t r) { return r & 15u; }
FE2O3_DEVICE uint32_t swz_v(uint32_t r) { return ((r & 3u) << 1) ^ ((r & 3u) << 2); }

// K and V of one head are read through buffer resources (base = the head,
// range = its seq * 256 bytes).  A partial last key tile (seq not a multiple
// of 64) has rows past seq: their loads take a VGPR offset past the range
// (the range check covers the VGPR offset, not the scalar tile offset), so
// the LDS-direct load writes zeros into the tile and the masked keys' P = 0
// meets V = 0 there, never a value of the next head, of another tile or of
// memory past the tensor.  One tile is 16 loads of 1 KiB (4 rows of
// 256 B), wave w issuing loads j = 0 .. 16/WAVES - 1 of rows
// 4 (WAVES j + w) .. +3.  The chunk swizzles depend on the row mod 16 only,
// and 4 WAVES is a multiple of 16, so a thread's byte offset within the tile
// is the same for every j up to the row-group step of 1024 WAVES bytes: one
// fixed VGPR offset per thread, the rest is scalar.
FE2O3_DEVICE __amdgpu_buffer_rsrc_t head_rsrc(const uint16_t* base, uint32_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, the raw-buffer setting for CDNA
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, (int)bytes,
                                           0x00020000);
}

template <bool IS_V>
FE2O3_DEVICE uint32_t tile_voffset() {
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t row = 4u * w + (lane >> 4);
  const uint32_t chunk = (lane & 15u) ^ (IS_V ? swz_v(row) : swz_k(row));
  return row * 256u + chunk * 16u;
}

constexpr int kLoadsPerTile = 16 / WAVES;  // 1 KiB loads per wave and tile
// LDS operand fragments are read this many MFMAs ahead of their MFMA (2, 4
// and 6 run within 1% of each other; reading each just before its MFMA, the
// scheduler's own choice, ran 3% slower)
constexpr int kAhead = 2;
// __builtin_amdgcn_sched_group_barrier instruction classes
constexpr int kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100;
static_assert(16 % (2 * kLoadsPerTile) == 0, "a tile's copies spread evenly over 16 MFMAs");

// past any head's range (seq * 256 < 2^31)
constexpr uint32_t kKeyOutOfRange = 0x80000000u;

// Load j of this thread's chunk of the tile at byte tile_byte.  RAGGED
// (seq not a multiple of 64): a chunk of a row at or past the head's `bytes`
// (seq * 256) loads zeros; otherwise every row of every tile is in range.
template <bool RAGGED>
FE2O3_DEVICE void copy_load(__amdgpu_buffer_rsrc_t src, uint32_t voff, uint32_t tile_byte,
                            uint32_t bytes, uint8_t* lds, uint32_t wave, int j) {
  const uint32_t soff = tile_byte + 1024u * WAVES * j;
  const uint32_t off = !RAGGED || voff + soff < bytes ? voff : kKeyOutOfRange;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (lds_void_t*)(lds + (WAVES * j + wave) * 1024u),
                                           16, off, soff, 0, 0);
}

template <bool RAGGED>
FE2O3_DEVICE void issue_tile(__amdgpu_buffer_rsrc_t src, uint32_t voff, uint32_t tile_byte,
                             uint32_t bytes, uint8_t* lds, uint32_t wave) {
#pragma unroll
  for (int j = 0; j < kLoadsPerTile; ++j)
    copy_load<RAGGED>(src, voff, tile_byte, bytes, lds, wave, j);
}

// V^T operand of one O^T MFMA (d rows 32*db.., keys of half h of 32-key block
// kb) with ds_read_b64_tr_b16.  Within each 16-lane group the instruction
// hands lane i the element M[4e + i/4][i%4] (e = 0..3) of the 16 x 4 block
// whose row r is the 4 bf16 at lane r's address.  Lane i = l%16 of group
// G = l/16 addresses V[kb0 + i/4][dg + 4*(i%4)] with dg = 32*db + 16*(G&1),
// so it receives V[kb0 + e][dg + i]: one d per lane (l%32 over the half
// wave) and 4 consecutive keys kb0 = 32kb + 16h + 4(G>>1) (+8 for the second
// read) -- the keys the S^T registers hold for MFMA k-slots 8(l/32) + 0..7.
FE2O3_DEVICE bf16x8_t read_vt(const uint8_t* vt, uint32_t db, uint32_t kb, uint32_t h) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t G = lane >> 4, i = lane & 15u;
  const uint32_t d = db * 32u + 16u * (G & 1u) + 4u * (i & 3u);
  const uint32_t key = kb * 32u + 16u * h + 4u * (G >> 1) + (i >> 2);
  const uint32_t off0 = key * 256u + (((d >> 3) ^ swz_v(key)) << 4) + (d & 7u) * 2u;
  const uint32_t off1 = (key + 8u) * 256u + (((d >> 3) ^ swz_v(key + 8u)) << 4) + (d & 7u) * 2u;
  const bf16x4_t r0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(vt + off0));
  const bf16x4_t r1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(vt + off1));
  return __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
}

// RAGGED: seq is not a multiple of 64, so the last key tile is partial and
// its copies mask the rows past seq (copy_load).
template <bool CAUSAL, bool RAGGED = false>
__global__ void __launch_bounds__(THREADS, 8 / WAVES) flash_fwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, float* __restrict__ lse,
    uint32_t seq, uint32_t heads, float scale_log2, uint32_t paired, uint32_t xcds) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t lr = lane & 31u, g = lane >> 5;
  // Workgroup order.  Workgroup id i runs on XCD i % xcds (the device's XCD
  // count, 8 on MI355X).  When xcds divides heads the ids are laid out so
  // that XCD x walks heads x, x + xcds, x + 2 xcds, ... and, for each, all of
  // its query tiles back to back: the tiles of one head run together on one
  // XCD and share their K/V through that XCD's L2.  Within a head the causal
  // order is heaviest tile (most key tiles) first.
  // With `paired`, a workgroup runs two query tiles of one head, r then
  // nq-1-r, so every causal workgroup does the same nq+1 key tiles.
  const uint32_t nq = (seq + BQ - 1u) / BQ;  // the last tile may be partial
  const uint32_t per_head = paired ? nq / 2u : nq;
  uint32_t bh, rank;
  if (xcds > 1u && heads % xcds == 0u) {
    const uint32_t xcd = blockIdx.x % xcds, slot = blockIdx.x / xcds;
    bh = (slot / per_head) * xcds + xcd;
    rank = slot % per_head;
  } else {
    bh = blockIdx.x / per_head;
    rank = blockIdx.x % per_head;
  }
  const uint64_t head = (uint64_t)bh * seq * D;
  const uint16_t* qh = q + head;
  const uint16_t* kh = k + head;
  const uint16_t* vh = v + head;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(w);  // wave-uniform
  const uint32_t head_bytes = seq * (uint32_t)(D * 2);
  const __amdgpu_buffer_rsrc_t ksrc = head_rsrc(kh, head_bytes);
  const __amdgpu_buffer_rsrc_t vsrc = head_rsrc(vh, head_bytes);
  const uint32_t k_off = tile_voffset<false>(), v_off = tile_voffset<true>();
  for (uint32_t item = 0; item < (paired ? 2u : 1u); ++item) {
  // heaviest first: the higher query tile of the pair, or rank order reversed
  const uint32_t qt = paired ? (item == 0u ? nq - 1u - rank : rank)
                             : (CAUSAL ? nq - 1u - rank : rank);
  const uint32_t q_row0 = qt * BQ + w * 32u;  // first query row of this wave
  const uint32_t my_q = q_row0 + lr;
  // rows past seq (a partial last tile) compute on row seq-1 and store nothing
  const uint32_t q_load = my_q < seq ? my_q : seq - 1u;

  // Q fragments (second MFMA operand): lane holds row my_q, d = 16*ds + 8*g .. +7
  bf16x8_t qf[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds)
    qf[ds] = *reinterpret_cast<const bf16x8_t*>(qh + (uint64_t)q_load * D + ds * 16 + g * 8);

  f32x16_t acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
  float m_ref = -INFINITY;  // exp reference, log2 domain (>= running max - slack)
  float l_run = 0.0f;       // this lane's partial row sum of exp2(s*c - m_ref)

  const uint32_t kv_tiles = (seq + BKV - 1u) / BKV;
  const uint32_t n_kv = CAUSAL ? min((qt + 1u) * (BQ / BKV), kv_tiles) : kv_tiles;
  issue_tile<RAGGED>(ksrc, k_off, 0u, head_bytes, smem, wave);
  issue_tile<RAGGED>(vsrc, v_off, 0u, head_bytes, smem + TILE_BYTES, wave);
  wait_vmcnt0();
  lds_barrier();

  for (uint32_t j = 0; j < n_kv; ++j) {
    const uint8_t* cur = smem + (j & 1u) * STAGE_BYTES;
    uint8_t* nxt = smem + ((j + 1u) & 1u) * STAGE_BYTES;
    // next tile's k offset; the last tile copies itself again (into a buffer
    // nobody reads) so that every tile issues the same copies
    const uint32_t nt =
        __builtin_amdgcn_readfirstlane((j + 1u < n_kv ? j + 1u : j) * (uint32_t)TILE_BYTES);
    const uint32_t key0 = j * BKV;
    // keys key0..key0+63 vs. rows q_row0..q_row0+31
    const bool active = !CAUSAL || key0 <= q_row0 + 31u;
    if (!active) {
      issue_tile<RAGGED>(ksrc, k_off, nt, head_bytes, nxt, wave);
      issue_tile<RAGGED>(vsrc, v_off, nt, head_bytes, nxt + TILE_BYTES, wave);
    }
    if (active) {
      // S^T = K Q^T : two 32-key blocks.  MFMA i (0..15) is key block kb = i%2
      // at d slice ds = i/2, so consecutive MFMAs feed the two accumulators
      // in turn (each accumulator still sums its d slices in order).  Each K
      // fragment is read kAhead MFMAs before its MFMA, and the group
      // barriers keep that order (read, MFMA, copy) against the
      // scheduler, which otherwise reads each fragment just before its use
      // and waits for it there.  The next tile's copies go one per two
      // MFMAs (K loads, then V).
      f32x16_t s[2];
      constexpr int kCopyEvery = 16 / (2 * kLoadsPerTile);
      auto kread = [&](int i) {
        const uint32_t krow = (uint32_t)(i & 1) * 32u + lr;
        const uint32_t c = 2u * (uint32_t)(i >> 1) + g;
        return *reinterpret_cast<const bf16x8_t*>(cur + krow * 256u + ((c ^ swz_k(krow)) << 4));
      };
      bf16x8_t kf[16];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) kf[i] = kread(i);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kAhead, 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int ds = i >> 1, kb = i & 1;
        if (i + kAhead < 16) kf[i + kAhead] = kread(i + kAhead);
        s[kb] = ds == 0 ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i], qf[0], f32x16_t{}, 0, 0, 0)
                        : __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i], qf[ds], s[kb], 0, 0, 0);
        if (i % kCopyEvery == 0) {
          const int n = i / kCopyEvery, jj = n % kLoadsPerTile;
          const bool is_v = n >= kLoadsPerTile;
          copy_load<RAGGED>(is_v ? vsrc : ksrc, is_v ? v_off : k_off, nt, head_bytes,
                    nxt + (is_v ? TILE_BYTES : 0), wave, jj);
        }
        if (i + kAhead < 16) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (i % kCopyEvery == 0) __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
      }
      // keys past seq (the partial last tile; causal rows below seq mask
      // them as future keys)
      if (!CAUSAL && key0 + (uint32_t)BKV > seq) {
        // key = key0 + 4g + c(kb, e) is past seq when c >= lim
        const int lim = (int)(seq - key0) - 4 * (int)g;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (kb * 32 + 8 * (e >> 2) + (e & 3) >= lim) s[kb][e] = -INFINITY;
      }
      // mask the diagonal tile
      if (CAUSAL && key0 + 63u > q_row0) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const uint32_t key = key0 + kb * 32u + 8u * (e >> 2) + 4u * g + (e & 3);
            if (key > my_q) s[kb][e] = -INFINITY;
          }
      }
      bf16x8_t pf[2][2];
      float psum;
      auto probabilities = [&] {
        psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float pv[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
              pv[jj] =
                  __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][h * 8 + jj], scale_log2, -m_ref));
              psum += pv[jj];
            }
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) pf[kb][h][jj] = (__bf16)pv[jj];
          }
      };
      probabilities();
      // The reference is raised only when some lane's sum of this tile is not
      // <= 2^slack: every p is at most that sum, and the first tile (reference
      // -inf) gives +inf or NaN.  Then the row's tile max, the rescale, and
      // this tile's probabilities again.
      if (__any(!(psum <= kLazyBound))) {
        float mloc = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, s[kb][e]);
        mloc = fmaxf(mloc, swap_half(mloc)) * scale_log2;
        const float m_new = fmaxf(m_ref, mloc);
        const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
        m_ref = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[db][e] *= alpha;
        probabilities();
      }
      l_run += psum;
      // O^T += V^T P^T.  Each SIMD runs one wave of each of two workgroups; a
      // wave raises its issue priority while it issues these MFMAs, so the
      // matrix core is fed first and the other wave's softmax fills the gaps
      // (measured: +3.6% over not raising it, and about as much over raising
      // it for the S^T MFMAs as well or instead).
      const uint8_t* vt = cur + TILE_BYTES;
      __builtin_amdgcn_s_setprio(1);
      // MFMA i (0..15) is d block db = i%4 of key half (kb = i/8, h = (i/4)%2):
      // consecutive MFMAs update different accumulators, each accumulator
      // still sums its key halves in order.  The V^T operand (two
      // transposing reads) is read kAhead MFMAs ahead, as the K fragments.
      auto vread = [&](int i) {
        return read_vt(vt, (uint32_t)(i & 3), (uint32_t)(i >> 3), (uint32_t)((i >> 2) & 1));
      };
      bf16x8_t vf[16];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) vf[i] = vread(i);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * kAhead, 1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i + kAhead < 16) vf[i + kAhead] = vread(i + kAhead);
        const int db = i & 3, kb = i >> 3, h = (i >> 2) & 1;
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[i], pf[kb][h], acc[db], 0, 0, 0);
        if (i + kAhead < 16) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 1);
      }
      __builtin_amdgcn_s_setprio(0);
    }
    wait_vmcnt0();
    lds_barrier();
  }

  // finalize: full row sum across the lane pair, normalize, store
  const float l_tot = l_run + swap_half(l_run);
  const float inv = 1.0f / l_tot;
  uint16_t* oh = o + head + (uint64_t)my_q * D;
  if (my_q < seq) {
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const uint32_t d = db * 32u + 8u * qd + 4u * g;
      u32x2_t packed;
      packed[0] = pack_bf16x2(acc[db][4 * qd + 0] * inv, acc[db][4 * qd + 1] * inv);
      packed[1] = pack_bf16x2(acc[db][4 * qd + 2] * inv, acc[db][4 * qd + 3] * inv);
      *reinterpret_cast<u32x2_t*>(oh + d) = packed;
    }
  }
  if (lse != nullptr && g == 0 && my_q < seq) {
    // natural-log statistic: max(s)*scale + ln(sum) = (m_ref + log2(sum)) * ln 2
    lse[(uint64_t)bh * seq + my_q] = (m_ref + __log2f(l_tot)) * 0.69314718055994531f;
  }
  }  // item
}

// kernels behind each entry point (fe2o3_kernel_resources)
const fe2o3_host::KernelRegistrar kRegistered[] = {
    fe2o3_host::KernelRegistrar({"fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1", "flash_profile_kernel", (const void*)flash_profile_kernel, 64, 0}),
    fe2o3_host::KernelRegistrar({"fe2o3_flash_attention_fwd", "flash_fwd_kernel<false>", (const void*)flash_fwd_kernel<false>, THREADS, SMEM_BYTES}),
    fe2o3_host::KernelRegistrar({"fe2o3_flash_attention_fwd", "flash_fwd_kernel<true>", (const void*)flash_fwd_kernel<true>, THREADS, SMEM_BYTES}),
    fe2o3_host::KernelRegistrar({"fe2o3_flash_attention_fwd", "flash_fwd_kernel<false, ragged>", (const void*)flash_fwd_kernel<false, true>, THREADS, SMEM_BYTES}),
    fe2o3_host::KernelRegistrar({"fe2o3_flash_attention_fwd", "flash_fwd_kernel<true, ragged>", (const void*)flash_fwd_kernel<true, true>, THREADS, SMEM_BYTES})};

}  // namespace

extern "C" {

int32_t fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1(const float* q, uint64_t q_len,
                                                          const float* k, uint64_t k_len,
                                                          const float* v, uint64_t v_len,
                                                          float* output, uint64_t output_len,
                                                          void* stream) {
  FE2O3_ENTRY("fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1");
  const uint64_t n = P_N * P_D;
  if (q_len != n || k_len != n || v_len != n || output_len != n) return FE2O3_ERR_LENGTH;
  if (!q || !k || !v || !output) return FE2O3_ERR_NULL;
  uint32_t* status = fe2o3_host::status_word();
  if (status == nullptr) return (int32_t)hipErrorInvalidSymbol;
  flash_profile_kernel<<<1, 64, 0, (hipStream_t)stream>>>(q, k, v, output, status);
  return fe2o3_host::after_launch();
}

int32_t fe2o3_flash_attention_fwd(const uint16_t* q, uint64_t q_len, const uint16_t* k,
                                  uint64_t k_len, const uint16_t* v, uint64_t v_len, uint16_t* o,
                                  uint64_t o_len, float* lse, uint64_t lse_len, uint32_t batch,
                                  uint32_t heads, uint32_t seq, uint32_t head_dim, int32_t causal,
                                  float scale, void* stream) {
  FE2O3_ENTRY("fe2o3_flash_attention_fwd");
  if (head_dim != D) return FE2O3_ERR_SHAPE;
  const uint64_t bh = (uint64_t)batch * heads;
  const uint64_t n = bh * seq * head_dim;
  if (q_len != n || k_len != n || v_len != n || o_len != n) return FE2O3_ERR_LENGTH;
  if (lse != nullptr && lse_len != bh * seq) return FE2O3_ERR_LENGTH;
  if (n == 0) return FE2O3_OK;
  if (bh > 0xffffffffu) return FE2O3_ERR_SHAPE;
  // K/V of one head are addressed through a 32-bit buffer range
  if ((uint64_t)seq * D * 2 > 0x7fffffffu) return FE2O3_ERR_SHAPE;
  if (!q || !k || !v || !o) return FE2O3_ERR_NULL;
  if ((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) & 15u) != 0)
    return FE2O3_ERR_ALIGNMENT;
  if (!(scale > 0.0f) || !__builtin_isfinite(scale)) return FE2O3_ERR_SHAPE;
  const float scale_log2 = scale * 1.4426950408889634f;
  static const int32_t lds_rc = fe2o3_host::set_dynamic_lds(
      {(const void*)flash_fwd_kernel<true>, (const void*)flash_fwd_kernel<false>,
       (const void*)flash_fwd_kernel<true, true>, (const void*)flash_fwd_kernel<false, true>},
      SMEM_BYTES);
  if (lds_rc != FE2O3_OK) return lds_rc;
  // one linear workgroup id per (query tile, batch*head); see the kernel
  // causal: pairs of query tiles per workgroup (every workgroup the same
  // work) when the tile count is even; non-causal tiles are equal already
  const uint32_t nq = (seq + BQ - 1u) / BQ;  // query tiles per head, the last maybe partial
  const uint32_t paired = causal && nq % 2u == 0u ? 1u : 0u;
  const uint64_t wgs = (uint64_t)nq / (paired ? 2u : 1u) * bh;
  if (wgs > 0x7fffffffu) return FE2O3_ERR_SHAPE;
  tile_plan::Topology topo;
  const int32_t topo_rc = fe2o3_host::device_topology(&topo);
  if (topo_rc != FE2O3_OK) return topo_rc;
  const dim3 grid((unsigned)wgs);
  hipStream_t s = (hipStream_t)stream;
  const bool ragged = seq % BKV != 0u;  // a partial last key tile
  if (causal && ragged)
    flash_fwd_kernel<true, true><<<grid, THREADS, SMEM_BYTES, s>>>(
        q, k, v, o, lse, seq, (uint32_t)bh, scale_log2, paired, topo.xcds);
  else if (causal)
    flash_fwd_kernel<true><<<grid, THREADS, SMEM_BYTES, s>>>(
        q, k, v, o, lse, seq, (uint32_t)bh, scale_log2, paired, topo.xcds);
  else if (ragged)
    flash_fwd_kernel<false, true><<<grid, THREADS, SMEM_BYTES, s>>>(
        q, k, v, o, lse, seq, (uint32_t)bh, scale_log2, paired, topo.xcds);
  else
    flash_fwd_kernel<false><<<grid, THREADS, SMEM_BYTES, s>>>(
        q, k, v, o, lse, seq, (uint32_t)bh, scale_log2, paired, topo.xcds);
  return fe2o3_host::after_launch();
}

}  // extern "C"
